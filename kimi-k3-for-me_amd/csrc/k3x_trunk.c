/* k3x_trunk.c - host side of the trunk's bf16 products (include/k3x_trunk.h): upload and
 * tiling of a matrix, argument checks, the workspace, the host-pointer form.  T <= 8 rows
 * run the GEMV on the tiled copy; more rows run a plain GEMM on hipBLASLt over a row-major
 * copy (k3x_blas.cpp; fp32 rows as two bf16 GEMMs, hi then lo accumulated), or the
 * hand-written dense GEMM over the tiled copy when the library offers no kernel. */
#include "k3x_internal.h"
#include "../../include/k3x_trunk.h"

#include <hip/hip_runtime_api.h>
#include <stdlib.h>

#define TRUNK_RETIRED 16   /* workspaces outgrown, kept until destroy */

struct k3x_trunk {
    int       device, in, out;
    uint16_t *w;              /* tiled bf16 [out][in]                        */
    uint16_t *wr;             /* row-major bf16 [out][in] (the library GEMM)  */
    int       blas;           /* the library GEMM is available               */
    uint16_t *planes;         /* workspace for T > K3X_DECODE_MAX_T           */
    size_t    planes_bytes;
    uint16_t *retired[TRUNK_RETIRED];   /* earlier workspaces: a graph recorded over
                                           one of them still reads it            */
    int       nretired;
    float    *hx, *hy;        /* device staging of the host-pointer form      */
    size_t    hcap;           /* floats of each                               */
};

/* The workspace for `need` bytes: grown (at least doubled, so few generations exist)
 * outside capture only; the outgrown one is retired, not freed, since a graph captured
 * over it may replay later. */
static int trunk_workspace(k3x_trunk *t, size_t need, void *stream)
{
    if (need <= t->planes_bytes) return 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) return K3X_E_HIP;
    if (cs != hipStreamCaptureStatusNone) return K3X_E_SHAPE;
    if (t->planes && t->nretired == TRUNK_RETIRED) return K3X_E_NOMEM;
    if (need < 2 * t->planes_bytes) need = 2 * t->planes_bytes;
    if (need > ((size_t)1 << 31)) need = (size_t)1 << 31;
    if (hipSetDevice(t->device) != hipSuccess) return K3X_E_HIP;
    uint16_t *p = NULL;
    if (hipMalloc((void **)&p, need) != hipSuccess) return K3X_E_NOMEM;
    if (t->planes) t->retired[t->nretired++] = t->planes;
    t->planes = p;
    t->planes_bytes = need;
    return 0;
}

int k3x_trunk_reserve(k3x_trunk *t, int max_T)
{
    if (!t || max_T < 0) return K3X_E_ARG;
    if (max_T <= K3X_DECODE_MAX_T) return 0;
    const size_t need = (size_t)max_T * t->in * 4;
    if (need > ((size_t)1 << 31)) return K3X_E_SHAPE;      /* 32-bit buffer offsets */
    return trunk_workspace(t, need, NULL);
}

int k3x_trunk_create(const uint16_t *W, int in, int out, int device, k3x_trunk **t)
{
    if (!W || !t || in <= 0 || out <= 0) return K3X_E_ARG;
    *t = NULL;
    if (in % 128 || out % 16) return K3X_E_SHAPE;
    int rc = k3x_dev_check(device);
    if (rc) return rc;
    if (hipSetDevice(device) != hipSuccess) return K3X_E_NODEV;
    k3x_trunk *m = (k3x_trunk *)calloc(1, sizeof *m);
    if (!m) return K3X_E_NOMEM;
    m->device = device; m->in = in; m->out = out;
    const size_t n = (size_t)in * out * 2;
    void *stage = NULL;
    rc = K3X_E_NOMEM;
    if (hipMalloc((void **)&m->w, n) != hipSuccess || hipMalloc(&stage, n) != hipSuccess)
        goto fail;
    rc = K3X_E_HIP;
    if (hipMemcpy(stage, W, n, hipMemcpyHostToDevice) != hipSuccess) goto fail;
    if ((rc = k3x_dev_tile_bf16(m->w, (const uint16_t *)stage, out, in, NULL))) goto fail;
    if (hipDeviceSynchronize() != hipSuccess) { rc = K3X_E_HIP; goto fail; }
    /* the row-major upload stays as the library GEMM's operand */
    m->wr = (uint16_t *)stage;
    m->blas = k3x_blas_init(device) == 0;
    *t = m;
    return 0;
fail:
    if (stage) hipFree(stage);
    k3x_trunk_destroy(m);
    return rc;
}

void k3x_trunk_destroy(k3x_trunk *t)
{
    if (!t) return;
    hipSetDevice(t->device);
    hipDeviceSynchronize();
    if (t->w) hipFree(t->w);
    if (t->wr) hipFree(t->wr);
    if (t->planes) hipFree(t->planes);
    for (int i = 0; i < t->nretired; i++) hipFree(t->retired[i]);
    if (t->hx) hipFree(t->hx);
    if (t->hy) hipFree(t->hy);
    free(t);
}

int k3x_trunk_apply(k3x_trunk *t, float *Y, int ldy, const void *X, int x_dtype, int ldx,
                    int T, void *stream)
{
    if (!t || T < 0 || (T > 0 && (!Y || !X))) return K3X_E_ARG;
    if (x_dtype != K3X_F32 && x_dtype != K3X_BF16) return K3X_E_ARG;
    if (ldx < t->in || ldy < t->out || (ldx & 7) || ((uintptr_t)X & 15)) return K3X_E_ARG;
    if (T == 0) return 0;
    if (T <= K3X_DECODE_MAX_T)
        return k3x_dev_trunk_gemv(t->w, t->in, t->out, Y, ldy, X, x_dtype, ldx, T, stream);
    const size_t need = (size_t)T * t->in * 4;
    if (need > ((size_t)1 << 31)) return K3X_E_SHAPE;      /* 32-bit buffer offsets */
    int rc = trunk_workspace(t, need, stream);
    if (rc) return rc;
    if (t->blas) {
        if (x_dtype == K3X_BF16) {
            rc = k3x_blas_gemm_bf16(t->device, t->wr, t->in, t->out, Y, ldy,
                                    (const uint16_t *)X, ldx, T, 0, stream);
        } else {
            /* X = hi + lo: Y = W.hi, then Y += W.lo */
            uint16_t *hi = t->planes, *lo = t->planes + (size_t)T * t->in;
            rc = k3x_dev_split_rows((const float *)X, ldx, T, t->in, hi, lo, stream);
            if (!rc)
                rc = k3x_blas_gemm_bf16(t->device, t->wr, t->in, t->out, Y, ldy, hi, t->in,
                                        T, 0, stream);
            if (!rc)
                rc = k3x_blas_gemm_bf16(t->device, t->wr, t->in, t->out, Y, ldy, lo, t->in,
                                        T, 1, stream);
        }
        if (rc != K3X_E_HIP) return rc;
        /* a shape the library does not serve (the same answer for every call of that
         * shape): the dense kernel computes the whole product instead, over Y */
        if (hipGetLastError() != hipSuccess) return K3X_E_HIP;
    }
    return k3x_dev_trunk_gemm(t->w, t->in, t->out, Y, ldy, X, x_dtype, ldx, T, t->planes,
                              stream);
}

int k3x_trunk_apply_host(k3x_trunk *t, float *Y, const float *X, int T)
{
    if (!t || T < 0 || (T > 0 && (!Y || !X))) return K3X_E_ARG;
    if (T == 0) return 0;
    if (hipSetDevice(t->device) != hipSuccess) return K3X_E_HIP;
    const size_t nx = (size_t)T * t->in, ny = (size_t)T * t->out;
    const size_t need = nx > ny ? nx : ny;
    if (need > t->hcap) {
        if (t->hx) hipFree(t->hx);
        if (t->hy) hipFree(t->hy);
        t->hx = t->hy = NULL;
        t->hcap = 0;
        if (hipMalloc((void **)&t->hx, need * 4) != hipSuccess ||
            hipMalloc((void **)&t->hy, need * 4) != hipSuccess)
            return K3X_E_NOMEM;
        t->hcap = need;
    }
    if (hipMemcpy(t->hx, X, nx * 4, hipMemcpyHostToDevice) != hipSuccess) return K3X_E_HIP;
    int rc = k3x_trunk_apply(t, t->hy, t->out, t->hx, K3X_F32, t->in, T, NULL);
    if (rc) return rc;
    if (hipMemcpy(Y, t->hy, ny * 4, hipMemcpyDeviceToHost) != hipSuccess) return K3X_E_HIP;
    return 0;
}
