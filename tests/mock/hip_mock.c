/* hip_mock.c - a recording stand-in for the few HIP runtime calls and device launchers
 * that the trunk's host layer (kimi-k3-for-me_amd/csrc/k3x_trunk.c) makes, so that its
 * workspace logic (growth, retirement, refusal under capture) runs on a host without a
 * GPU.  Test infrastructure: built by tests/test_trunk_host.py together with k3x_trunk.c
 * into a temporary library, never into the product. */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int   capturing;            /* what hipStreamIsCapturing reports          */
static long  n_malloc, n_free;     /* calls made                                  */
static void *live[256];            /* allocations not yet freed                   */
static int   n_live;
static void *last_planes;          /* the workspace the last GEMM launch was given */
static long  n_gemm, n_gemv;       /* products of more than / at most 8 rows      */
static int   blas;                 /* what k3x_blas_init reports: library present */
static long  n_blas;               /* library GEMM calls                           */

void mock_reset(void)
{
    capturing = 0; n_malloc = n_free = 0; n_live = 0; last_planes = NULL;
    n_gemm = n_gemv = 0; n_blas = 0;
}
void  mock_set_blas(int on) { blas = on; }
long  mock_blas_calls(void) { return n_blas; }
void  mock_set_capturing(int on) { capturing = on; }
long  mock_mallocs(void) { return n_malloc; }
long  mock_frees(void) { return n_free; }
int   mock_live(void) { return n_live; }
void *mock_last_planes(void) { return last_planes; }
long  mock_gemms(void) { return n_gemm; }
int   mock_is_live(void *p)
{
    for (int i = 0; i < n_live; i++) if (live[i] == p) return 1;
    return 0;
}

hipError_t hipMalloc(void **p, size_t n)
{
    n_malloc++;
    if (n_live == 256) return hipErrorOutOfMemory;
    *p = malloc(n ? n : 1);
    if (!*p) return hipErrorOutOfMemory;
    live[n_live++] = *p;
    return hipSuccess;
}

hipError_t hipFree(void *p)
{
    n_free++;
    for (int i = 0; i < n_live; i++)
        if (live[i] == p) { live[i] = live[--n_live]; free(p); return hipSuccess; }
    return hipErrorInvalidValue;           /* a double free or a foreign pointer */
}

hipError_t hipSetDevice(int d) { (void)d; return hipSuccess; }
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }
hipError_t hipMemcpy(void *dst, const void *src, size_t n, hipMemcpyKind k)
{
    (void)k;
    memcpy(dst, src, n);
    return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus *st)
{
    (void)s;
    *st = capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
    return hipSuccess;
}

int k3x_dev_check(int device) { (void)device; return 0; }
hipError_t hipGetLastError(void) { return hipSuccess; }
int k3x_blas_init(int device) { (void)device; return blas ? 0 : -5; }
int k3x_blas_gemm_bf16(int device, const uint16_t *W, int in, int out, float *Y, int ldy,
                       const uint16_t *X, int ldx, int T, int accumulate, void *stream)
{
    (void)device; (void)W; (void)in; (void)out; (void)Y; (void)ldy; (void)X; (void)ldx;
    (void)T; (void)accumulate; (void)stream;
    n_blas++;
    return 0;
}
/* the fp32 rows' split into the workspace: the library path's one use of it (counted as
 * that path's product, with the workspace it was given) */
int k3x_dev_split_rows(const float *x, int ldx, int T, int n, uint16_t *hi, uint16_t *lo,
                       void *stream)
{
    (void)x; (void)ldx; (void)T; (void)n; (void)lo; (void)stream;
    n_gemm++;
    last_planes = hi;
    return 0;
}
int k3x_dev_tile_bf16(uint16_t *dst, const uint16_t *src, int R, int K, void *stream)
{
    (void)stream;
    memcpy(dst, src, (size_t)R * K * 2);
    return 0;
}
int k3x_dev_trunk_gemv(const uint16_t *W, int in, int out, float *y, int ldy, const void *x,
                       int x_dtype, int ldx, int T, void *stream)
{
    (void)W; (void)in; (void)out; (void)y; (void)ldy; (void)x; (void)x_dtype; (void)ldx;
    (void)T; (void)stream;
    n_gemv++;
    return 0;
}
int k3x_dev_trunk_gemm(const uint16_t *W, int in, int out, float *y, int ldy, const void *x,
                       int x_dtype, int ldx, int T, uint16_t *planes, void *stream)
{
    (void)W; (void)in; (void)out; (void)y; (void)ldy; (void)x; (void)x_dtype; (void)ldx;
    (void)T; (void)stream;
    n_gemm++;
    last_planes = planes;
    return 0;
}
