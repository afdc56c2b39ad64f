/* k3x_moe.c - the C host side of the MoE block: layer upload, call validation and the
 * drop-in entry points.  Kernels live in k3x_kernels.hip behind the k3x_dev_* launchers.
 *
 * Follows the reference's MoE entry points (include/k3/k3.h:571-637, src/core/
 * k3_ops.c:1862-2132) and its expert supplier contract (K3ExpertSrc, k3.h:518-544);
 * the differences are listed in include/k3x_moe.h (weights resident in HBM, status codes
 * instead of abort()).
 */
#include "k3x_internal.h"
#include "../../include/k3x_store.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

long k3x_expert_drops = 0;

const char *k3x_strerror(int s)
{
    switch (s) {
    case K3X_OK:      return "ok";
    case K3X_E_ARG:   return "invalid argument";
    case K3X_E_SHAPE: return "unsupported shape";
    case K3X_E_HIP:   return "HIP runtime error";
    case K3X_E_NOMEM: return "out of memory";
    case K3X_E_DROP:  return "expert could not be fetched";
    case K3X_E_NODEV: return "no usable gfx950 device";
    case K3X_E_WAIT:  return "decode workgroup gave up waiting for the selection";
    default:          return "unknown status";
    }
}

#define HIPCHK(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "k3x: %s failed: %s\n", #call, hipGetErrorString(e_));     \
            rc = (e_ == hipErrorOutOfMemory) ? K3X_E_NOMEM : K3X_E_HIP;                \
            goto fail;                                                                 \
        }                                                                              \
    } while (0)

#define RCCHK(call)                                                                    \
    do {                                                                               \
        rc = (call);                                                                   \
        if (rc) goto fail;                                                             \
    } while (0)

static int cfg_ok(const k3x_cfg *c)
{
    if (!c) return K3X_E_ARG;
    if (c->hidden <= 0 || c->n_experts <= 0 || c->topk <= 0 || c->moe_inter <= 0 ||
        c->n_shared < 0)
        return K3X_E_SHAPE;
    if (c->hidden % 128 || c->moe_inter % 128) return K3X_E_SHAPE;
    if (c->group != 32) return K3X_E_SHAPE;
    if (c->topk > K3X_MAX_TOPK || c->topk > c->n_experts) return K3X_E_SHAPE;
    if (c->n_experts > 1024) return K3X_E_SHAPE;
    if (c->latent < 0 || c->latent % 128) return K3X_E_SHAPE;
    return 0;
}

static void layout(k3x_moe_layer *L)
{
    const int X = L->XL, I = L->cfg.moe_inter;
    const size_t gu = k3x_fp4_matrix_bytes(I, X), dn = k3x_fp4_matrix_bytes(X, I);
    L->gate_off = 0;
    L->up_off = gu;
    L->down_off = 2 * gu;
    L->expert_bytes = (2 * gu + dn + 255) & ~(size_t)255;
}

static int dmalloc(void **p, size_t n, size_t *total)
{
    n = (n + 255) & ~(size_t)255;
    if (hipMalloc(p, n ? n : 256) != hipSuccess) { *p = NULL; return K3X_E_NOMEM; }
    *total += n;
    return 0;
}

/* Allocate every device region of a layer; weights are filled by the caller. */
static int layer_alloc(k3x_moe_layer *L)
{
    const k3x_cfg *c = &L->cfg;
    const int H = c->hidden, E = c->n_experts, I = c->moe_inter, K = c->topk;
    int rc;
    L->lat = c->latent > 0;
    L->XL = L->lat ? c->latent : H;
    /* a beta of 2^64 or more caps nothing any layer produces (b * tanhf(v / b) == v) */
    L->b1 = (c->situ_b1 >= 0x1p64f || c->situ_b1 <= -0x1p64f) ? 0.0f : c->situ_b1;
    L->b2 = (c->situ_b2 >= 0x1p64f || c->situ_b2 <= -0x1p64f) ? 0.0f : c->situ_b2;
    layout(L);
    L->SI = c->moe_inter * c->n_shared;
    L->tdec = K3X_DECODE_MAX_T;
    size_t *b = &L->bytes;
    RCCHK(dmalloc((void **)&L->router, (size_t)E * H * 4, b));
    RCCHK(dmalloc((void **)&L->bias, (size_t)E * 4, b));
    RCCHK(dmalloc((void **)&L->experts, (size_t)(L->nslot ? L->nslot : E) * L->expert_bytes, b));
    if (L->nslot) RCCHK(dmalloc((void **)&L->slot_dev, (size_t)E * 4, b));
    if (L->SI > 0) {
        RCCHK(dmalloc((void **)&L->sh_gate, k3x_bf16_matrix_bytes(L->SI, H), b));
        RCCHK(dmalloc((void **)&L->sh_up, k3x_bf16_matrix_bytes(L->SI, H), b));
        RCCHK(dmalloc((void **)&L->sh_down, k3x_bf16_matrix_bytes(H, L->SI), b));
        if (2 * L->SI <= H) {
            RCCHK(dmalloc((void **)&L->sh_gu_rm, (size_t)2 * L->SI * H * 2, b));
            RCCHK(dmalloc((void **)&L->sh_down_rm, (size_t)H * L->SI * 2, b));
        }
        RCCHK(dmalloc((void **)&L->shB, (size_t)L->SI * 2 * K3X_DECODE_MAX_T * 2, b));
        if (hipStreamCreateWithFlags((hipStream_t *)&L->pf_side, hipStreamNonBlocking) !=
                hipSuccess ||
            hipEventCreateWithFlags((hipEvent_t *)&L->pf_ev[0], hipEventDisableTiming) !=
                hipSuccess ||
            hipEventCreateWithFlags((hipEvent_t *)&L->pf_ev[1], hipEventDisableTiming) !=
                hipSuccess)
            return K3X_E_HIP;
    }
    RCCHK(dmalloc((void **)&L->score, (size_t)K3X_DECODE_MAX_T * E * 4, b));
    RCCHK(dmalloc((void **)&L->choice, (size_t)K3X_DECODE_MAX_T * E * 4, b));
    RCCHK(dmalloc((void **)&L->slack, (size_t)K3X_DECODE_MAX_T * (E + 1) * 4, b));
    L->ninv = L->slack + (size_t)K3X_DECODE_MAX_T * E;
    RCCHK(dmalloc((void **)&L->idx, (size_t)K3X_DECODE_MAX_T * K * 4, b));
    RCCHK(dmalloc((void **)&L->wt, (size_t)K3X_DECODE_MAX_T * K * 4, b));
    RCCHK(dmalloc((void **)&L->route, sizeof(k3x_route), b));
    if (!L->lat && H % 256 == 0)
        RCCHK(dmalloc((void **)&L->pacc, (size_t)K3X_WIDE_PMAX * K3X_DECODE_MAX_T * H * 4, b));
    if (L->lat) {
        const int X = L->XL;
        const size_t xs = (size_t)(X + 511) / 512 * 512;
        RCCHK(dmalloc((void **)&L->ldown, k3x_bf16_matrix_bytes(X, H), b));
        RCCHK(dmalloc((void **)&L->lup, k3x_bf16_matrix_bytes(H, X), b));
        RCCHK(dmalloc((void **)&L->ldown_rm, (size_t)X * H * 2, b));
        RCCHK(dmalloc((void **)&L->lup_rm, (size_t)H * X * 2, b));
        RCCHK(dmalloc((void **)&L->zB, xs * 2 * K3X_DECODE_MAX_T * 2, b));
        const size_t np = K3X_WIDE_PMAX > K3X_DECODE_PARTS ? K3X_WIDE_PMAX : K3X_DECODE_PARTS;
        RCCHK(dmalloc((void **)&L->accL, np * K3X_DECODE_MAX_T * X * 4, b));
        RCCHK(dmalloc((void **)&L->latB, xs * 2 * K3X_DECODE_MAX_T * 2, b));
    }
    if (c->latent_norm) RCCHK(dmalloc((void **)&L->lnw, (size_t)L->XL * 4, b));
    if (hipMemset(L->route, 0, sizeof(k3x_route)) != hipSuccess ||
        hipMemset(L->slack, 0, (size_t)K3X_DECODE_MAX_T * (E + 1) * 4) != hipSuccess)
        return K3X_E_HIP;
    {
        /* the call tag starts at 1: words tagged 0 (the zeroed buffers) match no call */
        const unsigned one = 1u;
        if (hipMemcpy(&L->route->seq, &one, sizeof one, hipMemcpyHostToDevice) != hipSuccess)
            return K3X_E_HIP;
    }
    {
        const char *tr = getenv("K3X_TRACE");
        if (tr && tr[0] == '1') {
            L->tr_cap = E + L->SI / 16 + 1 + K3X_DECODE_MAX_T * K * (I / 16) +
                        K3X_DECODE_PARTS * (L->XL / 16);
            RCCHK(dmalloc((void **)&L->tr, (size_t)3 * L->tr_cap * 24, b));
        }
    }
    /* B sets of 2*DECODE_MAX_T columns over whole super-quads (512 elements) */
    const size_t hs = (size_t)(H + 511) / 512 * 512, is = (size_t)(I + 511) / 512 * 512;
    RCCHK(dmalloc((void **)&L->xB, hs * 2 * K3X_DECODE_MAX_T * 2, b));
    RCCHK(dmalloc((void **)&L->actB, (size_t)K3X_DECODE_MAX_T * K * is * 2 * K3X_DECODE_MAX_T * 2, b));
    if (hipMemset(L->bias, 0, (size_t)E * 4) != hipSuccess) return K3X_E_HIP;
    /* the prefill's plain products (the shared expert's, the latent projections) run on
     * the library where it is present */
    L->blas = k3x_blas_init(L->device) == 0;
    return 0;
fail:
    return rc;
}

static void layer_free(k3x_moe_layer *L)
{
    if (!L) return;
    void *p[] = {L->router, L->bias, L->experts, L->sh_gate, L->sh_up, L->sh_down, L->shB,
                 L->sh_gu_rm, L->sh_down_rm, L->ldown_rm, L->lup_rm,
                 L->score, L->choice, L->slack, L->idx, L->wt, L->route,
                 L->xB, L->actB, L->pf.base, L->h_dev_x, L->h_dev_out,
                 L->ldown, L->lup, L->lnw, L->zB, L->accL, L->latB, L->tr,
                 L->pacc};
    for (size_t i = 0; i < sizeof p / sizeof p[0]; i++)
        if (p[i]) hipFree(p[i]);
    for (int i = 0; i < L->pf.nretired; i++) hipFree(L->pf.retired[i]);
    if (L->slot_dev) hipFree(L->slot_dev);
    for (int i = 0; i < K3X_CACHE_IO; i++) {
        if (L->c_dbuf[i]) hipFree(L->c_dbuf[i]);
        if (L->c_hbuf[i]) hipHostFree(L->c_hbuf[i]);
    }
    if (L->c_sel) hipHostFree(L->c_sel);
    free(L->res_mask);
    if (L->c_route) hipHostFree(L->c_route);
    free(L->slot_of); free(L->key_of); free(L->used_at); free(L->pinned);
    for (int i = 0; i < 8; i++)
        if (L->ev[i]) hipEventDestroy((hipEvent_t)L->ev[i]);
    for (int i = 0; i < 2; i++)
        if (L->pf_ev[i]) hipEventDestroy((hipEvent_t)L->pf_ev[i]);
    if (L->pf_side) hipStreamDestroy((hipStream_t)L->pf_side);
    free(L);
}

void k3x_moe_layer_destroy(k3x_moe_layer *L)
{
    if (!L) return;
    hipSetDevice(L->device);
    hipDeviceSynchronize();
    layer_free(L);
}

size_t k3x_moe_layer_bytes(const k3x_moe_layer *L)
{
    return L ? L->bytes + L->pf.bytes + L->pf.retired_bytes : 0;
}

int k3x_moe_layer_reserve(k3x_moe_layer *L, int max_T)
{
    if (!L || max_T < 0) return K3X_E_ARG;
    if (max_T <= L->tdec || L->nslot) return 0;
    if (hipSetDevice(L->device) != hipSuccess) return K3X_E_HIP;
    return k3x_pf_reserve(L, max_T, NULL);
}

static int new_layer_slots(const k3x_cfg *c, int device, int nslot, k3x_moe_layer **out);

static int new_layer(const k3x_cfg *c, int device, k3x_moe_layer **out)
{
    return new_layer_slots(c, device, 0, out);
}

static int new_layer_slots(const k3x_cfg *c, int device, int nslot, k3x_moe_layer **out)
{
    int rc = cfg_ok(c);
    if (rc) return rc;
    if ((rc = k3x_dev_check(device))) return rc;
    if (hipSetDevice(device) != hipSuccess) return K3X_E_NODEV;
    k3x_moe_layer *L = (k3x_moe_layer *)calloc(1, sizeof *L);
    if (!L) return K3X_E_NOMEM;
    L->cfg = *c;
    L->device = device;
    L->wait_ticks = K3X_ROUTE_WAIT_DEFAULT;
    L->nslot = nslot;
    if ((rc = layer_alloc(L))) { layer_free(L); return rc; }
    *out = L;
    return 0;
}

/* Shared expert upload: three bf16 matrices, re-laid out on the device (and kept
 * row-major as well where the layer holds those copies). */
static int upload_shared(k3x_moe_layer *L, const uint16_t *sh1, const uint16_t *sh3,
                         const uint16_t *sh2)
{
    const int H = L->cfg.hidden, SI = L->SI;
    int rc = 0;
    void *stage = NULL;
    if (SI <= 0) return 0;
    if (!sh1 || !sh3 || !sh2) return K3X_E_ARG;
    const size_t n = (size_t)SI * H * 2, ne = (size_t)SI * H;
    uint16_t *g = L->sh_gu_rm, *u = L->sh_gu_rm ? L->sh_gu_rm + ne : NULL, *d = L->sh_down_rm;
    if (!g) {
        HIPCHK(hipMalloc(&stage, n));
        g = u = d = (uint16_t *)stage;
    }
    HIPCHK(hipMemcpy(g, sh1, n, hipMemcpyHostToDevice));
    RCCHK(k3x_dev_tile_bf16(L->sh_gate, g, SI, H, NULL));
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipMemcpy(u, sh3, n, hipMemcpyHostToDevice));
    RCCHK(k3x_dev_tile_bf16(L->sh_up, u, SI, H, NULL));
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipMemcpy(d, sh2, n, hipMemcpyHostToDevice));
    RCCHK(k3x_dev_tile_bf16(L->sh_down, d, H, SI, NULL));
    HIPCHK(hipDeviceSynchronize());
fail:
    if (stage) hipFree(stage);
    return rc;
}

/* Latent projections: bf16 down [XL][H] and up [H][XL] re-laid out on the device, and the
 * latent RMSNorm weights.  Nothing without a latent projection (the norm weights are
 * still taken when latent_norm is set). */
static int upload_latent(k3x_moe_layer *L, const uint16_t *down, const uint16_t *up,
                         const float *nw)
{
    const int H = L->cfg.hidden, X = L->XL;
    int rc = 0;
    if (L->cfg.latent_norm) {
        if (!nw) return K3X_E_ARG;
        HIPCHK(hipMemcpy(L->lnw, nw, (size_t)X * 4, hipMemcpyHostToDevice));
    }
    if (!L->lat) return 0;
    if (!down || !up) return K3X_E_ARG;
    const size_t n = (size_t)X * H * 2;
    /* the row-major uploads stay: the prefill's library products read them */
    HIPCHK(hipMemcpy(L->ldown_rm, down, n, hipMemcpyHostToDevice));
    RCCHK(k3x_dev_tile_bf16(L->ldown, L->ldown_rm, X, H, NULL));
    HIPCHK(hipMemcpy(L->lup_rm, up, n, hipMemcpyHostToDevice));
    RCCHK(k3x_dev_tile_bf16(L->lup, L->lup_rm, H, X, NULL));
    HIPCHK(hipDeviceSynchronize());
fail:
    return rc;
}

/* Bit m of the result: matrix m (0 gate, 1 up, 2 down) has a scale byte outside 1..252,
 * where a weight can be zero-scaled, subnormal-scaled or infinite and the kernels take
 * the exact dequantisation path. */
static int scale_flags(const k3x_expert_q *q, size_t sg)
{
    const unsigned char *s[3] = {q->s1, q->s3, q->s2};
    int f = 0;
    for (int m = 0; m < 3; m++)
        for (size_t i = 0; i < sg; i++)
            if (s[m][i] == 0 || s[m][i] >= 253) { f |= 1 << m; break; }
    return f;
}

/* One expert: its six arrays copied to a staging area, then tiled into the arena. */
static int upload_expert(k3x_moe_layer *L, int e, const k3x_expert_q *q, uint8_t *stage)
{
    const int H = L->XL, I = L->cfg.moe_inter;
    const size_t pg = (size_t)I * H / 2, sg = (size_t)I * H / 32;
    uint8_t *base = L->experts + (size_t)e * L->expert_bytes;
    int rc = 0;
    if (!q->p1 || !q->s1 || !q->p3 || !q->s3 || !q->p2 || !q->s2) return K3X_E_ARG;
    /* staging: p1 s1 p3 s3 p2 s2, each at its own offset */
    uint8_t *p1 = stage, *s1 = p1 + pg, *p3 = s1 + sg, *s3 = p3 + pg, *p2 = s3 + sg,
            *s2 = p2 + pg;
    HIPCHK(hipMemcpy(p1, q->p1, pg, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(s1, q->s1, sg, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(p3, q->p3, pg, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(s3, q->s3, sg, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(p2, q->p2, pg, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(s2, q->s2, sg, hipMemcpyHostToDevice));
    RCCHK(k3x_dev_tile_fp4(base + L->gate_off, p1, s1, I, H, NULL));
    RCCHK(k3x_dev_tile_fp4(base + L->up_off, p3, s3, I, H, NULL));
    RCCHK(k3x_dev_tile_fp4(base + L->down_off, p2, s2, H, I, NULL));
    HIPCHK(hipDeviceSynchronize());
fail:
    return rc;
}

int k3x_moe_layer_create(const k3x_cfg *c, const k3x_moe_w *w, int device,
                         k3x_moe_layer **out)
{
    if (!c || !w || !out || !w->gate || (!w->src && !w->bank)) return K3X_E_ARG;
    if (w->src && !w->src->get) return K3X_E_ARG;
    *out = NULL;
    k3x_moe_layer *L = NULL;
    int rc = new_layer(c, device, &L);
    if (rc) return rc;
    const int H = c->hidden, E = c->n_experts, I = c->moe_inter, X = L->XL;
    uint8_t *stage = NULL;
    HIPCHK(hipMemcpy(L->router, w->gate, (size_t)E * H * 4, hipMemcpyHostToDevice));
    if (w->bias) HIPCHK(hipMemcpy(L->bias, w->bias, (size_t)E * 4, hipMemcpyHostToDevice));
    RCCHK(upload_shared(L, w->sh1, w->sh3, w->sh2));
    RCCHK(upload_latent(L, w->down, w->up, w->latent_norm));
    HIPCHK(hipMalloc((void **)&stage, 3 * ((size_t)I * X / 2 + (size_t)I * X / 32)));
    for (int e = 0; e < E; e++) {
        k3x_expert_q q;
        if (w->src && w->src->getmany && e % 16 == 0) {
            /* the next 16 experts' reads issued together (k3_ops.c:1905-1906); a short
             * or failed return only means that get() reads the rest itself */
            int batch[16];
            const int nb = E - e < 16 ? E - e : 16;
            for (int i = 0; i < nb; i++) batch[i] = e + i;
            (void)w->src->getmany(w->src, w->layer, batch, nb);
        }
        if (w->src) {
            memset(&q, 0, sizeof q);
            if (w->src->get(w->src, w->layer, e, &q) != 0) {
                k3x_expert_drops++;
                fprintf(stderr, "EXPERT DROP: layer %d expert %d failed to load\n", w->layer,
                        e);
                rc = K3X_E_DROP;
                goto fail;
            }
        } else {
            q = w->bank[e];
        }
        RCCHK(upload_expert(L, e, &q, stage));
        L->special |= scale_flags(&q, (size_t)I * X / 32);
    }
    hipFree(stage);
    *out = L;
    return 0;
fail:
    if (stage) hipFree(stage);
    layer_free(L);
    return rc;
}

/* ---------------------------------------------------------------- from a store ---- */
/* An expert's matrices have the layer's shapes: w1 (gate) and w3 (up) [I][X], w2 (down)
 * [X][I], X the experts' width. */
static int store_shape_ok(const k3x_expert_ref *r, int I, int X)
{
    const int rows[3] = {I, X, I}, width[3] = {X, I, X};
    for (int i = 0; i < 3; i++)
        if (r->m[i].rows != rows[i] || r->m[i].pcols * 2 != width[i] || r->m[i].scols * 32 != width[i])
            return 0;
    return 1;
}

int k3x_moe_layer_create_from_store(const k3x_cfg *c, const k3x_moe_w *w, k3x_store *st,
                                    int layer, int device, k3x_moe_layer **out)
{
    if (!c || !w || !st || !out || !w->gate) return K3X_E_ARG;
    *out = NULL;
    k3x_moe_layer *L = NULL;
    int rc = new_layer(c, device, &L);
    if (rc) return rc;
    const int H = c->hidden, E = c->n_experts, I = c->moe_inter, X = L->XL;
    const size_t run = 3 * ((size_t)I * X / 2 + (size_t)I * X / 32);
    unsigned char *hb[2] = {NULL, NULL};
    uint8_t *db[2] = {NULL, NULL};
    hipEvent_t ev[2] = {NULL, NULL};
    hipStream_t sm = NULL;
    HIPCHK(hipMemcpy(L->router, w->gate, (size_t)E * H * 4, hipMemcpyHostToDevice));
    if (w->bias) HIPCHK(hipMemcpy(L->bias, w->bias, (size_t)E * 4, hipMemcpyHostToDevice));
    RCCHK(upload_shared(L, w->sh1, w->sh3, w->sh2));
    RCCHK(upload_latent(L, w->down, w->up, w->latent_norm));
    /* two pinned host buffers and two device staging areas in turn: run e is read from
     * the shard while run e-1 is copied and re-laid out on the stream */
    HIPCHK(hipStreamCreate(&sm));
    for (int b = 0; b < 2; b++) {
        HIPCHK(hipHostMalloc((void **)&hb[b], run, hipHostMallocDefault));
        HIPCHK(hipMalloc((void **)&db[b], run));
        HIPCHK(hipEventCreateWithFlags(&ev[b], hipEventDisableTiming));
    }
    for (int e = 0; e < E; e++) {
        const int b = e & 1;
        if (e >= 2) HIPCHK(hipEventSynchronize(ev[b]));
        k3x_expert_ref r;
        if (k3x_store_expert_ref(st, layer, e, &r) || !store_shape_ok(&r, I, X) ||
            (size_t)r.nbytes > run || k3x_store_expert_load(st, &r, hb[b]) != r.nbytes) {
            k3x_expert_drops++;
            fprintf(stderr, "EXPERT DROP: layer %d expert %d could not be read from the store\n",
                    layer, e);
            rc = K3X_E_DROP;
            goto fail;
        }
        const k3x_expert_q q = {hb[b] + r.m[0].p_off, hb[b] + r.m[0].s_off,
                                hb[b] + r.m[2].p_off, hb[b] + r.m[2].s_off,
                                hb[b] + r.m[1].p_off, hb[b] + r.m[1].s_off};
        L->special |= scale_flags(&q, (size_t)I * X / 32);
        uint8_t *base = L->experts + (size_t)e * L->expert_bytes;
        HIPCHK(hipMemcpyAsync(db[b], hb[b], (size_t)r.nbytes, hipMemcpyHostToDevice, sm));
        RCCHK(k3x_dev_tile_fp4(base + L->gate_off, db[b] + r.m[0].p_off, db[b] + r.m[0].s_off, I, X, sm));
        RCCHK(k3x_dev_tile_fp4(base + L->up_off, db[b] + r.m[2].p_off, db[b] + r.m[2].s_off, I, X, sm));
        RCCHK(k3x_dev_tile_fp4(base + L->down_off, db[b] + r.m[1].p_off, db[b] + r.m[1].s_off, X, I, sm));
        HIPCHK(hipEventRecord(ev[b], sm));
    }
    HIPCHK(hipStreamSynchronize(sm));
    for (int b = 0; b < 2; b++) {
        hipEventDestroy(ev[b]);
        hipFree(db[b]);
        hipHostFree(hb[b]);
    }
    hipStreamDestroy(sm);
    *out = L;
    return 0;
fail:
    if (sm) hipStreamSynchronize(sm);
    for (int b = 0; b < 2; b++) {
        if (ev[b]) hipEventDestroy(ev[b]);
        if (db[b]) hipFree(db[b]);
        if (hb[b]) hipHostFree(hb[b]);
    }
    if (sm) hipStreamDestroy(sm);
    layer_free(L);
    return rc;
}

/* ---------------------------------------------------------------- expert cache ---- */
/* A layer whose expert arena holds nslot experts (k3_cache.c's K3Cache, with the arena in
 * HBM instead of host RAM): after a decode call's selection the experts it names are made
 * resident; the misses are read from the store together (K3X_CACHE_IO at a time, each
 * into its own pinned buffer, as cache_getmany issues its preads together,
 * k3_cache.c:394-512), then copied to the device and re-laid out into slots; victims are
 * the least recently used unpinned slots not named by the call.  The kernels reach an
 * expert through the slot table (slot_dev). */
static size_t expert_run_bytes(const k3x_moe_layer *L)
{
    return 3 * ((size_t)L->cfg.moe_inter * L->XL / 2 + (size_t)L->cfg.moe_inter * L->XL / 32);
}

static int create_cached(const k3x_cfg *c, const k3x_moe_w *w, k3x_store *st,
                         k3x_expert_src *src, int layer, int nslot, int device,
                         k3x_moe_layer **out)
{
    *out = NULL;
    if (nslot < c->topk + 1 || nslot > c->n_experts) return K3X_E_ARG;
    k3x_moe_layer *L = NULL;
    int rc = new_layer_slots(c, device, nslot, &L);
    if (rc) return rc;
    const int H = c->hidden, E = c->n_experts;
    const size_t run = expert_run_bytes(L);
    L->st = st; L->st_layer = layer; L->c_src = src;
    L->slot_of = (int *)malloc((size_t)E * sizeof(int));
    L->key_of = (int *)malloc((size_t)nslot * sizeof(int));
    L->used_at = (uint64_t *)calloc((size_t)nslot, sizeof(uint64_t));
    L->pinned = (unsigned char *)calloc((size_t)nslot, 1);
    if (!L->slot_of || !L->key_of || !L->used_at || !L->pinned) { rc = K3X_E_NOMEM; goto fail; }
    for (int e = 0; e < E; e++) L->slot_of[e] = -1;
    for (int i = 0; i < nslot; i++) L->key_of[i] = -1;
    L->c_nio = nslot < K3X_CACHE_IO ? nslot : K3X_CACHE_IO;
    for (int i = 0; i < L->c_nio; i++) {
        HIPCHK(hipHostMalloc((void **)&L->c_hbuf[i], run, hipHostMallocDefault));
        HIPCHK(hipMalloc((void **)&L->c_dbuf[i], run));
    }
    HIPCHK(hipHostMalloc((void **)&L->c_route, sizeof(k3x_route), hipHostMallocDefault));
    HIPCHK(hipMemcpy(L->slot_dev, L->slot_of, (size_t)E * 4, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(L->router, w->gate, (size_t)E * H * 4, hipMemcpyHostToDevice));
    if (w->bias) HIPCHK(hipMemcpy(L->bias, w->bias, (size_t)E * 4, hipMemcpyHostToDevice));
    RCCHK(upload_shared(L, w->sh1, w->sh3, w->sh2));
    RCCHK(upload_latent(L, w->down, w->up, w->latent_norm));
    *out = L;
    return 0;
fail:
    layer_free(L);
    return rc;
}

int k3x_moe_layer_create_cached(const k3x_cfg *c, const k3x_moe_w *w, k3x_store *st,
                                int layer, int nslot, int device, k3x_moe_layer **out)
{
    if (!c || !w || !st || !out || !w->gate) return K3X_E_ARG;
    return create_cached(c, w, st, NULL, layer, nslot, device, out);
}

int k3x_moe_layer_create_cached_src(const k3x_cfg *c, const k3x_moe_w *w, int nslot,
                                    int device, k3x_moe_layer **out)
{
    if (!c || !w || !out || !w->gate || !w->src || !w->src->get) return K3X_E_ARG;
    return create_cached(c, w, NULL, w->src, w->layer, nslot, device, out);
}

/* A miss through the supplier: its getmany() (when it has one) for the batch, then, one
 * expert at a time (get()'s pointers last until the next get()), the six arrays copied
 * into the pinned buffer as a run laid out [p1 s1 p3 s3 p2 s2]; ok[i] = 0 for a failed
 * fetch. */
static void src_fetch(k3x_moe_layer *L, const int *miss, int nb, int *ok, k3x_expert_ref *ref)
{
    const size_t I = (size_t)L->cfg.moe_inter, X = (size_t)L->XL;
    const int64_t pb = (int64_t)(I * X / 2), sb = (int64_t)(I * X / 32);
    k3x_expert_src *src = L->c_src;
    if (src->getmany) (void)src->getmany(src, L->st_layer, miss, nb);
    for (int i = 0; i < nb; i++) {
        k3x_expert_q q;
        memset(&q, 0, sizeof q);
        ok[i] = src->get(src, L->st_layer, miss[i], &q) == 0 && q.p1 && q.s1 && q.p3 &&
                q.s3 && q.p2 && q.s2;
        if (!ok[i]) continue;
        k3x_expert_ref *r = &ref[i];
        memset(r, 0, sizeof *r);
        /* m[0] gate (w1), m[1] down (w2), m[2] up (w3), as the store's runs */
        r->m[0].p_off = 0;           r->m[0].s_off = pb;
        r->m[2].p_off = pb + sb;     r->m[2].s_off = 2 * pb + sb;
        r->m[1].p_off = 2 * pb + 2 * sb; r->m[1].s_off = 3 * pb + 2 * sb;
        r->nbytes = 3 * (pb + sb);
        unsigned char *hb = L->c_hbuf[i];
        memcpy(hb + r->m[0].p_off, q.p1, (size_t)pb); memcpy(hb + r->m[0].s_off, q.s1, (size_t)sb);
        memcpy(hb + r->m[2].p_off, q.p3, (size_t)pb); memcpy(hb + r->m[2].s_off, q.s3, (size_t)sb);
        memcpy(hb + r->m[1].p_off, q.p2, (size_t)pb); memcpy(hb + r->m[1].s_off, q.s2, (size_t)sb);
    }
}

/* The least recently used unpinned slot whose expert the call does not name (want[key]
 * == 0) and that no other miss of the batch took (taken[slot]), empty slots first. */
static int cache_victim(const k3x_moe_layer *L, const unsigned char *want,
                        const unsigned char *taken)
{
    int v = -1;
    for (int i = 0; i < L->nslot; i++) {
        if (L->pinned[i] || taken[i]) continue;
        const int k = L->key_of[i];
        if (k >= 0 && want && want[k]) continue;
        if (k < 0) return i;
        if (v < 0 || L->used_at[i] < L->used_at[v]) v = i;
    }
    return v;
}

/* Experts miss[0 .. n-1] (distinct, none resident) into slots: per batch of c_nio, the
 * victims are chosen, the runs read from the store concurrently (one thread and one
 * pinned buffer each), then copied and re-laid out on s, one synchronisation a batch.
 * A run that cannot be read counts in k3x_expert_drops; the others are still loaded. */
static int cache_load_many(k3x_moe_layer *L, const int *miss, int n, const unsigned char *want,
                           hipStream_t s)
{
    const int I = L->cfg.moe_inter, X = L->XL;
    const size_t run = expert_run_bytes(L);
    unsigned char *taken = (unsigned char *)calloc((size_t)L->nslot, 1);
    if (!taken) return K3X_E_NOMEM;
    int rc = 0, dropped = 0;
    for (int b0 = 0; b0 < n && !rc; b0 += L->c_nio) {
        const int nb = n - b0 < L->c_nio ? n - b0 : L->c_nio;
        int vic[K3X_CACHE_IO], ok[K3X_CACHE_IO];
        k3x_expert_ref ref[K3X_CACHE_IO];
        memset(taken, 0, (size_t)L->nslot);
        for (int i = 0; i < nb; i++) {
            vic[i] = cache_victim(L, want, taken);
            if (vic[i] < 0) { rc = K3X_E_SHAPE; break; }    /* every slot pinned or in use */
            taken[vic[i]] = 1;
        }
        if (rc) break;
        if (!L->st) {
            src_fetch(L, miss + b0, nb, ok, ref);
        } else {
#ifdef _OPENMP
#pragma omp parallel for num_threads(nb) schedule(static, 1)
#endif
            for (int i = 0; i < nb; i++) {
                k3x_expert_ref *r = &ref[i];
                ok[i] = !k3x_store_expert_ref(L->st, L->st_layer, miss[b0 + i], r) &&
                        store_shape_ok(r, I, X) && (size_t)r->nbytes <= run &&
                        k3x_store_expert_load(L->st, r, L->c_hbuf[i]) == r->nbytes;
            }
        }
        for (int i = 0; i < nb; i++) {
            const int e = miss[b0 + i], v = vic[i];
            if (!ok[i]) {
                k3x_expert_drops++;
                dropped = 1;
                fprintf(stderr, "EXPERT DROP: layer %d expert %d could not be %s\n",
                        L->st_layer, e, L->st ? "read from the store" : "fetched");
                continue;
            }
            const k3x_expert_ref *r = &ref[i];
            unsigned char *hb = L->c_hbuf[i];
            const k3x_expert_q q = {hb + r->m[0].p_off, hb + r->m[0].s_off,
                                    hb + r->m[2].p_off, hb + r->m[2].s_off,
                                    hb + r->m[1].p_off, hb + r->m[1].s_off};
            L->special |= scale_flags(&q, (size_t)I * X / 32);
            if (L->key_of[v] >= 0) {
                L->slot_of[L->key_of[v]] = -1;
                L->key_of[v] = -1;
                L->evictions++;
            }
            uint8_t *base = L->experts + (size_t)v * L->expert_bytes, *db = L->c_dbuf[i];
            if (hipMemcpyAsync(db, hb, (size_t)r->nbytes, hipMemcpyHostToDevice, s) != hipSuccess ||
                k3x_dev_tile_fp4(base + L->gate_off, db + r->m[0].p_off, db + r->m[0].s_off, I, X, s) ||
                k3x_dev_tile_fp4(base + L->up_off, db + r->m[2].p_off, db + r->m[2].s_off, I, X, s) ||
                k3x_dev_tile_fp4(base + L->down_off, db + r->m[1].p_off, db + r->m[1].s_off, X, I, s)) {
                rc = K3X_E_HIP;
                break;
            }
            L->key_of[v] = e;
            L->slot_of[e] = v;
            L->used_at[v] = ++L->clock;
            L->bytes_read += (uint64_t)r->nbytes;
            L->misses++;
        }
        L->c_dirty = 1;
        /* the pinned buffers and the staging areas are reused by the next batch */
        if (hipStreamSynchronize(s) != hipSuccess && !rc) rc = K3X_E_HIP;
    }
    free(taken);
    return rc ? rc : (dropped ? K3X_E_DROP : 0);
}

static int cache_publish(k3x_moe_layer *L, hipStream_t s)
{
    if (!L->c_dirty) return 0;
    if (hipMemcpyAsync(L->slot_dev, L->slot_of, (size_t)L->cfg.n_experts * 4,
                       hipMemcpyHostToDevice, s) != hipSuccess)
        return K3X_E_HIP;
    L->c_dirty = 0;
    return 0;
}

/* Make experts e[0 .. n-1] resident (the named ones: hits refresh their stamp, misses
 * are read together). */
static int cache_make_resident(k3x_moe_layer *L, const int *ex, int n, hipStream_t s)
{
    const int E = L->cfg.n_experts;
    if (n > L->nslot) return K3X_E_SHAPE;       /* more experts than slots in one call */
    unsigned char *want = (unsigned char *)calloc((size_t)E, 1);
    int *miss = (int *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    if (!want || !miss) { free(want); free(miss); return K3X_E_NOMEM; }
    for (int u = 0; u < n; u++) {
        if (ex[u] < 0 || ex[u] >= E) { free(want); free(miss); return K3X_E_ARG; }
        want[ex[u]] = 1;
    }
    int nm = 0;
    for (int u = 0; u < n; u++) {
        const int e = ex[u];
        if (L->slot_of[e] >= 0) {
            L->hits++;
            L->used_at[L->slot_of[e]] = ++L->clock;
        } else if (want[e] == 1) {
            want[e] = 2;                          /* listed once */
            miss[nm++] = e;
        }
    }
    int rc = nm ? cache_load_many(L, miss, nm, want, s) : 0;
    free(want);
    free(miss);
    const int rp = cache_publish(L, s);
    return rc ? rc : rp;
}

int k3x_cache_slots_fit(const k3x_cfg *c, int device, double fraction)
{
    if (!c || fraction <= 0.0 || fraction > 1.0 || c->hidden <= 0 || c->moe_inter <= 0)
        return K3X_E_ARG;
    const int X = c->latent > 0 ? c->latent : c->hidden, I = c->moe_inter;
    const size_t per = 2 * k3x_fp4_matrix_bytes(I, X) + k3x_fp4_matrix_bytes(X, I);
    size_t fr = 0, tot = 0;
    if (hipSetDevice(device) != hipSuccess || hipMemGetInfo(&fr, &tot) != hipSuccess)
        return K3X_E_NODEV;
    /* the layer's other weights (router, shared expert, projections) and its buffers */
    const size_t SI = (size_t)I * c->n_shared;
    const size_t fixed = (size_t)c->n_experts * c->hidden * 4 + 3 * SI * c->hidden * 2 +
                         (c->latent > 0 ? 2 * (size_t)X * c->hidden * 2 : 0) + ((size_t)256 << 20);
    const double room = (double)fr * fraction - (double)fixed;
    if (room <= 0.0) return 0;
    const double n = room / (double)per;
    return n > (double)c->n_experts ? c->n_experts : (int)n;
}

int k3x_cache_getmany(k3x_moe_layer *L, const int *experts, int n)
{
    if (!L || !L->nslot || n < 0 || (n && !experts)) return K3X_E_ARG;
    if (hipSetDevice(L->device) != hipSuccess) return K3X_E_NODEV;
    hipStream_t s = NULL;
    if (hipStreamCreate(&s) != hipSuccess) return K3X_E_HIP;
    int rc = cache_make_resident(L, experts, n, s);
    if (hipStreamSynchronize(s) != hipSuccess && !rc) rc = K3X_E_HIP;
    hipStreamDestroy(s);
    if (rc) return rc;
    int got = 0;
    for (int i = 0; i < n; i++) got += L->slot_of[experts[i]] >= 0;
    return got;
}

int k3x_cache_resident(const k3x_moe_layer *L, int expert)
{
    if (!L || expert < 0 || expert >= L->cfg.n_experts) return K3X_E_ARG;
    return L->nslot ? L->slot_of[expert] >= 0 : 1;
}

/* ---------------------------------------------------------- cache-only routing ---- */
int k3x_moe_layer_set_cache_only(k3x_moe_layer *L, int on, const unsigned char *resident)
{
    if (!L || (on != 0 && on != 1)) return K3X_E_ARG;
    const int E = L->cfg.n_experts, K = L->cfg.topk;
    if (hipSetDevice(L->device) != hipSuccess) return K3X_E_NODEV;
    if (on && !L->c_sel &&
        hipHostMalloc((void **)&L->c_sel, (size_t)2 * K3X_DECODE_MAX_T * K * sizeof(int),
                      hipHostMallocDefault) != hipSuccess)
        return K3X_E_NOMEM;
    if (on && !L->c_route &&
        hipHostMalloc((void **)&L->c_route, sizeof(k3x_route), hipHostMallocDefault) != hipSuccess)
        return K3X_E_NOMEM;
    if (on && resident) {
        if (!L->res_mask && !(L->res_mask = (unsigned char *)malloc((size_t)E))) return K3X_E_NOMEM;
        for (int e = 0; e < E; e++) L->res_mask[e] = resident[e] ? 1 : 0;
    } else {
        free(L->res_mask);
        L->res_mask = NULL;
    }
    L->cache_only = on;
    return 0;
}

static int is_resident(const k3x_moe_layer *L, int e)
{
    if (e < 0 || e >= L->cfg.n_experts) return 0;
    if (L->res_mask) return L->res_mask[e];
    return L->nslot ? L->slot_of[e] >= 0 : 1;
}

/* The draft's routing (k3_ops.c:1887-1896) applied to T tokens' selections sel_i/sel_w
 * [T][K]: each token's resident experts compacted to the front in top-k order, their
 * weights divided by their float sum when positive, the router's entries left after them
 * (as the reference's in-place loop leaves them).  The route is rebuilt over the kept
 * experts as the selection would have built it: unique experts in first-seen order over
 * (token, slot), each token's weight for an expert the sum of its kept slots' weights in
 * slot order. */
static void cache_only_filter(const k3x_moe_layer *L, int T, int *sel_i, float *sel_w,
                              k3x_route *r)
{
    const int K = L->cfg.topk;
    int nu = 0;
    for (int t = 0; t < T; t++) {
        int *it = sel_i + (size_t)t * K;
        float *wt = sel_w + (size_t)t * K;
        int m = 0;
        float wsum = 0.0f;
        for (int j = 0; j < K; j++)
            if (is_resident(L, it[j])) { it[m] = it[j]; wt[m] = wt[j]; wsum += wt[j]; m++; }
        if (wsum > 0.0f) for (int j = 0; j < m; j++) wt[j] /= wsum;
        for (int j = 0; j < m; j++) {
            int u = 0;
            while (u < nu && r->uniq[u] != it[j]) u++;
            if (u == nu) {
                r->uniq[nu++] = it[j];
                for (int tt = 0; tt < K3X_DECODE_MAX_T; tt++) r->wtok[u][tt] = 0.0f;
            }
            r->wtok[u][t] += wt[j];
        }
    }
    r->nu = nu;
}

int k3x_route_host(k3x_moe_layer *L, void *stream, int T, int *uidx, float *uwt)
{
    hipStream_t s = (hipStream_t)stream;
    const int K = L->cfg.topk, TK = T * K;
    k3x_route *r = (k3x_route *)L->c_route;
    const size_t head = offsetof(k3x_route, uniq) + sizeof(r->uniq);
    int *sel_i = L->c_sel;
    float *sel_w = L->c_sel ? (float *)(L->c_sel + (size_t)K3X_DECODE_MAX_T * K) : NULL;
    if (hipMemcpyAsync(r, L->route, head, hipMemcpyDeviceToHost, s) != hipSuccess) return K3X_E_HIP;
    if (L->cache_only &&
        (hipMemcpyAsync(sel_i, L->idx, (size_t)TK * 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
         hipMemcpyAsync(sel_w, L->wt, (size_t)TK * 4, hipMemcpyDeviceToHost, s) != hipSuccess))
        return K3X_E_HIP;
    if (hipStreamSynchronize(s) != hipSuccess) return K3X_E_HIP;
    if (r->nu < 0 || r->nu > K3X_DECODE_MAX_T * K3X_MAX_TOPK) return K3X_E_HIP;
    if (L->cache_only) {
        cache_only_filter(L, T, sel_i, sel_w, r);
        if (hipMemcpyAsync(&L->route->nu, &r->nu, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess ||
            (r->nu && (hipMemcpyAsync(L->route->uniq, r->uniq, (size_t)r->nu * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
                       hipMemcpyAsync(L->route->wtok, r->wtok, (size_t)r->nu * sizeof(r->wtok[0]),
                                      hipMemcpyHostToDevice, s) != hipSuccess)))
            return K3X_E_HIP;
        if (uidx && (hipMemcpyAsync(uidx, sel_i, (size_t)TK * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
                     hipMemcpyAsync(uwt, sel_w, (size_t)TK * 4, hipMemcpyHostToDevice, s) != hipSuccess))
            return K3X_E_HIP;
    }
    int rc = 0;
    if (L->nslot) rc = cache_make_resident(L, r->uniq, r->nu, s);
    /* the copies above read the pinned host buffers, which the next call (perhaps on
     * another stream) rewrites */
    if (!rc && L->cache_only && hipStreamSynchronize(s) != hipSuccess) rc = K3X_E_HIP;
    return rc;
}

int k3x_cache_stats(const k3x_moe_layer *L, k3x_cache_stat *st)
{
    if (!L || !st) return K3X_E_ARG;
    memset(st, 0, sizeof *st);
    st->nslot = L->nslot;
    for (int i = 0; i < L->nslot; i++) st->resident += L->key_of[i] >= 0;
    st->hits = L->hits; st->misses = L->misses;
    st->evictions = L->evictions; st->bytes_read = L->bytes_read;
    return 0;
}

int k3x_cache_pin(k3x_moe_layer *L, int expert, int pin)
{
    if (!L || !L->nslot || expert < 0 || expert >= L->cfg.n_experts) return K3X_E_ARG;
    int rc = 0;
    if (hipSetDevice(L->device) != hipSuccess) return K3X_E_NODEV;
    if (L->slot_of[expert] < 0) {
        if (!pin) return 0;
        int np = 0;
        for (int i = 0; i < L->nslot; i++) np += L->pinned[i];
        if (np + 1 > L->nslot - L->cfg.topk) return K3X_E_SHAPE;   /* keep topk slots free */
        hipStream_t s = NULL;
        HIPCHK(hipStreamCreate(&s));
        rc = cache_load_many(L, &expert, 1, NULL, s);
        if (!rc) rc = cache_publish(L, s);
        if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = K3X_E_HIP;
        hipStreamDestroy(s);
        if (rc) return rc;
    }
    L->pinned[L->slot_of[expert]] = pin ? 1 : 0;
    return 0;
fail:
    return rc;
}

int k3x_moe_layer_read_expert(const k3x_moe_layer *L, int e, unsigned char *p1,
                              unsigned char *s1, unsigned char *p3, unsigned char *s3,
                              unsigned char *p2, unsigned char *s2)
{
    if (!L || e < 0 || e >= L->cfg.n_experts) return K3X_E_ARG;
    if (L->nslot && L->slot_of[e] < 0) return K3X_E_ARG;        /* not resident */
    const int H = L->XL, I = L->cfg.moe_inter;
    const size_t pg = (size_t)I * H / 2, sg = (size_t)I * H / 32;
    const uint8_t *base = L->experts + (size_t)(L->nslot ? L->slot_of[e] : e) * L->expert_bytes;
    uint8_t *st = NULL;
    int rc = 0;
    HIPCHK(hipSetDevice(L->device));
    HIPCHK(hipMalloc((void **)&st, pg + sg));
    const struct { const uint8_t *src; int R, K; unsigned char *p, *s; } m[3] = {
        {base + L->gate_off, I, H, p1, s1},
        {base + L->up_off, I, H, p3, s3},
        {base + L->down_off, H, I, p2, s2}};
    for (int i = 0; i < 3; i++) {
        RCCHK(k3x_dev_untile_fp4(st, st + pg, m[i].src, m[i].R, m[i].K, NULL));
        HIPCHK(hipDeviceSynchronize());
        if (m[i].p) HIPCHK(hipMemcpy(m[i].p, st, pg, hipMemcpyDeviceToHost));
        if (m[i].s) HIPCHK(hipMemcpy(m[i].s, st + pg, sg, hipMemcpyDeviceToHost));
    }
fail:
    if (st) hipFree(st);
    return rc;
}

int k3x_moe_layer_dequant(const k3x_moe_layer *L, int e, int m, float *out)
{
    if (!L || !out || e < 0 || e >= L->cfg.n_experts || m < 0 || m > 2) return K3X_E_ARG;
    if (L->nslot && L->slot_of[e] < 0) return K3X_E_ARG;        /* not resident */
    const int X = L->XL, I = L->cfg.moe_inter;
    const int R = m == 2 ? X : I, K = m == 2 ? I : X;
    const size_t off[3] = {L->gate_off, L->up_off, L->down_off};
    const uint8_t *src = L->experts + (size_t)(L->nslot ? L->slot_of[e] : e) * L->expert_bytes +
                         off[m];
    float *d = NULL;
    int rc = 0;
    HIPCHK(hipSetDevice(L->device));
    HIPCHK(hipMalloc((void **)&d, (size_t)R * K * 4));
    RCCHK(k3x_dev_dequant_fp4(d, src, R, K, (L->special >> m) & 1, NULL));
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipMemcpy(out, d, (size_t)R * K * 4, hipMemcpyDeviceToHost));
fail:
    if (d) hipFree(d);
    return rc;
}

/* Prefill working buffers for min(T, the chunk) tokens per pipeline run: one
 * allocation, carved into 256-byte-aligned regions.  Grown, to at least twice the old
 * capacity, when a larger T arrives; the old allocation is not freed (a graph recorded
 * over it may still be replayed) but kept until the layer is destroyed.  Growing
 * allocates, so it is refused while `stream` is being captured: a caller that captures
 * prefill calls reserves first (k3x_moe_layer_reserve). */
int k3x_pf_reserve(k3x_moe_layer *L, int T, void *stream)
{
    k3x_prefill_buf *B = &L->pf;
    const int chunk = k3x_pf_chunk_tokens(L);
    if (T > chunk) T = chunk;
    if (T <= B->cap_T) return 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) return K3X_E_HIP;
    if (cs != hipStreamCaptureStatusNone) {
        fprintf(stderr, "k3x: prefill of %d tokens needs its buffers reserved before capture "
                        "(k3x_moe_layer_reserve); %d reserved\n", T, B->cap_T);
        return K3X_E_SHAPE;
    }
    if (B->nretired == K3X_PF_RETIRED) return K3X_E_NOMEM;
    if (B->base && T < 2 * B->cap_T) T = 2 * B->cap_T < chunk ? 2 * B->cap_T : chunk;
    const size_t total = k3x_pf_layout(L, T, NULL, NULL);
    void *base = NULL;
    if (hipSetDevice(L->device) != hipSuccess) return K3X_E_HIP;
    if (hipMalloc(&base, total) != hipSuccess) return K3X_E_NOMEM;
    if (B->base) {
        B->retired[B->nretired++] = B->base;
        B->retired_bytes += B->bytes;
    }
    k3x_pf_layout(L, T, (char *)base, B);
    B->base = base;
    return 0;
}

size_t k3x_pf_layout(const k3x_moe_layer *L, int T, char *p, k3x_prefill_buf *B)
{
    const k3x_cfg *c = &L->cfg;
    const size_t E = (size_t)c->n_experts, K = (size_t)c->topk,
                 I = (size_t)c->moe_inter, SI = (size_t)L->SI, t = (size_t)T;
    /* rows of the widest activation (hidden, or a latent width above it) */
    const size_t H = (size_t)(L->XL > c->hidden ? L->XL : c->hidden), X = (size_t)L->XL;
    /* GEMM tiles: at most ceil(rows/64) row blocks by (T*K/16 + E + 1) column blocks */
    const int ndg = (int)(((I + 63) / 64) * (t * K / 16 + E + 1));
    const int ndd = (int)(((H + 63) / 64) * (t * K / 16 + E + 1));
    const size_t sz[] = {
        t * H * 4,                 /* xhl     */
        t * E * 4, t * E * 4,      /* score, choice */
        t * K * 4, t * K * 4,      /* idx, wt */
        E * 4, (E + 1) * 4, E * 4, /* counts, offsets, cursor */
        2 * (E + 1) * 4, 2 * (E + 1) * 4,  /* tb_gu, tb_dn: small and large tile classes */
        t * K * 4, t * K * 4, t * K * 4,   /* perm_tok, perm_w, pos_of */
        t * K * I * 4,             /* act     */
        (SI ? t * SI * 4 : 256),   /* act_sh  */
        (t * K + t) * H * 4,       /* y       */
        t * K * H * 4,             /* xp      */
        L->lat ? t * X * 4 : 256,  /* zf      */
        L->lat ? t * X * 4 : 256,  /* zhl     */
        (size_t)ndg * 16,          /* desc_gu */
        (size_t)ndd * 16,          /* desc_dn */
    };
    enum { N = sizeof sz / sizeof sz[0] };
    size_t off[N], total = 0;
    for (int i = 0; i < N; i++) {
        off[i] = total;
        total += (sz[i] + 255) & ~(size_t)255;
    }
    if (!p || !B) return total;
    B->bytes = total; B->cap_T = T;
    B->xhl = (uint16_t *)(p + off[0]);
    B->score = (float *)(p + off[1]);   B->choice = (float *)(p + off[2]);
    B->idx = (int *)(p + off[3]);       B->wt = (float *)(p + off[4]);
    B->counts = (int *)(p + off[5]);    B->offsets = (int *)(p + off[6]);
    B->cursor = (int *)(p + off[7]);
    B->tb_gu = (int *)(p + off[8]);     B->tb_dn = (int *)(p + off[9]);
    B->perm_tok = (int *)(p + off[10]); B->perm_w = (float *)(p + off[11]);
    B->pos_of = (int *)(p + off[12]);
    B->act = (uint16_t *)(p + off[13]); B->act_sh = (uint16_t *)(p + off[14]);
    B->y = (float *)(p + off[15]);
    B->xp = (uint16_t *)(p + off[16]);
    B->zf = (float *)(p + off[17]);     B->zhl = (uint16_t *)(p + off[18]);
    B->desc_gu = p + off[19]; B->ndesc_gu = ndg;
    B->desc_dn = p + off[20]; B->ndesc_dn = ndd;
    return total;
}

/* ---------------------------------------------------------------- forward ---- */
int k3x_moe_forward(k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                    const float *resid, int *idx, float *wt, void *stream)
{
    if (!L || (T > 0 && (!out || !x))) return K3X_E_ARG;
    if (T < 0 || (x_dtype != K3X_F32 && x_dtype != K3X_BF16)) return K3X_E_ARG;
    if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)resid & 15)) return K3X_E_ARG;
    if ((idx == NULL) != (wt == NULL)) return K3X_E_ARG;
    if (T == 0) return 0;
    if (T <= L->tdec)
        return k3x_dev_decode(L, out, x, x_dtype, T, resid, idx, wt, NULL, 0.0f, stream);
    if (L->nslot || L->cache_only) {
        /* a cached layer, or cache-only routing: decode-path calls of tdec tokens (each
         * token's routing is its own; its output bits follow the sub-call's shape, within
         * the parity bar of any other grouping; the reference runs such calls token by
         * token, k3_ops.c:2018) */
        const size_t es = (x_dtype == K3X_BF16) ? 2 : 4;
        const int H = L->cfg.hidden, K = L->cfg.topk;
        for (int t0 = 0; t0 < T; t0 += L->tdec) {
            const int n = T - t0 < L->tdec ? T - t0 : L->tdec;
            const int rc = k3x_dev_decode(L, out + (size_t)t0 * H, (const char *)x + (size_t)t0 * H * es,
                                          x_dtype, n, resid ? resid + (size_t)t0 * H : NULL,
                                          idx ? idx + (size_t)t0 * K : NULL,
                                          wt ? wt + (size_t)t0 * K : NULL, NULL, 0.0f, stream);
            if (rc) return rc;
        }
        return 0;
    }
    return k3x_dev_prefill(L, out, x, x_dtype, T, resid, idx, wt, stream);
}

int k3x_moe_route(k3x_moe_layer *L, int *idx, float *wt, const void *x, int x_dtype, int T,
                  void *stream)
{
    if (!L || (T > 0 && (!x || !idx || !wt))) return K3X_E_ARG;
    if (T < 0 || (x_dtype != K3X_F32 && x_dtype != K3X_BF16)) return K3X_E_ARG;
    if ((uintptr_t)x & 15) return K3X_E_ARG;
    if (T == 0) return 0;
    return k3x_dev_route(L, idx, wt, x, x_dtype, T, stream);
}

int k3x_moe_prefill_noalloc(k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                            const float *resid, int *idx, float *wt, void *stream)
{
    if (!L || !out || !x || T < 0 || (x_dtype != K3X_F32 && x_dtype != K3X_BF16)) return K3X_E_ARG;
    if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)resid & 15)) return K3X_E_ARG;
    if ((idx == NULL) != (wt == NULL)) return K3X_E_ARG;
    if (L->nslot || L->cache_only) return K3X_E_ARG;  /* host work between the kernels */
    if (T <= L->tdec) return K3X_E_SHAPE;     /* the decode path: k3x_moe_forward */
    return k3x_dev_prefill_noalloc(L, out, x, x_dtype, T, resid, idx, wt, stream);
}

int k3x_moe_layer_trace(k3x_moe_layer *L, int kernel, unsigned long long *out, int max_wg)
{
    if (!L || !out || kernel < 0 || kernel > 2 || max_wg < 0) return K3X_E_ARG;
    if (!L->tr) return 0;
    const int n = L->tr_n[kernel] < max_wg ? L->tr_n[kernel] : max_wg;
    if (hipSetDevice(L->device) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, L->tr + (size_t)kernel * L->tr_cap * 3, (size_t)n * 24,
                  hipMemcpyDeviceToHost) != hipSuccess)
        return K3X_E_HIP;
    return n;
}

int k3x_moe_layer_set_route_wait(k3x_moe_layer *L, unsigned long long ticks, int publish)
{
    if (!L) return K3X_E_ARG;
    L->wait_ticks = ticks;
    L->no_publish = !publish;
    return 0;
}

int k3x_moe_layer_check(k3x_moe_layer *L)
{
    if (!L) return K3X_E_ARG;
    if (hipSetDevice(L->device) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return K3X_E_HIP;
    int err = 0;
    if (hipMemcpy(&err, &L->route->err, sizeof err, hipMemcpyDeviceToHost) != hipSuccess)
        return K3X_E_HIP;
    if (!err) return 0;
    const int zero = 0;
    if (hipMemcpy(&L->route->err, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess)
        return K3X_E_HIP;
    return K3X_E_WAIT;
}

int k3x_moe_layer_exact_count(k3x_moe_layer *L, int *n)
{
    if (!L || !n) return K3X_E_ARG;
    if (hipSetDevice(L->device) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
        return K3X_E_HIP;
    if (hipMemcpy(n, &L->route->nexact, sizeof *n, hipMemcpyDeviceToHost) != hipSuccess)
        return K3X_E_HIP;
    return 0;
}

int k3x_moe_layer_last_route(k3x_moe_layer *L, int T, int *idx, float *wt)
{
    if (!L || !idx || !wt || T <= 0 || T > K3X_DECODE_MAX_T) return K3X_E_ARG;
    const size_t n = (size_t)T * L->cfg.topk;
    if (hipSetDevice(L->device) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(idx, L->idx, n * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(wt, L->wt, n * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return K3X_E_HIP;
    return 0;
}

int k3x_attn_res(float *h, const float *blocks, int maxb, int nb, const float *pref,
                 const float *fold, int n, int T, float eps, void *stream)
{
    if (!h || !pref || !fold || n <= 0 || T < 0 || nb < 0 || (nb > 0 && (!blocks || maxb < nb)))
        return K3X_E_ARG;
    if (T == 0) return 0;
    return k3x_dev_attn_res(h, blocks, maxb, nb, NULL, 0, pref, fold, n, T, eps, stream);
}

int k3x_attn_res_v(float *h, const float *blocks, int maxb, const int *nbv, int nbs,
                   const float *pref, const float *fold, int n, int T, float eps, void *stream)
{
    if (!h || !pref || !fold || !nbv || n <= 0 || T < 0 || maxb < 0 || (nbs != 0 && nbs != 1))
        return K3X_E_ARG;
    if (T == 0) return 0;
    return k3x_dev_attn_res(h, blocks, maxb, 0, nbv, nbs, pref, fold, n, T, eps, stream);
}

/* The MoE half with the rows' block counts either one host value (nbv NULL) or read on
 * the device (nbv[t * nbs]). */
static int moe_half(k3x_moe_layer *L, float *h, float *pref, const float *blocks, int maxb,
                    int nb, const int *nbv, int nbs, const float *fold,
                    const float *post_norm, float eps, int T, float *hin, void *stream)
{
    if (!L || !post_norm || !hin || T < 0) return K3X_E_ARG;
    if (T == 0) return 0;
    const int H = L->cfg.hidden;
    int rc = nbv ? k3x_attn_res_v(h, blocks, maxb, nbv, nbs, pref, fold, H, T, eps, stream)
                 : k3x_attn_res(h, blocks, maxb, nb, pref, fold, H, T, eps, stream);
    if (!rc) rc = k3x_rmsnorm(hin, h, post_norm, H, T, eps, stream);
    if (!rc) rc = k3x_moe_forward(L, pref, hin, K3X_F32, T, pref, NULL, NULL, stream);
    if (!rc) rc = k3x_dev_copy_f32(h, pref, (size_t)T * H, stream);
    return rc;
}

int k3x_moe_half(k3x_moe_layer *L, float *h, float *pref, const float *blocks, int maxb,
                 int nb, const float *fold, const float *post_norm, float eps, int T,
                 float *hin, void *stream)
{
    return moe_half(L, h, pref, blocks, maxb, nb, NULL, 0, fold, post_norm, eps, T, hin,
                    stream);
}

int k3x_moe_half_v(k3x_moe_layer *L, float *h, float *pref, const float *blocks, int maxb,
                   const int *nbv, int nbs, const float *fold, const float *post_norm,
                   float eps, int T, float *hin, void *stream)
{
    if (!nbv) return K3X_E_ARG;
    return moe_half(L, h, pref, blocks, maxb, 0, nbv, nbs, fold, post_norm, eps, T, hin,
                    stream);
}

int k3x_rmsnorm(float *y, const float *x, const float *w, int n, int T, float eps,
                void *stream)
{
    if (!y || !x || !w || n <= 0 || T < 0) return K3X_E_ARG;
    return k3x_dev_rmsnorm(y, x, w, n, T, eps, stream);
}

/* Host-pointer drop-ins: stage x and out through device buffers held by the layer.
 * idx/wt receive the last token's routing, except for a prefill call of several tokens,
 * which leaves them as they were: k3_moe_prefill's batched path routes into buffers of
 * its own (k3_ops.c:2018-2053) and only its per-token fallback, k3_moe (for one token,
 * or for cache-only routing), writes them. */
static int host_call(k3x_moe_layer *L, float *out, const float *x, int T, int *idx,
                     float *wt, int prefill)
{
    if (!L || (T > 0 && (!out || !x))) return K3X_E_ARG;
    if (prefill && T > 1 && !L->cache_only) idx = NULL, wt = NULL;
    if (T <= 0) return T < 0 ? K3X_E_ARG : 0;
    const k3x_cfg *c = &L->cfg;
    const size_t n = (size_t)T * c->hidden * 4;
    const size_t nr = (size_t)T * c->topk * 4;
    int rc = 0;
    HIPCHK(hipSetDevice(L->device));
    if (L->h_cap < n + 2 * nr) {
        if (L->h_dev_x) hipFree(L->h_dev_x);
        if (L->h_dev_out) hipFree(L->h_dev_out);
        L->h_dev_x = L->h_dev_out = NULL;
        L->h_cap = 0;
        HIPCHK(hipMalloc(&L->h_dev_x, n + 2 * nr + 512));
        HIPCHK(hipMalloc(&L->h_dev_out, n));
        L->h_cap = n + 2 * nr;
    }
    {
        char *dx = (char *)L->h_dev_x;
        int *didx = (int *)(dx + ((n + 255) & ~(size_t)255));
        float *dwt = (float *)((char *)didx + ((nr + 255) & ~(size_t)255));
        HIPCHK(hipMemcpy(dx, x, n, hipMemcpyHostToDevice));
        RCCHK(k3x_moe_forward(L, (float *)L->h_dev_out, dx, K3X_F32, T, NULL, didx, dwt, NULL));
        /* synchronises, then reports (and clears) a decode workgroup that gave up its
         * bounded wait: that call's output is not valid, and the caller has no other way
         * to learn of it */
        RCCHK(k3x_moe_layer_check(L));
        HIPCHK(hipMemcpy(out, L->h_dev_out, n, hipMemcpyDeviceToHost));
        if (idx) {
            const size_t last = (size_t)(T - 1) * c->topk;
            HIPCHK(hipMemcpy(idx, didx + last, (size_t)c->topk * 4, hipMemcpyDeviceToHost));
        }
        if (wt) {
            const size_t last = (size_t)(T - 1) * c->topk;
            HIPCHK(hipMemcpy(wt, dwt + last, (size_t)c->topk * 4, hipMemcpyDeviceToHost));
        }
    }
fail:
    return rc;
}

int k3x_moe(k3x_moe_layer *L, float *out, const float *x, int T, int *idx, float *wt)
{
    return host_call(L, out, x, T, idx, wt, 0);
}

int k3x_moe_prefill(k3x_moe_layer *L, float *out, const float *x, int T, int *idx,
                    float *wt)
{
    return host_call(L, out, x, T, idx, wt, 1);
}

int k3x_moe_layer_set_prefill_mode(k3x_moe_layer *L, int mode)
{
    if (!L || (mode != K3X_PREFILL_EXACT && mode != K3X_PREFILL_MXFP8)) return K3X_E_ARG;
    if (mode == K3X_PREFILL_MXFP8 && L->special) return K3X_E_SHAPE;
    L->pf_mode = mode;
    return 0;
}

/* ---------------------------------------------------------------- timing ---- */
int k3x_moe_layer_set_timing(k3x_moe_layer *L, int on)
{
    if (!L) return K3X_E_ARG;
    if (on) {
        for (int i = 0; i < 8; i++)
            if (!L->ev[i] &&
                hipEventCreateWithFlags((hipEvent_t *)&L->ev[i], hipEventDisableSystemFence) !=
                    hipSuccess)
                return K3X_E_HIP;
    }
    L->timing = on ? 1 : 0;
    L->n_ev_used = 0;
    return 0;
}

int k3x_moe_layer_last_ms(k3x_moe_layer *L, float *ms)
{
    if (!L || !ms || !L->timing || L->n_ev_used < 2) return K3X_E_ARG;
    for (int i = 0; i + 1 < L->n_ev_used; i++) {
        if (hipEventSynchronize((hipEvent_t)L->ev[i + 1]) != hipSuccess) return K3X_E_HIP;
        if (hipEventElapsedTime(&ms[i], (hipEvent_t)L->ev[i], (hipEvent_t)L->ev[i + 1]) !=
            hipSuccess)
            return K3X_E_HIP;
    }
    return L->n_ev_used - 1;
}

/* ---------------------------------------------------------------- synthetic ---- */
static uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

uint64_t k3x_synth_key(uint64_t seed, int layer, int stream, int sub)
{
    uint64_t k = mix64(seed + 0x9E3779B97F4A7C15ull * (uint64_t)(layer + 1));
    k = mix64(k ^ (0xD1B54A32D192ED03ull * (uint64_t)(stream + 1)));
    return mix64(k + (uint64_t)(uint32_t)sub);
}

/* Box-Muller on the two 32-bit halves of one draw, in double, rounded to float once. */
static double normal_of(uint64_t u)
{
    const double u1 = ((double)(u >> 32) + 0.5) * 0x1p-32;
    const double u2 = ((double)(u & 0xFFFFFFFFull) + 0.5) * 0x1p-32;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void k3x_synth_normal_f32(float *dst, size_t n, uint64_t key, double mu, double sigma)
{
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) dst[i] = (float)(mu + sigma * normal_of(draw(key, i)));
}

static uint16_t to_bf16(float f)
{
    union { float f; uint32_t u; } v = {f};
    if ((v.u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((v.u >> 16) | 0x40u);
    return (uint16_t)((v.u + 0x7FFFu + ((v.u >> 16) & 1u)) >> 16);
}

void k3x_synth_normal_bf16(uint16_t *dst, size_t n, uint64_t key, double mu, double sigma)
{
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++)
        dst[i] = to_bf16((float)(mu + sigma * normal_of(draw(key, i))));
}

int k3x_synth_layer_create(const k3x_cfg *c, const k3x_synth_spec *s, int device,
                           k3x_moe_layer **out)
{
    if (!c || !s || !out) return K3X_E_ARG;
    if (s->scale_lo < 0 || s->scale_hi > 255 || s->scale_lo > s->scale_hi) return K3X_E_ARG;
    *out = NULL;
    k3x_moe_layer *L = NULL;
    int rc = new_layer(c, device, &L);
    if (rc) return rc;
    const int H = c->hidden, E = c->n_experts, I = c->moe_inter, SI = L->SI, X = L->XL;
    float *hf = NULL;
    uint16_t *hb = NULL;
    hf = (float *)malloc((size_t)E * H * 4);
    if (!hf) { rc = K3X_E_NOMEM; goto fail; }
    k3x_synth_normal_f32(hf, (size_t)E * H, k3x_synth_key(s->seed, s->layer, K3X_STREAM_ROUTER, 0),
                         0.0, s->router_sigma);
    HIPCHK(hipMemcpy(L->router, hf, (size_t)E * H * 4, hipMemcpyHostToDevice));
    if (s->zipf_alpha > 0.0) {
        int *perm = (int *)malloc((size_t)E * sizeof(int));
        if (!perm) { rc = K3X_E_NOMEM; goto fail; }
        const uint64_t key = k3x_synth_key(s->seed, s->layer, K3X_STREAM_BIAS, 0);
        for (int e = 0; e < E; e++) perm[e] = e;
        for (int e = E - 1; e > 0; e--) {
            const int j = (int)(draw(key, (uint64_t)e) % (uint64_t)(e + 1));
            const int t = perm[e]; perm[e] = perm[j]; perm[j] = t;
        }
        for (int e = 0; e < E; e++) hf[e] = (float)(s->zipf_alpha * pow((double)(perm[e] + 1), -s->zipf_s));
        free(perm);
    } else {
        k3x_synth_normal_f32(hf, (size_t)E, k3x_synth_key(s->seed, s->layer, K3X_STREAM_BIAS, 0),
                             0.0, s->bias_sigma);
    }
    HIPCHK(hipMemcpy(L->bias, hf, (size_t)E * 4, hipMemcpyHostToDevice));
    free(hf);
    hf = NULL;
    if (SI > 0) {
        hb = (uint16_t *)malloc((size_t)SI * H * 2 * 3);
        if (!hb) { rc = K3X_E_NOMEM; goto fail; }
        const size_t n = (size_t)SI * H;
        k3x_synth_normal_bf16(hb, n, k3x_synth_key(s->seed, s->layer, K3X_STREAM_SH1, 0), 0.0,
                              s->shared_sigma);
        k3x_synth_normal_bf16(hb + n, n, k3x_synth_key(s->seed, s->layer, K3X_STREAM_SH3, 0),
                              0.0, s->shared_sigma);
        k3x_synth_normal_bf16(hb + 2 * n, n, k3x_synth_key(s->seed, s->layer, K3X_STREAM_SH2, 0),
                              0.0, s->shared_sigma);
        RCCHK(upload_shared(L, hb, hb + n, hb + 2 * n));
        free(hb);
        hb = NULL;
    }
    if (L->lat || c->latent_norm) {
        const size_t n = (size_t)X * H;
        if (L->lat) {
            hb = (uint16_t *)malloc(n * 2 * 2);
            if (!hb) { rc = K3X_E_NOMEM; goto fail; }
            k3x_synth_normal_bf16(hb, n, k3x_synth_key(s->seed, s->layer, K3X_STREAM_DOWN, 0),
                                  0.0, s->trunk_sigma);
            k3x_synth_normal_bf16(hb + n, n, k3x_synth_key(s->seed, s->layer, K3X_STREAM_UP, 0),
                                  0.0, s->trunk_sigma);
        }
        if (c->latent_norm) {
            hf = (float *)malloc((size_t)X * 4);
            if (!hf) { rc = K3X_E_NOMEM; goto fail; }
            k3x_synth_normal_f32(hf, (size_t)X, k3x_synth_key(s->seed, s->layer, K3X_STREAM_LNORM, 0),
                                 1.0, 0.1);
        }
        RCCHK(upload_latent(L, hb, hb ? hb + n : NULL, hf));
        free(hb);
        hb = NULL;
        free(hf);
        hf = NULL;
    }
    L->special = (s->scale_lo < 1 || s->scale_hi > 252) ? 7 : 0;
    for (int e = 0; e < E; e++) {
        uint8_t *base = L->experts + (size_t)e * L->expert_bytes;
        const struct { size_t off; int R, K, m; } mm[3] = {
            {L->gate_off, I, X, 0}, {L->up_off, I, X, 1}, {L->down_off, X, I, 2}};
        for (int i = 0; i < 3; i++)
            RCCHK(k3x_dev_synth_fp4(base + mm[i].off, mm[i].R, mm[i].K,
                                    k3x_synth_key(s->seed, s->layer, K3X_STREAM_CODES, 3 * e + mm[i].m),
                                    k3x_synth_key(s->seed, s->layer, K3X_STREAM_SCALES, 3 * e + mm[i].m),
                                    s->scale_lo, s->scale_hi, NULL));
    }
    HIPCHK(hipDeviceSynchronize());
    *out = L;
    return 0;
fail:
    free(hf);
    free(hb);
    layer_free(L);
    return rc;
}

/* ---------------------------------------------------------------- stacks ---- */
#define K3X_STACK_MAX 256
struct k3x_stack {
    int             n, max_T, device, H;
    float           eps;
    k3x_moe_layer  *layers[K3X_STACK_MAX];
    const float    *norm_w[K3X_STACK_MAX];
    float          *y;              /* [max_T][H] normalised activations */
    hipStream_t     cap;            /* private stream the sequence is recorded on */
    hipGraph_t      graph;
    hipGraphExec_t  exec;
    float          *g_h;            /* (h, T) the recorded graph is bound to */
    int             g_T;
};

int k3x_stack_create(k3x_moe_layer *const *layers, const float *const *norm_w, int n_layers,
                     float eps, int max_T, k3x_stack **out)
{
    if (!layers || !norm_w || !out || n_layers <= 0 || n_layers > K3X_STACK_MAX || max_T <= 0)
        return K3X_E_ARG;
    *out = NULL;
    const int H = layers[0] ? layers[0]->cfg.hidden : 0, dev = layers[0] ? layers[0]->device : 0;
    for (int l = 0; l < n_layers; l++) {
        if (!layers[l] || !norm_w[l]) return K3X_E_ARG;
        if (layers[l]->cfg.hidden != H || layers[l]->device != dev) return K3X_E_SHAPE;
        if (layers[l]->timing || layers[l]->nslot || layers[l]->cache_only) return K3X_E_ARG;
    }
    k3x_stack *S = (k3x_stack *)calloc(1, sizeof *S);
    if (!S) return K3X_E_NOMEM;
    int rc = 0;
    S->n = n_layers; S->max_T = max_T; S->device = dev; S->H = H; S->eps = eps;
    for (int l = 0; l < n_layers; l++) { S->layers[l] = layers[l]; S->norm_w[l] = norm_w[l]; }
    HIPCHK(hipSetDevice(dev));
    if (hipMalloc((void **)&S->y, (size_t)max_T * H * 4) != hipSuccess) { rc = K3X_E_NOMEM; goto fail; }
    HIPCHK(hipStreamCreateWithFlags(&S->cap, hipStreamNonBlocking));
    /* every allocation a call can make happens here, never while recording */
    if (max_T > K3X_DECODE_MAX_T)
        for (int l = 0; l < n_layers; l++) RCCHK(k3x_pf_reserve(layers[l], max_T, NULL));
    *out = S;
    return 0;
fail:
    k3x_stack_destroy(S);
    return rc;
}

static int stack_record(k3x_stack *S, float *h, int T)
{
    int rc = 0;
    if (S->exec) { hipGraphExecDestroy(S->exec); S->exec = NULL; }
    if (S->graph) { hipGraphDestroy(S->graph); S->graph = NULL; }
    HIPCHK(hipStreamBeginCapture(S->cap, hipStreamCaptureModeThreadLocal));
    for (int l = 0; l < S->n && !rc; l++) {
        k3x_moe_layer *L = S->layers[l];
        const float *nw = S->norm_w[l];
        if (T <= L->tdec && !L->lat && S->H <= 8192 && !((uintptr_t)nw & 15)) {
            /* decode: the norm is worked out inside the router launch */
            rc = k3x_dev_decode(L, h, h, K3X_F32, T, h, NULL, NULL, nw, S->eps, S->cap);
        } else {
            rc = k3x_rmsnorm(S->y, h, nw, S->H, T, S->eps, S->cap);
            if (!rc) rc = k3x_moe_forward(L, h, S->y, K3X_F32, T, h, NULL, NULL, S->cap);
        }
    }
    hipGraph_t g = NULL;
    const hipError_t ec = hipStreamEndCapture(S->cap, &g);
    if (rc) { if (g) hipGraphDestroy(g); return rc; }
    if (ec != hipSuccess || !g) return K3X_E_HIP;
    S->graph = g;
    HIPCHK(hipGraphInstantiate(&S->exec, S->graph, NULL, NULL, 0));
    S->g_h = h; S->g_T = T;
fail:
    return rc;
}

int k3x_stack_forward(k3x_stack *S, float *h, int T, void *stream)
{
    if (!S || !h || T <= 0 || ((uintptr_t)h & 15)) return K3X_E_ARG;
    if (T > S->max_T) return K3X_E_SHAPE;
    int rc = 0;
    HIPCHK(hipSetDevice(S->device));
    if (!S->exec || S->g_h != h || S->g_T != T) RCCHK(stack_record(S, h, T));
    HIPCHK(hipGraphLaunch(S->exec, (hipStream_t)stream));
fail:
    return rc;
}

void k3x_stack_destroy(k3x_stack *S)
{
    if (!S) return;
    if (S->exec) hipGraphExecDestroy(S->exec);
    if (S->graph) hipGraphDestroy(S->graph);
    if (S->cap) hipStreamDestroy(S->cap);
    if (S->y) hipFree(S->y);
    free(S);
}
