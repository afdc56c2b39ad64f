/* ref_driver.c - a thin harness around the COMPILED REFERENCE (test infrastructure).
 *
 * Built only by oracle/Makefile's `ref` target, together with the reference's own
 * src/core/k3_ops.c compiled where it lies, into oracle/_ref/libk3ref.so.  It exists so
 * the tests can run the reference's k3_moe / k3_moe_prefill on a K2-class layer or a K3
 * LatentMoE layer and compare the oracle's restatement against it bit for bit.
 *
 * The K2 layer is expressed with the reference's own types (k3.h:94-102, 507-569):
 * latent = hidden with bf16 identity down/up projections, latent_norm off, SiTU betas
 * 2^64 (SwiGLU), one shared expert, experts served through a K3ExpertSrc whose get()
 * points into caller-owned packed MXFP4 arrays.
 */
#include "k3.h"

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const unsigned char *p1, *s1, *p3, *s3, *p2, *s2;
} drv_expert;

typedef struct {
    K3ExpertSrc       src;     /* first member: get() casts self back */
    const drv_expert *bank;
    int               n;
    const int        *fail;    /* optional [n]: 1 makes get() fail (a forced drop) */
    const int        *res;     /* optional [n]: resident() reports res[e] != 0 */
    long              gets;
} drv_src;

static int drv_get(K3ExpertSrc *self, int layer, int e, K3ExpertQ *out)
{
    drv_src *s = (drv_src *)self;
    (void)layer;
    s->gets++;
    if (e < 0 || e >= s->n) return -1;
    if (s->fail && s->fail[e]) return -1;
    out->p1 = s->bank[e].p1; out->s1 = s->bank[e].s1;
    out->p3 = s->bank[e].p3; out->s3 = s->bank[e].s3;
    out->p2 = s->bank[e].p2; out->s2 = s->bank[e].s2;
    return 0;
}

static int drv_resident(K3ExpertSrc *self, int layer, int e, K3ExpertQ *out)
{
    drv_src *s = (drv_src *)self;
    (void)layer;
    if (e < 0 || e >= s->n || (s->res && !s->res[e])) return 0;
    if (out) {
        out->p1 = s->bank[e].p1; out->s1 = s->bank[e].s1;
        out->p3 = s->bank[e].p3; out->s3 = s->bank[e].s3;
        out->p2 = s->bank[e].p2; out->s2 = s->bank[e].s2;
    }
    return 1;
}

static uint16_t *identity_bf16(int n)
{
    uint16_t *m = (uint16_t *)calloc((size_t)n * n, sizeof(uint16_t));
    if (!m) return NULL;
    for (int i = 0; i < n; i++) m[(size_t)i * n + i] = 0x3F80; /* 1.0 */
    return m;
}

/* Runs k3_moe (prefill == 0) or k3_moe_prefill (prefill == 1) over T tokens.
 * idx/wt receive the LAST token's routing (what the reference leaves there).
 * Returns the change in k3_expert_drops; *gets receives the number of get() calls. */
long refdrv_moe(float *out, const float *x, int T, int hidden, int n_experts, int topk,
                int inter, int n_shared, float routed_scale, int renorm,
                const float *gate, const float *bias, const drv_expert *bank,
                const int *fail, const uint16_t *sh1, const uint16_t *sh3,
                const uint16_t *sh2, int prefill, int *idx, float *wt, long *gets)
{
    K3Cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = hidden;
    c.n_experts = n_experts;
    c.topk = topk;
    c.n_shared = n_shared;
    c.latent = hidden;
    c.moe_inter = inter;
    c.routed_scale = routed_scale;
    c.moe_renorm = renorm;
    c.latent_norm = 0;
    c.situ_b1 = 0x1p64f;
    c.situ_b2 = 0x1p64f;
    c.rms_eps = 1e-5f;

    uint16_t *eye = identity_bf16(hidden);
    if (!eye) return -1000000;
    drv_src s;
    memset(&s, 0, sizeof s);
    s.src.get = drv_get;
    s.bank = bank;
    s.n = n_experts;
    s.fail = fail;

    K3MoeW w;
    memset(&w, 0, sizeof w);
    w.gate = gate;
    w.bias = bias;
    w.down = eye;
    w.up = eye;
    w.sh1 = sh1;
    w.sh3 = sh3;
    w.sh2 = sh2;
    w.wdt = K3_WBF16;
    w.src = &s.src;
    w.layer = 0;

    float *scratch = (float *)malloc(k3_moe_scratch(&c, T) * sizeof(float));
    if (!scratch) { free(eye); return -1000000; }
    const long d0 = k3_expert_drops;
    if (prefill) k3_moe_prefill(out, x, &w, &c, T, idx, wt, scratch);
    else         k3_moe(out, x, &w, &c, T, idx, wt, scratch);
    const long dd = k3_expert_drops - d0;
    if (gets) *gets = s.gets;
    free(scratch);
    free(eye);
    return dd;
}

/* The layer in general form (the K3 LatentMoE, or anything K3Cfg expresses): k3_moe
 * (prefill == 0) or k3_moe_prefill (prefill == 1) with the trunk matrices down/up/sh*
 * as given (bf16 when trunk_f32 == 0, else fp32) and experts from the same get() source
 * as refdrv_moe.  Same return and outputs as refdrv_moe. */
typedef struct {
    int   hidden, latent, n_experts, topk, inter, n_shared, renorm, latent_norm;
    float routed_scale, rms_eps, situ_b1, situ_b2;
} drv_cfg;

long refdrv_moe_cfg(float *out, const float *x, int T, const drv_cfg *dc, const float *gate,
                    const float *bias, const drv_expert *bank, const int *fail,
                    const void *down, const void *up, const float *lnorm, const void *sh1,
                    const void *sh3, const void *sh2, int trunk_f32, int prefill, int *idx,
                    float *wt, long *gets)
{
    K3Cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = dc->hidden;
    c.latent = dc->latent;
    c.n_experts = dc->n_experts;
    c.topk = dc->topk;
    c.moe_inter = dc->inter;
    c.n_shared = dc->n_shared;
    c.routed_scale = dc->routed_scale;
    c.moe_renorm = dc->renorm;
    c.latent_norm = dc->latent_norm;
    c.situ_b1 = dc->situ_b1;
    c.situ_b2 = dc->situ_b2;
    c.rms_eps = dc->rms_eps;

    drv_src s;
    memset(&s, 0, sizeof s);
    s.src.get = drv_get;
    s.bank = bank;
    s.n = dc->n_experts;
    s.fail = fail;

    K3MoeW w;
    memset(&w, 0, sizeof w);
    w.gate = gate;
    w.bias = bias;
    w.down = down;
    w.up = up;
    w.latent_norm = lnorm;
    w.sh1 = sh1;
    w.sh3 = sh3;
    w.sh2 = sh2;
    w.wdt = trunk_f32 ? K3_WF32 : K3_WBF16;
    w.src = &s.src;
    w.layer = 0;

    float *scratch = (float *)malloc(k3_moe_scratch(&c, T) * sizeof(float));
    if (!scratch) return -1000000;
    const long d0 = k3_expert_drops;
    if (prefill) k3_moe_prefill(out, x, &w, &c, T, idx, wt, scratch);
    else         k3_moe(out, x, &w, &c, T, idx, wt, scratch);
    const long dd = k3_expert_drops - d0;
    if (gets) *gets = s.gets;
    free(scratch);
    return dd;
}

/* The decoder layer's MLP half (k3_decoder_layer_core, k3_ops.c:2546-2589) with the
 * reference's own k3_attn_res, k3_rmsnorm and k3_moe_prefill, for rows whose block counts
 * are nbv[t * nbs] (K3_NB, :2493): per row the sources are its nb block residuals then
 * pref (:2548-2557), h = AttnRes of them; hin = RMSNorm(h; post_norm); tmp = MoE(hin);
 * pref += tmp; h = pref.  The layer as refdrv_moe_cfg takes it; dc->latent == 0 is the
 * K2 form, expressed as refdrv_moe does (identity bf16 projections at the hidden width,
 * 2^64 betas, no latent norm).  Returns the change in k3_expert_drops. */
long refdrv_moe_half_v(float *h, float *pref, const float *blocks, int maxb, const int *nbv,
                       int nbs, const float *fold, const float *post_norm, float eps, int T,
                       const drv_cfg *dc, const float *gate, const float *bias,
                       const drv_expert *bank, const void *down, const void *up,
                       const float *lnorm, const void *sh1, const void *sh3, const void *sh2)
{
    const int E = dc->hidden;
    drv_cfg kc = *dc;
    uint16_t *eye = NULL;
    if (dc->latent == 0) {
        eye = identity_bf16(E);
        if (!eye) return -1000000;
        kc.latent = E;
        kc.latent_norm = 0;
        kc.situ_b1 = kc.situ_b2 = 0x1p64f;
        down = up = eye;
        lnorm = NULL;
    }
    int nbmax = 0;
    for (int t = 0; t < T; t++) nbmax = nbv[(size_t)t * nbs] > nbmax ? nbv[(size_t)t * nbs] : nbmax;
    float *src = (float *)malloc((size_t)(nbmax + 1) * E * sizeof(float));
    float *hin = (float *)malloc((size_t)T * E * sizeof(float));
    float *tmp = (float *)malloc((size_t)T * E * sizeof(float));
    if (!src || !hin || !tmp) { free(eye); free(src); free(hin); free(tmp); return -1000000; }
    for (int t = 0; t < T; t++) {
        const int nb = nbv[(size_t)t * nbs];
        for (int b = 0; b < nb; b++)
            memcpy(src + (size_t)b * E, blocks + ((size_t)t * maxb + b) * E,
                   (size_t)E * sizeof(float));
        memcpy(src + (size_t)nb * E, pref + (size_t)t * E, (size_t)E * sizeof(float));
        k3_attn_res(h + (size_t)t * E, src, fold, nb + 1, E, eps);
    }
    for (int t = 0; t < T; t++)
        k3_rmsnorm(hin + (size_t)t * E, h + (size_t)t * E, post_norm, E, eps);
    int idx[K3_MAX_TOPK];
    float wt[K3_MAX_TOPK];
    const long dd = refdrv_moe_cfg(tmp, hin, T, &kc, gate, bias, bank, NULL, down, up, lnorm,
                                   sh1, sh3, sh2, 0, 1, idx, wt, NULL);
    for (size_t i = 0; i < (size_t)T * E; i++) pref[i] += tmp[i];
    memcpy(h, pref, (size_t)T * E * sizeof(float));
    free(eye); free(src); free(hin); free(tmp);
    return dd;
}

/* One K2-class layer over T tokens with the reference's own kernels and nothing else:
 * k3_router, then per selected expert 3 x k3_matmul_mxfp4 + k3_situ_glu and the float
 * combine in top-k order (k3_ops.c:1879-1942), then the shared expert with
 * k3_matmul_bf16 + k3_situ_glu (moe_shared, :1848-1860).  Without the identity latent
 * projections of refdrv_moe this is the reference's work for the layer, which is what
 * the CPU baseline times.  Bit-identical to refdrv_moe's output. idx/wt: [T][K]. */
long refdrv_k2_tokens(float *out, const float *x, int T, int H, int E, int K, int I,
                      int SI, float routed_scale, int renorm, const float *gate,
                      const float *bias, const drv_expert *bank, const uint16_t *sh1,
                      const uint16_t *sh3, const uint16_t *sh2, int *idx, float *wt)
{
    float *gu = (float *)malloc((size_t)2 * I * sizeof(float));
    float *act = (float *)malloc((size_t)I * sizeof(float));
    float *edn = (float *)malloc((size_t)H * sizeof(float));
    float *sgu = (float *)malloc((size_t)2 * (SI > 0 ? SI : 1) * sizeof(float));
    float *sdn = (float *)malloc((size_t)H * sizeof(float));
    if (!gu || !act || !edn || !sgu || !sdn) return -1;
    const float b = 0x1p64f;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * H;
        float *acc = out + (size_t)t * H;
        int *it = idx + (size_t)t * K;
        float *wtt = wt + (size_t)t * K;
        k3_router(it, wtt, xt, gate, bias, H, E, K, renorm, routed_scale);
        for (int i = 0; i < H; i++) acc[i] = 0.0f;
        for (int j = 0; j < K; j++) {
            const drv_expert *q = &bank[it[j]];
            k3_matmul_mxfp4(gu, xt, q->p1, q->s1, H, I, K3_MXFP4_GROUP);
            k3_matmul_mxfp4(gu + I, xt, q->p3, q->s3, H, I, K3_MXFP4_GROUP);
            k3_situ_glu(act, gu, I, b, b);
            k3_matmul_mxfp4(edn, act, q->p2, q->s2, I, H, K3_MXFP4_GROUP);
            for (int i = 0; i < H; i++) acc[i] += wtt[j] * edn[i];
        }
        if (SI > 0) {
            k3_matmul_bf16(sgu, xt, sh1, H, SI);
            k3_matmul_bf16(sgu + SI, xt, sh3, H, SI);
            k3_situ_glu(sgu, sgu, SI, b, b);
            k3_matmul_bf16(sdn, sgu, sh2, SI, H);
            for (int i = 0; i < H; i++) acc[i] += sdn[i];
        }
    }
    free(gu); free(act); free(edn); free(sgu); free(sdn);
    return 0;
}

/* One K2-class layer over a prefill chunk of T tokens with the reference's own kernels,
 * in the order of its k3_moe_prefill (k3_ops.c:2008-2053) without the identity latent
 * projections of refdrv_moe: per sub-chunk of 64 positions (MOE_DEDUP_CHUNK, :1993)
 * route every token with k3_router and list the unique experts in first-seen order
 * (:2067-2082), apply each unique expert once to every (token, slot) that chose it,
 * 3 x k3_matmul_mxfp4 + k3_situ_glu (:2086-2113), and sum each token's slots in top-k
 * order (:2115-2130); then the shared expert over all T positions with the batched bf16
 * products k3_mmw_batch_ld (moe_shared, :1848-1860).  What the CPU baseline of a prefill
 * chunk times.  Bit-identical to refdrv_moe(..., prefill = 1).  idx/wt: [T][K]. */
long refdrv_k2_prefill(float *out, const float *x, int T, int H, int E, int K, int I,
                       int SI, float routed_scale, int renorm, const float *gate,
                       const float *bias, const drv_expert *bank, const uint16_t *sh1,
                       const uint16_t *sh3, const uint16_t *sh2, int *idx, float *wt)
{
    enum { SUB = 64 };
    const float b = 0x1p64f;
    float *gu = (float *)malloc((size_t)2 * I * sizeof(float));
    float *act = (float *)malloc((size_t)I * sizeof(float));
    float *contrib = (float *)malloc((size_t)SUB * K * H * sizeof(float));
    int *uniq = (int *)malloc((size_t)E * sizeof(int));
    unsigned char *seen = (unsigned char *)malloc((size_t)E);
    float *sgu = (float *)malloc((size_t)T * 2 * (SI > 0 ? SI : 1) * sizeof(float));
    float *sdn = (float *)malloc((size_t)T * H * sizeof(float));
    long rc = 0;
    if (!gu || !act || !contrib || !uniq || !seen || !sgu || !sdn) { rc = -1; goto done; }
    for (int t0 = 0; t0 < T; t0 += SUB) {
        const int n = T - t0 < SUB ? T - t0 : SUB;
        memset(seen, 0, (size_t)E);
        int nu = 0;
        for (int t = 0; t < n; t++) {
            int *it = idx + (size_t)(t0 + t) * K;
            k3_router(it, wt + (size_t)(t0 + t) * K, x + (size_t)(t0 + t) * H, gate, bias, H,
                      E, K, renorm, routed_scale);
            for (int j = 0; j < K; j++)
                if (it[j] >= 0 && it[j] < E && !seen[it[j]]) { seen[it[j]] = 1; uniq[nu++] = it[j]; }
        }
        for (int u = 0; u < nu; u++) {
            const drv_expert *q = &bank[uniq[u]];
            for (int t = 0; t < n; t++) {
                const int *it = idx + (size_t)(t0 + t) * K;
                const float *xt = x + (size_t)(t0 + t) * H;
                for (int j = 0; j < K; j++) {
                    if (it[j] != uniq[u]) continue;
                    float *cb = contrib + ((size_t)t * K + j) * H;
                    k3_matmul_mxfp4(gu, xt, q->p1, q->s1, H, I, K3_MXFP4_GROUP);
                    k3_matmul_mxfp4(gu + I, xt, q->p3, q->s3, H, I, K3_MXFP4_GROUP);
                    k3_situ_glu(act, gu, I, b, b);
                    k3_matmul_mxfp4(cb, act, q->p2, q->s2, I, H, K3_MXFP4_GROUP);
                }
            }
        }
        for (int t = 0; t < n; t++) {
            const int *it = idx + (size_t)(t0 + t) * K;
            const float *wtt = wt + (size_t)(t0 + t) * K;
            float *acc = out + (size_t)(t0 + t) * H;
            for (int i = 0; i < H; i++) acc[i] = 0.0f;
            for (int j = 0; j < K; j++) {
                if (it[j] < 0) continue;
                const float *cb = contrib + ((size_t)t * K + j) * H;
                for (int i = 0; i < H; i++) acc[i] += wtt[j] * cb[i];
            }
        }
    }
    if (SI > 0) {
        k3_mmw_batch_ld(sgu, 2 * SI, x, H, sh1, K3_WBF16, H, SI, T);
        k3_mmw_batch_ld(sgu + SI, 2 * SI, x, H, sh3, K3_WBF16, H, SI, T);
        for (int t = 0; t < T; t++) {
            float *sg = sgu + (size_t)t * 2 * SI;
            k3_situ_glu(sg, sg, SI, b, b);
        }
        k3_mmw_batch_ld(sdn, H, sgu, 2 * SI, sh2, K3_WBF16, SI, H, T);
        for (size_t i = 0; i < (size_t)T * H; i++) out[i] += sdn[i];
    }
done:
    free(gu); free(act); free(contrib); free(uniq); free(seen); free(sgu); free(sdn);
    return rc;
}

/* One layer of a stack of K2-class layers for T rows: h = h + MoE(RMSNorm(h; norm_w)),
 * the RMSNorm by the reference's k3_rmsnorm and the layer as refdrv_k2_tokens computes it
 * (k3_moe's work, row by row).  What the stack's CPU baseline times, layer by layer.
 * idx/wt: [T][K]. */
long refdrv_k2_norm_layer(float *h, int T, const float *norm_w, float eps, int H, int E,
                          int K, int I, int SI, float routed_scale, int renorm,
                          const float *gate, const float *bias, const drv_expert *bank,
                          const uint16_t *sh1, const uint16_t *sh3, const uint16_t *sh2,
                          int *idx, float *wt)
{
    float *hin = (float *)malloc((size_t)T * H * sizeof(float));
    float *tmp = (float *)malloc((size_t)T * H * sizeof(float));
    long rc = -1;
    if (hin && tmp) {
        for (int t = 0; t < T; t++)
            k3_rmsnorm(hin + (size_t)t * H, h + (size_t)t * H, norm_w, H, eps);
        rc = refdrv_k2_tokens(tmp, hin, T, H, E, K, I, SI, routed_scale, renorm, gate, bias,
                              bank, sh1, sh3, sh2, idx, wt);
        if (rc == 0)
            for (size_t i = 0; i < (size_t)T * H; i++) h[i] += tmp[i];
    }
    free(hin); free(tmp);
    return rc;
}

#ifdef K3X_ADAPTER
/* The reference-side binding of libk3x (kimi-k3-for-me_amd/csrc/k3x_ref_adapter.c). */
int    k3_moe_gpu(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                  int *idx, float *wt, float *scratch);
int    k3_moe_prefill_gpu(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                          int *idx, float *wt, float *scratch);
size_t k3_moe_gpu_scratch(const K3Cfg *c, int T);
void   k3_moe_gpu_release(void);

void refdrv_gpu_release(void) { k3_moe_gpu_release(); }
#endif

/* One call of the layer in general form through a chosen entry point: mode 0 k3_moe,
 * 1 k3_moe_prefill (the reference's CPU path), 2 k3_moe_gpu, 3 k3_moe_prefill_gpu (the
 * GPU binding, in the library built with it; elsewhere *status = -2).  cache_only sets
 * K3MoeW.cache_only with a resident() reporting res[e] != 0 (every expert when res is
 * NULL); trunk_f32 tags the trunk matrices fp32.  *status receives the GPU entry's
 * return (0 or -1; 0 for the CPU modes), *gets the supplier's get() calls.  Returns the
 * change in k3_expert_drops. */
long refdrv_moe_entry(float *out, const float *x, int T, const drv_cfg *dc, const float *gate,
                      const float *bias, const drv_expert *bank, const int *fail,
                      const void *down, const void *up, const float *lnorm, const void *sh1,
                      const void *sh3, const void *sh2, int trunk_f32, int mode,
                      int cache_only, const int *res, int *idx, float *wt, int *status,
                      long *gets)
{
    K3Cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = dc->hidden;
    c.latent = dc->latent;
    c.n_experts = dc->n_experts;
    c.topk = dc->topk;
    c.moe_inter = dc->inter;
    c.n_shared = dc->n_shared;
    c.routed_scale = dc->routed_scale;
    c.moe_renorm = dc->renorm;
    c.latent_norm = dc->latent_norm;
    c.situ_b1 = dc->situ_b1;
    c.situ_b2 = dc->situ_b2;
    c.rms_eps = dc->rms_eps;

    static drv_src s;          /* outlives the call: the binding keeps the layer */
    memset(&s, 0, sizeof s);
    s.src.get = drv_get;
    s.src.resident = drv_resident;
    s.bank = bank;
    s.n = dc->n_experts;
    s.fail = fail;
    s.res = res;

    static K3MoeW w;
    memset(&w, 0, sizeof w);
    w.gate = gate;
    w.bias = bias;
    w.down = down;
    w.up = up;
    w.latent_norm = lnorm;
    w.sh1 = sh1;
    w.sh3 = sh3;
    w.sh2 = sh2;
    w.wdt = trunk_f32 ? K3_WF32 : K3_WBF16;
    w.src = &s.src;
    w.layer = 0;
    w.cache_only = cache_only;

    *status = 0;
    const long d0 = k3_expert_drops;
    if (mode <= 1) {
        float *scratch = (float *)malloc(k3_moe_scratch(&c, T) * sizeof(float));
        if (!scratch) return -1000000;
        if (mode == 1) k3_moe_prefill(out, x, &w, &c, T, idx, wt, scratch);
        else           k3_moe(out, x, &w, &c, T, idx, wt, scratch);
        free(scratch);
    } else {
#ifdef K3X_ADAPTER
        if (k3_moe_gpu_scratch(&c, T) != 0) { *status = -3; return 0; }
        *status = mode == 3 ? k3_moe_prefill_gpu(out, x, &w, &c, T, idx, wt, NULL)
                            : k3_moe_gpu(out, x, &w, &c, T, idx, wt, NULL);
#else
        *status = -2;
#endif
    }
    if (gets) *gets = s.gets;
    return k3_expert_drops - d0;
}
