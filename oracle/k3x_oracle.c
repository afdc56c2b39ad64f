/* k3x_oracle.c - CPU restatement of the reference MoE arithmetic (test infrastructure).
 *
 * Only tests/, the smoke check and bench.py's CPU-baseline leg use this file; the product
 * library never links it.  Build: oracle/Makefile, flags -O3 -ffp-contract=off -fopenmp
 * (the reference's own flags, Makefile:135-139); -ffp-contract=off is load-bearing: every
 * product and sum below is rounded exactly where the reference rounds it.
 *
 * How each function is pinned (beyond re-reading the reference):
 *   ko_e2m1/ko_e8m0/ko_mxfp4_dequant  reference fixture mxfp4.json (real checkpoint bytes,
 *                                     exact) and its swapped-nibble negative; closed form.
 *   ko_matmul_mxfp4                   bitwise against the compiled reference
 *                                     (oracle/_ref) on cancelling data where any other
 *                                     accumulation order changes the bits; within 1e-6
 *                                     of dequantise-then-double-dot (test_expert.c:227).
 *   ko_matmul_bf16 / ko_matmul_f32    bitwise against oracle/_ref on cancelling data.
 *   ko_router                         reference fixture router.json (index sets and
 *                                     weights); bitwise against oracle/_ref; brute-force
 *                                     top-k with lower-index ties.
 *   ko_situ_glu                       situ_glu.json; closed form of SwiGLU at 2^64 betas.
 *   ko_rmsnorm                        rmsnorm.json.
 *   ko_attn_res                       attnres.json; bitwise against oracle/_ref's
 *                                     k3_attn_res; one source returns it unchanged.
 *   ko_moe_half / ko_moe_half_v       bitwise against the reference's k3_attn_res,
 *                                     k3_rmsnorm and k3_moe_prefill composed as the
 *                                     decoder layer's MLP half (oracle/ref_driver.c,
 *                                     refdrv_moe_half_v) with per-row block counts; with
 *                                     no block residual, one ko_stack_step.
 *   ko_moe / ko_moe_prefill           bitwise against the reference's k3_moe /
 *                                     k3_moe_prefill (oracle/_ref) on the same layer,
 *                                     expressed with identity latent projections.
 */
#include "k3x_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ----------------------------------------------------------------- tables ---- */
/* OCP MX E2M1, bit 3 is the sign: k3_ops.c:2624-2627. */
static const float E2M1[16] = {
    0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
   -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f
};

float ko_e2m1(int code) { return E2M1[code & 15]; }

/* E8M0: 2^(b-127), and the NaN byte 255 maps to zero (k3_ops.c:3125-3132). ldexpf gives
 * the subnormal 2^-127 for byte 0, as the reference's table does. */
float ko_e8m0(int b) { return (b == 255) ? 0.0f : ldexpf(1.0f, b - 127); }

/* k3_ops.c:143 */
float ko_sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

/* --------------------------------------------------------------- rmsnorm ---- */
/* k3_ops.c:132-140: double sum of squares, inv rounded to float once, y = w*x*inv
 * evaluated left to right in float. */
void ko_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (int i = 0; i < n; i++) y[i] = w[i] * x[i] * inv;
}

/* -------------------------------------------------------------- SiTU-GLU ---- */
/* k3_ops.c:148-161. x = [gate | up], n each; y may alias the gate half. With
 * b1 = b2 = 2^64, b*tanhf(v/b) returns v for every float the layers produce, and this is
 * (g*sigmoid(g))*u, i.e. SwiGLU, with the reference's rounding. */
void ko_situ_glu(float *y, const float *x, int n, float b1, float b2)
{
    const float *gate = x, *up = x + n;
    for (int i = 0; i < n; i++) {
        const float g = gate[i];
        const float a = b1 * tanhf(g / b1) * ko_sigmoidf(g);
        const float u = b2 * tanhf(up[i] / b2);
        y[i] = a * u;
    }
}

/* ---------------------------------------------------------------- router ---- */
/* k3_ops.c:1624-1719. Each logit is ONE sequential chain of double adds over i in
 * ascending order, starting at 0.0; the product of two floats is exact in double so
 * fusing it or not changes nothing.  score = 1/(1+expf(-(float)logit)), choice =
 * score + bias in float.  Top-k by repeated maximum with strict '>' (lowest index wins a
 * tie), taken entries set to -inf; weights are the UNBIASED scores; renorm divides by the
 * double sum plus 1e-20 through a float reciprocal; then routed_scale. */
void ko_router(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale)
{
    float *score  = (float *)malloc((size_t)n_experts * sizeof(float));
    float *choice = (float *)malloc((size_t)n_experts * sizeof(float));
    if (!score || !choice) abort();
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n_experts >= 64)
#endif
    for (int e = 0; e < n_experts; e++) {
        const float *row = W + (size_t)e * hidden;
        double acc = 0.0;
        for (int i = 0; i < hidden; i++) acc += (double)row[i] * (double)x[i];
        score[e]  = 1.0f / (1.0f + expf(-(float)acc));
        choice[e] = score[e] + (bias ? bias[e] : 0.0f);
    }
    for (int j = 0; j < topk; j++) {
        int best = -1; float bv = -INFINITY;
        for (int e = 0; e < n_experts; e++)
            if (choice[e] > bv) { bv = choice[e]; best = e; }
        if (best < 0) { idx[j] = 0; w[j] = 0.0f; continue; }
        idx[j] = best;
        w[j] = score[best];
        choice[best] = -INFINITY;
    }
    if (renorm && topk > 1) {
        double s = 0.0;
        for (int j = 0; j < topk; j++) s += (double)w[j];
        const float inv = (float)(1.0 / (s + 1e-20));
        for (int j = 0; j < topk; j++) w[j] *= inv;
    }
    for (int j = 0; j < topk; j++) w[j] *= routed_scale;
    free(score); free(choice);
}

/* ----------------------------------------------------------------- MXFP4 ---- */
/* The x86 FLAT ROW contract of k3_matmul_mxfp4 (k3_ops.c:3427-3527, reproduced by the
 * AVX-512 form at :3159-3281; written out in tests/unit/test_matmul_exact.c:22-31):
 *   - weight w_i = (double)(float)(E2M1[code_i] * E8M0[scale of i's group]) -- the
 *     product is formed in FLOAT, then widened;
 *   - element i goes to accumulator a[i % 16], ascending i, one fma each;
 *   - a 16-element chunk whose group scale byte is 255 is skipped entirely;
 *   - reduction q_l = (a_l + a_{l+8}) + (a_{l+4} + a_{l+12}), then (q0+q2)+(q1+q3);
 *   - a serial fma tail for in % 16 (not skipped for byte 255), y = (float)acc with no
 *     NaN canonicalisation.
 * Low nibble = even element (k3_ops.c:3801-3803). Requires group % 16 == 0. */
static double mxfp4_row(const uint8_t *pr, const uint8_t *sr, const float *x, int in,
                        int group)
{
    double a[16] = {0};
    const int cpg = group >> 4;
    int i = 0, g = 0, c = 0;
    for (; i + 15 < in; i += 16) {
        const int sb = sr[g];
        if (sb != 255) {
            const float sc = ko_e8m0(sb);
            for (int l = 0; l < 16; l++) {
                const int by = pr[(i + l) >> 1];
                const int nib = ((i + l) & 1) ? (by >> 4) : (by & 15);
                const double wv = (double)(float)(E2M1[nib] * sc);
                a[l] = fma(wv, (double)x[i + l], a[l]);
            }
        }
        if (++c == cpg) { c = 0; g++; }
    }
    double q[4];
    for (int l = 0; l < 4; l++) q[l] = (a[l] + a[l + 8]) + (a[l + 4] + a[l + 12]);
    double acc = (q[0] + q[2]) + (q[1] + q[3]);
    for (; i < in; i++) {
        const int by = pr[i >> 1];
        const int nib = (i & 1) ? (by >> 4) : (by & 15);
        acc = fma((double)(float)(E2M1[nib] * ko_e8m0(sr[i / group])), (double)x[i], acc);
    }
    return acc;
}

int ko_matmul_mxfp4(float *y, const float *x, const uint8_t *packed,
                    const uint8_t *scales, int in, int rows, int group)
{
    if ((in & 1) || group <= 0 || (group & 15)) return -1;
    const int pcols = in / 2, ngrp = (in + group - 1) / group;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (rows > 64)
#endif
    for (int r = 0; r < rows; r++)
        y[r] = (float)mxfp4_row(packed + (size_t)r * pcols, scales + (size_t)r * ngrp, x,
                                in, group);
    return 0;
}

/* k3_ops.c:3778-3808: exact dequantisation, E8M0 255 -> 0. */
void ko_mxfp4_dequant(float *y, const uint8_t *packed, const uint8_t *scales, int rows,
                      int pcols, int group)
{
    const int in = 2 * pcols, ngrp = (in + group - 1) / group;
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < in; i++) {
            const int by = packed[(size_t)r * pcols + (i >> 1)];
            const int nib = (i & 1) ? (by >> 4) : (by & 15);
            y[(size_t)r * in + i] = E2M1[nib] * ko_e8m0(scales[(size_t)r * ngrp + i / group]);
        }
}

/* ------------------------------------------------------- bf16 / fp32 GEMV ---- */
/* k3_ops.c:380-420 and 2686-2692: sixteen double accumulators, element i fused into
 * a[i % 16] in ascending i; k3_tree16; sequential fma tail; every NaN result stored as
 * the one quiet NaN 0x7FC00000. bf16 widens by a 16-bit shift (k3.h:369-376). */
static double tree16(const double *a)
{
    const double b0 = (a[0] + a[4]) + (a[8]  + a[12]);
    const double b1 = (a[1] + a[5]) + (a[9]  + a[13]);
    const double b2 = (a[2] + a[6]) + (a[10] + a[14]);
    const double b3 = (a[3] + a[7]) + (a[11] + a[15]);
    return (b0 + b1) + (b2 + b3);
}

static float out_f32(double acc)
{
    union { uint32_t u; float f; } v;
    v.f = (float)acc;
    if (v.f != v.f) v.u = 0x7FC00000u;
    return v.f;
}

static float bf16f(uint16_t h)
{
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)h << 16;
    return v.f;
}

void ko_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out)
{
    const int n16 = in & ~15;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) {
        const uint16_t *row = W + (size_t)o * in;
        double a[16] = {0};
        for (int i = 0; i < n16; i += 16)
            for (int l = 0; l < 16; l++)
                a[l] = fma((double)bf16f(row[i + l]), (double)x[i + l], a[l]);
        double acc = tree16(a);
        for (int i = n16; i < in; i++) acc = fma((double)bf16f(row[i]), (double)x[i], acc);
        y[o] = out_f32(acc);
    }
}

void ko_matmul_f32(float *y, const float *x, const float *W, int in, int out)
{
    const int n16 = in & ~15;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (out > 64)
#endif
    for (int o = 0; o < out; o++) {
        const float *row = W + (size_t)o * in;
        double a[16] = {0};
        for (int i = 0; i < n16; i += 16)
            for (int l = 0; l < 16; l++)
                a[l] = fma((double)row[i + l], (double)x[i + l], a[l]);
        double acc = tree16(a);
        for (int i = n16; i < in; i++) acc = fma((double)row[i], (double)x[i], acc);
        y[o] = out_f32(acc);
    }
}

/* --------------------------------------------------------------- MoE layer ---- */
/* k3_moe / k3_moe_prefill (k3_ops.c:1862-1952, 2008-2132).  The LatentMoE order
 * (k3_ops.c:1793-1811): route on the full-width x; z = down . x; the selected experts at
 * the latent width, their outputs summed in float in top-k order; RMSNorm of that
 * aggregate when latent_norm; out = up . aggregate; then the shared expert on the
 * ORIGINAL x, added unweighted.  Every trunk product (down, up, sh1, sh3, sh2) is the
 * reference's k3_mmw_batch, which is bit-identical per position to the single-position
 * GEMV (k3.h:437-444), so the oracle applies ko_matmul_bf16 / ko_matmul_f32 per token.
 *
 * With cfg.latent == 0 there is no projection: the reference's K2 emulation uses identity
 * down/up, and those products are exact (row o of an identity matrix has one non-zero
 * product, 1 * v, and fifteen accumulators of signed zeros, so k3_tree16 returns v and
 * (float) gives v back), so z = x and out = aggregate before the shared expert. */

typedef struct {
    float *gu, *act, *edn, *sgu, *sdn, *z, *acc;
} moe_tmp;

static int latent_of(const ko_cfg *c) { return c->latent > 0 ? c->latent : c->hidden; }

static int moe_tmp_alloc(moe_tmp *m, const ko_cfg *c)
{
    const size_t I = (size_t)c->moe_inter, H = (size_t)c->hidden;
    const size_t L = (size_t)latent_of(c);
    const size_t SI = I * (size_t)c->n_shared;
    m->gu  = (float *)malloc(2 * I * sizeof(float));
    m->act = (float *)malloc(I * sizeof(float));
    m->edn = (float *)malloc(L * sizeof(float));
    m->sgu = (float *)malloc((2 * SI + 1) * sizeof(float));
    m->sdn = (float *)malloc(H * sizeof(float));
    m->z   = (float *)malloc(L * sizeof(float));
    m->acc = (float *)malloc(L * sizeof(float));
    return (m->gu && m->act && m->edn && m->sgu && m->sdn && m->z && m->acc) ? 0 : -1;
}

static void moe_tmp_free(moe_tmp *m)
{
    free(m->gu); free(m->act); free(m->edn); free(m->sgu); free(m->sdn); free(m->z);
    free(m->acc);
}

/* A trunk product (k3_mmw_batch per position): bf16 or fp32 weights. */
static void trunk_mm(float *y, const float *x, const void *W, int f32, int in, int out)
{
    if (f32) ko_matmul_f32(y, x, (const float *)W, in, out);
    else     ko_matmul_bf16(y, x, (const uint16_t *)W, in, out);
}

/* Expert e fetched for use: 0, or non-zero for a drop (the get() contract).  The
 * resident fp32 bank needs no fetch (k3_ops.c:1932-1938). */
static int expert_get(const ko_weights *w, int e, ko_expert *q)
{
    if (!w->get) { memset(q, 0, sizeof *q); return 0; }
    return w->get(w->ctx, e, q);
}

/* One expert applied to one latent row z: k3_ops.c:1928-1931 (MXFP4 gate, up, SiTU,
 * down) or :1932-1938 (the resident fp32 bank through k3_matmul). */
static void expert_apply(float *edn, const float *z, int e, const ko_expert *q,
                         const ko_cfg *c, const ko_weights *w, const moe_tmp *m)
{
    const int L = latent_of(c), I = c->moe_inter;
    if (!w->get) {
        const float *e1 = w->w1 + (size_t)e * I * L;
        const float *e3 = w->w3 + (size_t)e * I * L;
        const float *e2 = w->w2 + (size_t)e * L * I;
        ko_matmul_f32(m->gu,     z, e1, L, I);
        ko_matmul_f32(m->gu + I, z, e3, L, I);
        ko_situ_glu(m->act, m->gu, I, c->situ_b1, c->situ_b2);
        ko_matmul_f32(edn, m->act, e2, I, L);
        return;
    }
    ko_matmul_mxfp4(m->gu,     z, q->p1, q->s1, L, I, c->group);
    ko_matmul_mxfp4(m->gu + I, z, q->p3, q->s3, L, I, c->group);
    ko_situ_glu(m->act, m->gu, I, c->situ_b1, c->situ_b2);
    ko_matmul_mxfp4(edn, m->act, q->p2, q->s2, I, L, c->group);
}

/* moe_shared, k3_ops.c:1848-1860: [sh1.x | sh3.x], SiTU over the gate half, sh2, then
 * out += sdn (unweighted, in float). */
static void shared_add(float *out, const float *xt, const ko_cfg *c, const ko_weights *w,
                       const moe_tmp *m)
{
    const int H = c->hidden, SI = c->moe_inter * c->n_shared;
    if (!w->sh1 || c->n_shared <= 0) return;
    trunk_mm(m->sgu,      xt, w->sh1, w->trunk_f32, H, SI);
    trunk_mm(m->sgu + SI, xt, w->sh3, w->trunk_f32, H, SI);
    ko_situ_glu(m->sgu, m->sgu, SI, c->situ_b1, c->situ_b2);
    trunk_mm(m->sdn, m->sgu, w->sh2, w->trunk_f32, SI, H);
    for (int i = 0; i < H; i++) out[i] += m->sdn[i];
}

/* The latent input of token xt: down . x, or x itself without a projection. */
static const float *latent_in(const float *xt, const ko_cfg *c, const ko_weights *w,
                              float *z)
{
    if (c->latent <= 0) return xt;
    trunk_mm(z, xt, w->down, w->trunk_f32, c->hidden, c->latent);
    return z;
}

/* After the routed aggregate acc of one token: the latent RMSNorm (k3_ops.c:1946), then
 * out = up . acc (:1950); without a projection acc already is out. */
static void latent_out(float *out, float *acc, const ko_cfg *c, const ko_weights *w)
{
    const int L = latent_of(c);
    if (c->latent_norm) ko_rmsnorm(acc, acc, w->latent_norm, L, c->rms_eps);
    if (c->latent > 0) trunk_mm(out, acc, w->up, w->trunk_f32, L, c->hidden);
}

long ko_moe(float *out, const float *x, int T, const ko_cfg *c, const ko_weights *w,
            int *idx, float *wt)
{
    const int H = c->hidden, K = c->topk, L = latent_of(c);
    long drops = 0;
    moe_tmp m;
    if (moe_tmp_alloc(&m, c)) abort();
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * H;
        float *ot = out + (size_t)t * H;
        float *acc = c->latent > 0 ? m.acc : ot;
        int *it = idx + (size_t)t * K;
        float *wtt = wt + (size_t)t * K;
        const float *z = latent_in(xt, c, w, m.z);
        ko_router(it, wtt, xt, w->gate, w->bias, H, c->n_experts, K, c->renorm,
                  c->routed_scale);
        for (int i = 0; i < L; i++) acc[i] = 0.0f;
        for (int j = 0; j < K; j++) {
            ko_expert q;
            if (expert_get(w, it[j], &q) != 0) { drops++; continue; }
            expert_apply(m.edn, z, it[j], &q, c, w, &m);
            const float wj = wtt[j];
            for (int i = 0; i < L; i++) acc[i] += wj * m.edn[i];
        }
        latent_out(ot, acc, c, w);
        shared_add(ot, xt, c, w, &m);
    }
    moe_tmp_free(&m);
    return drops;
}

/* k3_moe with cache_only set (the draft model's routing, k3_ops.c:1884-1896, :1905-1926):
 * each token's top-k is filtered to the experts res[] marks resident, in top-k order,
 * compacted to the front of idx/wt (the slots past the kept count keep the router's
 * values), the kept weights divided by their float sum (when it is positive); only the
 * kept experts are computed, no getmany, and a kept expert is applied without get() (the
 * cache serves it) -- a failed fetch is skipped without a drop.  k3_moe_prefill with
 * cache_only runs this per-token path for every T (:2018). */
long ko_moe_cache_only(float *out, const float *x, int T, const ko_cfg *c,
                       const ko_weights *w, const int *res, int *idx, float *wt)
{
    const int H = c->hidden, K = c->topk, L = latent_of(c);
    moe_tmp m;
    if (moe_tmp_alloc(&m, c)) abort();
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * H;
        float *ot = out + (size_t)t * H;
        float *acc = c->latent > 0 ? m.acc : ot;
        int *it = idx + (size_t)t * K;
        float *wtt = wt + (size_t)t * K;
        const float *z = latent_in(xt, c, w, m.z);
        ko_router(it, wtt, xt, w->gate, w->bias, H, c->n_experts, K, c->renorm,
                  c->routed_scale);
        int nk = 0;
        float wsum = 0.0f;
        for (int j = 0; j < K; j++) {
            const int e = it[j];
            if (e >= 0 && e < c->n_experts && res[e]) {
                it[nk] = it[j]; wtt[nk] = wtt[j]; wsum += wtt[j]; nk++;
            }
        }
        if (wsum > 0.0f) for (int j = 0; j < nk; j++) wtt[j] /= wsum;
        for (int i = 0; i < L; i++) acc[i] = 0.0f;
        for (int j = 0; j < nk; j++) {
            ko_expert q;
            if (expert_get(w, it[j], &q) != 0) continue;
            expert_apply(m.edn, z, it[j], &q, c, w, &m);
            const float wj = wtt[j];
            for (int i = 0; i < L; i++) acc[i] += wj * m.edn[i];
        }
        latent_out(ot, acc, c, w);
        shared_add(ot, xt, c, w, &m);
    }
    moe_tmp_free(&m);
    return 0;
}

/* k3_moe_prefill / moe_prefill_routed, k3_ops.c:2008-2132: per 64-token sub-chunk
 * (MOE_DEDUP_CHUNK, :1993) route every token, collect unique experts in first-seen order,
 * apply each once to every (token, slot) that chose it, then sum each token's
 * contributions in the ORIGINAL top-k order.  T <= 1 falls back to ko_moe (:2018-2021). */
#define KO_DEDUP_CHUNK 64
long ko_moe_prefill(float *out, const float *x, int T, const ko_cfg *c,
                    const ko_weights *w, int *idx, float *wt, long *n_get)
{
    long gets = 0;
    if (T <= 1) {
        long d = ko_moe(out, x, T, c, w, idx, wt);
        if (n_get) *n_get = (long)T * c->topk;
        return d;
    }
    const int H = c->hidden, K = c->topk, L = latent_of(c);
    const int nmax = T < KO_DEDUP_CHUNK ? T : KO_DEDUP_CHUNK;
    float *contrib = (float *)malloc((size_t)nmax * K * L * sizeof(float));
    float *zc = (float *)malloc((size_t)nmax * L * sizeof(float));
    int *uniq = (int *)malloc((size_t)nmax * K * sizeof(int));
    char *seen = (char *)malloc((size_t)c->n_experts);
    int *ridx = (int *)malloc((size_t)nmax * K * sizeof(int));
    moe_tmp m;
    if (!contrib || !zc || !uniq || !seen || !ridx || moe_tmp_alloc(&m, c)) abort();
    long drops = 0;
    for (int t0 = 0; t0 < T; t0 += KO_DEDUP_CHUNK) {
        const int n = (T - t0) < KO_DEDUP_CHUNK ? (T - t0) : KO_DEDUP_CHUNK;
        memset(seen, 0, (size_t)c->n_experts);
        int nu = 0;
        const float *zt[KO_DEDUP_CHUNK];
        for (int t = 0; t < n; t++) {
            const float *xt = x + (size_t)(t0 + t) * H;
            zt[t] = latent_in(xt, c, w, zc + (size_t)t * L);
            int *it = idx + (size_t)(t0 + t) * K;
            ko_router(it, wt + (size_t)(t0 + t) * K, xt, w->gate, w->bias, H, c->n_experts,
                      K, c->renorm, c->routed_scale);
            for (int j = 0; j < K; j++) {
                ridx[t * K + j] = it[j];
                const int e = it[j];
                if (e >= 0 && e < c->n_experts && !seen[e]) { seen[e] = 1; uniq[nu++] = e; }
            }
        }
        for (int u = 0; u < nu; u++) {
            const int e = uniq[u];
            ko_expert q;
            gets++;
            if (expert_get(w, e, &q) != 0) {
                drops++;
                for (int i = 0; i < n * K; i++) if (ridx[i] == e) ridx[i] = -1;
                continue;
            }
            for (int t = 0; t < n; t++)
                for (int j = 0; j < K; j++) {
                    if (ridx[t * K + j] != e) continue;
                    expert_apply(contrib + ((size_t)t * K + j) * L, zt[t], e, &q, c, w, &m);
                }
        }
        for (int t = 0; t < n; t++) {
            float *ot = out + (size_t)(t0 + t) * H;
            float *acc = c->latent > 0 ? m.acc : ot;
            const float *wtt = wt + (size_t)(t0 + t) * K;
            for (int i = 0; i < L; i++) acc[i] = 0.0f;
            for (int j = 0; j < K; j++) {
                if (ridx[t * K + j] < 0) continue;
                const float wj = wtt[j];
                const float *cb = contrib + ((size_t)t * K + j) * L;
                for (int i = 0; i < L; i++) acc[i] += wj * cb[i];
            }
            latent_out(ot, acc, c, w);
        }
    }
    for (int t = 0; t < T; t++)
        shared_add(out + (size_t)t * H, x + (size_t)t * H, c, w, &m);
    moe_tmp_free(&m);
    free(contrib); free(zc); free(uniq); free(seen); free(ridx);
    if (n_get) *n_get = gets;
    return drops;
}

/* The MoE half of k3_decoder_layer_core (k3_ops.c:2559-2589) per layer:
 * hin = RMSNorm(h); tmp = MoE(hin); h += tmp. */
long ko_stack_step(float *h, int T, int n_layers, const ko_cfg *c,
                   const ko_weights *const *w, const float *const *norm_w, float eps)
{
    const int H = c->hidden, K = c->topk;
    float *hin = (float *)malloc((size_t)T * H * sizeof(float));
    float *tmp = (float *)malloc((size_t)T * H * sizeof(float));
    int *idx = (int *)malloc((size_t)T * K * sizeof(int));
    float *wt = (float *)malloc((size_t)T * K * sizeof(float));
    if (!hin || !tmp || !idx || !wt) abort();
    long drops = 0;
    for (int l = 0; l < n_layers; l++) {
        for (int t = 0; t < T; t++)
            ko_rmsnorm(hin + (size_t)t * H, h + (size_t)t * H, norm_w[l], H, eps);
        drops += ko_moe(tmp, hin, T, c, w[l], idx, wt);
        for (size_t i = 0; i < (size_t)T * H; i++) h[i] += tmp[i];
    }
    free(hin); free(tmp); free(idx); free(wt);
    return drops;
}

/* ------------------------------------------------------ decoder-layer glue ---- */
/* k3_attn_res, k3_ops.c:1722-1753: the key of a source is its RMS-normalised row (inv
 * rounded to float once, v*inv in float), dotted with fold (norm weight times projection,
 * folded at load) in one double chain; the maximum subtracted, expf, the double sum z;
 * p = (float)(e/z); out accumulated in float over sources in order, from 0. */
void ko_attn_res(float *out, const float *src, const float *fold, int nsrc, int n, float eps)
{
    float *score = (float *)malloc((size_t)(nsrc > 0 ? nsrc : 1) * sizeof(float));
    if (!score) abort();
    for (int s = 0; s < nsrc; s++) {
        const float *v = src + (size_t)s * n;
        double ss = 0.0;
        for (int i = 0; i < n; i++) ss += (double)v[i] * (double)v[i];
        const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
        double acc = 0.0;
        for (int i = 0; i < n; i++) acc += (double)(v[i] * inv) * (double)fold[i];
        score[s] = (float)acc;
    }
    float m = score[0];
    for (int s = 1; s < nsrc; s++) m = score[s] > m ? score[s] : m;
    double z = 0.0;
    for (int s = 0; s < nsrc; s++) {
        score[s] = expf(score[s] - m);
        z += score[s];
    }
    for (int i = 0; i < n; i++) out[i] = 0.0f;
    for (int s = 0; s < nsrc; s++) {
        const float p = (float)(score[s] / z);
        const float *v = src + (size_t)s * n;
        for (int i = 0; i < n; i++) out[i] += p * v[i];
    }
    free(score);
}

/* k3_decoder_layer_core's MLP half, k3_ops.c:2546-2589: row t's count is nbv[t * nbs]
 * (K3_NB, :2493), its sources gathered as :2548-2557. */
long ko_moe_half_v(float *h, float *pref, const float *blocks, int maxb, const int *nbv,
                   int nbs, const float *fold, const float *post_norm, float eps, int T,
                   const ko_cfg *c, const ko_weights *w)
{
    const int H = c->hidden, K = c->topk;
    int nbmax = 0;
    for (int t = 0; t < T; t++) {
        const int nb = nbv[(size_t)t * nbs];
        if (nb < 0 || nb > maxb) abort();
        nbmax = nb > nbmax ? nb : nbmax;
    }
    float *src = (float *)malloc((size_t)(nbmax + 1) * H * sizeof(float));
    float *hin = (float *)malloc((size_t)T * H * sizeof(float));
    float *tmp = (float *)malloc((size_t)T * H * sizeof(float));
    int *idx = (int *)malloc((size_t)T * K * sizeof(int));
    float *wt = (float *)malloc((size_t)T * K * sizeof(float));
    if (!src || !hin || !tmp || !idx || !wt) abort();
    for (int t = 0; t < T; t++) {
        const int nb = nbv[(size_t)t * nbs];
        for (int b = 0; b < nb; b++)
            memcpy(src + (size_t)b * H, blocks + ((size_t)t * maxb + b) * H, (size_t)H * sizeof(float));
        memcpy(src + (size_t)nb * H, pref + (size_t)t * H, (size_t)H * sizeof(float));
        ko_attn_res(h + (size_t)t * H, src, fold, nb + 1, H, eps);
        ko_rmsnorm(hin + (size_t)t * H, h + (size_t)t * H, post_norm, H, eps);
    }
    const long drops = ko_moe(tmp, hin, T, c, w, idx, wt);
    for (size_t i = 0; i < (size_t)T * H; i++) pref[i] += tmp[i];
    memcpy(h, pref, (size_t)T * H * sizeof(float));
    free(src); free(hin); free(tmp); free(idx); free(wt);
    return drops;
}

long ko_moe_half(float *h, float *pref, const float *blocks, int maxb, int nb,
                 const float *fold, const float *post_norm, float eps, int T,
                 const ko_cfg *c, const ko_weights *w)
{
    const int H = c->hidden, K = c->topk;
    float *src = (float *)malloc((size_t)(nb + 1) * H * sizeof(float));
    float *hin = (float *)malloc((size_t)T * H * sizeof(float));
    float *tmp = (float *)malloc((size_t)T * H * sizeof(float));
    int *idx = (int *)malloc((size_t)T * K * sizeof(int));
    float *wt = (float *)malloc((size_t)T * K * sizeof(float));
    if (!src || !hin || !tmp || !idx || !wt) abort();
    for (int t = 0; t < T; t++) {
        for (int b = 0; b < nb; b++)
            memcpy(src + (size_t)b * H, blocks + ((size_t)t * maxb + b) * H, (size_t)H * sizeof(float));
        memcpy(src + (size_t)nb * H, pref + (size_t)t * H, (size_t)H * sizeof(float));
        ko_attn_res(h + (size_t)t * H, src, fold, nb + 1, H, eps);
        ko_rmsnorm(hin + (size_t)t * H, h + (size_t)t * H, post_norm, H, eps);
    }
    const long drops = ko_moe(tmp, hin, T, c, w, idx, wt);
    for (size_t i = 0; i < (size_t)T * H; i++) pref[i] += tmp[i];
    memcpy(h, pref, (size_t)T * H * sizeof(float));
    free(src); free(hin); free(tmp); free(idx); free(wt);
    return drops;
}

/* ------------------------------------------------------- synthetic inputs ---- */
/* splitmix64 (Steele, Lea, Flood 2014): the i-th output of a stream started at key is
 * mix64(key + (i+1)*golden), so any element can be drawn on its own. */
uint64_t ko_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t ko_key(uint64_t seed, int layer, int stream, int sub)
{
    uint64_t k = ko_mix64(seed + 0x9E3779B97F4A7C15ull * (uint64_t)(layer + 1));
    k = ko_mix64(k ^ (0xD1B54A32D192ED03ull * (uint64_t)(stream + 1)));
    return ko_mix64(k + (uint64_t)(uint32_t)sub);
}

uint64_t ko_draw(uint64_t key, uint64_t i)
{
    return ko_mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

/* One normal per draw by Box-Muller on the draw's two 32-bit halves (both mapped to the
 * open interval (0,1) exactly), evaluated in double and rounded to float once. */
static double normal_of(uint64_t u)
{
    const double u1 = ((double)(u >> 32) + 0.5) * 0x1p-32;
    const double u2 = ((double)(u & 0xFFFFFFFFull) + 0.5) * 0x1p-32;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void ko_fill_normal_f32(float *dst, size_t n, uint64_t key, double mu, double sigma)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > 65536)
#endif
    for (size_t i = 0; i < n; i++) dst[i] = (float)(mu + sigma * normal_of(ko_draw(key, i)));
}

/* float -> bf16 round-to-nearest-even (NaN kept quiet). */
uint16_t ko_f32_to_bf16(float f)
{
    union { float f; uint32_t u; } v = { f };
    if ((v.u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((v.u >> 16) | 0x40u);
    const uint32_t r = 0x7FFFu + ((v.u >> 16) & 1u);
    return (uint16_t)((v.u + r) >> 16);
}

void ko_fill_normal_bf16(uint16_t *dst, size_t n, uint64_t key, double mu, double sigma)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > 65536)
#endif
    for (size_t i = 0; i < n; i++)
        dst[i] = ko_f32_to_bf16((float)(mu + sigma * normal_of(ko_draw(key, i))));
}

/* Packed E2M1 bytes: byte i is byte (i % 8) of draw i / 8, so every nibble is uniform
 * over the sixteen codes. */
void ko_fill_codes(uint8_t *dst, size_t n, uint64_t key)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > 65536)
#endif
    for (size_t i = 0; i < n; i++)
        dst[i] = (uint8_t)(ko_draw(key, i >> 3) >> (8 * (i & 7)));
}

/* E8M0 bytes uniform over [lo, hi]. */
void ko_fill_scales(uint8_t *dst, size_t n, uint64_t key, int lo, int hi)
{
    const uint64_t span = (uint64_t)(hi - lo + 1);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > 65536)
#endif
    for (size_t i = 0; i < n; i++)
        dst[i] = (uint8_t)(lo + (int)((ko_draw(key, i) >> 32) % span));
}

/* Zipf-skewed router bias: bias[e] = alpha * (pi(e)+1)^(-s), pi a seeded permutation
 * (Fisher-Yates on draws of key). */
void ko_zipf_bias(float *bias, int n_experts, uint64_t key, double alpha, double s)
{
    int *perm = (int *)malloc((size_t)n_experts * sizeof(int));
    if (!perm) abort();
    for (int e = 0; e < n_experts; e++) perm[e] = e;
    for (int e = n_experts - 1; e > 0; e--) {
        const int j = (int)(ko_draw(key, (uint64_t)e) % (uint64_t)(e + 1));
        const int t = perm[e]; perm[e] = perm[j]; perm[j] = t;
    }
    for (int e = 0; e < n_experts; e++)
        bias[e] = (float)(alpha * pow((double)(perm[e] + 1), -s));
    free(perm);
}

double ko_now(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int ko_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------- MXFP8-activation prefill mode ---- */
/* The opt-in prefill mode of the device library (K3X_PREFILL_MXFP8) has no counterpart
 * in the reference, whose expert products take fp32 activations.  Its oracle is the
 * reference's MoE arithmetic (k3_moe, k3_ops.c:1862-1952) with one documented change:
 * every activation row entering a routed expert product is first quantised to MXFP8
 * (OCP Microscaling Formats v1.0: blocks of 32 consecutive elements sharing one E8M0
 * scale 2^X, elements in FP8 E4M3, the "FN" encoding: bias 7, no infinities, 448 the
 * largest finite value, 0x7F/0xFF NaN), and the expert products are the exact
 * products of the MXFP4 weights (E2M1 x E8M0 as stored) with those elements, summed in
 * double and rounded to float once.  The quantisation:
 *   - X is the least integer with max|v| <= 448 * 2^X over the block's finite elements
 *     (max|v| = f * 2^E with f in [1, 2): X = E - 8, or E - 7 when f > 1.75), clamped
 *     to [-127, 127]; a block without a non-zero finite element has X = -127;
 *   - each finite element is v * 2^-X (exact) rounded to the nearest E4M3 value, ties
 *     to the even code; a non-finite element is the NaN code 0x7F (sign kept);
 *   - the scale byte is X + 127.
 * Where the quantisation happens: the routed experts' input (x, or z = down . x in a
 * LatentMoE layer) per token, and each expert's activation h = w_j * SiTU(gate, up)
 * with the routing weight w_j folded in before quantising (the device applies it in
 * the gate/up epilogue); the down products are then summed in float in top-k order
 * without a further weight.  Router, shared expert and latent projections are the
 * exact path's.  Pinned in tests/test_oracle_mx.py: the E4M3 rounding against a
 * brute-force nearest search over all 253 finite codes, the scale rule against its
 * definition, the product against dequantise-then-float64-dot, the identity on inputs
 * that MXFP8 represents exactly (the layer then equals ko_moe to float rounding). */

float ko_e4m3(int code)
{
    const int s = code & 0x80, e = (code >> 3) & 15, m = code & 7;
    float v;
    if (e == 15 && m == 7) return s ? -NAN : NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else        v = ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* |v| <= 448 (finite) to the nearest E4M3 value, ties to the even code. */
int ko_e4m3_rne(float v)
{
    const int sign = signbit(v) ? 0x80 : 0;
    const float a = fabsf(v);
    if (a < 0x1p-6f) {                              /* subnormal steps of 2^-9 */
        const int m = (int)nearbyintf(a * 512.0f);  /* 0 .. 8; 8 is 2^-6, code 0x08 */
        return sign | m;
    }
    int E;
    frexpf(a, &E);
    E -= 1;                                         /* a = f * 2^E, f in [1, 2) */
    const int m = (int)nearbyintf(ldexpf(a, 3 - E)); /* 8 .. 16 */
    if (m == 16) return sign | ((E + 8) << 3);
    return sign | ((E + 7) << 3) | (m - 8);
}

int ko_mx8_scale(const float *v, int n)
{
    float amax = 0.0f;
    for (int i = 0; i < n; i++)
        if (isfinite(v[i]) && fabsf(v[i]) > amax) amax = fabsf(v[i]);
    if (amax == 0.0f) return 0;
    uint32_t b;
    memcpy(&b, &amax, 4);
    int X = (int)((b >> 23) & 255u) - 127 - 8 + ((b & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    if (X < -127) X = -127;
    if (X > 127) X = 127;
    return X + 127;
}

void ko_mx8_quant(uint8_t *codes, uint8_t *scales, const float *x, int n)
{
    for (int b = 0; b < n / 32; b++) {
        const float *v = x + 32 * b;
        const int sb = ko_mx8_scale(v, 32);
        scales[b] = (uint8_t)sb;
        for (int i = 0; i < 32; i++) {
            if (!isfinite(v[i])) { codes[32 * b + i] = (uint8_t)((signbit(v[i]) ? 0x80 : 0) | 0x7F); continue; }
            codes[32 * b + i] = (uint8_t)ko_e4m3_rne(ldexpf(v[i], 127 - sb));
        }
    }
}

void ko_mx8_dequant(double *y, const uint8_t *codes, const uint8_t *scales, int n)
{
    for (int i = 0; i < n; i++) y[i] = ldexp((double)ko_e4m3(codes[i]), (int)scales[i / 32] - 127);
}

/* y[r] = sum_i W[r][i] * xq[i], exact products summed in double (ascending i), rounded
 * to float once; W MXFP4 (E2M1 codes, E8M0 scale per 32), xq MXFP8 (n % 32 == 0). */
void ko_matmul_mx(float *y, const uint8_t *xc, const uint8_t *xs, const uint8_t *packed,
                  const uint8_t *wscales, int in, int rows)
{
    double *xd = (double *)malloc((size_t)in * sizeof(double));
    if (!xd) abort();
    ko_mx8_dequant(xd, xc, xs, in);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (rows > 64)
#endif
    for (int r = 0; r < rows; r++) {
        const uint8_t *pr = packed + (size_t)r * (in / 2), *sr = wscales + (size_t)r * (in / 32);
        double acc = 0.0;
        for (int i = 0; i < in; i++) {
            const int by = pr[i >> 1];
            const int nib = (i & 1) ? (by >> 4) : (by & 15);
            const double wv = ldexp((double)E2M1[nib], (int)sr[i / 32] - 127);
            acc += wv * xd[i];
        }
        y[r] = (float)acc;
    }
    free(xd);
}

long ko_moe_mx(float *out, const float *x, int T, const ko_cfg *c, const ko_weights *w,
               int *idx, float *wt)
{
    const int H = c->hidden, K = c->topk, L = latent_of(c), I = c->moe_inter;
    if (!w->get || c->group != 32 || L % 32 || I % 32) return -1;
    long drops = 0;
    moe_tmp m;
    uint8_t *zc = (uint8_t *)malloc((size_t)L), *zs = (uint8_t *)malloc((size_t)L / 32);
    uint8_t *hc = (uint8_t *)malloc((size_t)I), *hs = (uint8_t *)malloc((size_t)I / 32);
    if (!zc || !zs || !hc || !hs || moe_tmp_alloc(&m, c)) abort();
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * H;
        float *ot = out + (size_t)t * H;
        float *acc = c->latent > 0 ? m.acc : ot;
        int *it = idx + (size_t)t * K;
        float *wtt = wt + (size_t)t * K;
        const float *z = latent_in(xt, c, w, m.z);
        ko_mx8_quant(zc, zs, z, L);
        ko_router(it, wtt, xt, w->gate, w->bias, H, c->n_experts, K, c->renorm,
                  c->routed_scale);
        for (int i = 0; i < L; i++) acc[i] = 0.0f;
        for (int j = 0; j < K; j++) {
            ko_expert q;
            if (expert_get(w, it[j], &q) != 0) { drops++; continue; }
            ko_matmul_mx(m.gu,     zc, zs, q.p1, q.s1, L, I);
            ko_matmul_mx(m.gu + I, zc, zs, q.p3, q.s3, L, I);
            ko_situ_glu(m.act, m.gu, I, c->situ_b1, c->situ_b2);
            const float wj = wtt[j];
            for (int i = 0; i < I; i++) m.act[i] = wj == 0.0f ? 0.0f : wj * m.act[i];
            ko_mx8_quant(hc, hs, m.act, I);
            ko_matmul_mx(m.edn, hc, hs, q.p2, q.s2, I, L);
            for (int i = 0; i < L; i++) acc[i] += m.edn[i];
        }
        latent_out(ot, acc, c, w);
        shared_add(ot, xt, c, w, &m);
    }
    moe_tmp_free(&m);
    free(zc); free(zs); free(hc); free(hs);
    return drops;
}
