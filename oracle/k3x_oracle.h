/* k3x_oracle.h - CPU restatement of the reference MoE arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or calls this
 * code; only tests/, the smoke check and the CPU-baseline leg of bench.py do, and only
 * to check device results (or, for the baseline, as the CPU path timed beside the GPU).
 *
 * Every function restates one routine of the reference engine's numeric core
 * (src/core/k3_ops.c) with the same floating-point contract: the same accumulator
 * partition, the same reduction tree, the same float/double conversions, compiled with
 * -ffp-contract=off and without -ffast-math.  The file:line each one follows is in its
 * comment.  ko_moe / ko_moe_prefill follow k3_moe / k3_moe_prefill for both forms of the
 * layer: the K3 LatentMoE (cfg.latent > 0: down projection, experts at the latent width,
 * aggregate RMSNorm, up projection, SiTU betas) and the K2-class layer (cfg.latent == 0:
 * no latent, SwiGLU, one shared expert), which the reference computes with latent =
 * hidden, identity down/up and SiTU betas of 2^64; the oracle writes the identity
 * products out (they are exact, see k3x_oracle.c).
 *
 * Parity status of each function (how it is pinned) is stated in its comment.
 */
#ifndef K3X_ORACLE_H
#define K3X_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- primitive kernels --------------------------------------------------------- */
float ko_e2m1(int code);                  /* k3_ops.c:2624-2627 */
float ko_e8m0(int byte);                  /* k3_ops.c:3125-3132 (255 -> 0) */
float ko_sigmoidf(float x);               /* k3_ops.c:143 */

void ko_rmsnorm(float *y, const float *x, const float *w, int n, float eps);
void ko_situ_glu(float *y, const float *x, int n, float b1, float b2);
void ko_router(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale);
/* returns 0, or -1 when in is odd or group is not a multiple of 16 (the x86 flat
 * contract this oracle restates covers group % 16 == 0 only) */
int  ko_matmul_mxfp4(float *y, const float *x, const uint8_t *packed,
                     const uint8_t *scales, int in, int rows, int group);
void ko_mxfp4_dequant(float *y, const uint8_t *packed, const uint8_t *scales, int rows,
                      int pcols, int group);
void ko_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out);
void ko_matmul_f32(float *y, const float *x, const float *W, int in, int out);

/* ---- the K2-class MoE layer ---------------------------------------------------- */
typedef struct {
    int   hidden, n_experts, topk, moe_inter, n_shared;
    int   renorm;
    float routed_scale;
    float situ_b1, situ_b2;        /* 2^64 for SwiGLU */
    int   group;                   /* MXFP4 group, 32 */
    /* the LatentMoE fields (K3Cfg, k3.h:94-102); all zero for the K2 form */
    int   latent;                  /* routed-expert width; 0: no projection (z = x) */
    int   latent_norm;             /* 1: RMSNorm of the routed aggregate (k3_ops.c:1946) */
    float rms_eps;
} ko_cfg;

typedef struct {
    const uint8_t *p1, *s1;        /* gate [I][H/2], [I][H/group] */
    const uint8_t *p3, *s3;        /* up   [I][H/2], [I][H/group] */
    const uint8_t *p2, *s2;        /* down [H][I/2], [H][I/group] */
} ko_expert;

/* Expert supplier, the K3ExpertSrc.get contract (k3.h:518-523): 0 on success. */
typedef int (*ko_get_fn)(void *ctx, int expert, ko_expert *q);

typedef struct {
    const float    *gate, *bias;   /* [n_experts][hidden] fp32, [n_experts] fp32 */
    ko_get_fn       get;
    void           *ctx;
    const void     *sh1, *sh3;     /* [n_shared*I][hidden] */
    const void     *sh2;           /* [hidden][n_shared*I] */
    /* LatentMoE (K3MoeW, k3.h:546-569): used when cfg.latent > 0 */
    const void     *down, *up;     /* [latent][hidden], [hidden][latent] */
    const float    *latent_norm;   /* [latent] fp32 */
    int             trunk_f32;     /* 0: down/up/sh* are bf16 (K3_WBF16); 1: fp32 */
    /* resident fp32 expert bank (the reference's w1/w3/w2, fixtures only), used when
     * get is NULL: w1/w3 [n_experts][I][latent], w2 [n_experts][latent][I] */
    const float    *w1, *w3, *w2;
} ko_weights;

/* Per token: route, run the top-k experts, combine in top-k order, add the shared
 * expert. idx/wt receive [T][topk] routing (the reference leaves only the last token's;
 * this keeps every token's for the tests). Returns the number of dropped experts. */
long ko_moe(float *out, const float *x, int T, const ko_cfg *c, const ko_weights *w,
            int *idx, float *wt);
/* The batched-prefill form (unique experts in first-seen order per 64-token sub-chunk,
 * contributions summed in top-k order). Bit-identical to ko_moe; get() is called once
 * per unique expert per sub-chunk, and *n_get receives the number of get() calls. */
long ko_moe_prefill(float *out, const float *x, int T, const ko_cfg *c,
                    const ko_weights *w, int *idx, float *wt, long *n_get);

/* Eight-layer stack step (BASELINE config 4 shape): h += MoE_l(RMSNorm_l(h)), layer by
 * layer, following the decoder layer's MoE half (k3_ops.c:2559-2589). */
long ko_stack_step(float *h, int T, int n_layers, const ko_cfg *c,
                   const ko_weights *const *w, const float *const *norm_w, float eps);

/* Block attention-residual aggregation (k3_attn_res, k3_ops.c:1722-1753): per source s
 * of nsrc rows of n, score_s = sum_i (v_i * inv_s) * fold_i in double (inv_s the row's
 * 1/rms), softmax of the scores (expf, double sum), out = sum_s p_s * v_s in float. */
void ko_attn_res(float *out, const float *src, const float *fold, int nsrc, int n, float eps);

/* The MoE half of a decoder layer (k3_decoder_layer_core, k3_ops.c:2546-2589) for T
 * rows: h[t] = attn_res(blocks[t][0 .. nb-1], pref[t]); hin = RMSNorm(h; post_norm);
 * tmp = MoE(hin); pref += tmp; h = pref.  blocks [T][maxb][H]. */
long ko_moe_half(float *h, float *pref, const float *blocks, int maxb, int nb,
                 const float *fold, const float *post_norm, float eps, int T,
                 const ko_cfg *c, const ko_weights *w);
/* The same with row t's block count nbv[t * nbs] (nbs 0: one shared count, 1: one per
 * row; k3_ops.c:2481-2493), as the speculative caller passes them (:2606-2613). */
long ko_moe_half_v(float *h, float *pref, const float *blocks, int maxb, const int *nbv,
                   int nbs, const float *fold, const float *post_norm, float eps, int T,
                   const ko_cfg *c, const ko_weights *w);

/* ---- synthetic inputs ---------------------------------------------------------- */
/* The counter-based generator shared by the tests and the product's synthetic-layer
 * builder: value i of a stream depends only on (seed, layer, stream, sub, i). */
/* k3_moe / k3_moe_prefill with K3MoeW.cache_only (k3_ops.c:1884-1926, :2018): each
 * token's top-k filtered to the experts with res[e] != 0, weights renormalised over them;
 * idx/wt [T][K] hold the kept experts first and the router's values after them. */
long ko_moe_cache_only(float *out, const float *x, int T, const ko_cfg *c,
                       const ko_weights *w, const int *res, int *idx, float *wt);

/* The opt-in MXFP8-activation prefill mode (no reference counterpart; the definition
 * is at the top of its section in k3x_oracle.c): E4M3 decode and round-to-nearest-even
 * (|v| <= 448), the block scale byte, MXFP8 quantisation and dequantisation of n % 32 == 0
 * elements, the MXFP4 x MXFP8 product, and the whole layer (drops counted as ko_moe). */
float ko_e4m3(int code);
int   ko_e4m3_rne(float v);
int   ko_mx8_scale(const float *v, int n);
void  ko_mx8_quant(uint8_t *codes, uint8_t *scales, const float *x, int n);
void  ko_mx8_dequant(double *y, const uint8_t *codes, const uint8_t *scales, int n);
void  ko_matmul_mx(float *y, const uint8_t *xc, const uint8_t *xs, const uint8_t *packed,
                   const uint8_t *wscales, int in, int rows);
long  ko_moe_mx(float *out, const float *x, int T, const ko_cfg *c, const ko_weights *w,
                int *idx, float *wt);

uint64_t ko_mix64(uint64_t z);
uint64_t ko_key(uint64_t seed, int layer, int stream, int sub);
uint64_t ko_draw(uint64_t key, uint64_t i);
void ko_fill_normal_f32(float *dst, size_t n, uint64_t key, double mu, double sigma);
void ko_fill_normal_bf16(uint16_t *dst, size_t n, uint64_t key, double mu, double sigma);
void ko_fill_codes(uint8_t *dst, size_t n, uint64_t key);
void ko_fill_scales(uint8_t *dst, size_t n, uint64_t key, int lo, int hi);
void ko_zipf_bias(float *bias, int n_experts, uint64_t key, double alpha, double s);
uint16_t ko_f32_to_bf16(float f);

/* ---- bench helper -------------------------------------------------------------- */
double ko_now(void);
int    ko_threads(void);

#ifdef __cplusplus
}
#endif
#endif
