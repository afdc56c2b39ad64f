/* k3x_internal.h - what the C host layer (k3x_moe.c) and the HIP kernels
 * (k3x_kernels.hip) share: the device layer record, the HBM layouts and the launchers.
 *
 * HBM layout of a layer (one allocation per region, all 256-byte aligned):
 *
 *   router   fp32 [n_experts][hidden]            as given (k3_router's W)
 *   bias     fp32 [n_experts]
 *   experts  n_experts records of K3X tiled MXFP4, each: gate tiles, up tiles, down tiles
 *            (gate/up [I][X], down [X][I], X = latent or hidden)
 *   shared   bf16 tiled gate, up, down (n_shared*moe_inter intermediate)
 *   latent   bf16 tiled down [latent][hidden] and up [hidden][latent], fp32 norm weights
 *   work     the per-call buffers (routing, activations in B-fragment layout, partials)
 *
 * K3X TILED MXFP4 (a matrix of R rows by K columns, R % 16 == 0, K % 128 == 0).
 *   The matrix is cut into R/16 row tiles, stored one after another.  A tile is K/128
 *   "quads" of 128 columns, grouped four to a "super-quad" of 4352 bytes (the last one
 *   padded with zero quads when K/128 is not a multiple of 4).  A super-quad holds the
 *   codes of its 4 quads, 1024 bytes each, then 256 bytes of scales:
 *     codes of quad q, lane l (m = l % 16, kq = l / 16): the 16 bytes of row 16*rt + m
 *       that hold columns 128*q + 32*kq .. +31 (one 32-column scale group, low nibble =
 *       even column, as in the reference's packed rows);
 *     scales, lane l: 4 bytes, byte j = scale byte of row 16*rt + m, group 4*(4*S+j)+kq
 *       (0 where quad 4*S+j does not exist).
 *   So one 16-byte load per lane reads a whole scale group, and a wave's load covers
 *   1024 contiguous bytes.  Lane (m, kq) is the matrix cores' A-operand lane for row m
 *   and k-slots 8*kq..8*kq+7 of v_mfma_f32_16x16x32_bf16; dword t of its 16 bytes feeds
 *   the t-th product of the quad, so product t of quad q pairs k-slot 8*kq + j with
 *   column 128*q + 32*kq + 8*t + j.  The B operand (activations) uses the same map.
 *
 * K3X TILED BF16 (R % 16 == 0, K % 128 == 0): R/16 tiles of K/128 quads of 4 KB; in quad
 *   q, product t, lane l holds row 16*rt + m, columns 128*q + 32*kq + 8*t .. +7.
 *
 * B FRAGMENTS (activations of up to 8 tokens): for a K-long vector set, [K/128][4][64]
 *   entries of 8 bf16: quad q, product t, lane l = n + 16*kq holds column n's elements
 *   128*q + 32*kq + 8*t .. +7.  Column 2*i is token i rounded to bf16 ("hi"), column
 *   2*i+1 the bf16 of the remainder ("lo"); hi + lo carries 16 significant bits.
 */
#ifndef K3X_INTERNAL_H
#define K3X_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "../../include/k3x_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

#define K3X_DECODE_MAX_T 8       /* tokens per call on the decode path (2 columns each) */
#define K3X_WIDE_PMAX 20         /* 2+ tokens: parts of the down products (k3_down_wide) */
#define K3X_DECODE_PARTS 8       /* latent form: parts the unique experts' down products
                                    are split into (partial aggregates, added in order) */
#define K3X_STAGE_MAX    65536   /* bytes of activation fragments a workgroup stages in LDS */
#define K3X_MAX_TOPK     64      /* K3_MAX_TOPK, k3.h:857-864 */
#define K3X_ROUTE_WAIT_DEFAULT 100000000ull  /* 1 s at 100 MHz: decode's bound on the wait */
#define K3X_PF_CHUNK     4096    /* prefill: most tokens per pipeline run */
#define K3X_NOALLOC_BYTES (64u << 20)  /* the no-allocation prefill's static device array */
#define K3X_CACHE_IO     8       /* expert-cache misses read from the store concurrently */
/* byte sizes of the tiled formats */
static inline size_t k3x_fp4_tile_bytes(int K)
{
    const int ns = (K / 128 + 3) / 4;
    return (size_t)ns * 4352;
}
static inline size_t k3x_fp4_matrix_bytes(int R, int K) { return (size_t)(R / 16) * k3x_fp4_tile_bytes(K); }
static inline size_t k3x_bf16_matrix_bytes(int R, int K) { return (size_t)R * K * 2; }

/* routing summary written by the router, read by the expert kernels */
typedef struct k3x_route {
    int   nu;                                   /* unique experts in this call        */
    unsigned seq;                               /* call sequence: 1 at creation, never
                                                   0; advanced by k1 before its use    */
    int   err;                                  /* a routed workgroup gave up waiting */
    int   nexact;                               /* router logits the last selection
                                                   worked out as the reference's chain */
    unsigned hkey[K3X_DECODE_MAX_T];            /* per token: the largest upper bound
                                                   (as a choice key) of a choice whose
                                                   logit is not proven; 0 = none.  Set
                                                   by the router (atomic maximum),
                                                   cleared by the selection that reads it */
    int   pad[60 - K3X_DECODE_MAX_T];
    int   uniq[K3X_DECODE_MAX_T * K3X_MAX_TOPK];        /* first-seen order           */
    float wtok[K3X_DECODE_MAX_T * K3X_MAX_TOPK][K3X_DECODE_MAX_T]; /* [u][token], 0 = not chosen */
    /* the same routing as k2's routed workgroups read it inside the launch that works it
       out: each word (seq << 32) | value, so that a word read with this call's seq holds
       this call's value whatever the order in which the words became visible */
    unsigned long long tnu;
    unsigned long long tuniq[K3X_DECODE_MAX_T * K3X_MAX_TOPK];
    unsigned long long twtok[K3X_DECODE_MAX_T * K3X_MAX_TOPK][K3X_DECODE_MAX_T];
} k3x_route;

/* prefill working buffers (one allocation), sized for cap_T tokens per pipeline run */
#define K3X_PF_RETIRED 24      /* earlier prefill allocations kept until the layer ends */
typedef struct k3x_prefill_buf {
    int       cap_T;
    void     *base;
    size_t    bytes;
    /* allocations replaced by a larger one: a HIP graph recorded over them may still be
     * replayed, so they stay allocated until the layer is destroyed (growth at least
     * doubles the capacity, so there are few) */
    void     *retired[K3X_PF_RETIRED];
    int       nretired;
    size_t    retired_bytes;
    uint16_t *xhl;          /* [T][H/8][2][8] bf16 hi/lo activation rows            */
    float    *score, *choice; /* [T][E]                                             */
    int      *idx;          /* [T][K]                                                */
    float    *wt;           /* [T][K]                                                */
    int      *counts;       /* [E] tokens per expert                                 */
    int      *offsets;      /* [E+1] first permuted row of each expert               */
    int      *cursor;       /* [E]                                                   */
    int      *tb_gu, *tb_dn;  /* [2][E+1] first GEMM tile of each expert in its class */
    void     *desc_gu, *desc_dn;   /* per GEMM tile {expert, row block, row, rows}      */
    int       ndesc_gu, ndesc_dn;  /* entries of each table                            */
    uint16_t *xp;           /* [2][H/8][T*K][8] gate/up activations, permuted rows    */
    int      *perm_tok;     /* [T*K] token of each permuted row                      */
    float    *perm_w;       /* [T*K] routing weight of each permuted row             */
    int      *pos_of;       /* [T*K] permuted row of each (token, slot)              */
    uint16_t *act;          /* [T*K][I/8][2][8] routed activations, hi/lo            */
    uint16_t *act_sh;       /* [T][SI/8][2][8] shared activations                    */
    float    *y;            /* [T*K + T][H] expert and shared output rows            */
    /* latent form (X = latent width) */
    float    *zf;           /* [T][X] z = down . x, then the routed aggregates        */
    uint16_t *zhl;          /* [2][X/8][T][8] hi/lo planes of the normalised
                               aggregates                                             */
    int       no_lib;       /* 1: no library GEMMs (the no-allocation entry point: a
                               library call may load code objects into device memory) */
} k3x_prefill_buf;

struct k3x_moe_layer {
    k3x_cfg   cfg;
    int       device;
    int       SI;                 /* n_shared * moe_inter */
    int       XL;                 /* the routed experts' width: cfg.latent, or hidden */
    int       lat;                /* 1: latent projections (cfg.latent > 0) */
    float     b1, b2;             /* SiTU betas; 0 where that half is uncapped */
    int       tdec;               /* tokens per decode-path call (<= K3X_DECODE_MAX_T) */
    /* weights */
    float    *router;             /* [E][H] */
    float    *bias;               /* [E] (zeros when absent) */
    uint8_t  *experts;            /* E * expert_bytes */
    size_t    expert_bytes, gate_off, up_off, down_off;
    int       special;            /* bit 0 gate, 1 up, 2 down: some expert's matrix has a
                                     scale byte outside 1..252 (the exact dequantisation
                                     kernels are launched) */
    uint16_t *sh_gate, *sh_up, *sh_down;   /* tiled bf16, NULL when SI == 0 */
    /* row-major bf16 copies for the prefill's library GEMMs, when 2*SI <= hidden (the
     * gate/up output then fits the shared rows of the prefill's output buffer): gate rows
     * then up rows [2*SI][H], and down [H][SI]; NULL otherwise */
    uint16_t *sh_gu_rm, *sh_down_rm;
    uint16_t *ldown_rm, *lup_rm;            /* row-major latent projections [XL][H], [H][XL] */
    int       blas;                         /* hipBLASLt is available on the device */
    uint16_t *ldown, *lup;        /* latent projections, tiled bf16 [XL][H] and [H][XL] */
    float    *lnw;                /* [XL] latent RMSNorm weights, or NULL */
    /* decode working buffers */
    float    *score, *choice;     /* [DECODE_MAX_T][E] */
    float    *slack;              /* [DECODE_MAX_T][E] choice slack: 0 where the router's
                                     float logit is proven to be the reference's chain's */
    float    *ninv;               /* [DECODE_MAX_T] 1/rms of the rows the router normalised
                                     (inside the slack allocation) */
    int      *idx;                /* [DECODE_MAX_T][K] */
    float    *wt;                 /* [DECODE_MAX_T][K] */
    k3x_route *route;
    uint16_t *xB;                 /* compact B set of x over whole super-quads of H */
    uint16_t *actB;               /* DECODE_MAX_T*K slots: B set of each unique expert's
                                     activation over whole super-quads of I */
    uint16_t *shB;                /* B set of the shared activation (SI/128 quads) */
    uint16_t *zB;                 /* latent: B set of z = down . x over whole super-quads */
    float    *accL;               /* latent: [max(DECODE_PARTS, WIDE_PMAX)][DECODE_MAX_T][XL] partial
                                     routed aggregates */
    uint16_t *latB;               /* latent: B set of the (normalised) aggregates */
    float    *pacc;               /* K2 form, 2+ tokens: [K3X_WIDE_PMAX][DECODE_MAX_T][H]
                                     part sums of k3_down_wide */
    /* diagnostics (K3X_TRACE=1 at creation): per-workgroup {id | ids, start, end} of the
     * last decode call's k1, k2 and k3, tr_cap records each */
    unsigned long long *tr;
    int       tr_cap, tr_n[3];
    k3x_prefill_buf pf;
    /* prefill: the shared expert's GEMMs run on a stream of their own, forked from the
     * caller's stream after the activation split and joined before the combine (events
     * 0 and 1); NULL when the layer has no shared expert */
    void     *pf_side, *pf_ev[2];
    int       pf_mode;            /* K3X_PREFILL_EXACT or K3X_PREFILL_MXFP8 */
    size_t    bytes;
    /* decode: bound on the routed workgroups' wait for the published selection (ticks of
     * the 100 MHz clock), and a failure-injection switch that withholds the flag */
    uint64_t  wait_ticks;
    int       no_publish;
    /* timing */
    int       timing;
    void     *ev[8];
    int       n_ev_used;
    /* host staging for the drop-in calls */
    void     *h_dev_x, *h_dev_out;
    size_t    h_cap;
    /* expert cache (k3x_moe_layer_create_cached): nslot slots of the expert arena hold the
     * resident experts; 0 when every expert sits at its own index */
    int       nslot;
    int      *slot_dev;           /* [E] slot of each expert, -1 when not resident   */
    int      *slot_of;            /* host copy of slot_dev                            */
    int      *key_of;             /* [nslot] expert held, -1 empty                    */
    uint64_t *used_at;            /* [nslot] LRU stamp                                */
    unsigned char *pinned;        /* [nslot] never evicted while set                  */
    uint64_t  clock, hits, misses, evictions, bytes_read;
    struct k3x_store *st;         /* where misses are read from, or NULL: from c_src   */
    int       st_layer;
    k3x_expert_src *c_src;        /* the supplier misses are fetched through (no store) */
    unsigned char *c_hbuf[K3X_CACHE_IO];  /* pinned host buffers, one expert run each  */
    uint8_t  *c_dbuf[K3X_CACHE_IO];       /* device staging, one expert run each        */
    int       c_nio;              /* staging pairs: misses read together               */
    int      *c_route;            /* pinned host copy of the routing summary (head,
                                     unique list, per-token weights)                 */
    int       c_dirty;            /* slot_of changed since slot_dev was last written   */
    /* cache-only (draft) routing: each token keeps its top-k experts that are resident */
    int       cache_only;
    unsigned char *res_mask;      /* [E] resident experts, or NULL: the HBM slots of a
                                     cached layer (every expert of a resident layer)   */
    int      *c_sel;              /* pinned [2][DECODE_MAX_T * topk]: the selection's
                                     indices, then its weights' bits                  */
};

/* After a decode call's selection (published in the route): with cache-only routing,
 * filter each token's experts to the resident ones and rewrite the route and the
 * caller's idx/wt; for a cached layer, make the named experts resident. */
int k3x_route_host(k3x_moe_layer *L, void *stream, int T, int *uidx, float *uwt);

/* ---- launchers (k3x_kernels.hip), all return 0 or K3X_E_HIP ---------------------- */
int k3x_dev_check(int device);
int k3x_dev_tile_fp4(uint8_t *dst, const uint8_t *packed, const uint8_t *scales, int R,
                     int K, void *stream);
int k3x_dev_tile_bf16(uint16_t *dst, const uint16_t *src, int R, int K, void *stream);
int k3x_dev_untile_fp4(uint8_t *packed, uint8_t *scales, const uint8_t *src, int R, int K,
                       void *stream);
int k3x_dev_dequant_fp4(float *out, const uint8_t *src, int R, int K, int exact,
                        void *stream);
int k3x_dev_synth_fp4(uint8_t *dst, int R, int K, uint64_t code_key, uint64_t scale_key,
                      int lo, int hi, void *stream);
/* norm_w != NULL: the MoE input is the RMSNorm of x (fp32, 16-byte aligned, hidden <=
 * 8192) with those weights and eps, worked out inside the router launch */
int k3x_dev_decode(struct k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                   const float *resid, int *idx, float *wt, const float *norm_w, float eps,
                   void *stream);
int k3x_dev_prefill(struct k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                    const float *resid, int *idx, float *wt, void *stream);
/* the router alone over T tokens (k3x_moe_route): pf_router and pf_topk per prefill chunk,
 * on the layer's prefill buffers (k3x_prefill.hip) */
int k3x_dev_route(struct k3x_moe_layer *L, int *idx, float *wt, const void *x, int x_dtype,
                  int T, void *stream);
/* prefill working buffers for runs of min(T, the chunk) tokens; refuses to grow while
 * `stream` is being captured (k3x_moe.c) */
int k3x_pf_reserve(struct k3x_moe_layer *L, int T, void *stream);
/* The prefill buffers of runs of T tokens carved from p (256-byte aligned regions) into
 * B; returns the bytes they take (with p or B NULL, only that) (k3x_moe.c) */
size_t k3x_pf_layout(const struct k3x_moe_layer *L, int T, char *p, k3x_prefill_buf *B);
/* the prefill pipeline over one run of T <= the chunk tokens with its working buffers
 * in the static device array, never allocating (k3x_prefill.hip) */
int k3x_dev_prefill_noalloc(struct k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                            int T, const float *resid, int *idx, float *wt, void *stream);
/* tokens per prefill pipeline run: at most K3X_PF_CHUNK, and the widest activation
 * planes of a run (T*K rows) stay under 1 GiB so 32-bit buffer offsets hold */
static inline int k3x_pf_chunk_tokens(const struct k3x_moe_layer *L)
{
    size_t wide = (size_t)(L->cfg.hidden > L->cfg.moe_inter ? L->cfg.hidden : L->cfg.moe_inter);
    if ((size_t)L->XL > wide) wide = (size_t)L->XL;
    size_t chunk = ((size_t)1 << 30) / ((size_t)L->cfg.topk * wide * 4);
    return chunk < 1 ? 1 : (chunk > K3X_PF_CHUNK ? K3X_PF_CHUNK : (int)chunk);
}
/* trunk products Y[t*ldy + o] = W[o] . X[t*ldx] over a tiled bf16 W [out][in]: T <= 8
 * (GEMV on the matrix cores) and any T (hi/lo planes into `planes`, T*in*4 bytes, then
 * the dense GEMM) */
/* decoder-layer glue (k3x_glue.hip) */
int k3x_dev_attn_res(float *h, const float *blocks, int maxb, int nb, const int *nbv, int nbs,
                     const float *pref, const float *fold, int n, int T, float eps,
                     void *stream);
int k3x_dev_copy_f32(float *dst, const float *src, size_t n, void *stream);
int k3x_dev_trunk_gemv(const uint16_t *W, int in, int out, float *y, int ldy, const void *x,
                       int x_dtype, int ldx, int T, void *stream);
int k3x_dev_trunk_gemm(const uint16_t *W, int in, int out, float *y, int ldy, const void *x,
                       int x_dtype, int ldx, int T, uint16_t *planes, void *stream);
int k3x_dev_rmsnorm(float *y, const float *x, const float *w, int n, int T, float eps,
                    void *stream);
/* the prefill shared expert's activation from its library gate/up product: ygu [T][2*SI]
 * fp32 (gate columns, then up) -> SiTU, split into bf16 hi and lo rows [T][SI] */
int k3x_dev_glu_rows(const float *ygu, int T, int SI, float b1, float b2, uint16_t *hi,
                     uint16_t *lo, void *stream);
/* fp32 rows [T][ldx] -> bf16 hi and lo rows [T][n] (hi + lo = 16 significant bits of x) */
int k3x_dev_split_rows(const float *x, int ldx, int T, int n, uint16_t *hi, uint16_t *lo,
                       void *stream);
/* plain bf16 GEMMs on hipBLASLt (k3x_blas.cpp): k3x_blas_init once per device, outside
 * graph capture; then Y[t*ldy + o] (+)= W[o] . X[t*ldx], W row-major bf16 [out][in], X
 * bf16 rows, Y fp32.  Non-zero when no kernel serves the shape (the caller falls back). */
int k3x_blas_init(int device);
/* 0 when a kernel serves the shape (chosen now and kept; nothing is enqueued) */
int k3x_blas_ready(int device, int in, int out, int T, int accumulate);
int k3x_blas_gemm_bf16(int device, const uint16_t *W, int in, int out, float *Y, int ldy,
                       const uint16_t *X, int ldx, int T, int accumulate, void *stream);

#ifdef __cplusplus
}
#endif
#endif
