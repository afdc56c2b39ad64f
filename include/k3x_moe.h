/* k3x_moe.h - MI355X (gfx950) MoE block behind a C ABI.
 *
 * The reference engine's MoE block (router scoring and top-k, dispatch, grouped SwiGLU
 * experts over packed MXFP4 weights with E8M0 per-32 scales, the shared expert and the
 * weighted combine) runs on the CPU through
 *
 *     void k3_moe        (float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
 *                         int T, int *idx, float *wt, float *scratch);   k3.h:629-630
 *     void k3_moe_prefill(float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
 *                         int T, int *idx, float *wt, float *scratch);   k3.h:636-637
 *
 * This library computes the same block on one GPU with the layer's weights resident in
 * HBM.  A layer is uploaded once (k3x_moe_layer_create, pulling every expert through the
 * same get() supplier contract as K3ExpertSrc) and then run any number of times, either
 * from host pointers with the k3_moe semantics (k3x_moe / k3x_moe_prefill) or on device
 * pointers on a caller's HIP stream (k3x_moe_forward).
 *
 * Everything here is plain C: pointers, sizes and status codes; no HIP or torch types.
 * Every call returns 0 or a negative K3X_E_* status (the reference aborts or counts a
 * drop instead; see each call).  Thread model: one layer handle is used by one host
 * thread at a time; kernels of one call run in order on the stream given.
 *
 * Variants covered (both with a sigmoid router and a selection bias, MXFP4 routed experts
 * and bf16 shared experts):
 *   - the K3 LatentMoE (k3_ops.c:1793-1811): route on the full width, down-project to the
 *     latent width, routed experts there with SiTU-GLU, the weighted sum RMSNormed, up-
 *     projected, plus the shared experts on the original input (cfg.latent > 0);
 *   - the K2-class layer: no latent projection, SwiGLU (cfg.latent == 0, betas 0).  In
 *     the reference's terms that is latent = hidden with identity down/up, latent_norm =
 *     0 and situ_b1 = situ_b2 = 2^64.
 */
#ifndef K3X_MOE_H
#define K3X_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ----------------------------------------------------------------- */
#define K3X_OK          0
#define K3X_E_ARG      -1   /* NULL pointer, T < 0, bad dtype                              */
#define K3X_E_SHAPE    -2   /* hidden or moe_inter not a multiple of 128, group != 32,
                               topk outside 1..64, T above the layer's limit             */
#define K3X_E_HIP      -3   /* a HIP runtime call or kernel launch failed                */
#define K3X_E_NOMEM    -4   /* device or host allocation failed                          */
#define K3X_E_DROP     -5   /* an expert could not be fetched (k3x_expert_drops counts it) */
#define K3X_E_NODEV    -6   /* no usable gfx950 device                                    */
#define K3X_E_WAIT     -7   /* a decode workgroup gave up waiting for the selection (never
                               expected: k3x_moe_layer_check reports it)                   */

/* Human-readable text of a status code (static storage). */
const char *k3x_strerror(int status);

/* ---- configuration: the MoE fields of K3Cfg (k3.h:94-102) -------------------------- */
typedef struct k3x_cfg {
    int   hidden;         /* 7168 */
    int   n_experts;      /* 384 */
    int   topk;           /* 8 */
    int   moe_inter;      /* 2048, routed and per shared expert */
    int   n_shared;       /* 1: shared intermediate = n_shared * moe_inter */
    int   moe_renorm;     /* 1: renormalise the top-k weights */
    float routed_scale;   /* 2.5 */
    int   group;          /* MXFP4 group size; only 32 is supported (K3_MXFP4_GROUP) */
    /* The LatentMoE fields.  All zero gives the K2-class layer. */
    int   latent;         /* 3584: the routed experts' width (a multiple of 128);
                             0: no projection, experts at hidden */
    int   latent_norm;    /* 1: RMSNorm of the routed aggregate (k3_ops.c:1946) */
    float rms_eps;        /* that norm's epsilon, 1e-5 */
    float situ_b1;        /* SiTU-GLU betas (k3_situ_glu, k3_ops.c:148-161): gate cap 4 */
    float situ_b2;        /*   and up cap 25; 0 (or >= 2^64) leaves that half uncapped,
                               so 0 and 0 is SwiGLU */
} k3x_cfg;

/* ---- one routed expert, still MXFP4: K3ExpertQ (k3.h:507-516) ----------------------
 * Row-major [out][in]: packed [rows][in/2] bytes (low nibble = even element),
 * scales [rows][in/group] E8M0 bytes.  With X the experts' width (latent, or hidden
 * when latent == 0): p1/s1 gate [I][X], p3/s3 up [I][X], p2/s2 down [X][I]. */
typedef struct k3x_expert_q {
    const unsigned char *p1, *s1;
    const unsigned char *p3, *s3;
    const unsigned char *p2, *s2;
} k3x_expert_q;

/* ---- expert supplier: K3ExpertSrc (k3.h:521-544) ----------------------------------
 * get() returns 0 and fills *out, or non-zero when the expert cannot be fetched. The
 * pointers need stay valid only until get() is called again.
 * getmany() (optional, may be NULL; k3.h:527-539): bring experts[0 .. n-1] resident with
 *   their reads issued together; returns how many are resident, or -1.  A short return
 *   is not an error: get() then fetches the rest itself.  Called before the get()s of a
 *   batch of experts (a layer's upload, 16 at a time).
 * resident() (optional, may be NULL; k3.h:540-542): 1 when the expert is resident (get()
 *   would read nothing), filling *out when out != NULL.
 * Zero the struct before setting what you have: the two optional members come last, so
 * a caller written for get/ctx alone stays valid when it zeroes the struct. */
typedef struct k3x_expert_src {
    int  (*get)(struct k3x_expert_src *self, int layer, int expert, k3x_expert_q *out);
    void *ctx;
    int  (*getmany)(struct k3x_expert_src *self, int layer, const int *experts, int n);
    int  (*resident)(struct k3x_expert_src *self, int layer, int expert, k3x_expert_q *out);
} k3x_expert_src;

/* ---- a layer's weights: K3MoeW (k3.h:546-569) with bf16 trunk matrices --------------
 * gate fp32 [n_experts][hidden], bias fp32 [n_experts] (may be NULL),
 * sh1/sh3 bf16 [n_shared*moe_inter][hidden], sh2 bf16 [hidden][n_shared*moe_inter]
 * (all three NULL when n_shared == 0).  Experts come from src, or from bank
 * ([n_experts] entries) when src is NULL.  With cfg.latent > 0: down bf16
 * [latent][hidden], up bf16 [hidden][latent], and latent_norm fp32 [latent] when
 * cfg.latent_norm (all ignored otherwise). */
typedef struct k3x_moe_w {
    const float        *gate, *bias;
    const uint16_t     *sh1, *sh3, *sh2;
    k3x_expert_src     *src;
    const k3x_expert_q *bank;
    int                 layer;
    const uint16_t     *down, *up;
    const float        *latent_norm;
} k3x_moe_w;

typedef struct k3x_moe_layer k3x_moe_layer;

/* Upload a layer to device `device` and keep it resident.  Every expert is fetched
 * once through src->get (or read from bank) and re-laid out for the matrix cores.
 * A failed fetch increments k3x_expert_drops and fails the call with K3X_E_DROP (the
 * reference would skip the term per token and leave the caller to check the counter:
 * k3_ops.c:1916-1926). Replaces the per-token expert fetches of k3_moe (k3_ops.c:1905-
 * 1931) by one upload. */
int  k3x_moe_layer_create(const k3x_cfg *c, const k3x_moe_w *w, int device,
                          k3x_moe_layer **out);
void k3x_moe_layer_destroy(k3x_moe_layer *L);

/* Bytes of device memory the layer holds (weights plus its working buffers). */
size_t k3x_moe_layer_bytes(const k3x_moe_layer *L);

/* Reserve the prefill working buffers for calls of up to max_T tokens (no-op for the
 * decode path's T <= 8 and for cached layers).  A forward call with more tokens than are
 * reserved grows the buffers itself, except while its stream is being captured into a
 * graph: then it returns K3X_E_SHAPE, so a caller that captures prefill calls reserves
 * first.  Growing never frees the old buffers (a graph recorded over them stays valid);
 * they are released with the layer.  No counterpart in the reference (k3_moe_scratch,
 * k3.h:574, sizes the caller's scratch instead). */
int  k3x_moe_layer_reserve(k3x_moe_layer *L, int max_T);

/* Matrix m (0 gate, 1 up, 2 down) of expert e, as the device's product kernels
 * dequantise it, into out (host, fp32 row-major [rows][width]): k3_mxfp4_dequant
 * (k3.h:866-867, k3_ops.c:3778-3808) of the layer's resident bytes, E8M0 byte 255 -> 0,
 * byte 0 -> 2^-127.  Every such value is a bf16 (or an infinity), so this is what the
 * matrix cores multiply.  For checking. */
int  k3x_moe_layer_dequant(const k3x_moe_layer *L, int e, int m, float *out);

/* Read expert e back from the device in the reference's row-major layout (host
 * buffers sized as in k3x_expert_q).  For checking and for handing experts back. */
int  k3x_moe_layer_read_expert(const k3x_moe_layer *L, int e, unsigned char *p1,
                               unsigned char *s1, unsigned char *p3, unsigned char *s3,
                               unsigned char *p2, unsigned char *s2);

/* ---- device-pointer forward --------------------------------------------------------
 * out  fp32 [T][hidden] device, overwritten (or resid + MoE when resid != NULL;
 *      resid may equal out).  x, out and resid are 16-byte aligned (else K3X_E_ARG).
 * x    [T][hidden] device, K3X_F32 or K3X_BF16.
 * idx/wt  optional device [T][topk]: every token's routing (expert indices in selection
 *      order, combine weights after renorm and routed_scale), as k3_router writes them
 *      (k3_ops.c:1700-1716).
 * stream  a hipStream_t, or NULL for the null stream.  Asynchronous: returns after
 *      enqueueing.  T <= 8 runs the decode path (fused dequant-GEMV on the matrix cores,
 *      every unique expert read once per call); larger T runs the prefill pipeline
 *      (device top-k, histogram, prefix sum, grouped GEMM, combine). */
#define K3X_F32  0
#define K3X_BF16 1
int  k3x_moe_forward(k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                     const float *resid, int *idx, float *wt, void *stream);

/* The router alone: every token's top-k experts and combine weights for T tokens of
 * device activations, the reference's k3_router (k3.h:294-313, k3_ops.c:1624-1719) over
 * the layer's router and bias: logits as its sequential double chain, score
 * sigmoid((float)logit), choice score + bias, the top-k by repeated maximum with the lower
 * index first among equal choices, the unbiased scores renormalised and scaled; idx and
 * wt bit for bit the reference's.  idx int [T][topk], wt fp32 [T][topk] device; x
 * [T][hidden] device, K3X_F32 or K3X_BF16, 16-byte aligned.  The plain router: a layer's
 * cache-only setting (draft routing, applied by the MoE call) does not apply.  Uses the
 * layer's prefill buffers, growing them on a first call of more tokens than before (not
 * while the stream is being captured: K3X_E_SHAPE then; reserve first with
 * k3x_moe_layer_reserve).  Asynchronous on stream. */
int  k3x_moe_route(k3x_moe_layer *L, int *idx, float *wt, const void *x, int x_dtype, int T,
                   void *stream);

/* The prefill path of k3x_moe_forward (8 < T tokens) for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops): same arguments, but
 * the working buffers come from a static device array of 64 MiB that each GPU holds until
 * the process ends, instead of the layer's buffers that k3x_moe_forward may grow.  Calls
 * no allocating routine: the plain products that k3x_moe_forward hands to hipBLASLt
 * (bf16 input: the shared expert's where 2*SI <= hidden, the latent projections), whose
 * first call of a shape may load code into device memory, run on the dense kernel here.
 * Results: the same selected experts and routing weights bit for bit; outputs bit for bit
 * where k3x_moe_forward uses no library product (fp32 input), else within fp32 rounding
 * of it (a different order of the same exact products).  One call's buffers must fit
 * the array (about 590 KB per token at the K2 shape: T <= 111 there); larger T, or
 * T <= 8 (k3x_moe_forward's decode path allocates nothing), returns K3X_E_SHAPE.  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU race, so order
 * them on one stream.  No counterpart in the reference; for callers that cannot
 * allocate. */
int  k3x_moe_prefill_noalloc(k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                             const float *resid, int *idx, float *wt, void *stream);

/* Prefill arithmetic of a layer (calls with more than 8 tokens; the decode path is always
 * exact).  K3X_PREFILL_EXACT (the default): the routed products take the activations as
 * bf16 hi + lo pairs against the exactly dequantised MXFP4 weights, within the parity bar
 * of the reference's fp32 path (k3_matmul_mxfp4, k3_ops.c:3323-3776).
 * K3X_PREFILL_MXFP8 (opt-in): the routed gate/up and down products run on the scaled
 * matrix cores with the weights as stored and the activations quantised to MXFP8 (E4M3
 * elements, one E8M0 scale per 32 consecutive k; the scale 2^X is the least power of two
 * with max|v| <= 448 * 2^X over the block's finite values, elements rounded to nearest,
 * ties to even; the routing weight is folded into the gate/up output before it is
 * quantised).  Router, shared expert and latent projections stay exact.  Results then
 * differ from the reference by the quantisation (about 1-3% relative L2 on N(0,1)
 * activations).  No counterpart in the reference.  Returns K3X_E_SHAPE for a layer
 * holding an E8M0 scale byte outside 1..252 (the matrix cores read 255 as NaN where the
 * reference reads zero) and K3X_E_ARG for an unknown mode. */
/* Cache-only (draft) routing, K3MoeW.cache_only (k3.h:564-568, k3_ops.c:1884-1926):
 * on = 1 makes every later forward call keep, per token, only those of its top-k experts
 * that are resident, in top-k order, with their weights divided by their float sum (so a
 * draft reads no expert bytes that are not already in place); idx/wt then hold the kept
 * experts first and the router's entries after them, as the reference leaves its arrays.
 * resident: a host array [n_experts] (copied; non-zero = resident), or NULL: for a cached
 * layer the experts in its HBM slots at each call, for a resident layer every expert
 * (which keeps the routing and renormalises the weights to sum 1).  Calls run the decode
 * path in groups of up to 8 tokens with a host step after each selection, as the
 * reference runs such calls token by token (:2018); k3x_moe_prefill_noalloc and the
 * stacked graph refuse such a layer (K3X_E_ARG).  on = 0 restores the exact routing. */
int  k3x_moe_layer_set_cache_only(k3x_moe_layer *L, int on, const unsigned char *resident);

#define K3X_PREFILL_EXACT 0
#define K3X_PREFILL_MXFP8 1
int  k3x_moe_layer_set_prefill_mode(k3x_moe_layer *L, int mode);

/* RMSNorm of T rows on the device: y = w * x * inv, inv = 1/sqrt(mean(x^2) + eps)
 * (k3_rmsnorm, k3_ops.c:132-140).  x, y fp32 [T][n], w fp32 [n], device pointers. */
int  k3x_rmsnorm(float *y, const float *x, const float *w, int n, int T, float eps,
                 void *stream);

/* ---- host-pointer drop-ins with the reference's semantics ---------------------------
 * k3x_moe mirrors k3_moe (k3.h:629-630): out [T][hidden] overwritten, x [T][hidden]
 * fp32, idx/wt [topk] left holding the LAST token's routing.  k3x_moe_prefill mirrors
 * k3_moe_prefill (k3.h:636-637): with T > 1 it leaves idx/wt untouched, as the
 * reference's batched path does (k3_ops.c:2018-2053); with T == 1 it writes them as
 * k3_moe.  On this device both run the same pipeline.  Identical calls repeat bit for
 * bit; one token's output in calls that group tokens differently (one token against
 * eight, decode against prefill) agrees within the parity bar but not bit for bit, since
 * the fp32 accumulation order of the products follows the call's shape (its token count
 * and its unique experts).  Synchronous; K3X_E_WAIT when a decode workgroup gave
 * up its wait (the output is then not valid).  The reference's scratch argument has no
 * counterpart: working memory lives in the layer. */
int  k3x_moe(k3x_moe_layer *L, float *out, const float *x, int T, int *idx, float *wt);
int  k3x_moe_prefill(k3x_moe_layer *L, float *out, const float *x, int T, int *idx,
                     float *wt);

/* k3_expert_drops (k3.h:576-580): experts that could not be fetched. */
extern long k3x_expert_drops;

/* ---- synthetic layers --------------------------------------------------------------
 * A layer whose weights come from a counter-based generator (splitmix64 per element),
 * so any element can be regenerated on its own on the CPU: the router fp32 N(0,
 * router_sigma); the bias N(0, bias_sigma), or Zipf-skewed alpha*(pi(e)+1)^-zipf_s over
 * a seeded permutation pi when zipf_alpha > 0; E2M1 codes uniform over 16; E8M0 scales
 * uniform over [scale_lo, scale_hi]; shared weights bf16 N(0, shared_sigma); for a
 * latent layer, down and up bf16 N(0, trunk_sigma) and latent-norm weights fp32 N(1, 0.1).
 * Expert bytes are generated directly in device memory. */
typedef struct k3x_synth_spec {
    uint64_t seed;
    int      layer;
    double   router_sigma;   /* 0.02 */
    double   bias_sigma;     /* 0.1 */
    double   zipf_alpha;     /* 0: normal bias */
    double   zipf_s;         /* 1.1 */
    int      scale_lo;       /* 121 */
    int      scale_hi;       /* 125 */
    double   shared_sigma;   /* 0.02 */
    double   trunk_sigma;    /* 0.02 */
} k3x_synth_spec;

int  k3x_synth_layer_create(const k3x_cfg *c, const k3x_synth_spec *s, int device,
                            k3x_moe_layer **out);

/* Generator stream ids and the element rule, exposed so a checker can regenerate any
 * tensor of a synthetic layer on the host. */
enum {
    K3X_STREAM_ROUTER = 0, K3X_STREAM_BIAS = 1, K3X_STREAM_X = 2, K3X_STREAM_SH1 = 3,
    K3X_STREAM_SH3 = 4, K3X_STREAM_SH2 = 5, K3X_STREAM_NORM = 6, K3X_STREAM_DOWN = 7,
    K3X_STREAM_UP = 8, K3X_STREAM_LNORM = 9, K3X_STREAM_CODES = 10, K3X_STREAM_SCALES = 11
};
uint64_t k3x_synth_key(uint64_t seed, int layer, int stream, int sub);
void     k3x_synth_normal_f32(float *dst, size_t n, uint64_t key, double mu, double sigma);
void     k3x_synth_normal_bf16(uint16_t *dst, size_t n, uint64_t key, double mu,
                               double sigma);

/* ---- decoder-layer glue ----------------------------------------------------------------
 * Block attention-residual aggregation (k3_attn_res, k3_ops.c:1722-1753, gathered as in
 * k3_decoder_layer_core, :2546-2555): for each of T rows the sources are blocks[t][0 ..
 * nb-1] (rows of n floats, maxb of them per row t) followed by pref[t]; h[t] = sum_s p_s
 * src_s, p the softmax over the sources of RMSNorm(src_s) . fold (fold = the norm weight
 * times the projection, one vector).  nb + 1 <= 64.  Device pointers, on stream. */
int  k3x_attn_res(float *h, const float *blocks, int maxb, int nb, const float *pref,
                  const float *fold, int n, int T, float eps, void *stream);

/* The MoE half of a decoder layer (k3_decoder_layer_core, k3_ops.c:2546-2589) on the
 * device: h = attn_res(blocks, pref); hin = RMSNorm(h; post_norm, eps); pref += MoE(hin);
 * h = pref.  hin is a caller workspace of T*hidden floats; all device pointers, 16-byte
 * aligned; asynchronous on stream (kernels only, so it can be captured in a graph). */
int  k3x_moe_half(k3x_moe_layer *L, float *h, float *pref, const float *blocks, int maxb,
                  int nb, const float *fold, const float *post_norm, float eps, int T,
                  float *hin, void *stream);

/* The same two calls with a block count per row, as k3_decoder_layer_core takes them
 * (k3_ops.c:2481-2483: token t's count is nbv[t * nbs], nbs 0 for one count shared by
 * every token, 1 for one per token; used per token at :2493 and :2549; the speculative
 * caller k3_decoder_layer_inc_logv, :2606-2613, passes nbs 1).  nbv is a DEVICE int
 * array read by the kernel when it runs, so a captured graph replays with the counts the
 * array then holds.  Rows with equal counts compute the same floats as k3x_attn_res /
 * k3x_moe_half.  A count outside 0 .. min(maxb, 63) (or above 0 with blocks NULL) fills
 * that row of h with quiet NaNs, which the MoE half carries to its outputs: the
 * reference reads past its block stack there. */
int  k3x_attn_res_v(float *h, const float *blocks, int maxb, const int *nbv, int nbs,
                    const float *pref, const float *fold, int n, int T, float eps,
                    void *stream);
int  k3x_moe_half_v(k3x_moe_layer *L, float *h, float *pref, const float *blocks, int maxb,
                    const int *nbv, int nbs, const float *fold, const float *post_norm,
                    float eps, int T, float *hin, void *stream);

/* ---- stacked layers ------------------------------------------------------------------
 * The MoE half of consecutive decoder layers (k3_decoder_layer_core, k3_ops.c:2547-2589,
 * without attention): for each layer l, h = h + MoE_l(RMSNorm(h; norm_w[l], eps)), the
 * norm as k3_rmsnorm (k3_ops.c:132-140) and the residual add as :2589.
 * k3x_stack_create takes n_layers device-resident layers of one hidden size on one
 * device (borrowed: they must outlive the stack; their timing hooks must be off) and
 * their RMSNorm weights (device fp32 [hidden] each, borrowed), and reserves working
 * memory for up to max_T tokens per call.
 * k3x_stack_forward runs the sequence on h (device fp32 [T][hidden], updated in place)
 * on `stream`.  The first call for a given (h, T) records the whole sequence into a HIP
 * graph; later calls with the same (h, T) replay it (a new (h, T) records a new graph).
 * Two calls on one stack must be ordered on one stream. */
typedef struct k3x_stack k3x_stack;
int  k3x_stack_create(k3x_moe_layer *const *layers, const float *const *norm_w, int n_layers,
                      float eps, int max_T, k3x_stack **out);
int  k3x_stack_forward(k3x_stack *S, float *h, int T, void *stream);
void k3x_stack_destroy(k3x_stack *S);

/* ---- timing hooks ---------------------------------------------------------------
 * The kernels the last k3x_moe_forward on L enqueued, bracketed by two HIP events on
 * the stream it used (recorded when timing is on).  ms receives the elapsed time of
 * the last timed call after a synchronize. */
/* Waits for the layer's work and reports (then clears) K3X_E_WAIT if any decode call since
 * the last check had a workgroup give up waiting for the published selection; 0 otherwise.
 * No counterpart in the reference (its CPU path has no cross-workgroup wait). */
int  k3x_moe_layer_check(k3x_moe_layer *L);
/* Failure injection for tests of the check above: sets the decode wait's bound (ticks of
 * the 100 MHz clock; the default is 100,000,000 = 1 s) and, with publish = 0, withholds
 * the flag, so that every routed workgroup gives up after `ticks` and leaves.  Calls made
 * so are not valid; restore with (100000000, 1).  No counterpart in the reference. */
int  k3x_moe_layer_set_route_wait(k3x_moe_layer *L, unsigned long long ticks, int publish);
int  k3x_moe_layer_set_timing(k3x_moe_layer *L, int on);
/* Diagnostics (a layer created with K3X_TRACE=1 in the environment): per workgroup of
 * decode kernel k (0 the router, 1 the gate/up products, 2 the down products, which is
 * traced when it runs as one part) of the last decode call, three words: the workgroup
 * index | XCD << 28 | hardware ids << 32, its start and its end (100 MHz clock).
 * Returns the number of workgroups copied (0 without the trace).  No counterpart in the
 * reference. */
int  k3x_moe_layer_trace(k3x_moe_layer *L, int kernel, unsigned long long *out, int max_wg);
/* Diagnostics: waits for the layer's work and stores in *n how many (token, expert)
 * router logits the last decode-path selection worked out again as the reference's
 * single double chain (k3_ops.c:1666-1688), because the parallel sum's float logit was
 * not proven equal to it and could change the selection or a selected weight.  No
 * counterpart in the reference (its router is that chain). */
int  k3x_moe_layer_exact_count(k3x_moe_layer *L, int *n);
/* Diagnostics: waits for the layer's work and copies the routing of the last decode-path
 * call on L (1 <= T <= 8 tokens, as that call carried; also the calls that the stacked
 * layers make): idx and wt [T][topk], as k3x_moe_forward returns them.  For callers that
 * do not see the selection, such as k3x_stack_forward.  No counterpart in the reference. */
int  k3x_moe_layer_last_route(k3x_moe_layer *L, int T, int *idx, float *wt);
int  k3x_moe_layer_last_ms(k3x_moe_layer *L, float *ms);

#ifdef __cplusplus
}
#endif
#endif
