// k3x_decode.hip - the decode path of the MoE block (T <= 8 tokens), three launches:
//
//   k1_router_bset    router logits in double, sigmoid, +bias (k3_router, k3_ops.c:1624-
//                     1694) for every expert, and x's B fragments for the products.  The
//                     router runs alone, so its 11 MB arrive first.
//   k2_gateup         workgroup 0 selects each token's top-k (:1700-1716) and lists the
//                     unique experts (the dedup of moe_prefill_routed, :2067-2081); the
//                     shared expert's gate/up products over the full K with SwiGLU
//                     (moe_shared, :1848-1857; k3_situ_glu at 2^64 betas, :148-161) stream
//                     meanwhile; then each unique expert's gate/up products
//                     (k3_matmul_mxfp4, :3323-3776) with SwiGLU and the routing weight
//                     folded in, once the selection is published.
//   k3_down           each unique expert's down product and the shared expert's (:1858)
//                     into one accumulator set per 16 output rows (the weighted combine,
//                     :1941-1942, plus the shared result, :1859), and an optional residual.
//                     With two or more tokens and 256 | H, k3_down_wide instead: 256 rows
//                     a workgroup over parts of the items, each item's B fragments loaded
//                     into LDS once for the workgroup; k3_reduce (K2 form) or
//                     k4_latent_norm (latent form) adds the parts in order.  Otherwise
//                     k3_down2: two 16-row tiles a workgroup, each B fragment read once
//                     for both.
//
// Each weight byte is read once per call.  Weights are dequantised in registers
// (E2M1 x 2^(s-127) is exact in bf16) and multiplied on v_mfma_f32_16x16x32_bf16 against
// activations split into bf16 hi + lo columns (16 significant bits: a bf16 activation
// exactly, an fp32 one within 2^-17): the products of the pair are exact, the sums fp32.
//
// Streaming.  A workgroup's weights are cut into wave-uniform items (an fp4 super-quad,
// 4352 bytes per 16 rows, or a bf16 quad, 4096 bytes) that its waves take interleaved,
// so the workgroup reads one contiguous window at a time.  Each wave keeps its next two
// items in flight through range-checked, non-temporal buffer loads; loads past a wave's
// last item carry an out-of-range offset, which returns zeros without touching memory,
// so every loop iteration issues the same loads and the compiler's wait counts stay
// exact.  The activations (B fragments, compact layout: k3x_device.h) are staged in LDS
// when they fit: their loads are issued before the first weights, so the loop waits on
// nothing but its own weight stream.
#include "k3x_device.h"
#include "k3x_stream.h"
#include "k3x_topk.h"

#define NT1 256     // k1 workgroup: 4 waves
#define NT  256     // k2 workgroup: 4 waves
#define NT3 512     // k3 workgroup: 8 waves
#define STAGE_MAX 65536u   // largest B set staged in LDS (bytes)
#define K3_LDS_MAX 73728u  // k3's dynamic LDS with the shared set: two workgroups per CU


// ------------------------------------------------------------------ selection
struct KSArgs {
    float         *score, *choice; // [T][E], from k1 (entries resolved below are rewritten)
    float         *slack;          // [T][E] choice slack from k1 (0: proven the reference's)
    unsigned      *hkey;           // [T] largest slack_key of each token's row (0: none)
    int            E, K, renorm;
    float          routed_scale;
    k3x_route     *route;          // unique experts and per-(expert, token) weights, for k2/k3
    int           *idx;  float *wt;        // internal [T][K]
    int           *uidx; float *uwt;       // optional caller copies
    int            T;
    // the router's inputs, for the logits worked out again as the reference's chain
    const float   *router, *bias;  // [E][H], [E]
    const void    *x;              // [T][H] raw rows (fp32 or bf16)
    int            x_bf16, H;
    const float   *norm_w, *ninv;  // RMSNorm weights [H] and each row's 1/rms, or NULL
};

// Stores of the published routing: written through to the device-coherent level, since
// the routed workgroups of the same launch read them, possibly on another XCD.
__device__ __forceinline__ void pub_i(int *p, int v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pub_f(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A tagged word of the in-launch handoff: (seq << 32) | v in one 64-bit atomic store.
__device__ __forceinline__ void pub_t(unsigned long long *p, unsigned seq, uint32_t v)
{
    __hip_atomic_store(p, ((unsigned long long)seq << 32) | v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// A workgroup's view of the routing, in LDS, and each wave's buffer for the products of
// a chain (ks_chain).
#define KS_CH 256            // elements of a chain chunk: four a lane
#define KS_CR 2              // chain chunks in flight per wave
#define KS_LIST 64           // experts worked out per pass of ks_resolve
struct KSLds {
    int    idx[K3X_DECODE_MAX_T][K3X_MAX_TOPK];
    float  w[K3X_DECODE_MAX_T][K3X_MAX_TOPK];
    int    first[1024];                          // per expert: its first (token, slot) item
    int    uq[K3X_DECODE_MAX_T * K3X_MAX_TOPK];  // unique experts, first-seen order
    int    wc[NT / WAVE];
    int    need[K3X_DECODE_MAX_T];               // token's selection needs ks_resolve
    int    list[KS_LIST], nlist;                 // ks_resolve's experts of a pass
    alignas(16) double pl[NT / WAVE][KS_CH];     // ks_chain's products
};

// The choice key (choice_key's order) just above choice + slack: an upper bound of the
// reference's choice for an expert whose logit is not proven.
__device__ __forceinline__ uint32_t slack_key(float choice, float slack)
{
    const uint32_t k = choice_key((float)((double)choice + (double)slack));
    return (k != 0u && k < 0xFF800000u) ? k + 1u : k;
}

// Whether an expert not proven could change a selection whose K-th choice is ck, or one
// of its weights: its choice may reach ck (hk: the token's largest slack_key, 0 = none).
// Every selected expert's choice is at least ck, so a selected one not proven counts.
__device__ __forceinline__ bool slack_reaches(uint32_t hk, float ck)
{
    return hk != 0u && hk >= choice_key(ck);
}

// The logit of (token t, expert e) as the reference computes it: one double chain
// acc += (double)W[e][i] * (double)x[i] for i = 0 .. H-1 in order (k3_ops.c:1666-1688),
// with x the row the router read (nw[i] * x[i] * inv for the RMSNorm of x).  The whole
// workgroup: in step g, wave w forms the products of chunk 4g + w (KS_CH elements, four a
// lane; exact in double, -0.0, the identity of the sum, past H) in its LDS buffer, with
// its next chunks' loads in flight (a ring of KS_CR); then thread 0 adds the step's
// 4 KS_CH products in order.  The value in thread 0 (every thread must call).
__device__ double ks_chain(const KSArgs &a, KSLds &l, int t, int e)
{
    constexpr int NW = NT / WAVE;
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const uint32_t H = (uint32_t)a.H, xb = a.x_bf16 ? 2u : 4u;
    const rsrc_t rw = make_rsrc(a.router + (size_t)e * H, H * 4u);
    const rsrc_t rx = make_rsrc((const uint8_t *)a.x + (size_t)t * H * xb, H * xb);
    const bool nrm = a.norm_w != nullptr;
    const rsrc_t rn = make_rsrc(nrm ? a.norm_w : a.router, nrm ? H * 4u : 0u);
    const float inv = nrm ? a.ninv[t] : 1.0f;
    const int steps = (int)((H + NW * KS_CH - 1) / (NW * KS_CH));
    double *pl = l.pl[wave];
    u32x4 w[KS_CR], nw[KS_CR];
    u32x2 xv[KS_CR][2];
    auto ld = [&](int i, int k) AI {
        const uint32_t el = (uint32_t)(k * NW + wave) * KS_CH + 4u * (uint32_t)lane;
        const bool on = k < steps;
        w[i] = bload16(rw, on ? el * 4u : K3X_OOB);
        // x in two 8-byte pieces (bf16: the first holds all four, the second loads
        // nothing), so that no load reaches past the row
        xv[i][0] = __builtin_amdgcn_raw_buffer_load_b64(rx, on ? el * xb : K3X_OOB, 0, 0);
        xv[i][1] = __builtin_amdgcn_raw_buffer_load_b64(rx, on && xb == 4u ? el * 4u + 8u : K3X_OOB,
                                                        0, 0);
        nw[i] = bload16(rn, on && nrm ? el * 4u : K3X_OOB);
    };
    double acc = 0.0;
    ring_prime<KS_CR>(ld);
    ring_loop<KS_CR>(steps, ld, [&](int i, int k) AI {
        const uint32_t el = (uint32_t)(k * NW + wave) * KS_CH + 4u * (uint32_t)lane;
        float xf[4];
        if (a.x_bf16) {
            xf[0] = bf2f(xv[i][0][0] & 0xFFFFu); xf[1] = bf2f(xv[i][0][0] >> 16);
            xf[2] = bf2f(xv[i][0][1] & 0xFFFFu); xf[3] = bf2f(xv[i][0][1] >> 16);
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) xf[q] = __uint_as_float(xv[i][q >> 1][q & 1]);
        }
        double p[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float xq = nrm ? __uint_as_float(nw[i][q]) * xf[q] * inv : xf[q];
            p[q] = el + q < H ? (double)__uint_as_float(w[i][q]) * (double)xq : -0.0;
        }
        *(f64x2 *)(pl + 4 * lane) = (f64x2){p[0], p[1]};
        *(f64x2 *)(pl + 4 * lane + 2) = (f64x2){p[2], p[3]};
        __syncthreads();
        if (threadIdx.x == 0) {
            const double *q = &l.pl[0][0];
            double s = acc;
#pragma unroll 4
            for (int j = 0; j < NW * KS_CH; j += 2) {
                const f64x2 v = *(const f64x2 *)(q + j);
                s += v[0];
                s += v[1];
            }
            acc = s;
        }
        __syncthreads();
    });
    return acc;
}

// Token t's selection where an expert whose logit is not proven may reach it
// (slack_reaches): wave 0 selects again from the rows in memory and lists the experts
// whose slack_key reaches the K-th choice (up to KS_LIST a pass, lowest index first); the
// workgroup works out each one's logit as the reference's chain (ks_chain) and stores
// its score, its choice and a slack of 0; until a pass lists none.  Each pass resolves
// at least one expert, so the loop ends.  Then every selected expert's choice and score
// are the reference's and every expert not proven lies below the K-th choice, as in the
// reference: the selection and its weights are the reference's.  Every thread calls;
// results as wave_topk's in s_idx/s_w, and in wave 0's out_e/out_w.  Returns the number
// of logits worked out again.
template <int NE>
__device__ int ks_resolve(const KSArgs &a, KSLds &l, int t, int *s_idx, float *s_w,
                          int *out_e = nullptr, float *out_w = nullptr)
{
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const uint32_t bytes = (uint32_t)(a.T * a.E * 4), ro = (uint32_t)(t * a.E * 4);
    const rsrc_t cr = make_rsrc(a.choice, bytes), sr = make_rsrc(a.score, bytes);
    const rsrc_t lr = make_rsrc(a.slack, bytes);
    int nex = 0;
    for (int pass = 0; pass <= a.E; pass++) {
        __threadfence();              // the stores below reach the loads of the next pass
        if (wave == 0) {
            float ck;
            wave_topk<NE, 0>(cr, sr, ro, a.E, a.K, a.renorm, a.routed_scale, s_idx, s_w, lane,
                             out_e, out_w, &ck);
            const uint32_t kk = choice_key(ck);
            uint32_t crit = 0u;
#pragma unroll
            for (int c = 0; c < NE; c++) {
                const int e = lane * NE + c;
                const uint32_t o = e < a.E ? ro + 4u * (uint32_t)e : K3X_OOB;
                const float sl = bload_f32<0>(lr, o);
                if (sl > 0.0f && slack_key(bload_f32<0>(cr, o), sl) >= kk) crit |= 1u << c;
            }
            int n = 0;
            for (; n < KS_LIST; n++) {             // lowest index first
                const uint64_t m = __ballot(crit != 0u);
                if (m == 0ull) break;
                const int l0 = (int)__builtin_ctzll(m);
                const int c = __builtin_ctz((uint32_t)__builtin_amdgcn_readlane((int)crit, l0));
                if (lane == l0) crit &= crit - 1u;
                if (lane == 0) l.list[n] = l0 * NE + c;
            }
            if (lane == 0) l.nlist = n;
        }
        __syncthreads();
        const int n = l.nlist;
        if (n == 0) break;
        for (int i = 0; i < n; i++) {
            const int e = l.list[i];
            const double v = ks_chain(a, l, t, e);
            if (threadIdx.x == 0) {
                const float sv = sigmoid_ref((float)v);
                const size_t o = (size_t)t * a.E + e;
                a.score[o] = sv;
                a.choice[o] = sv + a.bias[e];
                a.slack[o] = 0.0f;
            }
        }
        nex += n;
        __syncthreads();              // l.nlist is read before wave 0 writes it again
    }
    return nex;
}

// Token t's weight for expert e: the sum of its slots' weights for e (0 where not
// chosen; a slot repeated by a round that found nothing adds 0).
__device__ __forceinline__ float ks_weight(const KSLds &l, int K, int t, int e)
{
    float w = 0.0f;
    for (int j = 0; j < K; j++)
        if (l.idx[t][j] == e) w += l.w[t][j];
    return w;
}

// Routing of every token (one wave per token), then the unique experts in first-seen
// order over (token, slot), built in parallel: each expert's first item by an LDS
// minimum, the first items' slots by ballots.  Returns the number of unique experts.
// With `publish`, also writes the indices and weights, and the unique list and each
// unique expert's weight per token (written through) for k3 and the host.  With seq != 0,
// also the tagged copies that k2's routed workgroups read in the same launch.
template <int NE>
__device__ int ks_route(const KSArgs &a, KSLds &l, bool publish, unsigned seq = 0u)
{
    constexpr int NW = NT / WAVE;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const rsrc_t cr = make_rsrc(a.choice, (uint32_t)(a.T * a.E * 4));
    const rsrc_t sr = make_rsrc(a.score, (uint32_t)(a.T * a.E * 4));
    if (a.T == 1) {
        // one token, selected by wave 0 in its registers: lane j holds slot j; the unique
        // experts are the slots whose expert no lower slot holds, each with the sum of
        // its slots' weights in slot order.  The other waves stay for ks_resolve.
        int ex = 0;
        float w = 0.0f;
        if (wave == 0) {
            const uint32_t hk = __hip_atomic_load(&a.hkey[0], __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
            float ck;
            wave_topk<NE, 0>(cr, sr, 0u, a.E, a.K, a.renorm, a.routed_scale, l.idx[0], l.w[0],
                             lane, &ex, &w, &ck);
            if (lane == 0) {
                l.need[0] = slack_reaches(hk, ck);
                if (hk) a.hkey[0] = 0u;      // read: cleared for the next call's router
            }
        }
        __syncthreads();
        const int nex = l.need[0] ? ks_resolve<NE>(a, l, 0, l.idx[0], l.w[0], &ex, &w) : 0;
        if (wave != 0) return 0;
        const bool on = lane < a.K;
        bool first = on;
        float wsum = 0.0f;
        for (int i = 0; i < a.K; i++) {
            const int ei = __builtin_amdgcn_readlane(ex, i);
            const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), i));
            first = first && !(i < lane && ei == ex);
            wsum += ei == ex ? wi : 0.0f;
        }
        const uint64_t fm = __ballot(first);
        const int nu = __popcll(fm);
        if (first) l.uq[lanes_below(fm)] = ex;
        if (publish) {
            if (on) {
                a.idx[lane] = ex;
                a.wt[lane] = w;
                if (a.uidx) { a.uidx[lane] = ex; a.uwt[lane] = w; }
            }
            if (first) {
                const int slot = lanes_below(fm);
                pub_i(&a.route->uniq[slot], ex);
                pub_f(&a.route->wtok[slot][0], wsum);
                for (int t = 1; t < K3X_DECODE_MAX_T; t++) pub_f(&a.route->wtok[slot][t], 0.0f);
                if (seq) {
                    pub_t(&a.route->tuniq[slot], seq, (uint32_t)ex);
                    pub_t(&a.route->twtok[slot][0], seq, __float_as_uint(wsum));
                }
            }
            if (lane == 0) {
                pub_i(&a.route->nu, nu);
                pub_i(&a.route->nexact, nex);
                if (seq) pub_t(&a.route->tnu, seq, (uint32_t)nu);
            }
        }
        return nu;
    }
    // tokens wave and wave + NW together (at most eight tokens over four waves)
    static_assert(K3X_DECODE_MAX_T <= 2 * NW, "two tokens a wave at most");
    if (wave < a.T) {
        const int t1 = wave + NW < a.T ? wave + NW : wave;
        const uint32_t ro[2] = {(uint32_t)(wave * a.E * 4), (uint32_t)(t1 * a.E * 4)};
        int *const si[2] = {l.idx[wave], l.idx[t1]};
        float *const sw[2] = {l.w[wave], l.w[t1]};
        const int nt = wave + NW < a.T ? 2 : 1;
        const uint32_t hk0 = __hip_atomic_load(&a.hkey[wave], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t hk1 = nt == 2 ? __hip_atomic_load(&a.hkey[t1], __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT) : 0u;
        float ck[2];
        wave_topk_n<NE, 0, 2>(cr, sr, ro, nt, a.E, a.K, a.renorm, a.routed_scale, si, sw, lane, ck);
        if (lane == 0) {                     // read: cleared for the next call's router
            l.need[wave] = slack_reaches(hk0, ck[0]);
            if (hk0) a.hkey[wave] = 0u;
            if (nt == 2) {
                l.need[t1] = slack_reaches(hk1, ck[1]);
                if (hk1) a.hkey[t1] = 0u;
            }
        }
    }
    for (int e = threadIdx.x; e < a.E; e += NT) l.first[e] = 0x7FFFFFFF;
    __syncthreads();
    int nex = 0;
    for (int t = 0; t < a.T; t++)
        if (l.need[t]) nex += ks_resolve<NE>(a, l, t, l.idx[t], l.w[t]);
    const int TK = a.T * a.K;
    for (int i = threadIdx.x; i < TK; i += NT) {
        const int t = i / a.K, j = i % a.K;
        const int ex = l.idx[t][j];
        if (publish) {
            a.idx[i] = ex;
            a.wt[i] = l.w[t][j];
            if (a.uidx) { a.uidx[i] = ex; a.uwt[i] = l.w[t][j]; }
        }
        atomicMin(&l.first[ex], i);
    }
    __syncthreads();
    int base = 0;
    for (int c0 = 0; c0 < TK; c0 += NT) {          // uniform trip count
        const int i = c0 + threadIdx.x;
        const int ex = i < TK ? l.idx[i / a.K][i % a.K] : 0;
        const bool first = i < TK && l.first[ex] == i;
        const uint64_t m = __ballot(first);
        if (lane == 0) l.wc[wave] = __popcll(m);
        __syncthreads();
        int off = base, tot = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            off += w < wave ? l.wc[w] : 0;
            tot += l.wc[w];
        }
        if (first) {
            const int slot = off + lanes_below(m);
            l.uq[slot] = ex;
            if (publish) pub_i(&a.route->uniq[slot], ex);
            if (publish && seq) pub_t(&a.route->tuniq[slot], seq, (uint32_t)ex);
        }
        base += tot;
        __syncthreads();
    }
    if (publish) {
        for (int f = threadIdx.x; f < base * K3X_DECODE_MAX_T; f += NT) {
            const int slot = f / K3X_DECODE_MAX_T, t = f % K3X_DECODE_MAX_T;
            const float w = t < a.T ? ks_weight(l, a.K, t, l.uq[slot]) : 0.0f;
            pub_f(&a.route->wtok[slot][t], w);
            if (seq && t < a.T) pub_t(&a.route->twtok[slot][t], seq, __float_as_uint(w));
        }
        if (threadIdx.x == 0) {
            pub_i(&a.route->nu, base);
            pub_i(&a.route->nexact, nex);
            if (seq) pub_t(&a.route->tnu, seq, (uint32_t)base);
        }
    }
    return base;
}

// ------------------------------------------------------------------ K1
struct K1Args {
    const float *router;     // [E][H]
    const float *bias;       // [E]
    const void  *x;          // [T][H]
    int          x_bf16;
    int          T, H, E;
    float       *score, *choice;   // [T][E]
    float       *slack;            // [T][E] (choice_slack)
    unsigned    *hkey;             // [T] largest slack_key of each row (atomic maximum)
    float       *ninv;             // [T] 1/rms of each row, with norm_w
    uint16_t    *xB;               // compact B set of x over whole super-quads
    int          n_rwg;            // workgroups
    unsigned    *seq;              // the call sequence, advanced here
    const float *norm_w;           // RMSNorm weights [H] (fp32 x), or NULL
    float        eps;
    // latent form: z = down . x for the routed experts, and the selection (k1_zdown)
    const uint16_t *ldown;         // tiled bf16 [XL][H], or NULL
    int          XL;
    uint16_t    *zB;               // compact B set of z over whole super-quads of XL
    KSArgs       ks;
    unsigned long long *trace;     // diagnostics, or NULL
};

#define RWAVES 4                     // waves per expert row in the router
#define RCH    8                     // float4 chunks per lane held at once

// RMSNorm's 1/rms of every token (k3_rmsnorm, k3_ops.c:132-140) in the order of
// rmsnorm_kernel (k3x_layout.hip): thread i sums the squares of its float4 chunks i,
// i + 256, ... in double, a shuffle tree per wave, the four waves added in order; a row
// whose float 1/rms that order does not prove (rms_inv_proven) sums its squares again as
// the reference's chain, so the scale is the reference's, as rmsnorm_kernel's is.  Needs
// 256 threads, H <= 8192, and lds of 1152 floats.
__device__ void k1_norm_inv(const K1Args &a, float *lds, float *s_inv)
{
    static_assert(NT1 == 256 && RWAVES * WAVE == NT1, "one 256-thread workgroup per row");
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int nf4 = a.H >> 2;
    const float *x = (const float *)a.x;
    double *dl = (double *)lds;                                 // [4 waves][8]
    for (int t = 0; t < a.T; t++) {
        f32x4 xv[RCH];
#pragma unroll
        for (int c = 0; c < RCH; c++) {
            const int f = threadIdx.x + NT1 * c;
            xv[c] = f < nf4 ? *(const f32x4 *)(x + (size_t)t * a.H + 4 * f)
                            : (f32x4){0.f, 0.f, 0.f, 0.f};
        }
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < RCH; c++)
#pragma unroll
            for (int k = 0; k < 4; k++) ss += (double)xv[c][k] * (double)xv[c][k];
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        if (lane == 0) dl[wave * K3X_DECODE_MAX_T + t] = ss;
    }
    __syncthreads();
    int *redo = (int *)(dl + NT1 / WAVE * K3X_DECODE_MAX_T);   // [8]: rows to work out again
    if (threadIdx.x < a.T) {
        double tot = 0.0;
        for (int w = 0; w < NT1 / WAVE; w++) tot += dl[w * K3X_DECODE_MAX_T + threadIdx.x];
        s_inv[threadIdx.x] = rms_inv(tot, a.H, a.eps);
        redo[threadIdx.x] = !rms_inv_proven(tot, a.H, a.eps);
    }
    __syncthreads();
    // a row whose float 1/rms this order does not prove: its squares summed again as the
    // reference's chain (rare: about one row in 10^5 at the hidden width of 7168)
    for (int t = 0; t < a.T; t++) {
        if (!redo[t]) continue;                 // uniform
        const float *xr = x + (size_t)t * a.H;
        const double ss = wg_dot_chain(xr, 1.0f, xr, a.H, lds + 128, 512, NT1);
        if (threadIdx.x == 0) s_inv[t] = rms_inv(ss, a.H, a.eps);
        __syncthreads();
    }
}

// The slack of a choice whose logit v was summed in another order than the reference's
// single chain (k3_ops.c:1666-1688), from asum, the float sum of |W[e][i] x[i]|.  Each
// product here takes part in at most H/256 + 12 additions (a thread's run, the wave's
// shuffle tree, the four waves' pairs), so the reference's logit is a double within
// d = chain_gap of v, and its float lies in [(float)(v - d), (float)(v + d)]; where both
// ends round to (float)v, the float logit, and with it the score and the choice, are the
// reference's, and the slack is 0.  Otherwise the slack bounds the distance of the
// reference's choice from this one: a quarter of the float interval's half-width (the
// sigmoid's slope is at most 1/4) plus the roundings of the sigmoid and of the bias add (a
// few units in the last place of |choice| <= 2 + |bias|).  NaN logits give a NaN slack,
// which marks nothing (a NaN choice is never selected, here or in the reference).
__device__ __forceinline__ float choice_slack(double v, float asum, int H, float bias)
{
    const double d = chain_gap(abs_bound(asum, H), H);
    const float f = (float)v, lo = (float)(v - d), hi = (float)(v + d);
    if (lo == f && hi == f) return 0.0f;
    const double df = fmax((double)hi - (double)f, (double)f - (double)lo);
    return (float)((df * 0.25 + (2.0 + fabs((double)bias)) * 0x1p-21) * 1.01);
}

// A thread's RCH chunks of four activations of one row (chunk c: elements 4f .. 4f + 3,
// f = tl + NT1 c; zero past the row), all loads issued before any is used: one memory
// round trip per row.  (Loaded and converted chunk by chunk behind a range branch, each
// load was waited for on its own: eight round trips, about 1 us of the router's 5.5 us a
// workgroup.)
__device__ __forceinline__ void load_x_chunks(rsrc_t rx, int x_bf16, uint32_t row_el, int tl,
                                              int nf4, float (&xv)[RCH][4])
{
    if (x_bf16) {
        u32x2 r[RCH];
#pragma unroll
        for (int c = 0; c < RCH; c++) {
            const int f = tl + NT1 * c;
            r[c] = __builtin_amdgcn_raw_buffer_load_b64(
                rx, f < nf4 ? (row_el + 4u * (uint32_t)f) * 2u : K3X_OOB, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < RCH; c++) {
            xv[c][0] = bf2f(r[c][0] & 0xFFFFu); xv[c][1] = bf2f(r[c][0] >> 16);
            xv[c][2] = bf2f(r[c][1] & 0xFFFFu); xv[c][3] = bf2f(r[c][1] >> 16);
        }
    } else {
        u32x4 r[RCH];
#pragma unroll
        for (int c = 0; c < RCH; c++) {
            const int f = tl + NT1 * c;
            r[c] = bload16(rx, f < nf4 ? (row_el + 4u * (uint32_t)f) * 4u : K3X_OOB);
        }
#pragma unroll
        for (int c = 0; c < RCH; c++)
#pragma unroll
            for (int k = 0; k < 4; k++) xv[c][k] = __uint_as_float(r[c][k]);
    }
}

// Router logits: four waves per expert, sum_i W[e][i] x[i] in double (a product of two
// floats is exact in double; only the order of the additions differs from the
// reference's single chain), then score = sigmoid((float)logit), choice = score + bias,
// and the choice's slack (choice_slack; the float sum of |W[e][i] x[i]| runs beside).
// With a.norm_w, x[i] is the normalised nw[i] * x[i] * inv (float, the reference's order);
// the expert's weights are in flight while the norm is worked out.
template <int TM>
__device__ void k1_router(const K1Args &a, float *lds, float *s_inv, bool bset)
{
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int grp = wave / RWAVES, wq = wave % RWAVES;          // expert slot, quarter
    const int e = blockIdx.x * (NT1 / WAVE / RWAVES) + grp;
    const int nf4 = a.H >> 2;
    double acc[TM];
    float aa[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) { acc[t] = 0.0; aa[t] = 0.0f; }
    const int tl = wq * WAVE + lane;                            // 0..255 within the expert
    const rsrc_t rr = make_rsrc(a.router + (size_t)(e < a.E ? e : 0) * a.H,
                                e < a.E ? (uint32_t)a.H * 4u : 0u);
    const rsrc_t rx = make_rsrc(a.x, (uint32_t)(a.T * a.H) * (a.x_bf16 ? 2u : 4u));
    for (int f0 = 0; f0 < nf4; f0 += RWAVES * WAVE * RCH) {
        f32x4 w[RCH];
#pragma unroll
        for (int c = 0; c < RCH; c++) {
            const int f = f0 + tl + RWAVES * WAVE * c;
            w[c] = __builtin_bit_cast(f32x4, wld16(rr, f < nf4 ? 16u * (uint32_t)f : K3X_OOB));
        }
        // one token without the norm: its row's loads in flight with the weights
        float x0[RCH][4];
        const bool pre = TM == 1 && !a.norm_w;
        if (pre) load_x_chunks(rx, a.x_bf16, 0u, f0 + tl, nf4, x0);
        f32x4 nw[RCH];
        if (a.norm_w) {                         // uniform; then f0 == 0 (H <= 8192)
            k1_norm_inv(a, lds, s_inv);
            if (blockIdx.x == 0 && threadIdx.x < a.T) a.ninv[threadIdx.x] = s_inv[threadIdx.x];
#pragma unroll
            for (int c = 0; c < RCH; c++) {
                const int f = tl + RWAVES * WAVE * c;
                nw[c] = f < nf4 ? *(const f32x4 *)(a.norm_w + 4 * f) : (f32x4){0.f, 0.f, 0.f, 0.f};
            }
        }
        if (bset && f0 == 0) {
            // this workgroup's share of x's B set (of the normalised rows with norm_w),
            // while the router's weights are in flight
            const int nS = ((a.H >> 7) + 3) >> 2;
            const int tid = threadIdx.x * a.n_rwg + blockIdx.x, nth = a.n_rwg * NT1;
            x_to_bset((uint8_t *)a.xB, a.x, a.x_bf16, a.H, 2 * a.T, 4 * nS, tid, nth, a.norm_w,
                      s_inv);
        }
#pragma unroll
        for (int t = 0; t < TM; t++) {
            if (t < a.T) {
                float xv[RCH][4];
                if (pre) {
#pragma unroll
                    for (int c = 0; c < RCH; c++)
#pragma unroll
                        for (int k = 0; k < 4; k++) xv[c][k] = x0[c][k];
                } else {
                    load_x_chunks(rx, a.x_bf16, (uint32_t)(t * a.H), f0 + tl, nf4, xv);
                }
                if (a.norm_w) {
                    const float inv = s_inv[t];
#pragma unroll
                    for (int c = 0; c < RCH; c++)
#pragma unroll
                        for (int k = 0; k < 4; k++) xv[c][k] = nw[c][k] * xv[c][k] * inv;
                }
#pragma unroll
                for (int c = 0; c < RCH; c++)
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        acc[t] += (double)w[c][k] * (double)xv[c][k];
                        aa[t] = fmaf(fabsf(w[c][k]), fabsf(xv[c][k]), aa[t]);
                    }
            }
        }
    }
    double *dl = (double *)lds;                                 // [4 waves][8]
    float *al = (float *)(dl + NT1 / WAVE * K3X_DECODE_MAX_T);  // [4 waves][8]
#pragma unroll
    for (int t = 0; t < TM; t++) {
        if (t < a.T) {
            double v = acc[t];
            float av = aa[t];
            for (int off = 32; off >= 1; off >>= 1) {
                v += __shfl_xor(v, off);
                av += __shfl_xor(av, off);
            }
            if (lane == 0) {
                dl[wave * K3X_DECODE_MAX_T + t] = v;
                al[wave * K3X_DECODE_MAX_T + t] = av;
            }
        }
    }
    __syncthreads();
    if (wq == 0 && lane < a.T && e < a.E) {
        const int t = lane;
        const double *g = dl + grp * RWAVES * K3X_DECODE_MAX_T;
        const float *ga = al + grp * RWAVES * K3X_DECODE_MAX_T;
        const double v = (g[t] + g[K3X_DECODE_MAX_T + t]) +
                         (g[2 * K3X_DECODE_MAX_T + t] + g[3 * K3X_DECODE_MAX_T + t]);
        const float as = (ga[t] + ga[K3X_DECODE_MAX_T + t]) +
                         (ga[2 * K3X_DECODE_MAX_T + t] + ga[3 * K3X_DECODE_MAX_T + t]);
        const float sc = sigmoid_ref((float)v);
        const size_t o = (size_t)t * a.E + e;
        const float ch = sc + a.bias[e], sl = choice_slack(v, as, a.H, a.bias[e]);
        a.score[o] = sc;
        a.choice[o] = ch;
        a.slack[o] = sl;
        if (sl > 0.0f) atomicMax(&a.hkey[t], slack_key(ch, sl));
    }
}

// One quad of x's B fragments, raw (x rows ldx elements apart): lane (n, kq) holds token n/2's elements 128q + 32kq +
// 8t .. +7 for each product t (fp32: two float4; bf16: one 16-byte load, lo lanes zero).
// Split into bf16 hi/lo only when used, so the loads stay in flight in a ring.
struct XQ {
    f32x4 v[4][2];
};

__device__ __forceinline__ void xq_load(XQ &b, rsrc_t xr, int x_bf16, int ldx, int NC, int q,
                                        bool on, int lane)
{
    const int n0 = lane & 15, kq = lane >> 4;
    const int n = n0 < NC ? n0 : 0, tok = n >> 1, hl = n & 1;
    const uint32_t e0 = (uint32_t)(tok * ldx + q * 128 + kq * 32);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        if (x_bf16) {
            const u32x4 r = bload16(xr, on && !hl ? (e0 + 8u * t) * 2u : K3X_OOB);
            b.v[t][0] = __builtin_bit_cast(f32x4, r);
        } else {
            b.v[t][0] = __builtin_bit_cast(f32x4, bload16(xr, on ? (e0 + 8u * t) * 4u : K3X_OOB));
            b.v[t][1] = __builtin_bit_cast(f32x4, bload16(xr, on ? (e0 + 8u * t) * 4u + 16u : K3X_OOB));
        }
    }
}

__device__ __forceinline__ u32x4 xq_get(const XQ &b, int x_bf16, int t, int lane)
{
    if (x_bf16) return __builtin_bit_cast(u32x4, b.v[t][0]);
    const float v[8] = {b.v[t][0][0], b.v[t][0][1], b.v[t][0][2], b.v[t][0][3],
                        b.v[t][1][0], b.v[t][1][1], b.v[t][1][2], b.v[t][1][3]};
    return bfrag_of(v, lane & 1);
}

// One 16-row tile of a tiled bf16 matrix (K columns) times the T activation rows of x
// (row stride ldx elements, fp32 or bf16): four waves on interleaved quads, each quad's
// B fragments read from x with its weights (x is small and stays in the caches).  The
// workgroup's waves are summed in LDS; wave 0 ends with acc (per_token's layout).
__device__ __forceinline__ void bf16_tile_x(const uint16_t *wtile, int K, const void *x,
                                            int x_bf16, int ldx, int T, float *lds,
                                            float (&acc)[4])
{
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    constexpr int NW = NT1 / WAVE;
    const int nQ = K >> 7, NC = 2 * T;
    const int cnt = strided_count(wave, NW, nQ);
    const rsrc_t rw = make_rsrc(wtile, (uint32_t)nQ * 4096u);
    const rsrc_t xr = make_rsrc(x, (uint32_t)(((T - 1) * ldx + K) * (x_bf16 ? 2 : 4)));
    QB w[2];
    XQ b[2];
    auto ld = [&](int i, int k) AI {
        const bool on = k < cnt;
        const int q = wave + NW * k;
        qb_load(w[i], rw, on ? (uint32_t)q * 4096u : K3X_OOB, lane);
        xq_load(b[i], xr, x_bf16, ldx, NC, q, on, lane);
    };
    ring_prime<2>(ld);
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    ring_loop<2>(cnt, ld, [&](int i, int k) AI {
        u32x4 bb[4];
#pragma unroll
        for (int t = 0; t < 4; t++) bb[t] = xq_get(b[i], x_bf16, t, lane);
        qb_mfma(d, w[i], bb);
    });
    acc[0] = d[0]; acc[1] = d[1]; acc[2] = d[2]; acc[3] = d[3];
    wave_sum_lds<4, NW>(acc, lds, wave, lane);
}

// One 16-row tile of a tiled bf16 matrix (K columns) times x's compact B set (built by
// the router launch), staged in LDS: four waves on interleaved quads, as bf16_tile_x, so
// the same sums; ZR quads of weights in flight a wave (bf16_tile_x keeps two, its ring
// also holding x's fragments).
#define ZR 4
__device__ __forceinline__ void bf16_tile_bset(const uint16_t *wtile, int K, const uint16_t *xB,
                                               int NC, float *lds, float (&acc)[4])
{
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    constexpr int NW = NT1 / WAVE;
    const int nQ = K >> 7, nS = (nQ + 3) >> 2;
    const int cnt = strided_count(wave, NW, nQ);
    const uint32_t bbytes = (uint32_t)nS * 1024u * NC;
    Stage<8> st;
    st.issue(xB, bbytes, NT1);
    const rsrc_t rw = make_rsrc(wtile, (uint32_t)nQ * 4096u);
    QB w[ZR];
    auto ld = [&](int i, int k) AI {
        qb_load(w[i], rw, k < cnt ? (uint32_t)(wave + NW * k) * 4096u : K3X_OOB, lane);
    };
    ring_prime<ZR>(ld);
    st.commit(NT1);
    __syncthreads();
    BFrag<true> bf;
    bf.init(xB, bbytes, NC, lane);
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    ring_loop<ZR>(cnt, ld, [&](int i, int k) AI {
        const int q = wave + NW * k;
        u32x4 b[4];
#pragma unroll
        for (int t = 0; t < 4; t++) b[t] = bf.get(0u, q, t);
        qb_mfma(d, w[i], b);
    });
    acc[0] = d[0]; acc[1] = d[1]; acc[2] = d[2]; acc[3] = d[3];
    wave_sum_lds<4, NW>(acc, lds, wave, lane);
}

// The latent down projection z = down . x (k3_mmw_batch, k3_ops.c:1871) for rows
// 16*rt .. +15, and z's hi/lo B fragments into zB for k2's routed products.  LDSB: x's
// B set (the router launch's, with the same fragments bf16_tile_x forms from x) staged in
// LDS, for calls whose set fits (1 or 2 tokens).
template <bool LDSB>
__device__ void k1_down(const K1Args &a, float *lds, int rt)
{
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int NC = 2 * a.T;
    float acc[4];
    if (LDSB) bf16_tile_bset(a.ldown + (size_t)rt * 16 * a.H, a.H, a.xB, NC, lds, acc);
    else bf16_tile_x(a.ldown + (size_t)rt * 16 * a.H, a.H, a.x, a.x_bf16, a.H, a.T, lds, acc);
    // z's set holds whole super-quads; its quads past XL/128 stay zero
    const int nSX = ((a.XL >> 7) + 3) >> 2;
    if (rt == 0)
        for (uint32_t o = (uint32_t)(a.XL >> 7) * 256u * NC + threadIdx.x * 16u;
             o < (uint32_t)nSX * 1024u * NC; o += NT1 * 16u)
            *(u32x4 *)((uint8_t *)a.zB + o) = (u32x4){0u, 0u, 0u, 0u};
    if (wave != 0) return;
    per_token<4>(acc, NC, lane, [&](int r0, int tok, const float (&v)[4]) AI {
        for (int i = 0; i < 4; i++) {
            uint32_t hi, lo;
            split_bf16(v[i], hi, lo);
            const int r = rt * 16 + r0 + i;
            a.zB[bfrag_off(r, 2 * tok, NC)] = (uint16_t)hi;
            a.zB[bfrag_off(r, 2 * tok + 1, NC)] = (uint16_t)lo;
        }
    });
}

// The latent form's second launch: workgroup 0 selects each token's experts from the
// router's scores and publishes the routing (ks_route), the others work out z = down . x,
// 16 rows each.  The routed workgroups of k2_gateup then start on a published routing
// instead of waiting inside their own launch, where the selection's few loads queue
// behind the streaming workgroups' (about 14 us at the K3 shape).  A launch of its own:
// folded into k1_router_bset's grid, the two paths' register allocation merges badly
// (spills).
template <int NE, bool LDSB>
__global__ void __launch_bounds__(NT1) k1_zdown(K1Args a)
{
    __shared__ float lds[(NT1 / WAVE - 1) * 4 * WAVE];
    if (blockIdx.x == 0) {
        ks_route<NE>(a.ks, *(KSLds *)dyn_lds, true);
        return;
    }
    k1_down<LDSB>(a, lds, blockIdx.x - 1);
}

// Router logits of NT1 / WAVE / RWAVES experts (of the RMSNorm of x when norm_w is given),
// and a share of x's B set for k2; TM: the most tokens a call carries (1, or
// K3X_DECODE_MAX_T).
template <int TM>
__global__ void __launch_bounds__(NT1) k1_router_bset(K1Args a)
{
    __shared__ float lds[(NT1 / WAVE - 1) * 8 * WAVE];
    __shared__ float s_inv[K3X_DECODE_MAX_T];
    WgTrace tr;
    tr.start(a.trace);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const unsigned q = *a.seq + 1u;
        *a.seq = q ? q : 1u;                 // 0 tags nothing
    }
    // the B set's entries are dealt across the workgroups (a few per workgroup) and
    // converted while the router's weights are in flight
    k1_router<TM>(a, lds, s_inv, true);
    tr.end();
}

// Router logits of several tokens without the RMSNorm: RM_EPW experts per workgroup,
// x's rows (raw, bf16 or fp32) staged once in LDS for all of them, TG tokens at a time.
// Each expert's 256 threads take the chunks, the per-thread order and the reduction tree
// of k1_router, so every logit is bitwise the single-expert kernel's.  k1_router reads
// every token's x from L2 in each expert's workgroup, a load and its use at a time (8
// tokens of the K2 shape: 44 MB of 8-byte loads a call, 21 us a workgroup); staged once
// per two experts, a workgroup takes 12 us, most of it the double-precision products.
#define RM_EPW 2
#define RM_XLDS (120 * 1024)         // LDS for staged x rows

template <int TT, int TG, bool XBF>
__global__ void __launch_bounds__(NT1 * RM_EPW) k1_router_mt(K1Args a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    __shared__ double dl[RM_EPW * RWAVES][K3X_DECODE_MAX_T];
    __shared__ float al[RM_EPW * RWAVES][K3X_DECODE_MAX_T];
    WgTrace tr;
    tr.start(a.trace);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const unsigned q = *a.seq + 1u;
        *a.seq = q ? q : 1u;                 // 0 tags nothing
    }
    constexpr int XB = XBF ? 2 : 4;          // bytes per x element
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int grp = threadIdx.x / NT1, tl = threadIdx.x % NT1;
    const int e = blockIdx.x * RM_EPW + grp;
    const int nf4 = a.H >> 2;
    const float *row = a.router + (size_t)(e < a.E ? e : 0) * a.H;
    f32x4 w[RCH];
#pragma unroll
    for (int c = 0; c < RCH; c++) {
        const int f = tl + NT1 * c;
        w[c] = (f < nf4 && e < a.E) ? __builtin_nontemporal_load((const f32x4 *)(row + 4 * f))
                                    : (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    {
        // this workgroup's share of x's B set, as k1_router deals it over 256-thread groups
        const int nS = ((a.H >> 7) + 3) >> 2;
        const int tid = threadIdx.x * (int)gridDim.x + blockIdx.x, nth = (int)gridDim.x * NT1 * RM_EPW;
        x_to_bset((uint8_t *)a.xB, a.x, a.x_bf16, a.H, 2 * a.T, 4 * nS, tid, nth);
    }
    for (int t0 = 0; t0 < TT; t0 += TG) {
        const int ng = TT - t0 < TG ? TT - t0 : TG;
        // rows t0 .. t0 + ng - 1 into LDS, 16 bytes a thread at a time
        const size_t rowb = (size_t)a.H * XB;
        const uint8_t *src = (const uint8_t *)a.x + (size_t)t0 * rowb;
        const int n16 = (int)((size_t)ng * rowb / 16);
        if (t0) __syncthreads();             // the previous group's reads are done
        // eight loads in flight per thread before their stores (one at a time, each
        // would wait out its own latency)
        constexpr int NB = NT1 * RM_EPW, UNR = 8;
        for (int i0 = 0; i0 < n16; i0 += NB * UNR) {
            u32x4 r[UNR];
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int i = i0 + u * NB + (int)threadIdx.x;
                r[u] = i < n16 ? *(const u32x4 *)(src + (size_t)i * 16) : (u32x4){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int i = i0 + u * NB + (int)threadIdx.x;
                if (i < n16) *(u32x4 *)(xs + (size_t)i * 16) = r[u];
            }
        }
        __syncthreads();
        // one token at a time (a loop, not unrolled: unrolled, every token's widened x
        // would be live at once): this thread's chain, then the wave's sum
#pragma unroll 1
        for (int g = 0; g < ng; g++) {
            double v = 0.0;
            float av = 0.0f;
#pragma unroll
            for (int c = 0; c < RCH; c++) {
                const int f = tl + NT1 * c;
                float xv[4] = {0.f, 0.f, 0.f, 0.f};
                if (f < nf4) {
                    const uint8_t *px = xs + ((size_t)g * a.H + 4 * f) * XB;
                    if (XBF) {
                        const u32x2 r = *(const u32x2 *)px;
                        xv[0] = bf2f(r[0] & 0xFFFFu); xv[1] = bf2f(r[0] >> 16);
                        xv[2] = bf2f(r[1] & 0xFFFFu); xv[3] = bf2f(r[1] >> 16);
                    } else {
                        const f32x4 r = *(const f32x4 *)px;
                        xv[0] = r[0]; xv[1] = r[1]; xv[2] = r[2]; xv[3] = r[3];
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    v += (double)w[c][k] * (double)xv[k];
                    av = fmaf(fabsf(w[c][k]), fabsf(xv[k]), av);
                }
            }
            for (int off = 32; off >= 1; off >>= 1) {
                v += __shfl_xor(v, off);
                av += __shfl_xor(av, off);
            }
            if (lane == 0) {
                dl[wave][t0 + g] = v;
                al[wave][t0 + g] = av;
            }
        }
    }
    __syncthreads();
    const int wq = wave % RWAVES;
    if (wq == 0 && lane < TT && e < a.E) {
        const int t = lane, w0 = grp * RWAVES;
        const double v = (dl[w0][t] + dl[w0 + 1][t]) + (dl[w0 + 2][t] + dl[w0 + 3][t]);
        const float as = (al[w0][t] + al[w0 + 1][t]) + (al[w0 + 2][t] + al[w0 + 3][t]);
        const float sc = sigmoid_ref((float)v);
        const size_t o = (size_t)t * a.E + e;
        const float ch = sc + a.bias[e], sl = choice_slack(v, as, a.H, a.bias[e]);
        a.score[o] = sc;
        a.choice[o] = ch;
        a.slack[o] = sl;
        if (sl > 0.0f) atomicMax(&a.hkey[t], slack_key(ch, sl));
    }
    tr.end();
}

// The router launch: the multi-token kernel for 2 .. 8 tokens without the RMSNorm when a
// group of at least two rows fits the LDS, else k1_router_bset.  Returns the grid.
static unsigned launch_k1(const K1Args &a1, hipStream_t s)
{
    const int T = a1.T;
    const size_t rowb = (size_t)a1.H * (a1.x_bf16 ? 2 : 4);
    const int fit = (int)(RM_XLDS / rowb);
    if (T >= 2 && !a1.norm_w && fit >= 2 && a1.H <= RCH * NT1 * 4) {
        const dim3 g((unsigned)((a1.E + RM_EPW - 1) / RM_EPW)), b(NT1 * RM_EPW);
        const int tg = T <= fit ? T : (fit >= 4 ? 4 : 2);
        const size_t lds = (size_t)(tg < T ? tg : T) * rowb;
#define K1MT(TT_) \
        if (a1.x_bf16) { if (tg >= TT_) hipLaunchKernelGGL((k1_router_mt<TT_, TT_, true>), g, b, lds, s, a1); \
                         else if (tg >= 4) hipLaunchKernelGGL((k1_router_mt<TT_, (TT_ < 4 ? TT_ : 4), true>), g, b, lds, s, a1); \
                         else hipLaunchKernelGGL((k1_router_mt<TT_, 2, true>), g, b, lds, s, a1); } \
        else           { if (tg >= TT_) hipLaunchKernelGGL((k1_router_mt<TT_, TT_, false>), g, b, lds, s, a1); \
                         else if (tg >= 4) hipLaunchKernelGGL((k1_router_mt<TT_, (TT_ < 4 ? TT_ : 4), false>), g, b, lds, s, a1); \
                         else hipLaunchKernelGGL((k1_router_mt<TT_, 2, false>), g, b, lds, s, a1); }
        switch (T) {
        case 2: K1MT(2) break;
        case 3: K1MT(3) break;
        case 4: K1MT(4) break;
        case 5: K1MT(5) break;
        case 6: K1MT(6) break;
        case 7: K1MT(7) break;
        default: K1MT(8) break;
        }
#undef K1MT
        return g.x;
    }
    if (T == 1) hipLaunchKernelGGL(k1_router_bset<1>, dim3(a1.n_rwg), dim3(NT1), 0, s, a1);
    else hipLaunchKernelGGL(k1_router_bset<K3X_DECODE_MAX_T>, dim3(a1.n_rwg), dim3(NT1), 0, s, a1);
    return (unsigned)a1.n_rwg;
}

// ------------------------------------------------------------------ K2
struct K2Args {
    KSArgs         ks;             // the routing, worked out by workgroup 0
    const k3x_route *route;        // tnu / tuniq / twtok: the tagged routing of this launch
    const unsigned *seq;           // this call's sequence (advanced by k1)
    int           *err;            // set by a routed workgroup that gave up waiting
    uint64_t       wait_ticks;     // the routed workgroups' bound on the wait
    int            publish;        // 0 only to exercise the bound (failure-handling test)
    const uint8_t *experts;
    size_t         expert_bytes, gate_off, up_off;
    const uint16_t *xB;            // compact B set of x over whole super-quads
    uint16_t      *actB;           // one compact B set per unique expert (slot)
    int            T, H, I;
    int            n_sh;           // workgroups of the shared expert (the first ones)
    const uint16_t *sh_gate, *sh_up;
    int            SI;
    uint16_t      *shB;            // compact B set of the shared activation, for k3
    const uint16_t *rB;            // the routed experts' input set: xB, or z's in the latent form
    int            XL;             // its width (H, or the latent width)
    float          b1, b2;         // SiTU betas (0: that half uncapped)
    int            rtw;            // row tiles per routed workgroup (1, 2 or 4)
    int            sb;             // 1 (with rtw 2 and the input's B set past the LDS): each
                                   // super-quad's B fragments staged once for the four waves
    const int     *slot;           // expert -> arena slot (expert cache), or NULL: identity
    int            sel_done;       // 1: the routing was published by an earlier launch
                                   // (k1_zdown): no selection here, no wait
    unsigned long long *trace;     // diagnostics, or NULL
};

// Shared expert gate and up products for rows 16*rt .. +15 over the full K: four waves on
// interleaved quads (each wave both matrices of a quad, over one B read); SiTU-GLU
// (k3_situ_glu, k3_ops.c:148-161) per token and the activation's hi/lo B fragments into
// shB.  These workgroups come first: they stream while the routed ones
// work out the routing.
template <bool LDSB>
__device__ void k2_shared(const K2Args &a, float *lds, int rt)
{
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int NW = NT / WAVE;
    const int nQ = a.H >> 7, nS = (nQ + 3) >> 2, NC = 2 * a.T;
    const int cnt = strided_count(wave, NW, nQ);
    const uint32_t tbytes = (uint32_t)nQ * 4096u;
    const rsrc_t rg = make_rsrc(a.sh_gate + (size_t)rt * 16 * a.H, tbytes);
    const rsrc_t ru = make_rsrc(a.sh_up + (size_t)rt * 16 * a.H, tbytes);
    const uint32_t bbytes = (uint32_t)nS * 1024u * NC;
    Stage<8> st;
    if (LDSB) st.issue(a.xB, bbytes, NT);
    QB g[2], u[2];
    auto ld = [&](int i, int k) AI {
        const uint32_t o = k < cnt ? (uint32_t)(wave + NW * k) * 4096u : K3X_OOB;
        qb_load(g[i], rg, o, lane);
        qb_load(u[i], ru, o, lane);
    };
    ring_prime<2>(ld);
    if (LDSB) {
        st.commit(NT);
        __syncthreads();
    }
    BFrag<LDSB> bf;
    bf.init(a.xB, bbytes, NC, lane);
    f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
    ring_loop<2>(cnt, ld, [&](int i, int k) AI {
        const int q = wave + NW * k;
        u32x4 b[4];
#pragma unroll
        for (int t = 0; t < 4; t++) b[t] = bf.get(0u, q, t);
        qb_mfma(dg, g[i], b);
        qb_mfma(du, u[i], b);
    });
    float acc[8] = {dg[0], dg[1], dg[2], dg[3], du[0], du[1], du[2], du[3]};
    wave_sum_lds<8, NT / WAVE>(acc, lds, wave, lane);
    if (wave != 0) return;
    per_token<8>(acc, NC, lane, [&](int r0, int tok, const float (&v)[8]) AI {
        for (int i = 0; i < 4; i++) {
            uint32_t hi, lo;
            split_bf16(situ(v[i], v[4 + i], a.b1, a.b2), hi, lo);
            const int r = rt * 16 + r0 + i;
            a.shB[bfrag_off(r, 2 * tok, NC)] = (uint16_t)hi;
            a.shB[bfrag_off(r, 2 * tok + 1, NC)] = (uint16_t)lo;
        }
    });
}

// Workgroup 0 works out the routing (ks_route) and publishes it.  Next come the shared
// expert's workgroups, which need no routing and stream meanwhile; then the routed ones,
// which wait for it.  Workgroups are dispatched in order, so workgroup 0 is resident
// before any routed one waits, and it waits on nothing.  The handoff needs no ordering
// between memory locations: every word a routed workgroup reads (the unique count, its
// slot's expert, the slot's weight per token) is a 64-bit word (seq << 32) | value,
// written and read by relaxed atomic operations at agent scope, with seq the call's
// sequence number (advanced by k1 of the same call).  Atomic operations on one location
// are coherent, so a word read with this call's seq holds the value workgroup 0 stored
// in this call, and the reader needs neither a release/acquire pair nor the cache
// invalidation of an acquire fence (measured: 1.85 us of k2 at b = 1).  The wait is
// bounded (wait_ticks of the 100 MHz clock, by default 1 s, far above the selection's
// few microseconds, and above its worst case where every expert's logit of eight tokens
// is worked out again as the reference's chain, about 20 us each): a workgroup that
// gives up sets the error word (k3x_moe_layer_check reports it) and leaves without
// touching the expert weights.

// Gate and up products of rtw row tiles (16 rows each) of one unique expert: the waves
// are dealt over the tiles (4/rtw waves per tile, on interleaved super-quads of it);
// SiTU-GLU, the token's routing weight for this expert (0 where the token did not choose
// it) and the bf16 hi/lo split into the expert's activation slot.  Several tiles per
// workgroup when a tile has few super-quads (a narrow latent width), so that each wave
// streams a run of items and the per-workgroup staging and waits are amortised.
#ifndef K2SB_R
#define K2SB_R 2                       // stages of the shared-B path (super-quads)
#endif
#define K2SB_BL 4                      // its B loads per thread and super-quad (16 KB)
#define K2SB_STAGE (1024u * 2 * K3X_DECODE_MAX_T)   // LDS bytes of a stage's B
template <bool EXACT, bool LDSB, int NE>
__device__ void k2_gateup_body(const K2Args &a, float *lds, int *s_go_p);

template <bool EXACT, bool LDSB, int NE>
__global__ void __launch_bounds__(NT) k2_gateup(K2Args a)
{
    __shared__ float lds[(NT / WAVE - 1) * 8 * WAVE];
    __shared__ int s_go;
    WgTrace tr;
    tr.start(a.trace);
    k2_gateup_body<EXACT, LDSB, NE>(a, lds, &s_go);
    tr.end();
}

template <bool EXACT, bool LDSB, int NE>
__device__ void k2_gateup_body(const K2Args &a, float *lds, int *s_go_p)
{
    int &s_go = *s_go_p;
    if (blockIdx.x == 0) {
        // NE = 0: the launches after an earlier launch's selection (sel_done), built
        // without the selection's code and its registers
        if constexpr (NE > 0) {
            if (a.sel_done) return;
            // publish = 0 (the failure-handling test) leaves the tagged words unwritten,
            // so that the routed workgroups' bound runs out
            ks_route<NE>(a.ks, *(KSLds *)dyn_lds, true, a.publish ? *a.seq : 0u);
        }
        return;
    }
    if ((int)blockIdx.x <= a.n_sh) {
        k2_shared<LDSB>(a, lds, blockIdx.x - 1);
        return;
    }
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int NW = NT / WAVE;
    const int NC = 2 * a.T;
    const int RTW = a.rtw, WPT = NW / RTW;           // tiles per workgroup, waves per tile
    const int tw = wave % RTW, sw = wave / RTW;      // this wave's tile, its rank on it
    const int nGroups = (a.I >> 4) / RTW;
    const int blk = blockIdx.x - 1 - a.n_sh;
    const int u = blk / nGroups, g0 = (blk % nGroups) * RTW, rt = g0 + tw;
    const int nS = ((a.XL >> 7) + 3) >> 2;
    const uint32_t bbytes = (uint32_t)nS * 1024u * NC;
    if (LDSB) {                        // the input's B set into LDS while the routing is worked out
        Stage<8> st;
        st.issue(a.rB, bbytes, NT);
        st.commit(NT);
    }
    // the routing words this workgroup needs: the unique count, its slot's expert and the
    // slot's weight per token (into s_w); after an earlier launch's selection (sel_done)
    // the plain words, written before this launch began, else their tagged copies
    __shared__ float s_w[K3X_DECODE_MAX_T];
    __shared__ int s_e;
    const k3x_route *rte = a.route;
    if (a.sel_done) {
        if (wave == 0) {
            // lane 0 the unique count, lane 1 its slot's expert, lanes 2 .. T + 1 the slot's
            // weight per token: one load each, all at once
            const int nw = 2 + a.T;
            const int *p = lane == 0 ? &rte->nu
                         : lane == 1 ? &rte->uniq[u]
                                     : (const int *)&rte->wtok[u][lane < nw ? lane - 2 : 0];
            const int v = lane < nw ? *p : 0;
            const int nu = __shfl(v, 0), e = __shfl(v, 1);
            if (u < nu && lane >= 2 && lane < nw) s_w[lane - 2] = __int_as_float(v);
            if (lane == 0) {
                s_go = u < nu;
                s_e = u < nu ? e : 0;
            }
        }
    } else if (wave == 0) {
        // lane 0 reads the unique count, lane 1 its slot's expert, lanes 2 .. T + 1 the
        // slot's weight per token, all at once, until each carries this call's tag (or
        // the count does and this slot is past it); the bound ends the wait with an error
        const unsigned seq = *a.seq;
        const int nw = 2 + a.T;
        const unsigned long long *p = lane == 0 ? &rte->tnu
                                    : lane == 1 ? &rte->tuniq[u]
                                                : &rte->twtok[u][lane < nw ? lane - 2 : 0];
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        int go = 0, e = 0;
        for (;;) {
            const unsigned long long wv =
                lane < nw ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : (unsigned long long)seq << 32;
            const uint32_t v = (uint32_t)wv;
            const uint64_t ok = __ballot((unsigned)(wv >> 32) == seq);
            if ((ok & 1ull) && u >= (int)__shfl(v, 0)) break;
            if (ok == ~0ull) {
                go = 1;
                e = (int)__shfl(v, 1);
                if (lane >= 2 && lane < nw) s_w[lane - 2] = __uint_as_float(v);
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks) {
                if (lane == 0) __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) {
            s_go = go;
            s_e = e;
        }
    }
    __syncthreads();
    if (!s_go) return;
    int e = s_e;
    if (a.slot) e = a.slot[e];
    const uint32_t tb = (uint32_t)fp4_tile_bytes(a.XL);
    const uint8_t *ex = a.experts + (size_t)e * a.expert_bytes + (size_t)rt * tb;
    const rsrc_t rg = make_rsrc(ex + a.gate_off, tb);
    const rsrc_t ru = make_rsrc(ex + a.up_off, tb);
    f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
    if (!LDSB && a.sb) {
        // several tokens: wave (tw, sw) streams matrix sw (gate, up) of tile tw over every
        // super-quad; each super-quad's B fragments come straight into an LDS stage, once
        // for the four waves, with its weights.  K2SB_R stages: a wave has K2SB_R - 1
        // super-quads' loads in flight while it multiplies one.
        const rsrc_t rw = sw ? ru : rg;
        const uint32_t sqb = 1024u * (uint32_t)NC;           // B bytes of a super-quad
        const rsrc_t rbB = make_rsrc(a.rB, bbytes);
        constexpr int LPI = 5 + K2SB_BL;                      // vector loads per super-quad
        SQ w[K2SB_R];
        auto ld = [&](int i, int S) AI {
            const bool on = S < nS;
            sq_load(w[i], rw, on ? (uint32_t)S * SQ_BYTES : K3X_OOB, lane);
#pragma unroll
            for (int c = 0; c < K2SB_BL; c++) {
                const uint32_t o = threadIdx.x * 16u + (uint32_t)c * NT * 16u;
                const uint32_t go = (on && o < sqb) ? (uint32_t)S * sqb + o : K3X_OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rbB, (lds_void *)(dyn_lds + (uint32_t)i * K2SB_STAGE + (uint32_t)c * NT * 16u +
                                      (uint32_t)wave * WAVE * 16u), 16, go, 0, 0, 0);
            }
        };
        BFrag<true> bl;
        bl.init(nullptr, 0u, NC, lane);
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        auto mm = [&](const SQ &wq, int i) AI {
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    d = mfma(sq_a<EXACT>(wq, j, t), as_bf16x8(bl.get((uint32_t)i * K2SB_STAGE, j, t)), d);
        };
#pragma unroll
        for (int i = 0; i < K2SB_R - 1; i++) {
            SCHED_FENCE();
            ld(i, i);
        }
        SCHED_FENCE();
        // super-quad S + i: wait for its loads (those of the K2SB_R - 2 after it remain),
        // meet the other waves (so that stage i - 1 is no longer read), refill that stage
        // with super-quad S + i + K2SB_R - 1, multiply
        for (int S = 0; S < nS; S += K2SB_R) {
#pragma unroll
            for (int i = 0; i < K2SB_R; i++) {
                if (S + i < nS) {
                    meet<(K2SB_R - 2) * LPI>();
                    SCHED_FENCE();
                    ld((i + K2SB_R - 1) % K2SB_R, S + i + K2SB_R - 1);
                    SCHED_FENCE();
                    mm(w[i], i);
                }
            }
        }
        WAIT_VMCNT_LGKM0(0);
        if (sw) du = d;
        else    dg = d;
    } else {
        const int cnt = strided_count(sw, WPT, nS);
        SQ g[2], v[2];
        auto ld = [&](int i, int k) AI {
            const uint32_t o = k < cnt ? (uint32_t)(sw + WPT * k) * SQ_BYTES : K3X_OOB;
            sq_load(g[i], rg, o, lane);
            sq_load(v[i], ru, o, lane);
        };
        ring_prime<2>(ld);
        BFrag<LDSB> bf;
        bf.init(a.rB, bbytes, NC, lane);
        ring_loop<2>(cnt, ld, [&](int i, int k) AI {
            sq_mfma2<EXACT, LDSB>(dg, du, g[i], v[i], bf, sw + WPT * k);
        });
    }
    float acc[8] = {dg[0], dg[1], dg[2], dg[3], du[0], du[1], du[2], du[3]};
    // the waves of one tile summed into its rank-0 wave (waves tw + RTW*j)
    if (sw != 0)
        for (int i = 0; i < 8; i++) lds[((wave - 1) * 8 + i) * WAVE + lane] = acc[i];
    __syncthreads();
    if (sw == 0)
        for (int j = 1; j < WPT; j++)
            for (int i = 0; i < 8; i++) acc[i] += lds[((tw + RTW * j - 1) * 8 + i) * WAVE + lane];
    // the slot holds whole super-quads; its quads past I/128 stay zero
    const int nSI = ((a.I >> 7) + 3) >> 2;
    const uint32_t slot = (uint32_t)nSI * 1024u * NC;
    uint8_t *dst = (uint8_t *)a.actB + (size_t)u * slot;
    if (g0 == 0)
        for (uint32_t o = (uint32_t)(a.I >> 7) * 256u * NC + threadIdx.x * 16u; o < slot; o += NT * 16u)
            *(u32x4 *)(dst + o) = (u32x4){0u, 0u, 0u, 0u};
    if (sw != 0) return;
    uint16_t *d16 = (uint16_t *)dst;
    per_token<8>(acc, NC, lane, [&](int r0, int tok, const float (&s)[8]) AI {
        const float w = s_w[tok];
        for (int i = 0; i < 4; i++) {
            const float y = (w == 0.0f) ? 0.0f : w * situ(s[i], s[4 + i], a.b1, a.b2);
            uint32_t hi, lo;
            split_bf16(y, hi, lo);
            const int r = rt * 16 + r0 + i;
            d16[bfrag_off(r, 2 * tok, NC)] = (uint16_t)hi;
            d16[bfrag_off(r, 2 * tok + 1, NC)] = (uint16_t)lo;
        }
    });
}

// ------------------------------------------------------------------ K3
struct K3Args {
    const uint8_t *experts;
    size_t         expert_bytes, down_off;
    const k3x_route *route;
    const uint16_t *actB;
    const uint16_t *sh_down;       // shared expert down matrix (tiled bf16), or NULL
    const uint16_t *shB;           // compact B set of the shared activation
    int            SI;
    float         *out;            // [T][H] (or the latent aggregates [T][XL])
    const float   *resid;
    int            T, H, I, K;     // H: the output rows (the latent width in that form)
    uint32_t       lds_bytes;      // LDS for the routed activation sets
    uint32_t       sh_lds;         // LDS for the shared activation set (after them), or 0
    int            upp;            // unique experts per part: part blockIdx.y takes slots
                                   // upp*y .. upp*y + upp - 1 (the latent form's split)
    size_t         pstride;        // floats between parts' outputs (0: one part)
    const int     *slot;           // expert -> arena slot (expert cache), or NULL: identity
    unsigned long long *trace;     // diagnostics, or NULL
    float         *pacc;           // k3_down_wide: part sums, [part][DECODE_MAX_T][H]
    int            pr;             // k3_down_wide: parts of the routed items (the rest of
                                   // blockIdx.y: parts of the shared expert's quads)
};

// A bf16 quad of the shared down matrix with its B fragments (read from the shared
// activation's B set in global memory, which every workgroup reads: an L2 hit).
struct QBB {
    QB    a;
    u32x4 b[4];
};

// Down products of 16 output rows over every (unique expert, super-quad) item, then the
// shared expert's down product over its bf16 quads, eight waves interleaved, into one
// accumulator set.  Both rings are primed first, so the shared quads' loads are in
// flight while the routed items stream.
template <bool EXACT, bool LDSB, bool SHL>
__device__ __forceinline__ void k3_body(const K3Args &a, f32x4 &d, int wave, int lane, int u0,
                                        int nu)
{
    const int NW = NT3 / WAVE;
    const int NC = 2 * a.T;
    const int rt = blockIdx.x;
    const int nSI = ((a.I >> 7) + 3) >> 2;
    const uint32_t slot = (uint32_t)nSI * 1024u * NC;
    const uint32_t tb = (uint32_t)fp4_tile_bytes(a.I);
    const int cnt = strided_count(wave, NW, nu * nSI);
    const int nQS = (a.sh_down && blockIdx.y == 0) ? a.SI >> 7 : 0;
    const uint16_t *actB = a.actB + (size_t)u0 * (slot / 2);   // this part's slots
    Stage<8> st;
    if (LDSB) st.issue(actB, (uint32_t)nu * slot, NT3);
    Stage<1> st2;
    if (SHL) st2.issue(a.shB, (uint32_t)nQS * 256u * NC, NT3);
    SQ ring[2];
    auto ld = [&](int i, int k) AI {
        const int it = wave + NW * k;
        const bool on = k < cnt;
        const int u = on ? it / nSI : 0, S = on ? it % nSI : 0;
        int e = on ? a.route->uniq[u0 + u] : 0;
        if (a.slot) e = on ? a.slot[e] : 0;
        const rsrc_t r = make_rsrc(a.experts + (size_t)e * a.expert_bytes + a.down_off +
                                       (size_t)rt * tb, on ? tb : 0u);
        sq_load(ring[i], r, (uint32_t)S * SQ_BYTES, lane);
    };
    ring_prime<2>(ld);
    const int cs = strided_count(wave, NW, nQS);
    const rsrc_t rw = make_rsrc(a.sh_down + (size_t)rt * 16 * a.SI, (uint32_t)nQS * 4096u);
    const rsrc_t rb = make_rsrc(a.shB, (uint32_t)nQS * 256u * NC);
    const int n = lane & 15, kq = lane >> 4;
    const uint32_t boff = (uint32_t)((kq * NC + (n < NC ? n : 0)) * 16);
    QBB ring2[2];
    auto ld2 = [&](int i, int k) AI {
        const bool on = k < cs;
        const int q = wave + NW * k;
        qb_load(ring2[i].a, rw, on ? (uint32_t)q * 4096u : K3X_OOB, lane);
        if (!SHL) {
#pragma unroll
            for (int t = 0; t < 4; t++)
                ring2[i].b[t] = bload16(rb, on ? boff + (uint32_t)(q * 256 * NC + t * 64 * NC) : K3X_OOB);
        }
    };
    ring_prime<2>(ld2);
    if (LDSB) st.commit(NT3);
    if (SHL) st2.commit(NT3, a.lds_bytes);
    if (LDSB || SHL) __syncthreads();
    BFrag<LDSB> bf;
    bf.init(actB, (uint32_t)nu * slot, NC, lane);
    ring_loop<2>(cnt, ld, [&](int i, int k) AI {
        const int it = wave + NW * k;
        sq_mfma<EXACT, LDSB>(d, ring[i], bf, (uint32_t)(it / nSI) * slot, it % nSI);
    });
    BFrag<true> sbf;
    sbf.init(nullptr, 0u, NC, lane);
    ring_loop<2>(cs, ld2, [&](int i, int k) AI {
        if (SHL) {
            u32x4 b[4];
#pragma unroll
            for (int t = 0; t < 4; t++) b[t] = sbf.get(a.lds_bytes, wave + NW * k, t);
            qb_mfma(d, ring2[i].a, b);
        } else {
            qb_mfma(d, ring2[i].a, ring2[i].b);
        }
    });
}

template <bool EXACT>
__global__ void __launch_bounds__(NT3) k3_down(K3Args a)
{
    __shared__ float lds[(NT3 / WAVE - 1) * 4 * WAVE];
    WgTrace tr;
    tr.start(a.trace);
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int nall = a.route->nu;
    const int u0 = (int)blockIdx.y * a.upp;
    const int nu = nall - u0 < a.upp ? (nall > u0 ? nall - u0 : 0) : a.upp;
    const int nSI = ((a.I >> 7) + 3) >> 2;
    const uint32_t slot = (uint32_t)nSI * 1024u * 2 * a.T;
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    // both activation sets in LDS when they fit, else both read through L2
    if ((uint32_t)nu * slot <= a.lds_bytes && a.sh_lds)
        k3_body<EXACT, true, true>(a, d, wave, lane, u0, nu);
    else
        k3_body<EXACT, false, false>(a, d, wave, lane, u0, nu);
    float acc[4] = {d[0], d[1], d[2], d[3]};
    wave_sum_lds<4, NT3 / WAVE>(acc, lds, wave, lane);
    if (wave != 0) return;
    const int rt = blockIdx.x;
    float *out = a.out + blockIdx.y * a.pstride;
    per_token<4>(acc, 2 * a.T, lane, [&](int r0, int tok, const float (&v)[4]) AI {
        for (int i = 0; i < 4; i++) {
            const size_t o = (size_t)tok * a.H + rt * 16 + r0 + i;
            out[o] = a.resid ? a.resid[o] + v[i] : v[i];
        }
    });
    tr.end();
}

// Several tokens (K2 form): two 16-row tiles per workgroup, so that each B fragment read
// from memory (the activation sets no longer fit the LDS) serves both tiles' products.
#ifndef K3D2_R
#define K3D2_R 2
#endif
#ifndef K3D2_BPF
#define K3D2_BPF 1
#endif
template <bool EXACT>
__global__ void __launch_bounds__(NT3) k3_down2(K3Args a)
{
    __shared__ float lds[(NT3 / WAVE - 1) * 8 * WAVE];
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    constexpr int NW = NT3 / WAVE;
    const int NC = 2 * a.T;
    const int nall = a.route->nu;
    const int u0 = (int)blockIdx.y * a.upp;         // this part's unique experts
    const int nu = nall - u0 < a.upp ? (nall > u0 ? nall - u0 : 0) : a.upp;
    const int nSI = ((a.I >> 7) + 3) >> 2;
    const uint32_t slot = (uint32_t)nSI * 1024u * NC;
    const uint32_t tb = (uint32_t)fp4_tile_bytes(a.I);
    const int rt0 = 2 * blockIdx.x;
    const int cnt = strided_count(wave, NW, nu * nSI);
    const int nQS = (a.sh_down && blockIdx.y == 0) ? a.SI >> 7 : 0;
    const uint16_t *actB = a.actB + (size_t)u0 * (slot / 2);
    const int n = lane & 15, kq = lane >> 4;
    const uint32_t boff = (uint32_t)((kq * NC + (n < NC ? n : 0)) * 16);
    // an item's B fragments travel with its weights: a read of them at use would leave
    // its L2 latency in front of every item's products
    const rsrc_t ra = make_rsrc(actB, (uint32_t)nu * slot);
    SQ ring[K3D2_R][2];
    u32x4 bb[K3D2_BPF ? K3D2_R : 1][16];
    auto ld = [&](int i, int k) AI {
        const int it = wave + NW * k;
        const bool on = k < cnt;
        const int u = on ? it / nSI : 0, S = on ? it % nSI : 0;
        int e = on ? a.route->uniq[u0 + u] : 0;
        if (a.slot) e = on ? a.slot[e] : 0;
        const rsrc_t r = make_rsrc(a.experts + (size_t)e * a.expert_bytes + a.down_off +
                                       (size_t)rt0 * tb, on ? 2 * tb : 0u);
        sq_load(ring[i][0], r, (uint32_t)S * SQ_BYTES, lane);
        sq_load(ring[i][1], r, tb + (uint32_t)S * SQ_BYTES, lane);
#if K3D2_BPF
        const uint32_t bo = (uint32_t)u * slot + (uint32_t)(4 * S) * 256u * NC + boff;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int t = 0; t < 4; t++)
                bb[i][4 * j + t] = bload16(ra, on ? bo + (uint32_t)(j * 256 * NC + t * 64 * NC) : K3X_OOB);
#endif
    };
    ring_prime<K3D2_R>(ld);
    f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
    ring_loop<K3D2_R>(cnt, ld, [&](int i, int k) AI {
#if !K3D2_BPF
        const int it = wave + NW * k;
        const uint32_t bo = (uint32_t)(it / nSI) * slot + (uint32_t)(4 * (it % nSI)) * 256u * NC + boff;
#endif
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
#if K3D2_BPF
                const bf16x8 bv = as_bf16x8(bb[i][4 * j + t]);
#else
                const bf16x8 bv = as_bf16x8(bload16(ra, bo + (uint32_t)(j * 256 * NC + t * 64 * NC)));
#endif
                d0 = mfma(sq_a<EXACT>(ring[i][0], j, t), bv, d0);
                d1 = mfma(sq_a<EXACT>(ring[i][1], j, t), bv, d1);
            }
    });
    // then the shared expert's quads (two per wave at SI = 2048), their ring primed once
    // the routed one has drained, so that the two never hold registers together
    const int cs = strided_count(wave, NW, nQS);
    const uint32_t sbytes = (uint32_t)nQS * 4096u;
    const rsrc_t rw = make_rsrc(a.sh_down + (size_t)rt0 * 16 * a.SI, 2 * sbytes);
    const rsrc_t rb = make_rsrc(a.shB, (uint32_t)nQS * 256u * NC);
    QB w2[2][2];
    u32x4 b2[2][4];
    auto ld2 = [&](int i, int k) AI {
        const bool on = k < cs;
        const int q = wave + NW * k;
        qb_load(w2[i][0], rw, on ? (uint32_t)q * 4096u : K3X_OOB, lane);
        qb_load(w2[i][1], rw, on ? sbytes + (uint32_t)q * 4096u : K3X_OOB, lane);
#pragma unroll
        for (int t = 0; t < 4; t++)
            b2[i][t] = bload16(rb, on ? boff + (uint32_t)(q * 256 * NC + t * 64 * NC) : K3X_OOB);
    };
    ring_prime<2>(ld2);
    ring_loop<2>(cs, ld2, [&](int i, int k) AI {
        qb_mfma(d0, w2[i][0], b2[i]);
        qb_mfma(d1, w2[i][1], b2[i]);
    });
    float acc[8] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3]};
    wave_sum_lds<8, NW>(acc, lds, wave, lane);
    if (wave != 0) return;
    float *out = a.out + blockIdx.y * a.pstride;
    per_token<8>(acc, NC, lane, [&](int r0, int tok, const float (&v)[8]) AI {
        for (int tt = 0; tt < 2; tt++)
            for (int i = 0; i < 4; i++) {
                const size_t o = (size_t)tok * a.H + (rt0 + tt) * 16 + r0 + i;
                out[o] = a.resid ? a.resid[o] + v[4 * tt + i] : v[4 * tt + i];
            }
    });
}

// Several tokens, K2 form, H a multiple of 256: the down products of 256 output rows a
// workgroup (wave w: row tiles 2w, 2w + 1 of the group).  Workgroups blockIdx.y < pr
// each take one part of the (unique expert, super-quad) items, dealt in runs of equal
// length; the other rows take the shared expert's bf16 quads, quad q to the row q mod
// (gridDim.y - pr).
// All eight waves take the same item at once, so that its B fragments (16 KB at eight
// tokens) come straight into an LDS stage once for the workgroup, beside the waves'
// weights, through a ring of K3W_R stages: a wave has K3W_R - 1 items of weights in
// flight while it multiplies one.  Every workgroup writes its part sums, which k3_reduce
// adds up in part order (the shared expert's parts last).
#define K3W_R 4
#ifndef K3W_ON
#define K3W_ON 1
#endif
#ifndef K3W_TMIN
#define K3W_TMIN 2                                 // fewest tokens taking k3_down_wide
#endif
#define K3W_STAGE (1024u * 2 * K3X_DECODE_MAX_T)   // LDS bytes of a stage's B
#define K3W_LPI 12                                 // vector loads per item and wave

// The ring over n items: ld(i, k) issues item k's loads into stage i (K3W_LPI of them,
// any k; k >= n loads nothing), use(i) multiplies stage i.
template <class LD, class USE>
__device__ __forceinline__ void k3w_ring(int n, LD ld, USE use)
{
#pragma unroll
    for (int i = 0; i < K3W_R - 1; i++) {
        SCHED_FENCE();
        ld(i, i);
    }
    SCHED_FENCE();
    // item k + i: wait for its loads (those of the K3W_R - 2 items after it remain), meet
    // the other waves (stage i - 1 is then no longer read), refill that stage with item
    // k + i + K3W_R - 1, multiply
    int k = 0;
    for (; k + K3W_R <= n; k += K3W_R) {
#pragma unroll
        for (int i = 0; i < K3W_R; i++) {
            meet<(K3W_R - 2) * K3W_LPI>();
            SCHED_FENCE();
            ld((i + K3W_R - 1) % K3W_R, k + i + K3W_R - 1);
            SCHED_FENCE();
            use(i);
        }
    }
    // the last n - k items (fewer than K3W_R), without refills
#pragma unroll
    for (int i = 0; i < K3W_R - 1; i++) {
        if (k + i < n) {
            WAIT_VMCNT_LGKM0(0);
            __builtin_amdgcn_s_barrier();
            use(i);
        }
    }
    WAIT_VMCNT_LGKM0(0);
}

template <bool EXACT>
__global__ void __launch_bounds__(NT3) k3_down_wide(K3Args a)
{
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int NC = 2 * a.T;
    const int rg = blockIdx.x, p = blockIdx.y, P = a.pr;
    const int rt0 = rg * 16 + 2 * wave;
    const uint32_t stB = (uint32_t)wave * WAVE * 16u;
    BFrag<true> bl;
    bl.init(nullptr, 0u, NC, lane);
    f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
    SQ w[K3W_R][2];
    if (p < P) {
        const int nu = __builtin_amdgcn_readfirstlane(a.route->nu);
        const int nSI = ((a.I >> 7) + 3) >> 2;
        const uint32_t sqb = 1024u * (uint32_t)NC;      // B bytes of a super-quad
        const uint32_t slot = (uint32_t)nSI * sqb;      // B bytes of an expert
        const int nit = nu * nSI;
        const int ipp = (nit + P - 1) / P;
        const int i0 = p * ipp < nit ? p * ipp : nit;
        const int cnt = (i0 + ipp < nit ? i0 + ipp : nit) - i0;
        const uint32_t tb = (uint32_t)fp4_tile_bytes(a.I);
        const rsrc_t ra = make_rsrc(a.actB, (uint32_t)nu * slot);
        // the unique experts' arena slots in LDS, so that the loads of an item need no
        // load of their own (a global one would be waited for in front of every item's)
        __shared__ int s_ue[K3X_DECODE_MAX_T * K3X_MAX_TOPK];
        for (int u = threadIdx.x; u < nu; u += NT3) {
            const int e = a.route->uniq[u];
            s_ue[u] = a.slot ? a.slot[e] : e;
        }
        __syncthreads();
        // (expert, super-quad) of the next item: ld is called for k = 0, 1, 2, ...
        int cu = i0 / nSI, cS = i0 % nSI;
        k3w_ring(cnt, [&](int i, int k) AI {
            const bool on = k < cnt;
            const int e = __builtin_amdgcn_readfirstlane(s_ue[on ? cu : 0]);
            const rsrc_t r = make_rsrc(a.experts + (size_t)e * a.expert_bytes + a.down_off +
                                           (size_t)rt0 * tb, on ? 2 * tb : 0u);
            sq_load(w[i][0], r, (uint32_t)cS * SQ_BYTES, lane);
            sq_load(w[i][1], r, tb + (uint32_t)cS * SQ_BYTES, lane);
            const uint32_t gb = (uint32_t)cu * slot + (uint32_t)cS * sqb;
            const int wrap = cS + 1 == nSI;
            cu += wrap;
            cS = wrap ? 0 : cS + 1;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t o = threadIdx.x * 16u + (uint32_t)c * NT3 * 16u;
                const uint32_t go = (on & (o < sqb)) ? gb + o : K3X_OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra, (lds_void *)(dyn_lds + (uint32_t)i * K3W_STAGE + (uint32_t)c * NT3 * 16u + stB),
                    16, go, 0, 0, 0);
            }
        }, [&](int i) AI {
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const bf16x8 bv = as_bf16x8(bl.get((uint32_t)i * K3W_STAGE, j, t));
                    d0 = mfma(sq_a<EXACT>(w[i][0], j, t), bv, d0);
                    d1 = mfma(sq_a<EXACT>(w[i][1], j, t), bv, d1);
                }
        });
    } else {
        // the shared expert: quad q's two 16-row runs a wave (four 16-byte loads each, as
        // an fp4 super-quad's codes, plus two scale-slot loads that read nothing)
        const int nQS = a.sh_down ? a.SI >> 7 : 0;
        const int ps = p - P, PS = gridDim.y - P;
        const int cs = ps < nQS ? (nQS - 1 - ps) / PS + 1 : 0;
        const uint32_t sbytes = (uint32_t)nQS * 4096u;  // a tile's bytes
        const uint32_t qbB = 256u * (uint32_t)NC;       // B bytes of a quad
        const rsrc_t r = make_rsrc(a.sh_down + (size_t)rt0 * 16 * a.SI, 2 * sbytes);
        const rsrc_t rsb = make_rsrc(a.shB, (uint32_t)nQS * qbB);
        k3w_ring(cs, [&](int i, int k) AI {
            const bool on = k < cs;
            const int q = ps + PS * k;
            const uint32_t b0 = on ? (uint32_t)q * 4096u : K3X_OOB;
            sq_load(w[i][0], r, b0, lane);
            sq_load(w[i][1], r, on ? sbytes + b0 : K3X_OOB, lane);
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t o = threadIdx.x * 16u + (uint32_t)c * NT3 * 16u;
                const uint32_t go = (on & (o < qbB)) ? (uint32_t)q * qbB + o : K3X_OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rsb, (lds_void *)(dyn_lds + (uint32_t)i * K3W_STAGE + (uint32_t)c * NT3 * 16u + stB),
                    16, go, 0, 0, 0);
            }
        }, [&](int i) AI {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const bf16x8 bv = as_bf16x8(bl.get((uint32_t)i * K3W_STAGE, 0, t));
                d0 = mfma(as_bf16x8(w[i][0].c[t]), bv, d0);
                d1 = mfma(as_bf16x8(w[i][1].c[t]), bv, d1);
            }
        });
    }
    const float acc[8] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3]};
    float *dst = a.pacc + (size_t)p * K3X_DECODE_MAX_T * a.H;
    per_token<8>(acc, NC, lane, [&](int r0, int tok, const float (&v)[8]) AI {
        for (int tt = 0; tt < 2; tt++)
            for (int i = 0; i < 4; i++)
                dst[(size_t)tok * a.H + (rt0 + tt) * 16 + r0 + i] = v[4 * tt + i];
    });
}

// The same, four outputs a thread (16-byte aligned out, resid and parts, H % 4 == 0).
__global__ void __launch_bounds__(256) k3_reduce4(const float *pacc, int P, const float *resid,
                                                   float *out, int n4, int H)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const size_t o = (size_t)i * 4, ps = (size_t)K3X_DECODE_MAX_T * H;
    f32x4 v[K3X_WIDE_PMAX];
#pragma unroll
    for (int q = 0; q < K3X_WIDE_PMAX; q++)
        if (q < P) v[q] = *(const f32x4 *)(pacc + q * ps + o);
    f32x4 s = v[0];
#pragma unroll
    for (int q = 1; q < K3X_WIDE_PMAX; q++)
        if (q < P) { s[0] += v[q][0]; s[1] += v[q][1]; s[2] += v[q][2]; s[3] += v[q][3]; }
    if (resid) {
        const f32x4 r = *(const f32x4 *)(resid + o);
        s[0] = r[0] + s[0]; s[1] = r[1] + s[1]; s[2] = r[2] + s[2]; s[3] = r[3] + s[3];
    }
    *(f32x4 *)(out + o) = s;
}

// out = resid + the parts' sums of k3_down_wide, added in part order, over [T][H].
__global__ void __launch_bounds__(256) k3_reduce(const float *pacc, int P, const float *resid,
                                                  float *out, int n, int H)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const size_t ps = (size_t)K3X_DECODE_MAX_T * H;
    float v[K3X_WIDE_PMAX];
#pragma unroll
    for (int q = 0; q < K3X_WIDE_PMAX; q++)
        if (q < P) v[q] = pacc[q * ps + i];
    float s = v[0];
#pragma unroll
    for (int q = 1; q < K3X_WIDE_PMAX; q++)
        if (q < P) s += v[q];
    out[i] = resid ? resid[i] + s : s;
}

// ------------------------------------------------------------------ K4 (latent form)
// The routed aggregates (the sum of k3's parts, in part order), their RMSNorm (k3_rmsnorm
// on the aggregate, k3_ops.c:1946) and their B set for the up projection.  Every
// workgroup works out 1/rms of every token (a double sum of squares, as the reference),
// then writes its share of the set.
struct KNArgs {
    const float *acc;              // [P][T][XL] partial aggregates, pstride floats apart
    int          P;
    size_t       pstride;
    const float *nw;               // [XL], or NULL: no norm
    float        eps;
    int          T, XL;
    uint16_t    *latB;
};

#define NT4 1024                  // k4_latent_norm: 16 waves, 1024 set entries a workgroup

__device__ __forceinline__ float agg_at(const KNArgs &a, size_t i)
{
    float v = a.acc[i];
    for (int p = 1; p < a.P; p++) v += a.acc[p * a.pstride + i];
    return v;
}

// Four consecutive floats at o of each of P parts (pstride floats apart), added in part
// order.  The loads go out eight parts at a time (a part past P loads the last part again
// and is not added), not one part's load and add after another's.
__device__ __forceinline__ f32x4 parts_sum4(const float *acc, int P, size_t pstride, size_t o)
{
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < P; p0 += 8) {
        f32x4 w[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int p = p0 + j < P ? p0 + j : P - 1;
            w[j] = *(const f32x4 *)(acc + p * pstride + o);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (p0 + j >= P) break;
            if (p0 + j == 0) v = w[j];
            else { v[0] += w[j][0]; v[1] += w[j][1]; v[2] += w[j][2]; v[3] += w[j][3]; }
        }
    }
    return v;
}

// four consecutive aggregates (i a multiple of 4), each added over the parts in order
__device__ __forceinline__ f32x4 agg4(const KNArgs &a, size_t i)
{
    return parts_sum4(a.acc, a.P, a.pstride, i);
}

__global__ void __launch_bounds__(NT4) k4_latent_norm(KNArgs a)
{
    __shared__ double dl[NT4 / WAVE][K3X_DECODE_MAX_T];
    __shared__ float s_inv[K3X_DECODE_MAX_T];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (a.nw) {
        // every token's loads of a step in flight together
        double ss[K3X_DECODE_MAX_T];
#pragma unroll
        for (int t = 0; t < K3X_DECODE_MAX_T; t++) ss[t] = 0.0;
        for (int i = threadIdx.x * 4; i < a.XL; i += NT4 * 4) {
#pragma unroll
            for (int t = 0; t < K3X_DECODE_MAX_T; t++) {
                if (t >= a.T) break;
                const f32x4 v = agg4(a, (size_t)t * a.XL + i);
                ss[t] += (double)v[0] * (double)v[0] + (double)v[1] * (double)v[1] +
                         (double)v[2] * (double)v[2] + (double)v[3] * (double)v[3];
            }
        }
#pragma unroll
        for (int t = 0; t < K3X_DECODE_MAX_T; t++) {
            if (t >= a.T) break;
            double v = ss[t];
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) dl[wave][t] = v;
        }
        __syncthreads();
        if (threadIdx.x < a.T) {
            double tot = 0.0;
            for (int w = 0; w < NT4 / WAVE; w++) tot += dl[w][threadIdx.x];
            s_inv[threadIdx.x] = (float)(1.0 / sqrt(tot / (double)a.XL + (double)a.eps));
        }
        __syncthreads();
    }
    // entries of the compact set (whole super-quads; quads past XL/128 are zeros), as
    // x_to_bset lays them out
    const int NC = 2 * a.T, nQ = a.XL >> 7, nq = 4 * (((a.XL >> 7) + 3) >> 2);
    const int ne = nq * 16 * NC;
    for (int f = blockIdx.x * NT4 + threadIdx.x; f < ne; f += gridDim.x * NT4) {
        const int n = f % NC, kq = (f / NC) & 3, t = (f / (NC * 4)) & 3, q = f / (NC * 16);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (q < nQ) {
            const int c0 = q * 128 + kq * 32 + t * 8;
            const size_t base = (size_t)(n >> 1) * a.XL + c0;
            float xv[8];
            const f32x4 v0 = agg4(a, base), v1 = agg4(a, base + 4);
#pragma unroll
            for (int j = 0; j < 4; j++) { xv[j] = v0[j]; xv[4 + j] = v1[j]; }
            if (a.nw) {
                const float inv = s_inv[n >> 1];
#pragma unroll
                for (int j = 0; j < 8; j++) xv[j] = a.nw[c0 + j] * xv[j] * inv;
            }
            v = bfrag_of(xv, n & 1);
        }
        *(u32x4 *)((uint8_t *)a.latB + (size_t)f * 16) = v;
    }
}

// The up projection (k3_ops.c:1950) of the normalised aggregates and the shared expert's
// down product (moe_shared, :1858) for 16 output rows: eight waves on interleaved bf16
// quads of `up` and then of the shared down matrix, into two accumulator sets; out =
// up + shared (:1859), plus the residual.
//   FUSE: the workgroup works out the aggregates itself, while its first weights are in
//         flight: the parts of k3 added in order into LDS (fp32), each token's 1/rms, and
//         the normalised set's B fragments into LDS at 0 (else they come from
//         k4_latent_norm's set in global memory, read with each quad's weights).
//   SHL:  the shared activation's set staged in LDS after the aggregates' set (else read
//         from global memory with each quad's weights).
struct K4Args {
    const uint16_t *up;            // tiled bf16 [H][XL]
    const uint16_t *latB;          // B set of the normalised aggregates (not FUSE)
    KNArgs          kn;            // the parts and the norm (FUSE)
    const uint16_t *sh_down;       // tiled bf16 [H][SI], or NULL
    const uint16_t *shB;           // B set of the shared activation
    float          *out;
    const float    *resid;
    int             T, H, XL, SI;
};

#define K4_LDS_MAX 65536u          // with the static reduction area, two workgroups per CU

__host__ __device__ inline uint32_t k4_lds_bytes(bool fuse, bool shl, int T, int XL, int SI)
{
    const uint32_t NC = 2u * (uint32_t)T;
    return (fuse ? (uint32_t)(XL >> 7) * 256u * NC + (uint32_t)(T * XL) * 4u : 0u) +
           (shl ? (uint32_t)(SI >> 7) * 256u * NC : 0u);
}

// FUSE's preamble: aggregates into LDS (agg), 1/rms per token, the normalised B set into
// LDS at 0.  All NT3 threads; ends with a barrier.
__device__ __forceinline__ void k4_fuse_norm(const KNArgs &a, float *agg, double (*dl)[K3X_DECODE_MAX_T],
                                             float *s_inv)
{
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int n4 = a.XL >> 2;
    for (int t = 0; t < a.T; t++) {
        double ss = 0.0;
        for (int c = threadIdx.x; c < n4; c += NT3) {
            const size_t o = (size_t)t * a.XL + 4 * c;
            const f32x4 v = parts_sum4(a.acc, a.P, a.pstride, o);
            *(f32x4 *)(agg + o) = v;
#pragma unroll
            for (int k = 0; k < 4; k++) ss += (double)v[k] * (double)v[k];
        }
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        if (lane == 0) dl[wave][t] = ss;
    }
    __syncthreads();
    if (threadIdx.x < a.T) {
        double tot = 0.0;
        for (int w = 0; w < NT3 / WAVE; w++) tot += dl[w][threadIdx.x];
        s_inv[threadIdx.x] = a.nw ? (float)(1.0 / sqrt(tot / (double)a.XL + (double)a.eps)) : 1.0f;
    }
    __syncthreads();
    const int NC = 2 * a.T, ne = (a.XL >> 7) * 16 * NC;
    for (int f = threadIdx.x; f < ne; f += NT3) {
        const int n = f % NC, kq = (f / NC) & 3, t = (f / (NC * 4)) & 3, q = f / (NC * 16);
        const int c0 = q * 128 + kq * 32 + t * 8;
        const float *src = agg + (size_t)(n >> 1) * a.XL + c0;
        float xv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) xv[j] = src[j];
        if (a.nw) {
            const float inv = s_inv[n >> 1];
            float wv[8];
            load_x8(a.nw, 0, (size_t)c0, wv);
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = wv[j] * xv[j] * inv;
        }
        *(u32x4 *)(dyn_lds + (size_t)f * 16) = bfrag_of(xv, n & 1);
    }
}

template <bool FUSE, bool SHL>
__global__ void __launch_bounds__(NT3) k4_up(K4Args a)
{
    __shared__ float lds[(NT3 / WAVE - 1) * 8 * WAVE];
    __shared__ double dl[NT3 / WAVE][K3X_DECODE_MAX_T];
    __shared__ float s_inv[K3X_DECODE_MAX_T];
    constexpr int NW = NT3 / WAVE;
    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int NC = 2 * a.T, rt = blockIdx.x;
    const int nQL = a.XL >> 7, nQS = a.sh_down ? a.SI >> 7 : 0;
    const uint32_t lbytes = (uint32_t)nQL * 256u * NC, sbytes = (uint32_t)nQS * 256u * NC;
    const uint32_t sh_off = FUSE ? lbytes : 0u;            // the shared set's LDS offset
    Stage<4> st2;
    if (SHL) st2.issue(a.shB, sbytes, NT3);
    const int c1 = strided_count(wave, NW, nQL), c2 = strided_count(wave, NW, nQS);
    const rsrc_t rw1 = make_rsrc(a.up + (size_t)rt * 16 * a.XL, (uint32_t)nQL * 4096u);
    const rsrc_t rw2 = make_rsrc(nQS ? a.sh_down + (size_t)rt * 16 * a.SI : a.up,
                                 (uint32_t)nQS * 4096u);
    const rsrc_t rb1 = make_rsrc(a.latB, lbytes), rb2 = make_rsrc(a.shB, sbytes);
    const int n = lane & 15, kq = lane >> 4;
    const uint32_t boff = (uint32_t)((kq * NC + (n < NC ? n : 0)) * 16);
    QBB r1[2], r2[2];
    auto ldq = [&](QBB &it, rsrc_t rw, rsrc_t rb, int k, int cnt, bool gb) AI {
        const bool on = k < cnt;
        const int q = wave + NW * k;
        qb_load(it.a, rw, on ? (uint32_t)q * 4096u : K3X_OOB, lane);
        if (gb) {
#pragma unroll
            for (int t = 0; t < 4; t++)
                it.b[t] = bload16(rb, on ? boff + (uint32_t)(q * 256 * NC + t * 64 * NC) : K3X_OOB);
        }
    };
    auto ld1 = [&](int i, int k) AI { ldq(r1[i], rw1, rb1, k, c1, !FUSE); };
    auto ld2 = [&](int i, int k) AI { ldq(r2[i], rw2, rb2, k, c2, !SHL); };
    ring_prime<2>(ld1);
    ring_prime<2>(ld2);
    if (SHL) st2.commit(NT3, sh_off);
    if (FUSE)
        k4_fuse_norm(a.kn, (float *)(dyn_lds + sh_off + (SHL ? sbytes : 0u)), dl, s_inv);
    if (FUSE || SHL) __syncthreads();
    BFrag<true> bf;
    bf.init(nullptr, 0u, NC, lane);
    f32x4 d1 = {0.f, 0.f, 0.f, 0.f}, d2 = {0.f, 0.f, 0.f, 0.f};
    auto use = [&](f32x4 &d, const QBB &it, bool inlds, uint32_t sbase, int q) AI {
        if (inlds) {
            u32x4 b[4];
#pragma unroll
            for (int t = 0; t < 4; t++) b[t] = bf.get(sbase, q, t);
            qb_mfma(d, it.a, b);
        } else {
            qb_mfma(d, it.a, it.b);
        }
    };
    ring_loop<2>(c1, ld1, [&](int i, int k) AI { use(d1, r1[i], FUSE, 0u, wave + NW * k); });
    ring_loop<2>(c2, ld2, [&](int i, int k) AI { use(d2, r2[i], SHL, sh_off, wave + NW * k); });
    float acc[8] = {d1[0], d1[1], d1[2], d1[3], d2[0], d2[1], d2[2], d2[3]};
    wave_sum_lds<8, NW>(acc, lds, wave, lane);
    if (wave != 0) return;
    per_token<8>(acc, NC, lane, [&](int r0, int tok, const float (&v)[8]) AI {
        for (int i = 0; i < 4; i++) {
            const size_t o = (size_t)tok * a.H + rt * 16 + r0 + i;
            const float y = v[i] + v[4 + i];
            a.out[o] = a.resid ? a.resid[o] + y : y;
        }
    });
}

// ------------------------------------------------------------------ launcher
static inline int launch_ok(void) { return hipGetLastError() == hipSuccess ? 0 : K3X_E_HIP; }

static int record(k3x_moe_layer *L, int i, hipStream_t s)
{
    if (!L->timing || i >= 8) return 0;
    if (i + 1 > L->n_ev_used) L->n_ev_used = i + 1;
    return hipEventRecord((hipEvent_t)L->ev[i], s) == hipSuccess ? 0 : K3X_E_HIP;
}

template <int NE>
static void launch_k2(const K2Args &a, bool ex, bool st, dim3 grid, size_t lds, hipStream_t s)
{
    if (ex && st)  hipLaunchKernelGGL((k2_gateup<true, true, NE>), grid, dim3(NT), lds, s, a);
    else if (ex)   hipLaunchKernelGGL((k2_gateup<true, false, NE>), grid, dim3(NT), lds, s, a);
    else if (st)   hipLaunchKernelGGL((k2_gateup<false, true, NE>), grid, dim3(NT), lds, s, a);
    else           hipLaunchKernelGGL((k2_gateup<false, false, NE>), grid, dim3(NT), lds, s, a);
}

extern "C" int k3x_dev_decode(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                              int T, const float *resid, int *idx, float *wt,
                              const float *norm_w, float eps, void *stream)
{
    const k3x_cfg *c = &L->cfg;
    hipStream_t s = (hipStream_t)stream;
    const int H = c->hidden, I = c->moe_inter, NC = 2 * T, X = L->XL;
    const int nQ = H / 128, nS = (nQ + 3) / 4, nSI = (I / 128 + 3) / 4, nSX = (X / 128 + 3) / 4;
    int rc;
    if (L->nslot || L->cache_only) {
        // such a call reads the selection back to the host and synchronises, which a
        // stream under capture cannot do: refused before anything is enqueued
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) != hipSuccess) return K3X_E_HIP;
        if (cs != hipStreamCaptureStatusNone) return K3X_E_ARG;
    }

    K1Args a1;
    a1.router = L->router; a1.bias = L->bias; a1.x = x; a1.x_bf16 = (x_dtype == K3X_BF16);
    a1.T = T; a1.H = H; a1.E = c->n_experts;
    a1.score = L->score; a1.choice = L->choice; a1.xB = L->xB;
    a1.slack = L->slack; a1.ninv = L->ninv; a1.hkey = L->route->hkey;
    a1.n_rwg = (c->n_experts + NT1 / WAVE / RWAVES - 1) / (NT1 / WAVE / RWAVES);
    a1.seq = &L->route->seq;
    a1.norm_w = norm_w; a1.eps = eps;
    a1.ldown = L->lat ? L->ldown : NULL; a1.XL = X; a1.zB = L->zB;
    if (norm_w && (L->lat || x_dtype == K3X_BF16 || H > RCH * NT1 * 4 || ((uintptr_t)x & 15) ||
                   ((uintptr_t)norm_w & 15)))
        return K3X_E_ARG;
    unsigned long long *trb = L->tr;
    a1.trace = (trb && a1.n_rwg <= L->tr_cap) ? trb : NULL;
    if ((rc = record(L, 0, s))) return rc;
    const unsigned g1 = launch_k1(a1, s);
    if (trb) L->tr_n[0] = a1.trace ? (int)g1 : 0;
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, 1, s))) return rc;
    int ev = 2;                        // the next timing event
    KSArgs ks;
    ks.score = L->score; ks.choice = L->choice; ks.E = c->n_experts; ks.K = c->topk;
    ks.renorm = c->moe_renorm; ks.routed_scale = c->routed_scale; ks.route = L->route;
    ks.idx = L->idx; ks.wt = L->wt; ks.uidx = idx; ks.uwt = wt; ks.T = T;
    ks.slack = L->slack; ks.hkey = L->route->hkey; ks.router = L->router; ks.bias = L->bias; ks.x = x;
    ks.x_bf16 = a1.x_bf16; ks.H = H; ks.norm_w = norm_w; ks.ninv = L->ninv;
    if (L->lat) {
        a1.ks = ks;
        const dim3 gz(1 + X / 16);
        // x's B set staged in LDS where it fits beside two workgroups a CU
        const size_t xbb = (size_t)nS * 1024u * 2 * T;
        const bool zl = xbb <= 64 * 1024;
        const size_t lz = std::max(sizeof(KSLds), zl ? xbb : (size_t)0);
#define K1Z(NE_) \
        if (zl) hipLaunchKernelGGL((k1_zdown<NE_, true>), gz, dim3(NT1), lz, s, a1); \
        else    hipLaunchKernelGGL((k1_zdown<NE_, false>), gz, dim3(NT1), lz, s, a1);
        if (c->n_experts <= 128)      { K1Z(2) }
        else if (c->n_experts <= 256) { K1Z(4) }
        else if (c->n_experts <= 384) { K1Z(6) }
        else if (c->n_experts <= 512) { K1Z(8) }
        else                          { K1Z(16) }
#undef K1Z
        if ((rc = launch_ok())) return rc;
        if ((rc = record(L, ev++, s))) return rc;
    }

    K2Args a2;
    a2.trace = NULL;
    a2.ks = ks;
    a2.sel_done = L->lat;
    a2.route = L->route; a2.seq = &L->route->seq; a2.err = &L->route->err;
    a2.wait_ticks = L->wait_ticks; a2.publish = !L->no_publish;
    a2.experts = L->experts; a2.expert_bytes = L->expert_bytes;
    a2.gate_off = L->gate_off; a2.up_off = L->up_off;
    a2.xB = L->xB; a2.actB = L->actB; a2.T = T; a2.H = H; a2.I = I;
    a2.n_sh = L->SI > 0 ? L->SI / 16 : 0;
    a2.sh_gate = L->sh_gate; a2.sh_up = L->sh_up; a2.SI = L->SI; a2.shB = L->shB;
    a2.rB = L->lat ? L->zB : L->xB; a2.XL = X; a2.b1 = L->b1; a2.b2 = L->b2;
    // row tiles per routed workgroup: each wave streams at least a few super-quads, and
    // the grid stays near one workgroup per slot (two tiles a workgroup measured 1.3 us
    // faster than one at the hidden width of 7168, b = 1, and 15 us faster at T = 8)
    a2.rtw = nSX >= 6 ? 2 : 4;
    const int n_routed = T * c->topk * (I / 16) / a2.rtw;
    // the routed input's set and x's (the shared experts'): staged when both fit
    const uint32_t xset = (uint32_t)nS * 1024u * NC, rset = (uint32_t)nSX * 1024u * NC;
    const uint32_t bset = xset > rset ? xset : rset;
    const bool st2 = bset <= STAGE_MAX;
    size_t l2 = st2 ? bset : 0;
    if (l2 < sizeof(KSLds)) l2 = sizeof(KSLds);
    a2.sb = (!st2 && a2.rtw == 2) ? 1 : 0;
    if (a2.sb && l2 < (size_t)K2SB_R * K2SB_STAGE) l2 = (size_t)K2SB_R * K2SB_STAGE;
    auto k2_launch = [&](bool ex, dim3 g) {
        if (a2.sel_done)              launch_k2<0>(a2, ex, st2, g, l2, s);
        else if (c->n_experts <= 128) launch_k2<2>(a2, ex, st2, g, l2, s);
        else if (c->n_experts <= 256) launch_k2<4>(a2, ex, st2, g, l2, s);
        else if (c->n_experts <= 384) launch_k2<6>(a2, ex, st2, g, l2, s);
        else if (c->n_experts <= 512) launch_k2<8>(a2, ex, st2, g, l2, s);
        else                          launch_k2<16>(a2, ex, st2, g, l2, s);
    };
    a2.slot = L->nslot ? L->slot_dev : NULL;
    if (L->nslot || L->cache_only) {
        // expert cache or cache-only routing: the selection alone first (workgroup 0 of
        // k2 on a grid of one, or k1_zdown's in the latent form), then the host's part:
        // the draft filter, and the experts it names made resident (refused under
        // capture, before the first launch)
        if (!L->lat) {
            k2_launch(false, dim3(1));
            if ((rc = launch_ok())) return rc;
        }
        if ((rc = k3x_route_host(L, s, T, idx, wt))) return rc;
        a2.sel_done = 1;
    }
    const bool ex2 = (L->special & 3) != 0;
    const int g2 = 1 + a2.n_sh + n_routed;
    a2.trace = (trb && g2 <= L->tr_cap) ? trb + (size_t)L->tr_cap * 3 : NULL;
    if (trb) L->tr_n[1] = a2.trace ? g2 : 0;
    k2_launch(ex2, dim3(g2));
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, ev++, s))) return rc;

    // k3: the routed down products, plus the shared expert's into the same rows (K2 form),
    // or into the latent aggregates alone (latent form; the shared expert goes to k4)
    K3Args a3;
    a3.experts = L->experts; a3.expert_bytes = L->expert_bytes; a3.down_off = L->down_off;
    a3.slot = L->nslot ? L->slot_dev : NULL;
    a3.route = L->route; a3.actB = L->actB;
    a3.sh_down = (L->SI > 0 && !L->lat) ? L->sh_down : NULL; a3.shB = L->shB; a3.SI = L->SI;
    a3.out = L->lat ? L->accL : out; a3.resid = L->lat ? NULL : resid;
    a3.T = T; a3.H = X; a3.I = I; a3.K = c->topk;
    a3.trace = NULL;
    const uint32_t slot = (uint32_t)nSI * 1024u * NC;
    const size_t all = (size_t)T * c->topk * slot;
    a3.lds_bytes = slot <= STAGE_MAX ? (uint32_t)(all < STAGE_MAX ? all : (STAGE_MAX / slot) * slot) : 0u;
    // the shared activation set beside them when two workgroups still fit a CU (without
    // a shared expert here, an empty set)
    const uint32_t shb = a3.sh_down ? (uint32_t)(L->SI / 128) * 256u * NC : 0u;
    a3.sh_lds = (a3.lds_bytes && a3.lds_bytes + shb <= K3_LDS_MAX) ? (shb ? shb : 16u) : 0u;
    // the latent form splits the unique experts into parts whose activation sets fit the
    // LDS (at most K3X_DECODE_PARTS; k4_latent_norm adds the parts up); the K2 form writes
    // its rows in one part
    int parts = 1;
    a3.upp = T * c->topk;
    // latent form with the activation sets past the LDS: two row tiles a workgroup
    // (k3_down2, each B fragment read once for both) and parts for parallelism
    const bool lat2 = L->lat && !a3.lds_bytes && T >= 2 && X % 32 == 0;
    if (L->lat && a3.lds_bytes) {
        parts = (T * c->topk + (int)(a3.lds_bytes / slot) - 1) / (int)(a3.lds_bytes / slot);
        if (parts > K3X_DECODE_PARTS) parts = K3X_DECODE_PARTS;
        a3.upp = (T * c->topk + parts - 1) / parts;     // balanced parts
    } else if (lat2) {
        parts = T * c->topk < K3X_DECODE_PARTS ? T * c->topk : K3X_DECODE_PARTS;
        a3.upp = (T * c->topk + parts - 1) / parts;
    }
    a3.pstride = parts > 1 ? (size_t)K3X_DECODE_MAX_T * X : 0;
    const size_t l3 = (size_t)a3.lds_bytes + a3.sh_lds;
    const bool use2 = (!L->lat && T >= 2 && X % 32 == 0) || lat2;
    if (trb) {
        // k3_down's workgroups when they are one part (k3_down2 is not traced)
        const bool on = parts == 1 && !use2 && X / 16 <= L->tr_cap;
        a3.trace = on ? trb + (size_t)L->tr_cap * 6 : NULL;
        L->tr_n[2] = on ? X / 16 : 0;
    }
    // several tokens, X a multiple of 256: 256 rows a workgroup over parts of the items,
    // about one workgroup per CU; the parts' sums go to the K2 form's part buffer (added up
    // by k3_reduce) or to the latent form's partial aggregates (added up by k4_latent_norm)
    a3.pacc = L->lat ? L->accL : L->pacc;
    const bool wide = T >= K3W_TMIN && X % 256 == 0 && a3.pacc && K3W_ON;
    if (wide) {
        // about one workgroup per CU, the parts shared between the routed items (by the
        // unique experts a call can have) and the shared expert's quads in proportion
        int pw = 256 / (X / 256);
        if (pw < 2) pw = 2;
        if (pw > K3X_WIDE_PMAX) pw = K3X_WIDE_PMAX;
        const int nQS = a3.sh_down ? L->SI / 128 : 0;
        const int ue = T * c->topk < c->n_experts ? T * c->topk : c->n_experts;
        const int nit = ue * nSI;
        int pr = (int)(((long)pw * nit * 2 + (nit + nQS)) / (2L * (nit + nQS)));
        if (pr > pw - (nQS > 0)) pr = pw - (nQS > 0);
        if (pr < 1) pr = 1;
        a3.pr = pr;
        if (L->lat) {
            parts = pw;
            a3.pstride = (size_t)K3X_DECODE_MAX_T * X;
        }
        const dim3 gw(X / 256, pw);
        const size_t lw = (size_t)K3W_R * K3W_STAGE;
        if (L->special & 4) hipLaunchKernelGGL(k3_down_wide<true>, gw, dim3(NT3), lw, s, a3);
        else                hipLaunchKernelGGL(k3_down_wide<false>, gw, dim3(NT3), lw, s, a3);
        if (!L->lat) {
            if ((rc = launch_ok())) return rc;
            const int n = T * X;
            const bool v4 = X % 4 == 0 && ((uintptr_t)out % 16 | (uintptr_t)resid % 16) == 0;
            if (v4)
                hipLaunchKernelGGL(k3_reduce4, dim3((n / 4 + 255) / 256), dim3(256), 0, s,
                                   (const float *)L->pacc, pw, resid, out, n / 4, X);
            else
                hipLaunchKernelGGL(k3_reduce, dim3((n + 255) / 256), dim3(256), 0, s,
                                   (const float *)L->pacc, pw, resid, out, n, X);
        }
    } else if (use2) {
        if (L->special & 4) hipLaunchKernelGGL(k3_down2<true>, dim3(X / 32, parts), dim3(NT3), 0, s, a3);
        else                hipLaunchKernelGGL(k3_down2<false>, dim3(X / 32, parts), dim3(NT3), 0, s, a3);
    } else if (L->special & 4) hipLaunchKernelGGL(k3_down<true>, dim3(X / 16, parts), dim3(NT3), l3, s, a3);
    else                hipLaunchKernelGGL(k3_down<false>, dim3(X / 16, parts), dim3(NT3), l3, s, a3);
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, ev++, s))) return rc;
    if (!L->lat) return 0;

    KNArgs an;
    an.acc = L->accL; an.P = parts; an.pstride = a3.pstride;
    an.nw = c->latent_norm ? L->lnw : NULL; an.eps = c->rms_eps;
    an.T = T; an.XL = X; an.latB = L->latB;
    K4Args a4;
    a4.up = L->lup; a4.latB = L->latB; a4.kn = an;
    a4.sh_down = L->SI > 0 ? L->sh_down : NULL; a4.shB = L->shB;
    a4.out = out; a4.resid = resid; a4.T = T; a4.H = H; a4.XL = X; a4.SI = L->SI;
    // the norm inside k4 when its set (and the aggregates) fit the LDS, the shared set
    // beside them when that fits too; otherwise the norm kernel writes the set first
    const bool fuse = k4_lds_bytes(true, false, T, X, L->SI) <= K4_LDS_MAX;
    const bool shl = k4_lds_bytes(fuse, true, T, X, L->SI) <= K4_LDS_MAX;
    if (!fuse) {
        const int nent = 4 * nSX * 16 * NC;
        hipLaunchKernelGGL(k4_latent_norm, dim3((nent + NT4 - 1) / NT4), dim3(NT4), 0,
                           s, an);
        if ((rc = launch_ok())) return rc;
        if ((rc = record(L, ev++, s))) return rc;
    }
    const size_t l4 = k4_lds_bytes(fuse, shl, T, X, L->SI);
    const dim3 g4(H / 16);
    if (fuse && shl)  hipLaunchKernelGGL((k4_up<true, true>), g4, dim3(NT3), l4, s, a4);
    else if (fuse)    hipLaunchKernelGGL((k4_up<true, false>), g4, dim3(NT3), l4, s, a4);
    else if (shl)     hipLaunchKernelGGL((k4_up<false, true>), g4, dim3(NT3), l4, s, a4);
    else              hipLaunchKernelGGL((k4_up<false, false>), g4, dim3(NT3), l4, s, a4);
    if ((rc = launch_ok())) return rc;
    return record(L, ev, s);
}

// ------------------------------------------------------------------ trunk products
// A bf16 trunk matrix (tiled, [out][in]) times T <= 8 activation rows: one workgroup per
// 16 output rows, Y[t*ldy + o] = W[o] . X[t*ldx] (k3_mmw_batch_ld, k3_ops.c:624-976).
struct TrunkArgs {
    const uint16_t *W;
    int             in, out;
    const void     *x;
    int             x_bf16, ldx, T;
    float          *y;
    int             ldy;
};

__global__ void __launch_bounds__(NT1) trunk_gemv(TrunkArgs a)
{
    __shared__ float lds[(NT1 / WAVE - 1) * 4 * WAVE];
    const int rt = blockIdx.x, lane = threadIdx.x % WAVE;
    float acc[4];
    bf16_tile_x(a.W + (size_t)rt * 16 * a.in, a.in, a.x, a.x_bf16, a.ldx, a.T, lds, acc);
    if (wave_id() != 0) return;
    per_token<4>(acc, 2 * a.T, lane, [&](int r0, int tok, const float (&v)[4]) AI {
        for (int i = 0; i < 4; i++) a.y[(size_t)tok * a.ldy + rt * 16 + r0 + i] = v[i];
    });
}

extern "C" int k3x_dev_trunk_gemv(const uint16_t *W, int in, int out, float *y, int ldy,
                                  const void *x, int x_dtype, int ldx, int T, void *stream)
{
    TrunkArgs a;
    a.W = W; a.in = in; a.out = out; a.x = x; a.x_bf16 = (x_dtype == K3X_BF16); a.ldx = ldx;
    a.T = T; a.y = y; a.ldy = ldy;
    hipLaunchKernelGGL(trunk_gemv, dim3(out / 16), dim3(NT1), 0, (hipStream_t)stream, a);
    return launch_ok();
}
