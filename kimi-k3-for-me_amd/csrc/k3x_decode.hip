// k3x_decode.hip - the decode path of the MoE block (T <= 8 tokens), four launches:
//
//   k1_router_shared  router logits in double, sigmoid, +bias (k3_router, k3_ops.c:1624-
//                     1694) for every expert, and the shared expert's gate/up products
//                     with SwiGLU (moe_shared, :1848-1857) in the same launch.
//   k1b_select_shdown one workgroup selects each token's top-k (:1700-1716) and lists the
//                     unique experts (the dedup of moe_prefill_routed, :2067-2081) while
//                     the others stream the shared expert's down product (:1858).
//   k2_gateup         each unique expert's gate/up products (k3_matmul_mxfp4,
//                     :3323-3776) with SwiGLU (k3_situ_glu at 2^64 betas, :148-161) and the
//                     routing weight folded in.
//   k3_down           each unique expert's down product into one accumulator set per 16
//                     output rows (the weighted combine, :1941-1942), plus the shared
//                     result (:1859) and an optional residual.
//
// Each weight byte is read once per call, with non-temporal loads.  Weights are
// dequantised in registers (E2M1 x 2^(s-127) is exact in bf16) and multiplied on
// v_mfma_f32_16x16x32_bf16 against activations split into bf16 hi + lo columns: every
// product is exact and only the fp32 accumulation rounds.  The activations (B
// fragments, compact layout: k3x_device.h) are staged in LDS when they fit, so a
// workgroup's loop waits on nothing but its own weight stream.
#include "k3x_device.h"

#define NT1 1024    // k1 workgroup: 16 waves
#define NT  256     // k1b / k2 workgroup: 4 waves
#define NT3 512     // k3 workgroup: 8 waves
#define STAGE_MAX 65536u   // largest B set staged in LDS (bytes)

extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];

// B source over a compact set of `bytes` at `src` (NC columns): staged into dynamic LDS
// when `stage`, else read through a range-checked buffer.  Every thread must call it.
__device__ __forceinline__ BSrc make_bsrc(const void *src, uint32_t bytes, int NC, bool stage,
                                          int nthreads)
{
    BSrc b;
    b.NC = NC;
    b.r = make_rsrc(src, bytes);
    b.lds = nullptr;
    b.zero = 0;
    if (stage) {
        b.zero = stage_b(dyn_lds, src, bytes, threadIdx.x, nthreads);
        b.lds = dyn_lds;
        __syncthreads();
    }
    return b;
}

// ------------------------------------------------------------------ streaming loops
// The loops below are branch-free in steady state: a wave's range is walked in steps of
// four (two) quads; a quad past the range multiplies weights of the range's last quad (a
// valid address) by zero B fragments, so every load is issued unconditionally and the
// compiler keeps the prefetches in flight.

// Quads q0, q0 + st, ... (cnt of them) of a gate/up pair of fp4 tiles.  The waves of a
// workgroup take interleaved quads (q0 = wave, st = waves), so at any moment the
// workgroup reads one contiguous window of each matrix.  Weights are loaded four quads
// ahead into a ring (slot k % 4, refilled right after the quad is multiplied), B
// fragments one quad ahead.  pair_prime issues the first four quads' loads (as early as
// the addresses are known); pair_run consumes them.
struct PairRing {
    Q4 g[4], u[4];
};

__device__ __forceinline__ void pair_prime(PairRing &ring, const uint8_t *tg, const uint8_t *tu,
                                           int nQ, int q0, int st, int cnt, int lane)
{
    if (cnt <= 0) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = q0 + st * min(i, cnt - 1);
        q4_load(ring.g[i], tg, q, nQ, lane);
        q4_load(ring.u[i], tu, q, nQ, lane);
    }
}

template <bool EXACT>
__device__ __forceinline__ void pair_run(f32x4 &dg, f32x4 &du, PairRing &ring,
                                         const uint8_t *tg, const uint8_t *tu, int nQ,
                                         const BSrc &bs, int q0, int st, int cnt, int lane,
                                         bool live)
{
    if (cnt <= 0) return;
    B4 bc;
    b4_load(bc, bs, 0u, q0, lane, live);
    for (int k0 = 0; k0 < cnt; k0 += 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k = k0 + i;
            const int q = q0 + st * min(k, cnt - 1);
            B4 bn;
            b4_load(bn, bs, 0u, q0 + st * min(k + 1, cnt - 1), lane, live && k + 1 < cnt);
            q4_mfma<EXACT>(dg, ring.g[i], q & 3, bc, k < cnt);
            q4_mfma<EXACT>(du, ring.u[i], q & 3, bc, k < cnt);
            const int qn = q0 + st * min(k + 4, cnt - 1);
            q4_load(ring.g[i], tg, qn, nQ, lane);
            q4_load(ring.u[i], tu, qn, nQ, lane);
            bc = bn;
        }
    }
}

// Quads [fa, fb) of the flattened (unique expert u, quad q) stream of the down
// products of one output row tile; expert u's B fragments start at u * slot_bytes.
struct DownSrc {
    const uint8_t *experts;
    size_t         expert_bytes, down_off, tb;
    const int     *uniq;
    int            nQ, rt;
    uint32_t       slot_bytes;
};

__device__ __forceinline__ void down_load(Q4 &a, const DownSrc &s, int f, int lane)
{
    const int u = f / s.nQ, q = f % s.nQ;
    const uint8_t *tile = s.experts + (size_t)s.uniq[u] * s.expert_bytes + s.down_off +
                          (size_t)s.rt * s.tb;
    q4_load(a, tile, q, s.nQ, lane);
}

struct DownRing {
    Q4 a[4];
};

// Flattened indices f0, f0 + st, ... (cnt of them).
__device__ __forceinline__ void down_prime(DownRing &ring, const DownSrc &s, int f0, int st,
                                           int cnt, int lane)
{
    if (cnt <= 0) return;
#pragma unroll
    for (int i = 0; i < 4; i++) down_load(ring.a[i], s, f0 + st * min(i, cnt - 1), lane);
}

template <bool EXACT>
__device__ __forceinline__ void down_run(f32x4 &d, DownRing &ring, const DownSrc &s,
                                         const BSrc &bs, int f0, int st, int cnt, int lane,
                                         bool live)
{
    if (cnt <= 0) return;
    B4 bc;
    b4_load(bc, bs, (uint32_t)(f0 / s.nQ) * s.slot_bytes, f0 % s.nQ, lane, live);
    for (int k0 = 0; k0 < cnt; k0 += 4) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k = k0 + i;
            const int f = f0 + st * min(k, cnt - 1);
            const int fn = f0 + st * min(k + 1, cnt - 1);
            B4 bn;
            b4_load(bn, bs, (uint32_t)(fn / s.nQ) * s.slot_bytes, fn % s.nQ, lane,
                    live && k + 1 < cnt);
            q4_mfma<EXACT>(d, ring.a[i], (f % s.nQ) & 3, bc, k < cnt);
            down_load(ring.a[i], s, f0 + st * min(k + 4, cnt - 1), lane);
            bc = bn;
        }
    }
}

// One bf16 quad of a tiled matrix: four 16-byte A fragments per lane.
struct QB {
    u32x4 a[4];
};

__device__ __forceinline__ void qb_load(QB &a, const uint8_t *tile, int q, int lane)
{
    const uint8_t *p = tile + (size_t)q * 4096 + lane * 16;
#pragma unroll
    for (int t = 0; t < 4; t++) a.a[t] = ldw16(p + t * 1024);
}

__device__ __forceinline__ void qb_mfma(f32x4 &d, const QB &a, const B4 &b)
{
#pragma unroll
    for (int t = 0; t < 4; t++) d = mfma(as_bf16x8(a.a[t]), as_bf16x8(b.b[t]), d);
}

// Quads q0, q0 + st, ... (cnt of them) of one tiled bf16 matrix (two with PAIR,
// sharing the B fragments): weights two quads ahead, B one quad ahead; lb(b, q, on)
// loads quad q's fragments (zeros when !on).  bf16_prime issues the first two quads'
// loads.
struct BfRing {
    QB g[2], u[2];
};

template <bool PAIR>
__device__ __forceinline__ void bf16_prime(BfRing &ring, const uint8_t *tg, const uint8_t *tu,
                                           int q0, int st, int cnt, int lane)
{
    if (cnt <= 0) return;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int q = q0 + st * min(i, cnt - 1);
        qb_load(ring.g[i], tg, q, lane);
        if (PAIR) qb_load(ring.u[i], tu, q, lane);
    }
}

template <bool PAIR, class LB>
__device__ __forceinline__ void bf16_run(f32x4 &dg, f32x4 &du, BfRing &ring, const uint8_t *tg,
                                         const uint8_t *tu, LB lb, int q0, int st, int cnt,
                                         int lane)
{
    if (cnt <= 0) return;
    B4 bc;
    lb(bc, q0, true);
    for (int k0 = 0; k0 < cnt; k0 += 2) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int k = k0 + i;
            B4 bn;
            lb(bn, q0 + st * min(k + 1, cnt - 1), k + 1 < cnt);
            qb_mfma(dg, ring.g[i], bc);
            if (PAIR) qb_mfma(du, ring.u[i], bc);
            const int qn = q0 + st * min(k + 2, cnt - 1);
            qb_load(ring.g[i], tg, qn, lane);
            if (PAIR) qb_load(ring.u[i], tu, qn, lane);
            bc = bn;
        }
    }
}

// Number of indices w, w + st, ... below n.
__device__ __forceinline__ int strided_count(int w, int st, int n) { return w < n ? (n - 1 - w) / st + 1 : 0; }

// B fragments of quad q straight from activations x [T][H] (no staging): bf16 x is its
// own hi column (lo = 0) and is read through a range-checked buffer; fp32 x is split
// here.
__device__ __forceinline__ void bx_load(B4 &b, const void *x, int x_bf16, rsrc_t xr, int H,
                                        int q, int lane, bool live)
{
    const int n = lane & 15, kq = lane >> 4, tok = n >> 1, hl = n & 1;
    if (x_bf16) {
        const uint32_t off = (uint32_t)(((size_t)tok * H + (size_t)q * 128 + kq * 32) * 2);
#pragma unroll
        for (int t = 0; t < 4; t++) b.b[t] = bload16(xr, (live && !hl) ? off + 16u * t : K3X_OOB);
    } else {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            b.b[t] = (u32x4){0u, 0u, 0u, 0u};
            if (live) {
                float xv[8];
                load_x8(x, 0, (size_t)tok * H + (size_t)q * 128 + kq * 32 + t * 8, xv);
                b.b[t] = bfrag_of(xv, hl);
            }
        }
    }
}

// Compact B fragments of x [T][H] (NC = 2T columns: hi, lo per token), entries
// [e0, e1) of the set, written by `nthreads` threads from `tid`.
__device__ __forceinline__ void x_to_bfrags(uint8_t *dst, const void *x, int x_bf16, int H,
                                            int NC, int e0, int e1, int tid, int nthreads)
{
    for (int f = e0 + tid; f < e1; f += nthreads) {
        const int n = f % NC, kq = (f / NC) & 3, t = (f / (NC * 4)) & 3, q = f / (NC * 16);
        float xv[8];
        load_x8(x, x_bf16, (size_t)(n >> 1) * H + (size_t)q * 128 + kq * 32 + t * 8, xv);
        *(u32x4 *)(dst + (size_t)f * 16) = bfrag_of(xv, n & 1);
    }
}

// ------------------------------------------------------------------ K1
struct K1Args {
    const float *router;     // [E][H]
    const float *bias;       // [E]
    const void  *x;          // [T][H]
    int          x_bf16;
    int          T, H, E;
    float       *score, *choice;   // [T][E]
    uint16_t    *xB;               // compact B fragments of x, for k2
    int          n_rwg;            // router workgroups
    const uint16_t *sh_gate, *sh_up;
    int          SI;
    uint16_t    *shB;              // compact B fragments of the shared activation
    int          stage;            // shared workgroups build x's fragments in LDS
};

#define RWAVES 4                     // waves per expert row in the router
#define RCH    4                     // float4 chunks per lane held at once

// Router logits: four waves per expert, sum_i W[e][i] x[i] in double (a product of two
// floats is exact in double; only the order of the additions differs from the
// reference's single chain), then score = sigmoid((float)logit), choice = score + bias.
__device__ void k1_router(const K1Args &a, float *lds)
{
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int grp = wave / RWAVES, wq = wave % RWAVES;          // expert slot, quarter
    const int e = blockIdx.x * (NT1 / WAVE / RWAVES) + grp;
    const int nf4 = a.H >> 2;
    double acc[K3X_DECODE_MAX_T];
#pragma unroll
    for (int t = 0; t < K3X_DECODE_MAX_T; t++) acc[t] = 0.0;
    if (e < a.E) {
        const float *row = a.router + (size_t)e * a.H;
        const int tl = wq * WAVE + lane;                        // 0..255 within the expert
        for (int f0 = 0; f0 < nf4; f0 += RWAVES * WAVE * RCH) {
            f32x4 w[RCH];
#pragma unroll
            for (int c = 0; c < RCH; c++) {
                const int f = f0 + tl + RWAVES * WAVE * c;
                w[c] = f < nf4 ? __builtin_nontemporal_load((const f32x4 *)(row + 4 * f))
                               : (f32x4){0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int t = 0; t < K3X_DECODE_MAX_T; t++) {
                if (t < a.T) {
                    float xv[RCH][4];
#pragma unroll
                    for (int c = 0; c < RCH; c++) {
                        const int f = f0 + tl + RWAVES * WAVE * c;
                        if (f < nf4) load_x4(a.x, a.x_bf16, (size_t)t * a.H + 4 * f, xv[c]);
                        else xv[c][0] = xv[c][1] = xv[c][2] = xv[c][3] = 0.f;
                    }
#pragma unroll
                    for (int c = 0; c < RCH; c++)
#pragma unroll
                        for (int k = 0; k < 4; k++) acc[t] += (double)w[c][k] * (double)xv[c][k];
                }
            }
        }
    }
    double *dl = (double *)lds;                                 // [16 waves][8]
#pragma unroll
    for (int t = 0; t < K3X_DECODE_MAX_T; t++) {
        if (t < a.T) {
            double v = acc[t];
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) dl[wave * K3X_DECODE_MAX_T + t] = v;
        }
    }
    __syncthreads();
    if (wq == 0 && lane < a.T && e < a.E) {
        const int t = lane;
        const double *g = dl + grp * RWAVES * K3X_DECODE_MAX_T;
        const double v = (g[t] + g[K3X_DECODE_MAX_T + t]) +
                         (g[2 * K3X_DECODE_MAX_T + t] + g[3 * K3X_DECODE_MAX_T + t]);
        const float sc = sigmoid_ref((float)v);
        a.score[(size_t)t * a.E + e] = sc;
        a.choice[(size_t)t * a.E + e] = sc + a.bias[e];
    }
}

// Shared expert gate and up for 16 rows over the full K, sixteen waves splitting the
// quads, then SwiGLU (hi + lo columns summed first) into the shared activation's
// compact B fragments.
__device__ void k1_shared(const K1Args &a, float *lds, int rt)
{
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int NW = NT1 / WAVE;
    const int nQ = a.H >> 7, NC = 2 * a.T;
    const int n = lane & 15, kq = lane >> 4;
    const bool live = n < NC;
    const int cnt = strided_count(wave, NW, nQ);
    const uint8_t *tg = (const uint8_t *)(a.sh_gate + (size_t)rt * nQ * 2048);
    const uint8_t *tu = (const uint8_t *)(a.sh_up + (size_t)rt * nQ * 2048);
    f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
    BfRing ring;
    if (a.stage) {
        // x's fragments built once per workgroup in LDS
        const uint32_t bytes = (uint32_t)(a.H * NC * 2);
        x_to_bfrags(dyn_lds, a.x, a.x_bf16, a.H, NC, 0, nQ * 16 * NC, threadIdx.x, NT1);
        if (threadIdx.x == 0) *(u32x4 *)(dyn_lds + bytes) = (u32x4){0u, 0u, 0u, 0u};
        bf16_prime<true>(ring, tg, tu, wave, NW, cnt, lane);
        __syncthreads();
        BSrc bs;
        bs.NC = NC;
        bs.lds = dyn_lds;
        bs.zero = bytes;
        bf16_run<true>(dg, du, ring, tg, tu,
                       [&](B4 &b, int q, bool on) { b4_load(b, bs, 0u, q, lane, live && on); },
                       wave, NW, cnt, lane);
    } else {
        bf16_prime<true>(ring, tg, tu, wave, NW, cnt, lane);
        const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.T * a.H * 2));
        bf16_run<true>(dg, du, ring, tg, tu,
                       [&](B4 &b, int q, bool on) { bx_load(b, a.x, a.x_bf16, xr, a.H, q, lane, live && on); },
                       wave, NW, cnt, lane);
    }
    float acc[8] = {dg[0], dg[1], dg[2], dg[3], du[0], du[1], du[2], du[3]};
    wave_sum_lds<8, NT1 / WAVE>(acc, lds, wave, lane);
    if (wave != 0) return;
    const int tok = n >> 1;
    for (int i = 0; i < 4; i++) {
        const float g = acc[i] + __shfl_xor(acc[i], 1);
        const float v = acc[4 + i] + __shfl_xor(acc[4 + i], 1);
        if ((n & 1) == 0 && live) {
            uint32_t hi, lo;
            split_bf16(swiglu(g, v), hi, lo);
            const int r = rt * 16 + 4 * kq + i;
            a.shB[bfrag_off(r, 2 * tok, NC)] = (uint16_t)hi;
            a.shB[bfrag_off(r, 2 * tok + 1, NC)] = (uint16_t)lo;
        }
    }
}

__global__ void __launch_bounds__(NT1) k1_router_shared(K1Args a)
{
    __shared__ float lds[(NT1 / WAVE - 1) * 8 * WAVE];
    if ((int)blockIdx.x < a.n_rwg) {
        k1_router(a, lds);
        const int NC = 2 * a.T, ne = (a.H >> 7) * 16 * NC;
        x_to_bfrags((uint8_t *)a.xB, a.x, a.x_bf16, a.H, NC, 0, ne,
                    blockIdx.x * NT1 + threadIdx.x, a.n_rwg * NT1);
        return;
    }
    k1_shared(a, lds, blockIdx.x - a.n_rwg);
}

// ------------------------------------------------------------------ top-k
// Order-preserving key of a choice value: larger float -> larger key; -0 is +0 (they
// compare equal in the reference); NaN -> 0 (never selected); -inf -> K_NEG_INF (never
// selected either: the reference's strict '>' against -inf fails).
#define K_NEG_INF 0x007FFFFFu
__device__ __forceinline__ uint32_t choice_key(float f)
{
    uint32_t u = __float_as_uint(f);
    if (f != f) return 0u;
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int lanes_below(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ float bload_f32(rsrc_t r, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// One token's top-k by one wave, equal to the reference's repeated maximum
// (k3_ops.c:1700-1708): the K largest choices in descending order, the lower index first
// among equal values, NaN and -inf never taken (a pick with nothing left gives index 0,
// weight 0).  A 32-step bitwise search with ballot counts finds the k-th largest key;
// the k selected are then ranked.  Weights are the unbiased scores, renormalised through
// a double sum and a float reciprocal, then scaled (:1710-1716).  Results in s_idx/s_w.
template <int NC>
__device__ void wave_topk(rsrc_t cr, rsrc_t sr, uint32_t row_off, int E, int K, int renorm,
                          float routed_scale, int *s_idx, float *s_w, uint64_t *s_key,
                          int *s_e, float *s_sc, int lane)
{
    uint32_t key[NC];
    float sco[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int e = lane + WAVE * c;
        const uint32_t off = row_off + 4u * (uint32_t)e;
        const float v = bload_f32(cr, e < E ? off : K3X_OOB);
        sco[c] = bload_f32(sr, e < E ? off : K3X_OOB);
        key[c] = e < E ? choice_key(v) : 0u;
    }
    int nvalid = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) nvalid += __popcll(__ballot(key[c] > K_NEG_INF));
    const int ke = min(K, nvalid);
    uint32_t tau = 0xFFFFFFFFu;
    if (ke > 0) {
        tau = 0u;
        for (int b = 31; b >= 0; b--) {
            const uint32_t cand = tau | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int c = 0; c < NC; c++) cnt += __popcll(__ballot(key[c] >= cand));
            if (cnt >= ke) tau = cand;
        }
    }
    int ngt = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) ngt += __popcll(__ballot(key[c] > tau));
    int need = ke - ngt;                    // ties at tau, taken in ascending index
    int base = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const uint64_t eq = __ballot(ke > 0 && key[c] == tau);
        const int take = min(need, (int)__popcll(eq));
        need -= take;
        const bool sel = (ke > 0) && (key[c] > tau || (key[c] == tau && lanes_below(eq) < take));
        const uint64_t sm = __ballot(sel);
        if (sel) {
            const int pos = base + lanes_below(sm);
            const int e = lane + WAVE * c;
            s_key[pos] = ((uint64_t)key[c] << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
            s_e[pos] = e;
            s_sc[pos] = sco[c];
        }
        base += (int)__popcll(sm);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (lane < ke) {
        const uint64_t my = s_key[lane];
        int rank = 0;
        for (int i = 0; i < ke; i++) rank += s_key[i] > my;
        s_idx[rank] = s_e[lane];
        s_w[rank] = s_sc[lane];
    } else if (lane < K) {
        s_idx[lane] = 0;
        s_w[lane] = 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        if (renorm && K > 1) {
            double sum = 0.0;
            for (int j = 0; j < K; j++) sum += (double)s_w[j];
            const float inv = (float)(1.0 / (sum + 1e-20));
            for (int j = 0; j < K; j++) s_w[j] *= inv;
        }
        for (int j = 0; j < K; j++) s_w[j] *= routed_scale;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
}

// ------------------------------------------------------------------ K1b
struct KSArgs {
    const float   *score, *choice;
    int            E, K, renorm;
    float          routed_scale;
    k3x_route     *route;          // unique experts and per-(expert, token) weights, for k2/k3
    int           *idx;  float *wt;        // internal [T][K]
    int           *uidx; float *uwt;       // optional caller copies
    int            T, H;
    const uint16_t *sh_down, *shB;
    float         *ysh;            // [T][H] shared expert output
    int            SI;
    int            stage;          // shB staged in LDS
};

// Shared expert down product for 16 output rows: four waves splitting the quads.
__device__ void ks_shared_down(const KSArgs &a, float *lds, int rt)
{
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int nQS = a.SI >> 7, NC = 2 * a.T;
    const int n = lane & 15;
    const bool live = n < NC;
    const uint8_t *tile = (const uint8_t *)(a.sh_down + (size_t)rt * nQS * 2048);
    const int cnt = strided_count(wave, NT / WAVE, nQS);
    BfRing ring;
    bf16_prime<false>(ring, tile, tile, wave, NT / WAVE, cnt, lane);
    const BSrc bs = make_bsrc(a.shB, (uint32_t)(a.SI * NC * 2), NC, a.stage != 0, NT);
    f32x4 d = {0.f, 0.f, 0.f, 0.f}, unused = {0.f, 0.f, 0.f, 0.f};
    bf16_run<false>(d, unused, ring, tile, tile,
                    [&](B4 &b, int q, bool on) { b4_load(b, bs, 0u, q, lane, live && on); },
                    wave, NT / WAVE, cnt, lane);
    float acc[4] = {d[0], d[1], d[2], d[3]};
    wave_sum_lds<4, NT / WAVE>(acc, lds, wave, lane);
    if (wave != 0) return;
    const int kq = lane >> 4, tok = n >> 1;
    for (int i = 0; i < 4; i++) {
        const float y = acc[i] + __shfl_xor(acc[i], 1);
        if ((n & 1) == 0 && live) a.ysh[(size_t)tok * a.H + rt * 16 + 4 * kq + i] = y;
    }
}

// Routing of every token (one wave per token), then the unique experts in first-seen
// order over (token, slot) and each one's weight per token (0 where not chosen).
template <int NC>
__device__ void ks_select(const KSArgs &a)
{
    __shared__ int      s_idx[K3X_DECODE_MAX_T][K3X_MAX_TOPK];
    __shared__ float    s_w[K3X_DECODE_MAX_T][K3X_MAX_TOPK];
    __shared__ uint64_t s_key[NT / WAVE][K3X_MAX_TOPK];
    __shared__ int      s_e[NT / WAVE][K3X_MAX_TOPK];
    __shared__ float    s_sc[NT / WAVE][K3X_MAX_TOPK];
    __shared__ int      s_slot[1024];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const rsrc_t cr = make_rsrc(a.choice, (uint32_t)(a.T * a.E * 4));
    const rsrc_t sr = make_rsrc(a.score, (uint32_t)(a.T * a.E * 4));
    for (int t = wave; t < a.T; t += NT / WAVE)
        wave_topk<NC>(cr, sr, (uint32_t)(t * a.E * 4), a.E, a.K, a.renorm, a.routed_scale,
                      s_idx[t], s_w[t], s_key[wave], s_e[wave], s_sc[wave], lane);
    for (int e = threadIdx.x; e < a.E; e += NT) s_slot[e] = -1;
    __syncthreads();
    for (int i = threadIdx.x; i < a.T * a.K; i += NT) {
        const int t = i / a.K, j = i % a.K;
        a.idx[i] = s_idx[t][j];
        a.wt[i] = s_w[t][j];
        if (a.uidx) { a.uidx[i] = s_idx[t][j]; a.uwt[i] = s_w[t][j]; }
    }
    if (threadIdx.x == 0) {
        int nu = 0;
        for (int t = 0; t < a.T; t++)
            for (int j = 0; j < a.K; j++) {
                const int ex = s_idx[t][j];
                if (s_slot[ex] < 0) {
                    s_slot[ex] = nu;
                    a.route->uniq[nu] = ex;
                    for (int tt = 0; tt < K3X_DECODE_MAX_T; tt++) a.route->wtok[nu][tt] = 0.0f;
                    nu++;
                }
                a.route->wtok[s_slot[ex]][t] = s_w[t][j];
            }
        a.route->nu = nu;
    }
}

template <int NC>
__global__ void __launch_bounds__(NT) k1b_select_shdown(KSArgs a)
{
    __shared__ float lds[(NT / WAVE - 1) * 4 * WAVE];
    if (blockIdx.x == 0) { ks_select<NC>(a); return; }
    ks_shared_down(a, lds, blockIdx.x - 1);
}

// ------------------------------------------------------------------ K2
struct K2Args {
    const uint8_t *experts;
    size_t         expert_bytes, gate_off, up_off;
    const k3x_route *route;
    const int     *xflags;         // [E] bit 0 gate, 1 up, 2 down: scale bytes need EXACT
    const uint16_t *xB;            // compact B fragments of x
    uint16_t      *actB;           // compact B fragments of each unique expert's activation
    int            T, H, I;
    int            stage;
};

__global__ void __launch_bounds__(NT) k2_gateup(K2Args a)
{
    __shared__ float lds[(NT / WAVE - 1) * 8 * WAVE];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int nTiles = a.I >> 4;
    const int u = blockIdx.x / nTiles, rt = blockIdx.x % nTiles;
    if (u >= a.route->nu) return;
    const int e = a.route->uniq[u];
    const int NC = 2 * a.T;
    const size_t tb = fp4_tile_bytes(a.H);
    const uint8_t *ex = a.experts + (size_t)e * a.expert_bytes;
    const uint8_t *tg = ex + a.gate_off + (size_t)rt * tb;
    const uint8_t *tu = ex + a.up_off + (size_t)rt * tb;
    const int nQ = a.H >> 7;
    const int cnt = strided_count(wave, NT / WAVE, nQ);
    const int n = lane & 15;
    const bool live = n < NC;
    PairRing ring;
    pair_prime(ring, tg, tu, nQ, wave, NT / WAVE, cnt, lane);
    const int flags = a.xflags[e];
    const BSrc bs = make_bsrc(a.xB, (uint32_t)(a.H * NC * 2), NC, a.stage != 0, NT);
    f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
    if (flags & 3) pair_run<true>(dg, du, ring, tg, tu, nQ, bs, wave, NT / WAVE, cnt, lane, live);
    else           pair_run<false>(dg, du, ring, tg, tu, nQ, bs, wave, NT / WAVE, cnt, lane, live);
    float acc[8] = {dg[0], dg[1], dg[2], dg[3], du[0], du[1], du[2], du[3]};
    wave_sum_lds<8, NT / WAVE>(acc, lds, wave, lane);
    if (wave != 0) return;
    // hi + lo columns, SwiGLU, the token's routing weight for this expert (0 if the token
    // did not choose it), then the bf16 split for the down products
    const int kq = lane >> 4, tok = n >> 1;
    const float w = live ? a.route->wtok[u][tok] : 0.0f;
    uint16_t *dst = a.actB + (size_t)u * ((size_t)a.I * NC);
    for (int i = 0; i < 4; i++) {
        const float g = acc[i] + __shfl_xor(acc[i], 1);
        const float v = acc[4 + i] + __shfl_xor(acc[4 + i], 1);
        if ((n & 1) == 0 && live) {
            const float y = (w == 0.0f) ? 0.0f : w * swiglu(g, v);
            uint32_t hi, lo;
            split_bf16(y, hi, lo);
            const int r = rt * 16 + 4 * kq + i;
            dst[bfrag_off(r, 2 * tok, NC)] = (uint16_t)hi;
            dst[bfrag_off(r, 2 * tok + 1, NC)] = (uint16_t)lo;
        }
    }
}

// ------------------------------------------------------------------ K3
struct K3Args {
    const uint8_t *experts;
    size_t         expert_bytes, down_off;
    const k3x_route *route;
    const int     *xflags;
    const uint16_t *actB;
    const float   *ysh;            // shared output, or NULL
    float         *out;
    const float   *resid;
    int            T, H, I, K;
    int            stage;          // stage the routed activations when nu*I*NC*2 <= STAGE_MAX
};

__global__ void __launch_bounds__(NT3) k3_down(K3Args a)
{
    __shared__ float lds[(NT3 / WAVE - 1) * 4 * WAVE];
    __shared__ int   s_uniq[K3X_DECODE_MAX_T * K3X_MAX_TOPK];
    __shared__ int   s_exact;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int NW = NT3 / WAVE;
    const int rt = blockIdx.x;
    const int nu = a.route->nu;
    const int NC = 2 * a.T;
    if (threadIdx.x == 0) s_exact = 0;
    for (int u = threadIdx.x; u < nu; u += NT3) s_uniq[u] = a.route->uniq[u];
    __syncthreads();
    const uint32_t slot = (uint32_t)(a.I * NC * 2);
    const int nQI = a.I >> 7;
    const int n = lane & 15;
    const bool live = n < NC;
    DownSrc ds;
    ds.experts = a.experts; ds.expert_bytes = a.expert_bytes; ds.down_off = a.down_off;
    ds.tb = fp4_tile_bytes(a.I); ds.uniq = s_uniq; ds.nQ = nQI; ds.rt = rt;
    ds.slot_bytes = slot;
    const int nf = nu * nQI;
    const int cnt = strided_count(wave, NW, nf);
    DownRing ring;
    down_prime(ring, ds, wave, NW, cnt, lane);
    for (int u = threadIdx.x; u < nu; u += NT3)
        if (a.xflags[s_uniq[u]] & 4) s_exact = 1;
    const bool stage = a.stage && (uint32_t)nu * slot <= STAGE_MAX;
    const BSrc bs = make_bsrc(a.actB, stage ? (uint32_t)nu * slot : (uint32_t)(a.T * a.K) * slot,
                              NC, stage, NT3);
    __syncthreads();
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    if (s_exact) down_run<true>(d, ring, ds, bs, wave, NW, cnt, lane, live);
    else         down_run<false>(d, ring, ds, bs, wave, NW, cnt, lane, live);
    float acc[4] = {d[0], d[1], d[2], d[3]};
    wave_sum_lds<4, NT3 / WAVE>(acc, lds, wave, lane);
    if (wave != 0) return;
    const int kq = lane >> 4, tok = n >> 1;
    for (int i = 0; i < 4; i++) {
        const float y = acc[i] + __shfl_xor(acc[i], 1);
        if ((n & 1) == 0 && live) {
            const int r = rt * 16 + 4 * kq + i;
            const size_t o = (size_t)tok * a.H + r;
            const float ys = a.ysh ? y + a.ysh[o] : y;
            a.out[o] = a.resid ? a.resid[o] + ys : ys;
        }
    }
}

// ------------------------------------------------------------------ launcher
static inline int launch_ok(void) { return hipGetLastError() == hipSuccess ? 0 : K3X_E_HIP; }

static int record(k3x_moe_layer *L, int i, hipStream_t s)
{
    if (!L->timing || i >= 8) return 0;
    if (i + 1 > L->n_ev_used) L->n_ev_used = i + 1;
    return hipEventRecord((hipEvent_t)L->ev[i], s) == hipSuccess ? 0 : K3X_E_HIP;
}

extern "C" int k3x_dev_decode(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                              int T, const float *resid, int *idx, float *wt, void *stream)
{
    const k3x_cfg *c = &L->cfg;
    hipStream_t s = (hipStream_t)stream;
    const int NC = 2 * T;
    int rc;
    K1Args a1;
    a1.router = L->router; a1.bias = L->bias; a1.x = x; a1.x_bf16 = (x_dtype == K3X_BF16);
    a1.T = T; a1.H = c->hidden; a1.E = c->n_experts;
    a1.score = L->score; a1.choice = L->choice; a1.xB = L->xB;
    a1.n_rwg = (c->n_experts + NT1 / WAVE / RWAVES - 1) / (NT1 / WAVE / RWAVES);
    a1.sh_gate = L->sh_gate; a1.sh_up = L->sh_up; a1.SI = L->SI; a1.shB = L->shB;
    const uint32_t xbytes = (uint32_t)(c->hidden * NC * 2);
    a1.stage = xbytes <= STAGE_MAX;
    const int n_sh = L->SI > 0 ? L->SI / 16 : 0;
    if ((rc = record(L, 0, s))) return rc;
    hipLaunchKernelGGL(k1_router_shared, dim3(a1.n_rwg + n_sh), dim3(NT1),
                       a1.stage ? xbytes + 16 : 0, s, a1);
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, 1, s))) return rc;

    KSArgs as;
    as.score = L->score; as.choice = L->choice; as.E = c->n_experts; as.K = c->topk;
    as.renorm = c->moe_renorm; as.routed_scale = c->routed_scale; as.route = L->route;
    as.idx = L->idx; as.wt = L->wt; as.uidx = idx; as.uwt = wt; as.T = T; as.H = c->hidden;
    as.sh_down = L->sh_down; as.shB = L->shB; as.ysh = L->ysh; as.SI = L->SI;
    const uint32_t sbytes = (uint32_t)(L->SI * NC * 2);
    as.stage = L->SI > 0 && sbytes <= STAGE_MAX;
    const dim3 gs(1 + (L->SI > 0 ? c->hidden / 16 : 0));
    const size_t ls = as.stage ? sbytes + 16 : 0;
    if (c->n_experts <= 128)      hipLaunchKernelGGL(k1b_select_shdown<2>, gs, dim3(NT), ls, s, as);
    else if (c->n_experts <= 256) hipLaunchKernelGGL(k1b_select_shdown<4>, gs, dim3(NT), ls, s, as);
    else if (c->n_experts <= 384) hipLaunchKernelGGL(k1b_select_shdown<6>, gs, dim3(NT), ls, s, as);
    else if (c->n_experts <= 512) hipLaunchKernelGGL(k1b_select_shdown<8>, gs, dim3(NT), ls, s, as);
    else                          hipLaunchKernelGGL(k1b_select_shdown<16>, gs, dim3(NT), ls, s, as);
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, 2, s))) return rc;

    K2Args a2;
    a2.experts = L->experts; a2.expert_bytes = L->expert_bytes;
    a2.gate_off = L->gate_off; a2.up_off = L->up_off; a2.route = L->route;
    a2.xflags = L->xflags;
    a2.xB = L->xB; a2.actB = L->actB; a2.T = T; a2.H = c->hidden; a2.I = c->moe_inter;
    a2.stage = xbytes <= STAGE_MAX;
    hipLaunchKernelGGL(k2_gateup, dim3(T * c->topk * (c->moe_inter / 16)), dim3(NT),
                       a2.stage ? xbytes + 16 : 0, s, a2);
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, 3, s))) return rc;

    K3Args a3;
    a3.experts = L->experts; a3.expert_bytes = L->expert_bytes; a3.down_off = L->down_off;
    a3.route = L->route; a3.xflags = L->xflags; a3.actB = L->actB;
    a3.ysh = L->SI > 0 ? L->ysh : NULL;
    a3.out = out; a3.resid = resid; a3.T = T; a3.H = c->hidden; a3.I = c->moe_inter;
    a3.K = c->topk;
    a3.stage = 1;
    hipLaunchKernelGGL(k3_down, dim3(c->hidden / 16), dim3(NT3), STAGE_MAX + 16, s, a3);
    if ((rc = launch_ok())) return rc;
    return record(L, 4, s);
}

// Prefill, first form: the decode pipeline over consecutive groups of up to
// K3X_DECODE_MAX_T tokens.  Each token's result depends only on its own routing, so the
// grouping changes no result.
extern "C" int k3x_dev_prefill(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                               int T, const float *resid, int *idx, float *wt, void *stream)
{
    const int H = L->cfg.hidden, K = L->cfg.topk;
    const size_t es = (x_dtype == K3X_BF16) ? 2 : 4;
    for (int t0 = 0; t0 < T; t0 += K3X_DECODE_MAX_T) {
        const int n = min(K3X_DECODE_MAX_T, T - t0);
        const int rc = k3x_dev_decode(L, out + (size_t)t0 * H,
                                      (const char *)x + (size_t)t0 * H * es, x_dtype, n,
                                      resid ? resid + (size_t)t0 * H : NULL,
                                      idx ? idx + (size_t)t0 * K : NULL,
                                      wt ? wt + (size_t)t0 * K : NULL, stream);
        if (rc) return rc;
    }
    return 0;
}
