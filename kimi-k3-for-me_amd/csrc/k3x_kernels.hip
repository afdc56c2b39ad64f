// k3x_kernels.hip - gfx950 kernels of the MoE block and their C-ABI launchers.
//
// Decode path (T <= 8 tokens), three launches per layer:
//   k1_router_shared  router logits in double, sigmoid, +bias (k3_router, k3_ops.c:1624-
//                     1694); the last router workgroup does top-k, renorm, scale
//                     (:1700-1716) and the unique-expert list (the dedup of
//                     moe_prefill_routed, :2067-2081); other workgroups run the shared
//                     expert's gate/up products (moe_shared, :1848-1860) in parallel.
//   k2_gateup         every unique expert's gate and up products (k3_matmul_mxfp4,
//                     :3323-3776) on the matrix cores, SwiGLU (k3_situ_glu at 2^64 betas,
//                     :148-161), the routing weight folded in; shared SwiGLU finalised.
//   k3_down           every unique expert's down product and the shared down product
//                     accumulated in one set of accumulators per output row tile: the
//                     weighted combine (:1941-1942) and the shared add (:1859).
// Weights are dequantised in registers (v_cvt_scalef32_pk_bf16_fp4: E2M1 x 2^(s-127) is
// exact in bf16) and multiplied with v_mfma_f32_16x16x32_bf16 against activations split
// into bf16 hi + lo columns, so each product is exact and only fp32 accumulation rounds.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include "k3x_internal.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

#define WAVE 64
#define NT   256          // threads per workgroup on the decode path (4 waves)

// ------------------------------------------------------------------ small helpers
__device__ __forceinline__ uint32_t f2bf(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// v = hi + lo with hi, lo bf16: hi = rne(v), lo = rne(v - hi) (v - hi is exact).
__device__ __forceinline__ void split_bf16(float v, uint32_t &hi, uint32_t &lo)
{
    hi = f2bf(v);
    lo = f2bf(v - bf2f(hi));
}

// The reference's sigmoid, 1/(1+expf(-x)) in float (k3_ops.c:143).  exp is evaluated in
// double and rounded once, which gives the correctly rounded expf(-x) except within
// ~2^-29 relative of a rounding midpoint.
__device__ __forceinline__ float sigmoid_ref(float x)
{
    const float e = (float)exp(-(double)x);
    return 1.0f / (1.0f + e);
}

// SwiGLU as k3_situ_glu computes it at 2^64 betas: a = g*sigmoid(g), y = a*u, in float.
__device__ __forceinline__ float swiglu(float g, float u)
{
    const float a = g * sigmoid_ref(g);
    return a * u;
}

// E8M0 byte -> the fp32 scale operand of the fp4 converts.  Byte 255 (NaN, zero in the
// reference) is handled by zeroing the codes instead.
__device__ __forceinline__ float e8m0_f32(uint32_t b)
{
    return b == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(b << 23);
}

// 8 E2M1 codes (one dword, low nibble first) times a scale -> 8 bf16, exact.
__device__ __forceinline__ bf16x8 dq8(uint32_t codes, uint32_t sbyte)
{
    const uint32_t c = (sbyte == 255u) ? 0u : codes;
    const float s = e8m0_f32(sbyte == 255u ? 127u : sbyte);
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 0);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 1);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 2);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(c, s, 3);
    bf16x8 r = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

// Offsets inside a tiled fp4 matrix (see k3x_internal.h).
__device__ __forceinline__ size_t fp4_tile_bytes(int K)
{
    const int nq = K >> 7, ns = (nq + 3) >> 2;
    return (size_t)nq * 1024 + (size_t)ns * 256;
}

// Element offset (in bf16 units) of B-fragment entry (K-index r, column n).
__device__ __forceinline__ size_t bfrag_off(int r, int n)
{
    const int q = r >> 7, kq = (r & 127) >> 5, t = (r & 31) >> 3, j = r & 7;
    return ((((size_t)q * 4 + t) * 64 + (n + 16 * kq)) << 3) + j;
}

// Cross-wave sum of per-lane accumulators through LDS; wave 0 ends with the total.
template <int NV>
__device__ __forceinline__ void wave_sum_lds(float (&acc)[NV], float *lds, int wave, int lane)
{
    if (wave != 0)
        for (int v = 0; v < NV; v++) lds[((wave - 1) * NV + v) * WAVE + lane] = acc[v];
    __syncthreads();
    if (wave == 0)
        for (int w = 1; w < NT / WAVE; w++)
            for (int v = 0; v < NV; v++) acc[v] += lds[((w - 1) * NV + v) * WAVE + lane];
}

// ------------------------------------------------------------------ K1: router + shared gate/up
struct K1Args {
    const float *router;     // [E][H]
    const float *bias;       // [E]
    const void  *x;          // [T][H]
    int          x_bf16;
    int          T, H, E, K, renorm;
    float        routed_scale;
    float       *score, *choice;   // [T][E]
    int         *idx;  float *wt;  // [T][K] internal
    int         *uidx; float *uwt; // optional user copies
    unsigned    *counter;
    k3x_route   *route;
    uint16_t    *xB;               // B fragments of x
    int          n_rwg;            // router workgroups
    // shared gate/up
    const uint16_t *sh_gate, *sh_up;
    int          SI;
    float       *shpart;           // [2][2][SI][16]
};

// 4 and 8 consecutive activations (base a multiple of 4 / 8), widened to float.
__device__ __forceinline__ void load_x4(const void *x, int bf, size_t base, float (&v)[4])
{
    if (bf) {
        const u32x2 r = *(const u32x2 *)((const uint16_t *)x + base);
        v[0] = bf2f(r[0] & 0xFFFFu); v[1] = bf2f(r[0] >> 16);
        v[2] = bf2f(r[1] & 0xFFFFu); v[3] = bf2f(r[1] >> 16);
    } else {
        const f32x4 r = *(const f32x4 *)((const float *)x + base);
        v[0] = r[0]; v[1] = r[1]; v[2] = r[2]; v[3] = r[3];
    }
}

__device__ __forceinline__ void load_x8(const void *x, int bf, size_t base, float (&v)[8])
{
    if (bf) {
        const u32x4 r = ld16((const uint16_t *)x + base);
        for (int j = 0; j < 4; j++) { v[2 * j] = bf2f(r[j] & 0xFFFFu); v[2 * j + 1] = bf2f(r[j] >> 16); }
    } else {
        const f32x4 r0 = *(const f32x4 *)((const float *)x + base);
        const f32x4 r1 = *(const f32x4 *)((const float *)x + base + 4);
        for (int j = 0; j < 4; j++) { v[j] = r0[j]; v[4 + j] = r1[j]; }
    }
}

// One B fragment (8 bf16 of column hi or lo) from 8 activations.
__device__ __forceinline__ u32x4 bfrag_of(const float (&v)[8], int hl)
{
    uint32_t h[8];
    for (int j = 0; j < 8; j++) {
        uint32_t hi, lo;
        split_bf16(v[j], hi, lo);
        h[j] = hl ? lo : hi;
    }
    u32x4 r = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    return r;
}

// Top-k of one token by one wave, the reference's repeated maximum (k3_ops.c:1700-1708):
// strict '>' in ascending index, so the lowest index wins a tie; a taken entry becomes
// -inf.  vals is this wave's LDS copy of the token's choice row.
// Results go to this token's LDS rows s_idx/s_w (written by lane 0).
__device__ void wave_topk(float *vals, const float *score_row, int E, int K, int renorm,
                          float routed_scale, int *s_idx, float *s_w, int lane)
{
    for (int j = 0; j < K; j++) {
        float bv = -INFINITY;
        int   bi = 0x7FFFFFFF;
        for (int e = lane; e < E; e += WAVE) {
            const float v = vals[e];
            if (v > bv) { bv = v; bi = e; }
        }
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int   oi = __shfl_xor(bi, off);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) {
            if (bi == 0x7FFFFFFF) { s_idx[j] = 0; s_w[j] = 0.0f; }
            else { s_idx[j] = bi; s_w[j] = score_row[bi]; vals[bi] = -INFINITY; }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) {
        if (renorm && K > 1) {
            double s = 0.0;
            for (int j = 0; j < K; j++) s += (double)s_w[j];
            const float inv = (float)(1.0 / (s + 1e-20));
            for (int j = 0; j < K; j++) s_w[j] *= inv;
        }
        for (int j = 0; j < K; j++) s_w[j] *= routed_scale;
    }
}

__global__ void __launch_bounds__(NT) k1_router_shared(K1Args a)
{
    __shared__ float lds[(NT / WAVE) * 1024];          // reductions, top-k rows, dedup map
    __shared__ int   s_idx[K3X_DECODE_MAX_T][K3X_MAX_TOPK];
    __shared__ float s_w[K3X_DECODE_MAX_T][K3X_MAX_TOPK];
    __shared__ int   s_last;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;

    if ((int)blockIdx.x < a.n_rwg) {
        // ---- router logits: one expert per wave, one double chain per token
        const int e = blockIdx.x * (NT / WAVE) + wave;
        if (e < a.E) {
            double acc[K3X_DECODE_MAX_T];
            for (int t = 0; t < K3X_DECODE_MAX_T; t++) acc[t] = 0.0;
            const float *row = a.router + (size_t)e * a.H;
            for (int i = lane * 4; i < a.H; i += WAVE * 4) {
                const f32x4 w4 = *(const f32x4 *)(row + i);
#pragma unroll
                for (int t = 0; t < K3X_DECODE_MAX_T; t++) {
                    if (t < a.T) {
                        float xv[4];
                        load_x4(a.x, a.x_bf16, (size_t)t * a.H + i, xv);
                        acc[t] += (double)w4[0] * (double)xv[0];
                        acc[t] += (double)w4[1] * (double)xv[1];
                        acc[t] += (double)w4[2] * (double)xv[2];
                        acc[t] += (double)w4[3] * (double)xv[3];
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < K3X_DECODE_MAX_T; t++) {
                if (t >= a.T) break;
                double v = acc[t];
                for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
                if (lane == 0) {
                    const float s = sigmoid_ref((float)v);
                    a.score[(size_t)t * a.E + e] = s;
                    a.choice[(size_t)t * a.E + e] = s + a.bias[e];
                }
            }
        }
        // ---- B fragments of x for the routed gate/up products (columns < 2T)
        {
            const int nQ = a.H >> 7, cols = 2 * a.T;
            const int total = nQ * 4 * 4 * cols;          // [q][t][kq][n]
            for (int f = blockIdx.x * NT + threadIdx.x; f < total; f += a.n_rwg * NT) {
                const int n = f % cols, kq = (f / cols) & 3, t = (f / (cols * 4)) & 3;
                const int q = f / (cols * 16);
                const int tok = n >> 1, hl = n & 1;
                const size_t base = (size_t)tok * a.H + (size_t)q * 128 + kq * 32 + t * 8;
                float xv[8];
                load_x8(a.x, a.x_bf16, base, xv);
                const u32x4 v = bfrag_of(xv, hl);
                *(u32x4 *)(a.xB + ((((size_t)q * 4 + t) * 64 + (n + 16 * kq)) << 3)) = v;
            }
        }
        // ---- the last router workgroup selects
        __syncthreads();
        if (threadIdx.x == 0) {
            __threadfence();
            const unsigned ticket = atomicAdd(a.counter, 1u);
            s_last = (ticket == (unsigned)a.n_rwg - 1u);
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
        float *vals = lds + wave * 1024;          // E <= 1024 per wave row
        for (int t = wave; t < a.T; t += NT / WAVE) {
            for (int e = lane; e < a.E; e += WAVE)
                vals[e] = __builtin_nontemporal_load(a.choice + (size_t)t * a.E + e);
            __builtin_amdgcn_wave_barrier();
            wave_topk(vals, a.score + (size_t)t * a.E, a.E, a.K, a.renorm, a.routed_scale,
                      s_idx[t], s_w[t], lane);
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            // unique experts in first-seen order over (token, slot)
            int *slot_of = (int *)lds;             // [E], reuses the top-k rows
            for (int e = 0; e < a.E; e++) slot_of[e] = -1;
            int nu = 0;
            for (int t = 0; t < a.T; t++)
                for (int j = 0; j < a.K; j++) {
                    const int ex = s_idx[t][j];
                    if (slot_of[ex] < 0) {
                        slot_of[ex] = nu;
                        a.route->uniq[nu] = ex;
                        for (int tt = 0; tt < K3X_DECODE_MAX_T; tt++) a.route->wtok[nu][tt] = 0.0f;
                        nu++;
                    }
                    a.route->wtok[slot_of[ex]][t] = s_w[t][j];
                    a.idx[t * a.K + j] = ex;
                    a.wt[t * a.K + j] = s_w[t][j];
                    if (a.uidx) { a.uidx[t * a.K + j] = ex; a.uwt[t * a.K + j] = s_w[t][j]; }
                }
            a.route->nu = nu;
            *a.counter = 0u;
        }
        return;
    }

    // ---- shared expert gate/up partial products: (matrix, row tile, K half)
    const int sb = blockIdx.x - a.n_rwg;
    const int mat = sb & 1, half = (sb >> 1) & 1, rt = sb >> 2;
    const int nQ = a.H >> 7;
    const int qa = half ? nQ / 2 : 0, qb = half ? nQ : nQ / 2;
    const int per = (qb - qa + 3) / 4;
    const int q0 = qa + wave * per, q1 = min(qb, q0 + per);
    const uint16_t *tile = (mat ? a.sh_up : a.sh_gate) + (size_t)rt * nQ * 2048;
    const int n = lane & 15, kq = lane >> 4;
    const bool bcol = n < 2 * a.T;
    const int tok = n >> 1, hl = n & 1;
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    for (int q = q0; q < q1; q++) {
        u32x4 av[4];
        for (int t = 0; t < 4; t++)
            av[t] = ld16((const uint8_t *)tile + (size_t)q * 4096 + t * 1024 + lane * 16);
        for (int t = 0; t < 4; t++) {
            u32x4 bv = {0u, 0u, 0u, 0u};
            if (bcol) {
                float xv[8];
                load_x8(a.x, a.x_bf16, (size_t)tok * a.H + (size_t)q * 128 + kq * 32 + t * 8, xv);
                bv = bfrag_of(xv, hl);
            }
            d = mfma(as_bf16x8(av[t]), as_bf16x8(bv), d);
        }
    }
    float acc[4] = {d[0], d[1], d[2], d[3]};
    wave_sum_lds<4>(acc, lds, wave, lane);
    if (wave == 0) {
        float *dst = a.shpart + ((size_t)(mat * 2 + half) * a.SI) * 16;
        for (int i = 0; i < 4; i++) {
            const int r = rt * 16 + 4 * kq + i;
            dst[(size_t)r * 16 + n] = acc[i];
        }
    }
}

// ------------------------------------------------------------------ K2: routed gate/up
struct K2Args {
    const uint8_t *experts;
    size_t         expert_bytes, gate_off, up_off;
    const k3x_route *route;
    const uint16_t *xB;
    uint16_t      *actB;           // [slot][I/128][4][64][8]
    int            T, H, I;
    int            n_fin;          // shared-finalise workgroups
    const float   *shpart;         // [2][2][SI][16]
    uint16_t      *shB;
    int            SI;
};

__global__ void __launch_bounds__(NT) k2_gateup(K2Args a)
{
    __shared__ float lds[(NT / WAVE - 1) * 8 * WAVE];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;

    if ((int)blockIdx.x < a.n_fin) {
        // shared SwiGLU: sum the two K halves of gate and up, hi+lo columns
        const int f = blockIdx.x * NT + threadIdx.x;
        if (f >= a.SI * a.T) return;
        const int r = f % a.SI, tok = f / a.SI;
        const size_t hs = (size_t)a.SI * 16;
        const float *g = a.shpart, *u = a.shpart + 2 * hs;
        const size_t o = (size_t)r * 16 + 2 * tok;
        const float gv = (g[o] + g[o + 1]) + (g[hs + o] + g[hs + o + 1]);
        const float uv = (u[o] + u[o + 1]) + (u[hs + o] + u[hs + o + 1]);
        uint32_t hi, lo;
        split_bf16(swiglu(gv, uv), hi, lo);
        a.shB[bfrag_off(r, 2 * tok)] = (uint16_t)hi;
        a.shB[bfrag_off(r, 2 * tok + 1)] = (uint16_t)lo;
        return;
    }

    const int nTiles = a.I >> 4;
    const int b = blockIdx.x - a.n_fin;
    const int u = b / nTiles, rt = b % nTiles;
    if (u >= a.route->nu) return;
    const int e = a.route->uniq[u];
    const size_t tb = fp4_tile_bytes(a.H);
    const uint8_t *ex = a.experts + (size_t)e * a.expert_bytes;
    const uint8_t *tg = ex + a.gate_off + (size_t)rt * tb;
    const uint8_t *tu = ex + a.up_off + (size_t)rt * tb;
    const int nQ = a.H >> 7, nS = (nQ + 3) >> 2;
    const int s0 = (wave * nS) / 4, s1 = ((wave + 1) * nS) / 4;
    const int n = lane & 15;
    const bool bcol = n < 2 * a.T;
    f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
    for (int S = s0; S < s1; S++) {
        const int nq = min(4, nQ - 4 * S);
        const size_t so = (size_t)S * 4352;
        u32x4 cg[4], cu[4];
        for (int j = 0; j < 4; j++)
            if (j < nq) {
                cg[j] = ld16(tg + so + j * 1024 + lane * 16);
                cu[j] = ld16(tu + so + j * 1024 + lane * 16);
            }
        const uint32_t sg = *(const uint32_t *)(tg + so + nq * 1024 + lane * 4);
        const uint32_t su = *(const uint32_t *)(tu + so + nq * 1024 + lane * 4);
        for (int j = 0; j < 4; j++) {
            if (j >= nq) break;
            const uint32_t bg = (sg >> (8 * j)) & 255u, bu = (su >> (8 * j)) & 255u;
            for (int t = 0; t < 4; t++) {
                u32x4 bv = {0u, 0u, 0u, 0u};
                if (bcol) bv = ld16(a.xB + (((((size_t)(4 * S + j)) * 4 + t) * 64 + lane) << 3));
                dg = mfma(dq8(cg[j][t], bg), as_bf16x8(bv), dg);
                du = mfma(dq8(cu[j][t], bu), as_bf16x8(bv), du);
            }
        }
    }
    float acc[8] = {dg[0], dg[1], dg[2], dg[3], du[0], du[1], du[2], du[3]};
    wave_sum_lds<8>(acc, lds, wave, lane);
    if (wave != 0) return;
    // hi + lo columns, then SwiGLU and the routing weight
    const int kq = lane >> 4, tok = n >> 1;
    for (int i = 0; i < 4; i++) {
        const float g = acc[i] + __shfl_xor(acc[i], 1);
        const float v = acc[4 + i] + __shfl_xor(acc[4 + i], 1);
        if ((n & 1) == 0 && bcol) {
            const float w = a.route->wtok[u][tok];
            const float y = (w == 0.0f) ? 0.0f : w * swiglu(g, v);
            uint32_t hi, lo;
            split_bf16(y, hi, lo);
            const int r = rt * 16 + 4 * kq + i;
            uint16_t *dst = a.actB + (size_t)u * ((size_t)a.I * 16);
            dst[bfrag_off(r, 2 * tok)] = (uint16_t)hi;
            dst[bfrag_off(r, 2 * tok + 1)] = (uint16_t)lo;
        }
    }
}

// ------------------------------------------------------------------ K3: down + combine
struct K3Args {
    const uint8_t *experts;
    size_t         expert_bytes, down_off;
    const k3x_route *route;
    const uint16_t *actB, *shB, *sh_down;
    float         *out;
    const float   *resid;
    int            T, H, I, SI;
};

__global__ void __launch_bounds__(NT) k3_down(K3Args a)
{
    __shared__ float lds[(NT / WAVE - 1) * 4 * WAVE];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int rt = blockIdx.x;
    const int nu = a.route->nu;
    const int nQI = a.I >> 7, nSI = (nQI + 3) >> 2;
    const int nQS = a.SI >> 7;
    const int n_fp4 = nu * nSI, n_items = n_fp4 + nQS;
    const size_t tb = fp4_tile_bytes(a.I);
    const int n = lane & 15;
    const bool bcol = n < 2 * a.T;
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    for (int it = wave; it < n_items; it += NT / WAVE) {
        if (it < n_fp4) {
            const int u = it / nSI, S = it % nSI;
            const int e = a.route->uniq[u];
            const uint8_t *tile = a.experts + (size_t)e * a.expert_bytes + a.down_off +
                                  (size_t)rt * tb;
            const int nq = min(4, nQI - 4 * S);
            const size_t so = (size_t)S * 4352;
            u32x4 c[4];
            for (int j = 0; j < 4; j++)
                if (j < nq) c[j] = ld16(tile + so + j * 1024 + lane * 16);
            const uint32_t sc = *(const uint32_t *)(tile + so + nq * 1024 + lane * 4);
            const uint16_t *bsrc = a.actB + (size_t)u * ((size_t)a.I * 16);
            for (int j = 0; j < 4; j++) {
                if (j >= nq) break;
                const uint32_t sb = (sc >> (8 * j)) & 255u;
                for (int t = 0; t < 4; t++) {
                    u32x4 bv = {0u, 0u, 0u, 0u};
                    if (bcol) bv = ld16(bsrc + (((((size_t)(4 * S + j)) * 4 + t) * 64 + lane) << 3));
                    d = mfma(dq8(c[j][t], sb), as_bf16x8(bv), d);
                }
            }
        } else {
            const int q = it - n_fp4;
            const uint8_t *tile = (const uint8_t *)(a.sh_down + (size_t)rt * nQS * 2048);
            u32x4 av[4];
            for (int t = 0; t < 4; t++) av[t] = ld16(tile + (size_t)q * 4096 + t * 1024 + lane * 16);
            for (int t = 0; t < 4; t++) {
                u32x4 bv = {0u, 0u, 0u, 0u};
                if (bcol) bv = ld16(a.shB + ((((size_t)q * 4 + t) * 64 + lane) << 3));
                d = mfma(as_bf16x8(av[t]), as_bf16x8(bv), d);
            }
        }
    }
    float acc[4] = {d[0], d[1], d[2], d[3]};
    wave_sum_lds<4>(acc, lds, wave, lane);
    if (wave != 0) return;
    const int kq = lane >> 4, tok = n >> 1;
    for (int i = 0; i < 4; i++) {
        const float y = acc[i] + __shfl_xor(acc[i], 1);
        if ((n & 1) == 0 && bcol) {
            const int r = rt * 16 + 4 * kq + i;
            const size_t o = (size_t)tok * a.H + r;
            a.out[o] = a.resid ? a.resid[o] + y : y;
        }
    }
}

// ------------------------------------------------------------------ layout kernels
__global__ void tile_fp4_kernel(uint8_t *dst, const uint8_t *packed, const uint8_t *scales,
                                int R, int K)
{
    const int nQ = K >> 7, nS = (nQ + 3) >> 2, tiles = R >> 4;
    const size_t tb = fp4_tile_bytes(K);
    const long total = (long)tiles * nS * 64;
    for (long f = blockIdx.x * (long)blockDim.x + threadIdx.x; f < total;
         f += (long)gridDim.x * blockDim.x) {
        const int l = f & 63;
        const int S = (f >> 6) % nS;
        const int rt = (int)((f >> 6) / nS);
        const int m = l & 15, kq = l >> 4;
        const int row = rt * 16 + m;
        const int nq = min(4, nQ - 4 * S);
        uint8_t *so = dst + (size_t)rt * tb + (size_t)S * 4352;
        uint32_t sw = 0;
        for (int j = 0; j < nq; j++) {
            const int q = 4 * S + j;
            const uint8_t *src = packed + (size_t)row * (K / 2) + (size_t)(128 * q + 32 * kq) / 2;
            for (int b = 0; b < 16; b++) so[j * 1024 + l * 16 + b] = src[b];
            sw |= (uint32_t)scales[(size_t)row * (K / 32) + 4 * q + kq] << (8 * j);
        }
        *(uint32_t *)(so + nq * 1024 + l * 4) = sw;
    }
}

__global__ void untile_fp4_kernel(uint8_t *packed, uint8_t *scales, const uint8_t *src,
                                  int R, int K)
{
    const int nQ = K >> 7, nS = (nQ + 3) >> 2, tiles = R >> 4;
    const size_t tb = fp4_tile_bytes(K);
    const long total = (long)tiles * nS * 64;
    for (long f = blockIdx.x * (long)blockDim.x + threadIdx.x; f < total;
         f += (long)gridDim.x * blockDim.x) {
        const int l = f & 63;
        const int S = (f >> 6) % nS;
        const int rt = (int)((f >> 6) / nS);
        const int m = l & 15, kq = l >> 4;
        const int row = rt * 16 + m;
        const int nq = min(4, nQ - 4 * S);
        const uint8_t *so = src + (size_t)rt * tb + (size_t)S * 4352;
        const uint32_t sw = *(const uint32_t *)(so + nq * 1024 + l * 4);
        for (int j = 0; j < nq; j++) {
            const int q = 4 * S + j;
            uint8_t *d = packed + (size_t)row * (K / 2) + (size_t)(128 * q + 32 * kq) / 2;
            for (int b = 0; b < 16; b++) d[b] = so[j * 1024 + l * 16 + b];
            scales[(size_t)row * (K / 32) + 4 * q + kq] = (uint8_t)(sw >> (8 * j));
        }
    }
}

__global__ void tile_bf16_kernel(uint16_t *dst, const uint16_t *src, int R, int K)
{
    const int nQ = K >> 7;
    const long total = (long)(R >> 4) * nQ * 4 * 64;      // one 8-element run each
    for (long f = blockIdx.x * (long)blockDim.x + threadIdx.x; f < total;
         f += (long)gridDim.x * blockDim.x) {
        const int l = f & 63, t = (f >> 6) & 3;
        const long qt = f >> 8;
        const int q = qt % nQ, rt = (int)(qt / nQ);
        const int m = l & 15, kq = l >> 4;
        const uint16_t *s = src + (size_t)(rt * 16 + m) * K + 128 * q + 32 * kq + 8 * t;
        uint16_t *d = dst + (size_t)f * 8;
        for (int j = 0; j < 8; j++) d[j] = s[j];
    }
}

// splitmix64 finaliser and counter draw (the synthetic-layer rule, k3x_moe.h)
__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t draw(uint64_t key, uint64_t i)
{
    return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

// Synthetic expert matrix written straight into the tiled layout: code byte i of the
// row-major packed array is byte (i % 8) of draw(code_key, i / 8); scale byte i is
// lo + (draw(scale_key, i) >> 32) % (hi - lo + 1).
__global__ void synth_fp4_kernel(uint8_t *dst, int R, int K, uint64_t ck, uint64_t sk,
                                 int lo, int hi)
{
    const int nQ = K >> 7, nS = (nQ + 3) >> 2, tiles = R >> 4;
    const size_t tb = fp4_tile_bytes(K);
    const uint64_t span = (uint64_t)(hi - lo + 1);
    const long total = (long)tiles * nS * 64;
    for (long f = blockIdx.x * (long)blockDim.x + threadIdx.x; f < total;
         f += (long)gridDim.x * blockDim.x) {
        const int l = f & 63;
        const int S = (f >> 6) % nS;
        const int rt = (int)((f >> 6) / nS);
        const int m = l & 15, kq = l >> 4;
        const int row = rt * 16 + m;
        const int nq = min(4, nQ - 4 * S);
        uint8_t *so = dst + (size_t)rt * tb + (size_t)S * 4352;
        uint32_t sw = 0;
        for (int j = 0; j < nq; j++) {
            const int q = 4 * S + j;
            const uint64_t i0 = (uint64_t)row * (K / 2) + (uint64_t)(128 * q + 32 * kq) / 2;
            // i0 is a multiple of 16, so the 16 bytes are two whole draws
            const uint64_t d0 = draw(ck, i0 >> 3), d1 = draw(ck, (i0 >> 3) + 1);
            u32x4 v = {(uint32_t)d0, (uint32_t)(d0 >> 32), (uint32_t)d1, (uint32_t)(d1 >> 32)};
            *(u32x4 *)(so + j * 1024 + l * 16) = v;
            const uint64_t si = (uint64_t)row * (K / 32) + 4 * q + kq;
            sw |= (uint32_t)(lo + (int)((draw(sk, si) >> 32) % span)) << (8 * j);
        }
        *(uint32_t *)(so + nq * 1024 + l * 4) = sw;
    }
}

// ------------------------------------------------------------------ RMSNorm
__global__ void __launch_bounds__(NT) rmsnorm_kernel(float *y, const float *x, const float *w,
                                                      int n, float eps)
{
    __shared__ double red[NT / WAVE];
    const float *xr = x + (size_t)blockIdx.x * n;
    float *yr = y + (size_t)blockIdx.x * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += NT) ss += (double)xr[i] * (double)xr[i];
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / WAVE] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int i = 0; i < NT / WAVE; i++) tot += red[i];
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
    for (int i = threadIdx.x; i < n; i += NT) yr[i] = w[i] * xr[i] * inv;
}

// ------------------------------------------------------------------ launchers
static inline int hip_ok(hipError_t e) { return e == hipSuccess ? 0 : K3X_E_HIP; }
static inline int launch_ok(void) { return hip_ok(hipGetLastError()); }

static int grid_for(long total, int block)
{
    long g = (total + block - 1) / block;
    if (g < 1) g = 1;
    if (g > 65535L * 16) g = 65535L * 16;
    return (int)g;
}

extern "C" int k3x_dev_check(int device)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return K3X_E_NODEV;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) return K3X_E_NODEV;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) return K3X_E_NODEV;   // gfx950 only
    return 0;
}

extern "C" int k3x_dev_tile_fp4(uint8_t *dst, const uint8_t *packed, const uint8_t *scales,
                                int R, int K, void *stream)
{
    const long total = (long)(R >> 4) * (((K >> 7) + 3) >> 2) * 64;
    hipLaunchKernelGGL(tile_fp4_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       (hipStream_t)stream, dst, packed, scales, R, K);
    return launch_ok();
}

extern "C" int k3x_dev_untile_fp4(uint8_t *packed, uint8_t *scales, const uint8_t *src,
                                  int R, int K, void *stream)
{
    const long total = (long)(R >> 4) * (((K >> 7) + 3) >> 2) * 64;
    hipLaunchKernelGGL(untile_fp4_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       (hipStream_t)stream, packed, scales, src, R, K);
    return launch_ok();
}

extern "C" int k3x_dev_tile_bf16(uint16_t *dst, const uint16_t *src, int R, int K,
                                 void *stream)
{
    const long total = (long)(R >> 4) * (K >> 7) * 4 * 64;
    hipLaunchKernelGGL(tile_bf16_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       (hipStream_t)stream, dst, src, R, K);
    return launch_ok();
}

extern "C" int k3x_dev_synth_fp4(uint8_t *dst, int R, int K, uint64_t code_key,
                                 uint64_t scale_key, int lo, int hi, void *stream)
{
    const long total = (long)(R >> 4) * (((K >> 7) + 3) >> 2) * 64;
    hipLaunchKernelGGL(synth_fp4_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       (hipStream_t)stream, dst, R, K, code_key, scale_key, lo, hi);
    return launch_ok();
}

extern "C" int k3x_dev_rmsnorm(float *y, const float *x, const float *w, int n, int T,
                               float eps, void *stream)
{
    if (T <= 0) return 0;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(NT), 0, (hipStream_t)stream, y, x, w,
                       n, eps);
    return launch_ok();
}

static int record(k3x_moe_layer *L, int i, hipStream_t s)
{
    if (!L->timing) return 0;
    if (i >= 8) return 0;
    if (i + 1 > L->n_ev_used) L->n_ev_used = i + 1;
    return hip_ok(hipEventRecord((hipEvent_t)L->ev[i], s));
}

extern "C" int k3x_dev_decode(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                              int T, const float *resid, int *idx, float *wt, void *stream)
{
    const k3x_cfg *c = &L->cfg;
    hipStream_t s = (hipStream_t)stream;
    int rc;
    K1Args a1;
    a1.router = L->router; a1.bias = L->bias; a1.x = x; a1.x_bf16 = (x_dtype == K3X_BF16);
    a1.T = T; a1.H = c->hidden; a1.E = c->n_experts; a1.K = c->topk;
    a1.renorm = c->moe_renorm; a1.routed_scale = c->routed_scale;
    a1.score = L->score; a1.choice = L->choice; a1.idx = L->idx; a1.wt = L->wt;
    a1.uidx = idx; a1.uwt = wt; a1.counter = L->counter; a1.route = L->route; a1.xB = L->xB;
    a1.n_rwg = (c->n_experts + NT / WAVE - 1) / (NT / WAVE);
    a1.sh_gate = L->sh_gate; a1.sh_up = L->sh_up; a1.SI = L->SI; a1.shpart = L->shpart;
    const int n_sh = L->SI > 0 ? 4 * (L->SI / 16) : 0;
    if ((rc = record(L, 0, s))) return rc;
    hipLaunchKernelGGL(k1_router_shared, dim3(a1.n_rwg + n_sh), dim3(NT), 0, s, a1);
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, 1, s))) return rc;

    K2Args a2;
    a2.experts = L->experts; a2.expert_bytes = L->expert_bytes;
    a2.gate_off = L->gate_off; a2.up_off = L->up_off; a2.route = L->route;
    a2.xB = L->xB; a2.actB = L->actB; a2.T = T; a2.H = c->hidden; a2.I = c->moe_inter;
    a2.n_fin = L->SI > 0 ? (L->SI * T + NT - 1) / NT : 0;
    a2.shpart = L->shpart; a2.shB = L->shB; a2.SI = L->SI;
    const int n_rt = T * c->topk * (c->moe_inter / 16);
    hipLaunchKernelGGL(k2_gateup, dim3(a2.n_fin + n_rt), dim3(NT), 0, s, a2);
    if ((rc = launch_ok())) return rc;
    if ((rc = record(L, 2, s))) return rc;

    K3Args a3;
    a3.experts = L->experts; a3.expert_bytes = L->expert_bytes; a3.down_off = L->down_off;
    a3.route = L->route; a3.actB = L->actB; a3.shB = L->shB; a3.sh_down = L->sh_down;
    a3.out = out; a3.resid = resid; a3.T = T; a3.H = c->hidden; a3.I = c->moe_inter;
    a3.SI = L->SI;
    hipLaunchKernelGGL(k3_down, dim3(c->hidden / 16), dim3(NT), 0, s, a3);
    if ((rc = launch_ok())) return rc;
    return record(L, 3, s);
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
