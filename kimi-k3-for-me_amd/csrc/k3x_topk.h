// k3x_topk.h - one token's top-k selection by one wave, shared by the decode and the
// prefill kernels (the reference's repeated maximum, k3_ops.c:1700-1716).
#ifndef K3X_TOPK_H
#define K3X_TOPK_H

#include "k3x_device.h"

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

// Maximum of an unsigned value over the wave: DPP steps within quads and rows, then row
// broadcasts across rows (lane 63 ends with the total), then a read of lane 63.  Lanes
// that a step does not write take 0, the identity.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_max(uint32_t v)
{
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
    return o > v ? o : v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = dpp_max<0xB1, 0xF>(v);      // quad_perm [1,0,3,2]
    v = dpp_max<0x4E, 0xF>(v);      // quad_perm [2,3,0,1]
    v = dpp_max<0x124, 0xF>(v);     // row_ror:4
    v = dpp_max<0x128, 0xF>(v);     // row_ror:8: every lane holds its row's maximum
    v = dpp_max<0x142, 0xA>(v);     // row_bcast:15 into rows 1 and 3
    v = dpp_max<0x143, 0xC>(v);     // row_bcast:31 into rows 2 and 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// One token's top-k by one wave, the reference's repeated maximum (k3_ops.c:1700-1708):
// K rounds, each taking the largest remaining choice with the lower index first among
// equal values.  Lane l holds experts l*NE .. l*NE+NE-1 (so a lower lane holds lower
// indices) with their choice keys and scores, loaded once.  A round: each lane's best key
// (the lowest of its indices among equals), the wave maximum, and the lowest lane holding
// it by a ballot; that lane's expert and score are read as wave-uniform values and its key
// cleared.  NaN and -inf are never taken; a round with nothing left gives index 0, weight
// 0.  Weights are the unbiased scores, renormalised through a double sum in slot order and
// a float reciprocal, then scaled (:1710-1716).  Results in s_idx/s_w (K entries).
template <int NE>
__device__ void wave_topk(rsrc_t cr, rsrc_t sr, uint32_t row_off, int E, int K, int renorm,
                          float routed_scale, int *s_idx, float *s_w, int lane)
{
    uint32_t key[NE];
    float sc[NE];
#pragma unroll
    for (int c = 0; c < NE; c++) {
        const int e = lane * NE + c;
        const uint32_t o = e < E ? row_off + 4u * (uint32_t)e : K3X_OOB;
        const float v = bload_f32(cr, o);
        sc[c] = bload_f32(sr, o);
        const uint32_t k = choice_key(v);
        key[c] = (e < E && k > K_NEG_INF) ? k : 0u;
    }
    int mine_e = 0;               // lane j keeps round j's expert and score
    float mine_s = 0.0f;
    for (int j = 0; j < K; j++) {
        uint32_t bk = key[0];
        int bc = 0;
#pragma unroll
        for (int c = 1; c < NE; c++)
            if (key[c] > bk) { bk = key[c]; bc = c; }
        const uint32_t m = wave_max_u32(bk);
        const uint64_t holders = __ballot(m != 0u && bk == m);
        if (holders == 0ull) {                  // nothing left (uniform)
            if (lane == j) { mine_e = 0; mine_s = 0.0f; }
            continue;
        }
        const int w = (int)__builtin_ctzll(holders);
        float bs = sc[0];
#pragma unroll
        for (int c = 1; c < NE; c++)
            if (c == bc) bs = sc[c];
        const int wc = __builtin_amdgcn_readlane(bc, w);
        const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), w));
        if (lane == w) {
#pragma unroll
            for (int c = 0; c < NE; c++)
                if (c == bc) key[c] = 0u;
        }
        if (lane == j) { mine_e = w * NE + wc; mine_s = ws; }
    }
    float wgt = mine_s;
    if (renorm && K > 1) {
        double sum = 0.0;
        for (int j = 0; j < K; j++)
            sum += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine_s), j));
        const float inv = (float)(1.0 / (sum + 1e-20));
        wgt *= inv;
    }
    wgt *= routed_scale;
    if (lane < K) {
        s_idx[lane] = mine_e;
        s_w[lane] = wgt;
    }
}

#endif
