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

// One token's top-k by one wave, equal to the reference's repeated maximum
// (k3_ops.c:1700-1708): the K largest choices in descending order, the lower index first
// among equal values, NaN and -inf never taken (a pick with nothing left gives index 0,
// weight 0).  A 32-step bitwise search with ballot counts finds the k-th largest key;
// the k selected are then ranked.  Weights are the unbiased scores, renormalised through
// a double sum and a float reciprocal, then scaled (:1710-1716).  Results in s_idx/s_w.
// NE: 64-expert chunks held per lane.
template <int NE>
__device__ void wave_topk(rsrc_t cr, rsrc_t sr, uint32_t row_off, int E, int K, int renorm,
                          float routed_scale, int *s_idx, float *s_w, uint64_t *s_key,
                          int *s_e, float *s_sc, int lane)
{
    uint32_t key[NE];
    float sco[NE];
#pragma unroll
    for (int c = 0; c < NE; c++) {
        const int e = lane + WAVE * c;
        const uint32_t off = row_off + 4u * (uint32_t)e;
        const float v = bload_f32(cr, e < E ? off : K3X_OOB);
        sco[c] = bload_f32(sr, e < E ? off : K3X_OOB);
        key[c] = e < E ? choice_key(v) : 0u;
    }
    int nvalid = 0;
#pragma unroll
    for (int c = 0; c < NE; c++) nvalid += __popcll(__ballot(key[c] > K_NEG_INF));
    const int ke = min(K, nvalid);
    uint32_t tau = 0xFFFFFFFFu;
    if (ke > 0) {
        tau = 0u;
        for (int b = 31; b >= 0; b--) {
            const uint32_t cand = tau | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int c = 0; c < NE; c++) cnt += __popcll(__ballot(key[c] >= cand));
            if (cnt >= ke) tau = cand;
        }
    }
    int ngt = 0;
#pragma unroll
    for (int c = 0; c < NE; c++) ngt += __popcll(__ballot(key[c] > tau));
    int need = ke - ngt;                    // ties at tau, taken in ascending index
    int base = 0;
#pragma unroll
    for (int c = 0; c < NE; c++) {
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

#endif
