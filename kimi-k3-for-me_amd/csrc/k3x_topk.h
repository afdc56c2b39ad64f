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

// The choice value of a key (the inverse of choice_key on the values it keeps).
__device__ __forceinline__ float key_choice(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ int lanes_below(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

template <int CP>
__device__ __forceinline__ float bload_f32(rsrc_t r, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP));
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
// indices) as 64-bit words key << 32 | ~index, loaded once (CP: the loads' cache
// policy); in that order the entries still remaining after a round's winner W are exactly
// those below W.  A round: each lane's largest word below the previous winner, the wave
// maximum of their keys, the lowest lane holding it (a ballot: its word has the lowest
// index among equal keys), and that lane's index and score read as wave-uniform values.
// Branch-free.  NaN and -inf are never taken; a round with nothing left gives index 0,
// weight 0.  Weights are the unbiased scores, renormalised through a double sum in slot
// order and a float reciprocal, then scaled (:1710-1716).  Results in s_idx/s_w, and
// lane j's (slot j's) in out_e/out_w when given, and the last round's choice (the K-th
// largest; -inf when fewer than K were selectable) in out_ck.  This form takes the
// choices and scores in registers (lane l: experts l*NE + c); wave_topk below loads them
// first.
template <int NE>
__device__ void wave_topk_vals(const float (&cv)[NE], const float (&sc)[NE], int E, int K,
                               int renorm, float routed_scale, int *s_idx, float *s_w,
                               int lane, int *out_e = nullptr, float *out_w = nullptr,
                               float *out_ck = nullptr)
{
    uint64_t pk[NE];
#pragma unroll
    for (int c = 0; c < NE; c++) {
        const int e = lane * NE + c;
        const uint32_t k = choice_key(cv[c]);
        pk[c] = (e < E && k > K_NEG_INF) ? ((uint64_t)k << 32) | (uint64_t)(~(uint32_t)e) : 0ull;
    }
    uint64_t prev = ~0ull;        // the previous round's winner (none yet: above all)
    int mine_e = 0;               // lane j keeps round j's expert and score
    float mine_s = 0.0f;
    float ck = -__builtin_inff(); // the last round's choice (-inf when a round finds none:
                                  // the later rounds find none either)
    for (int j = 0; j < K; j++) {
        uint64_t best = 0ull;
        float bs = 0.0f;
#pragma unroll
        for (int c = 0; c < NE; c++) {
            const uint64_t v = pk[c] < prev ? pk[c] : 0ull;
            const bool gt = v > best;
            best = gt ? v : best;
            bs = gt ? sc[c] : bs;
        }
        const uint32_t bk = (uint32_t)(best >> 32);
        const uint32_t m = wave_max_u32(bk);
        const uint64_t holders = __ballot(m != 0u && bk == m);
        if (holders == 0ull) {                  // nothing left (uniform)
            if (lane == j) { mine_e = 0; mine_s = 0.0f; }
            ck = -__builtin_inff();
            continue;
        }
        const int w = (int)__builtin_ctzll(holders);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)best, w);
        const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), w));
        prev = ((uint64_t)m << 32) | lo;
        if (lane == j) { mine_e = (int)~lo; mine_s = ws; }
        ck = key_choice(m);
    }
    if (out_ck) *out_ck = ck;
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
    if (out_e) { *out_e = mine_e; *out_w = wgt; }
}

template <int NE, int CP>
__device__ void wave_topk(rsrc_t cr, rsrc_t sr, uint32_t row_off, int E, int K, int renorm,
                          float routed_scale, int *s_idx, float *s_w, int lane,
                          int *out_e = nullptr, float *out_w = nullptr,
                          float *out_ck = nullptr)
{
    float sc[NE], cv[NE];
#pragma unroll
    for (int c = 0; c < NE; c++) {
        const int e = lane * NE + c;
        const uint32_t o = e < E ? row_off + 4u * (uint32_t)e : K3X_OOB;
        cv[c] = bload_f32<CP>(cr, o);
        sc[c] = bload_f32<CP>(sr, o);
    }
    SCHED_FENCE();      // both rows' loads in flight together: one memory round trip
    wave_topk_vals<NE>(cv, sc, E, K, renorm, routed_scale, s_idx, s_w, lane, out_e, out_w,
                       out_ck);
}

// wave_topk for N tokens of one wave together (tokens past ntok load nothing and store
// nothing): every token's rows are loaded at once (one memory round trip for all), and
// each round runs for every token before the next, so that one token's wave maximum
// fills the other's latency.  Per token, the same operations in the same order as
// wave_topk, so the same results; out_ck[r] is token r's K-th choice.
template <int NE, int CP, int N>
__device__ void wave_topk_n(rsrc_t cr, rsrc_t sr, const uint32_t (&row_off)[N], int ntok, int E,
                            int K, int renorm, float routed_scale, int *const (&s_idx)[N],
                            float *const (&s_w)[N], int lane, float (&out_ck)[N])
{
    uint64_t pk[N][NE];
    float sc[N][NE], cv[N][NE];
#pragma unroll
    for (int r = 0; r < N; r++)
#pragma unroll
        for (int c = 0; c < NE; c++) {
            const int e = lane * NE + c;
            const uint32_t o = (e < E && r < ntok) ? row_off[r] + 4u * (uint32_t)e : K3X_OOB;
            cv[r][c] = bload_f32<CP>(cr, o);
            sc[r][c] = bload_f32<CP>(sr, o);
        }
    SCHED_FENCE();
#pragma unroll
    for (int r = 0; r < N; r++)
#pragma unroll
        for (int c = 0; c < NE; c++) {
            const int e = lane * NE + c;
            const uint32_t k = choice_key(cv[r][c]);
            pk[r][c] = (e < E && k > K_NEG_INF) ? ((uint64_t)k << 32) | (uint64_t)(~(uint32_t)e) : 0ull;
        }
    uint64_t prev[N];
    int mine_e[N];
    float mine_s[N], ck[N];
#pragma unroll
    for (int r = 0; r < N; r++) {
        prev[r] = ~0ull;
        mine_e[r] = 0;
        mine_s[r] = 0.0f;
        ck[r] = -__builtin_inff();
    }
    for (int j = 0; j < K; j++) {
#pragma unroll
        for (int r = 0; r < N; r++) {
            uint64_t best = 0ull;
            float bs = 0.0f;
#pragma unroll
            for (int c = 0; c < NE; c++) {
                const uint64_t v = pk[r][c] < prev[r] ? pk[r][c] : 0ull;
                const bool gt = v > best;
                best = gt ? v : best;
                bs = gt ? sc[r][c] : bs;
            }
            const uint32_t bk = (uint32_t)(best >> 32);
            const uint32_t m = wave_max_u32(bk);
            const uint64_t holders = __ballot(m != 0u && bk == m);
            if (holders == 0ull) {                  // nothing left (uniform)
                if (lane == j) { mine_e[r] = 0; mine_s[r] = 0.0f; }
                ck[r] = -__builtin_inff();
                continue;
            }
            const int w = (int)__builtin_ctzll(holders);
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)best, w);
            const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bs), w));
            prev[r] = ((uint64_t)m << 32) | lo;
            if (lane == j) { mine_e[r] = (int)~lo; mine_s[r] = ws; }
            ck[r] = key_choice(m);
        }
    }
#pragma unroll
    for (int r = 0; r < N; r++) out_ck[r] = ck[r];
#pragma unroll
    for (int r = 0; r < N; r++) {
        float wgt = mine_s[r];
        if (renorm && K > 1) {
            double sum = 0.0;
            for (int j = 0; j < K; j++)
                sum += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine_s[r]), j));
            const float inv = (float)(1.0 / (sum + 1e-20));
            wgt *= inv;
        }
        wgt *= routed_scale;
        if (r < ntok && lane < K) {
            s_idx[r][lane] = mine_e[r];
            s_w[r][lane] = wgt;
        }
    }
}

#endif
