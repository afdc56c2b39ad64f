// k3x_prefill.hip - the prefill path of the MoE block (more than 8 tokens per call):
//
//   pf_split    activations to bf16 hi/lo rows (the GEMMs' B source); clears the histogram
//   pf_router   router logits of every (token, expert) in double, one sequential chain per
//               pair in the reference's order (k3_router, k3_ops.c:1666-1688), so they
//               are the reference's logits bit for bit; sigmoid, + bias (:1691-1692)
//   pf_topk     each token's top-k by one wave (:1700-1716) and the per-expert histogram
//   pf_scan     per-expert offsets (prefix sum) and the GEMM tile lists
//   pf_scatter  each (token, slot) to its row in its expert's segment
//   pf_gather   the routed input's planes, rows in that order
//   pf_gemm32   grouped GEMMs: gate/up of every expert segment with SwiGLU and the
//               routing weight (k3_matmul_mxfp4 :3323-3776, k3_situ_glu :148-161), then
//               down (pf_gemm_mx in the MXFP8 mode)
//   pf_dense    the shared expert's bf16 products (:1848-1860), the latent projections
//               and the trunk matrices
//   pf_combine  per token, the K expert rows summed in top-k order (:1941-1942), plus
//               the shared row (:1951), plus an optional residual
//
// The GEMMs run on v_mfma_f32_32x32x16_bf16 with MXFP4 weights dequantised exactly in
// registers; the activations are bf16 hi + lo pairs (hi only when the input is bf16,
// whose lo part is zero), so products are exact and only the fp32 accumulation rounds.
#include "k3x_device.h"
#include "k3x_topk.h"

#include <stdio.h>
#include <string.h>

#include <mutex>

#define PF_NT 256

// ------------------------------------------------------------------ split
// Activation planes, the GEMMs' B source: x [T][H] (bf16 or fp32, rows ldx elements
// apart) -> xg [2][H/8][T][8] bf16, plane 0 the hi parts, plane 1 the lo parts, each
// k-group of 8 elements token-major, so that one k-group of consecutive rows is
// contiguous.  For bf16 rows the lo parts are zero and no GEMM reads plane 1 (they take
// one column per token, HL = 1): it is not written.  A workgroup transposes a tile of
// SP_T tokens by SP_G k-groups through LDS, so that both its reads (along the rows) and
// its writes (along the tokens of a k-group) are contiguous.  Block 0 also clears the
// expert histogram (when given).
#define SP_T 32
#define SP_G 32

static inline unsigned pf_split_grid(int T, int H)
{
    return (unsigned)(((T + SP_T - 1) / SP_T) * (((H >> 3) + SP_G - 1) / SP_G));
}

__global__ void __launch_bounds__(PF_NT) pf_split(const void *x, int x_bf16, int T, int H,
                                                  int ldx, uint16_t *xg, int *counts, int E)
{
    __shared__ u32x4 sh[2][SP_G][SP_T + 1];
    if (blockIdx.x == 0 && counts)
        for (int e = threadIdx.x; e < E; e += PF_NT) counts[e] = 0;
    const int G8 = H >> 3, ntg = (G8 + SP_G - 1) / SP_G;
    const int t0 = (blockIdx.x / ntg) * SP_T, g0 = (blockIdx.x % ntg) * SP_G;
#pragma unroll
    for (int j = 0; j < SP_T * SP_G / PF_NT; j++) {
        const int i = j * PF_NT + threadIdx.x, r = i / SP_G, g = i % SP_G;
        const int t = t0 + r, gi = g0 + g;
        u32x4 h = {0u, 0u, 0u, 0u}, l = {0u, 0u, 0u, 0u};
        const size_t src = (size_t)t * ldx + (size_t)gi * 8;
        if (t < T && gi < G8 && x_bf16) {
            h = *(const u32x4 *)((const uint16_t *)x + src);        // bf16: hi = x, lo = 0
        } else if (t < T && gi < G8) {
            float v[8];
            load_x8(x, 0, src, v);
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int k = 0; k < 8; k++) split_bf16(v[k], hi[k], lo[k]);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                h[k] = hi[2 * k] | (hi[2 * k + 1] << 16);
                l[k] = lo[2 * k] | (lo[2 * k + 1] << 16);
            }
        }
        sh[0][g][r] = h;
        sh[1][g][r] = l;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SP_T * SP_G / PF_NT; j++) {
        const int i = j * PF_NT + threadIdx.x, g = i / SP_T, r = i % SP_T;
        const int t = t0 + r, gi = g0 + g;
        if (t < T && gi < G8) {
            *(u32x4 *)(xg + ((size_t)gi * T + t) * 8) = sh[0][g][r];
            if (!x_bf16) *(u32x4 *)(xg + ((size_t)(G8 + gi) * T + t) * 8) = sh[1][g][r];
        }
    }
}

// ------------------------------------------------------------------ gather
// The routed experts' input planes in permuted order: xg[h][g][p][8] = part h of
// x[rowmap[p]][8g .. 8g+7], the layout pf_split writes, for TK rows.  A lane owns one
// permuted row p (consecutive lanes, consecutive p: each store of a k-group is 1 KB
// contiguous per wave) and walks PG_GS k-groups of its source row, eight at a time: the
// eight 16-byte pieces of a row's consecutive k-groups (32-byte for fp32 rows) share
// cache lines, so the walk reads every line once.  The row map is read once per lane
// and no LDS transpose is needed.
#define PG_GS 56

static inline unsigned pf_gather_grid(int TK, int H)
{
    const int ns = ((H >> 3) + PG_GS - 1) / PG_GS;
    return (unsigned)((((TK + WAVE - 1) / WAVE) * ns + PF_NT / WAVE - 1) / (PF_NT / WAVE));
}

__global__ void __launch_bounds__(PF_NT) pf_gather(const void *x, int x_bf16, int TK, int H,
                                                   int ldx, uint16_t *xg, const int *rowmap)
{
    const int G8 = H >> 3, ns = (G8 + PG_GS - 1) / PG_GS;
    const int w = blockIdx.x * (PF_NT / WAVE) + (int)(threadIdx.x / WAVE);
    const int pb = w / ns, sl = w % ns;
    const int p = pb * WAVE + (int)(threadIdx.x % WAVE);
    if (p >= TK) return;
    const size_t row = (size_t)rowmap[p] * ldx;
    const int g0 = sl * PG_GS, g1 = min(G8, g0 + PG_GS);
    const size_t plane = (size_t)G8 * TK * 8;
    // G8 is a multiple of 16 (H of 128), so every step of 8 k-groups is whole
    for (int g = g0; g < g1; g += 8) {
        if (x_bf16) {
            u32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = ld16((const uint16_t *)x + row + (size_t)(g + j) * 8);
#pragma unroll
            for (int j = 0; j < 8; j++) *(u32x4 *)(xg + ((size_t)(g + j) * TK + p) * 8) = v[j];
        } else {
            f32x4 v[8][2];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float *src = (const float *)x + row + (size_t)(g + j) * 8;
                v[j][0] = *(const f32x4 *)src;
                v[j][1] = *(const f32x4 *)(src + 4);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t hi[8], lo[8];
#pragma unroll
                for (int k = 0; k < 8; k++) split_bf16(v[j][k >> 2][k & 3], hi[k], lo[k]);
                u32x4 h, l;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    h[k] = hi[2 * k] | (hi[2 * k + 1] << 16);
                    l[k] = lo[2 * k] | (lo[2 * k + 1] << 16);
                }
                const size_t o = ((size_t)(g + j) * TK + p) * 8;
                *(u32x4 *)(xg + o) = h;
                *(u32x4 *)(xg + plane + o) = l;
            }
        }
    }
}

// ------------------------------------------------------------------ router
// Logits of every (token, expert) pair in double, each one sequential chain over
// i = 0 .. H-1 in the reference's order (k3_router, k3_ops.c:1666-1688), on the FP64
// matrix cores.  v_mfma_f64_16x16x4f64 adds its four k terms to each output one after
// another, k in lane-group order, each a fused multiply-add (held bitwise against a
// sequential fma chain on wide-exponent cancelling data); a product of two floats is
// exact in double, so the chain equals the reference's fma-free loop bit for bit.  A
// chain cannot be split over k, so the parallelism is the number of 16x16 output tiles:
// a workgroup takes 48 experts x 64 tokens as twelve waves of one tile each (three waves
// a SIMD, whose independent chains keep its matrix core fed; 12 tiles per CU at 2048
// tokens x 384 experts).  K is staged 64 at a time in LDS as float, element k of a chunk
// at (k % 4) * 16 + k / 4 of its row, so that one 16-byte read gives a lane its operands
// of four consecutive MFMA steps; the next chunk is fetched into registers during the
// current one.  Workgroups are dealt expert block fastest, so that with 8 expert blocks
// each XCD keeps one block's router rows in L2.
#define RM_E  48
#define RM_T  64
#define RM_KC 64
#define RM_S  (RM_KC + 4)
#define RM_NT 768

struct PfRouterArgs {
    const void  *x;
    int          x_bf16;
    const float *W, *bias;
    int          T, H, E;
    float       *score, *choice;
};

typedef double f64x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(RM_NT) pf_router(PfRouterArgs a)
{
    __shared__ __attribute__((aligned(16))) float lds[2][RM_E + RM_T][RM_S];
    const int nEB = (a.E + RM_E - 1) / RM_E;
    const int e0 = (blockIdx.x % nEB) * RM_E, t0 = (blockIdx.x / nEB) * RM_T;
    const int tid = threadIdx.x, wave = tid / WAVE, r = tid % 16, g = (tid % WAVE) / 16;
    const int et = wave % 3, tt = wave / 3;          // this wave's expert and token tiles
    // staging roles: W row tid/16 (48 rows), k 4*(tid%16) .. +3; x (threads below 512) row
    // tid/8, k 8*(tid%8) .. +7
    const int wk = 4 * (tid % 16), xk = 8 * (tid % 8);
    const bool xst = tid < RM_T * 8;
    f32x4 wv;
    float xv[8];
    auto fetch = [&](int k0) AI {
        const int e = e0 + tid / 16;
        wv = e < a.E ? *(const f32x4 *)(a.W + (size_t)e * a.H + k0 + wk) : (f32x4){0.f, 0.f, 0.f, 0.f};
        if (xst) {
            const int t = t0 + tid / 8;
            if (t < a.T) load_x8(a.x, a.x_bf16, (size_t)t * a.H + k0 + xk, xv);
            else
#pragma unroll
                for (int q = 0; q < 8; q++) xv[q] = 0.f;
        }
    };
    auto stage = [&](int b) AI {
#pragma unroll
        for (int q = 0; q < 4; q++) lds[b][tid / 16][q * 16 + tid % 16] = wv[q];
        if (xst)
#pragma unroll
            for (int q = 0; q < 8; q++)
                lds[b][RM_E + tid / 8][(q % 4) * 16 + xk / 4 + q / 4] = xv[q];
    };
    f64x4 acc = {0.0, 0.0, 0.0, 0.0};
    fetch(0);
    stage(0);
    __syncthreads();
    const int nk = a.H / RM_KC;
    for (int kc = 0; kc < nk; kc++) {
        const int b = kc & 1;
        if (kc + 1 < nk) fetch((kc + 1) * RM_KC);
#pragma unroll
        for (int j0 = 0; j0 < RM_KC / 4; j0 += 4) {
            const f32x4 xq = *(const f32x4 *)&lds[b][RM_E + 16 * tt + r][g * 16 + j0];
            const f32x4 wq = *(const f32x4 *)&lds[b][16 * et + r][g * 16 + j0];
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64((double)wq[jj], (double)xq[jj], acc, 0, 0, 0);
        }
        if (kc + 1 < nk) stage(b ^ 1);
        __syncthreads();
    }
    // element i of lane (r, g): expert 16 et + g + 4i, token 16 tt + r
    const int t = t0 + 16 * tt + r;
    if (t >= a.T) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = e0 + 16 * et + g + 4 * i;
        if (e < a.E) {
            const float sc = sigmoid_ref((float)acc[i]);
            a.score[(size_t)t * a.E + e] = sc;
            a.choice[(size_t)t * a.E + e] = sc + a.bias[e];
        }
    }
}

// ------------------------------------------------------------------ top-k
struct PfTopkArgs {
    const float *score, *choice;
    int          T, E, K, renorm;
    float        routed_scale;
    int         *idx;   float *wt;       // [T][K]
    int         *uidx;  float *uwt;      // optional caller copies
    int         *counts;                 // [E] histogram
};

// One wave per token, TK_W tokens a workgroup.  The per-expert histogram is counted in LDS
// first and added to the global counts once per workgroup and expert: a device-scope
// atomic per (token, slot) serialised on the busiest experts' counters (the Zipf chunk's
// first expert takes every token).
#define TK_W 8
template <int NE>
__global__ void __launch_bounds__(TK_W * WAVE) pf_topk(PfTopkArgs a)
{
    __shared__ int      s_idx[TK_W][K3X_MAX_TOPK];
    __shared__ float    s_w[TK_W][K3X_MAX_TOPK];
    __shared__ int      hist[1024];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int t = blockIdx.x * TK_W + wave;
    if (a.counts)
        for (int e = threadIdx.x; e < a.E; e += TK_W * WAVE) hist[e] = 0;
    __syncthreads();
    if (t < a.T) {                                       // uniform over the wave
        const rsrc_t cr = make_rsrc(a.choice, (uint32_t)((size_t)a.T * a.E * 4));
        const rsrc_t sr = make_rsrc(a.score, (uint32_t)((size_t)a.T * a.E * 4));
        wave_topk<NE, 0>(cr, sr, (uint32_t)((size_t)t * a.E * 4), a.E, a.K, a.renorm,
                         a.routed_scale, s_idx[wave], s_w[wave], lane);
        __builtin_amdgcn_wave_barrier();
        if (lane < a.K) {
            const size_t o = (size_t)t * a.K + lane;
            const int e = s_idx[wave][lane];
            a.idx[o] = e;
            a.wt[o] = s_w[wave][lane];
            if (a.uidx) { a.uidx[o] = e; a.uwt[o] = s_w[wave][lane]; }
            if (a.counts) atomicAdd(&hist[e], 1);
        }
    }
    if (!a.counts) return;                               // uniform
    __syncthreads();
    for (int e = threadIdx.x; e < a.E; e += TK_W * WAVE)
        if (hist[e]) atomicAdd(&a.counts[e], hist[e]);
}

// ------------------------------------------------------------------ scan
// One workgroup of 1024 threads (E <= 1024): offsets[e] = sum of counts below e, and the
// tile bases of the two routed GEMMs.  Each GEMM has two tile classes: an expert with at
// most tpb_s tokens takes nrb_s tiles of tpb_s columns (one column block), a larger one
// nrb_b x ceil(count/tpb_b) tiles of tpb_b columns.  tb[0..E] are the small class's bases
// (tb[E] = its tile count), tb[E+1 .. 2E+1] the large class's.  Cursors cleared.  Five
// inclusive scans, one element per thread (shuffles within each wave, then the waves'
// totals).
struct PfScanArgs {
    const int *counts;
    int        E;
    int       *offsets, *cursor;
    int       *tb[2];                   // gate/up, down
    int        tpb_s[2], tpb_b[2];      // columns of a tile, small and large class
    int        nrb_s[2], nrb_b[2];      // row blocks, small and large class
};

__global__ void __launch_bounds__(1024) pf_scan(PfScanArgs a)
{
    __shared__ int wsum[5][16], woff[5][16];
    const int e = threadIdx.x, E = a.E, wave = e / WAVE, lane = e % WAVE;
    const int c = e < E ? a.counts[e] : 0;
    int v[5];
    v[0] = c;
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const bool big = c > a.tpb_s[m];
        v[1 + 2 * m] = big ? 0 : a.nrb_s[m] * ((c + a.tpb_s[m] - 1) / a.tpb_s[m]);
        v[2 + 2 * m] = big ? a.nrb_b[m] * ((c + a.tpb_b[m] - 1) / a.tpb_b[m]) : 0;
    }
    if (e < E) a.cursor[e] = 0;
    // inclusive sums: within each wave by shuffles, then the waves' totals (wave 0)
    int in[5];
#pragma unroll
    for (int i = 0; i < 5; i++) {
        in[i] = v[i];
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const int t = __shfl_up(in[i], o);
            if (lane >= o) in[i] += t;
        }
        if (lane == WAVE - 1) wsum[i][wave] = in[i];
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
#pragma unroll
        for (int i = 0; i < 5; i++) {
            int x = wsum[i][lane], inc = x;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const int t = __shfl_up(inc, o, 16);
                if (lane >= o) inc += t;
            }
            woff[i][lane] = inc - x;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 5; i++) in[i] += woff[i][wave];
    // the exclusive value of e is its inclusive sum less its own
    if (e < E) {
        a.offsets[e] = in[0] - v[0];
#pragma unroll
        for (int m = 0; m < 2; m++) {
            a.tb[m][e] = in[1 + 2 * m] - v[1 + 2 * m];
            a.tb[m][E + 1 + e] = in[2 + 2 * m] - v[2 + 2 * m];
        }
    }
    if (e == E - 1) {
        a.offsets[E] = in[0];
#pragma unroll
        for (int m = 0; m < 2; m++) {
            a.tb[m][E] = in[1 + 2 * m];
            a.tb[m][2 * E + 1] = in[2 + 2 * m];
        }
    }
}

// ------------------------------------------------------------------ scatter
// Each (token, slot) to a row of its expert's segment: a workgroup ranks its items per
// expert in LDS, reserves each expert's run with one device-scope atomic, and places its
// items in that run (the order within a segment is free: every row's products are its
// own, and the combine finds each row through pos_of).
__global__ void __launch_bounds__(PF_NT) pf_scatter(const int *idx, const float *wt, int TK, int K,
                                                    int E, const int *offsets, int *cursor,
                                                    int *perm_tok, float *perm_w, int *pos_of)
{
    __shared__ int cnt[1024], base[1024];
    for (int e = threadIdx.x; e < E; e += PF_NT) cnt[e] = 0;
    __syncthreads();
    const int i = blockIdx.x * PF_NT + threadIdx.x;
    const int e = i < TK ? idx[i] : 0;
    const int r = i < TK ? atomicAdd(&cnt[e], 1) : 0;
    __syncthreads();
    for (int f = threadIdx.x; f < E; f += PF_NT)
        if (cnt[f]) base[f] = offsets[f] + atomicAdd(&cursor[f], cnt[f]);
    __syncthreads();
    if (i >= TK) return;
    const int p = base[e] + r;
    perm_tok[p] = i / K;
    perm_w[p] = wt[i];
    pos_of[i] = p;
}

// ------------------------------------------------------------------ tile tables
// One descriptor per GEMM tile: {group, row block, first permuted row, tokens}; expert e
// owns tiles tb[e] .. of its class's list (the small class's list first, then the large
// class's from desc + tb[E]), row blocks outer, column blocks inner.
__global__ void __launch_bounds__(PF_NT) pf_tiles(const int *counts, const int *offsets,
                                                  PfScanArgs a, int4 *desc_gu, int4 *desc_dn)
{
    const int e = blockIdx.x, c = counts[e], off = offsets[e], E = a.E;
    for (int m = 0; m < 2; m++) {
        const bool big = c > a.tpb_s[m];
        const int tpb = big ? a.tpb_b[m] : a.tpb_s[m], nrb = big ? a.nrb_b[m] : a.nrb_s[m];
        const int *tb = a.tb[m];
        int4 *desc = (m ? desc_dn : desc_gu) + (big ? tb[E] + tb[E + 1 + e] : tb[e]);
        const int nc = (c + tpb - 1) / tpb;
        for (int rel = threadIdx.x; rel < nrb * nc; rel += PF_NT) {
            const int rb = rel / nc, cb = rel % nc;
            desc[rel] = make_int4(e, rb, off + cb * tpb, min(tpb, c - cb * tpb));
        }
    }
}

// ------------------------------------------------------------------ GEMMs
// Y[p][r] = sum_k W_g[r][k] B[p][k] over the rows p of group g: an expert's segment of
// permuted rows (the grouped GEMMs, pf_gemm32 and pf_gemm_mx), or all rows of one dense
// product (pf_dense).
//
// K advances through a ring of slots: a slot holds one step's weights (registers,
// range-checked buffer loads, or LDS) and its B block (LDS, filled by buffer loads
// straight to LDS: lane i of a load writes 16 bytes at the load's LDS base + 16 i; rows
// past the block's tokens read out of range and land as zeros).  Each step waits for its
// own slot's loads, meets the other waves at one barrier (after which every wave's share
// of the block is in LDS and the slot used by the previous step is free), refills that
// slot and runs the step's MFMAs.
//
// B sources are activation planes [2][K/8][rows][8] bf16 (hi, lo; each k-group
// row-major over rows), so the 16-byte pieces of one k-group over consecutive rows are
// contiguous.
struct PfGemmArgs {
    const uint8_t  *wm[2];      // group 0's matrices (gate, up) or (down), tiled
    size_t          gstride;    // bytes between groups' records
    int             R, K;       // rows and inner dimension of each matrix
    const int4     *desc;       // per tile {group, row block, first row, rows}, or NULL:
                                // one group of n0 rows
    const int      *ntile;      // tiles in this launch's list
    const int      *dbase;      // the list starts at desc + *dbase, or NULL: at desc
    int             n0;
    const uint16_t *bsrc;       // B planes [2][K/8][brows][8] bf16
    int             brows;      // rows of each B plane
    const int      *perm;       // B row of permuted row p, or NULL: row_base + p
    int             row_base;
    const float    *pw;         // weight of permuted row p (gate/up epilogue), or NULL: 1
    uint16_t       *act;        // gate/up output planes [2][R/8][arows][8] bf16
    int             arows;
    float          *y;          // down output rows [*][R] fp32
    int             out_base;   // output row = out_base + p
    float           b1, b2;     // SiTU betas of the gate/up epilogue (0: uncapped)
    int             ldy;        // floats between output rows (0: R)
    // MXFP8 mode (pf_gemm_mx): B codes [K/16][brows][16] bytes and scales [K/128][brows]
    // dwords (byte b = the 32-k block 4q + b); the gate/up output in the same two forms
    // over R, arows rows
    const uint8_t  *b8;
    const uint32_t *b8s;
    uint8_t        *o8, *o8s;
};


// ------------------------------------------------------------------ dense GEMM
// One dense product Y[p][r] = sum_k W[r][k] B[p][k] with bf16 weights (the shared
// experts, the latent projections, the trunk matrices): W in the 16-row tile layout
// (per 128-k quad, 16-byte runs at t*1024 + (row + 16*kq)*16 for k = 32kq + 8t .. +7), B
// the activation planes.  Both operands go through LDS, fetched by loads straight to LDS,
// so that every weight byte a workgroup reads serves all of its columns and every B byte
// all of its rows; the four waves (2 x 2) take RW x CW tiles of 32 x 32 each (NMAT
// matrices: gate and up of the same rows together) on v_mfma_f32_32x32x16_bf16.
//
// K advances 64 at a time through a ring of NS stages.  A stage holds the workgroup's
// A block as [matrix][k-group g][row][8] and its B block as [g][column][8] (16-byte runs),
// so that the 32 lanes of an MFMA operand that share a k-group read 512 consecutive
// bytes.  Each step waits for its stage (the loads issued after it are the NS - 2 stages
// ahead: stages past the end load out of range, which reads nothing and keeps the count
// exact), meets the other waves, refills the stage freed by the previous step and runs
// its 16 k-steps' MFMAs.
template <int NMAT, int RW, int CW, int HL, bool GU, int NS>
__global__ void __launch_bounds__(PF_NT) pf_dense(PfGemmArgs a)
{
    constexpr int BM = 2 * RW * 32;                // rows of each matrix per workgroup
    constexpr int BN = 2 * CW * 32;                // B columns per workgroup
    constexpr int TPB = BN / HL;                   // tokens per workgroup
    constexpr int SA = NMAT * BM * 128;            // A bytes per stage (64 k)
    constexpr int SB = BN * 128;
    constexpr int SS = SA + SB;
    constexpr int NJA = SA / (PF_NT * 16), NJB = SB / (PF_NT * 16);
    constexpr int LPS = NJA + NJB;                 // vector loads per stage per wave
    static_assert(NJA * PF_NT * 16 == SA && NJB * PF_NT * 16 == SB, "stage must split evenly");
    static_assert(NS >= 2 && (NS - 2) * LPS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) uint8_t sm[NS * SS];

    const int wave = wave_id(), lane = threadIdx.x % WAVE, tid = threadIdx.x;
    const int wr = wave >> 1, wc = wave & 1;
    int rb, p0, ntok;
    {
        // tiles dealt to the 8 XCDs in contiguous runs (workgroups go round-robin), so
        // that the column blocks of a row block run back to back on one XCD and read its
        // weights from that XCD's L2; the grid is a multiple of 8, surplus workgroups
        // leave at once
        const int nrb = (a.R + BM - 1) / BM, nc = (a.n0 + TPB - 1) / TPB, ntiles = nrb * nc;
        const int per = (ntiles + 7) >> 3;
        const int k = blockIdx.x >> 3, dt = (blockIdx.x & 7) * per + k;
        if (k >= per || dt >= ntiles) return;
        rb = dt / nc;
        p0 = (dt % nc) * TPB;
        ntok = min(TPB, a.n0 - p0);
    }
    const int nst = a.K >> 6;

    // ---- A: the row block's weights of each matrix; rows past R read out of range
    const uint32_t tbytes = (uint32_t)a.K * 32u;
    const int t16 = rb * (BM / 16), R16 = a.R >> 4;
    const uint32_t ntl = (uint32_t)(R16 - t16 < BM / 16 ? R16 - t16 : BM / 16);
    rsrc_t ra[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
        ra[m] = make_rsrc(a.wm[m] + (size_t)t16 * tbytes, ntl * tbytes);
    // load j of a stage: 16-byte run c = j*256 + tid -> (matrix, g, row) of the A block,
    // or (g, column) of the B block; its offset in the stage's source, less the stage's
    // own step (A: (st>>1)*4096 + (st&1)*512, B: st*8 k-groups)
    uint32_t aoff[NJA], boff[NJB];
#pragma unroll
    for (int j = 0; j < NJA; j++) {
        const int c = j * PF_NT + tid;
        const int rem = c % (BM * 8), g = rem / BM, r = rem % BM;
        aoff[j] = (uint32_t)(r >> 4) * tbytes + (uint32_t)(g & 3) * 1024u +
                  (uint32_t)((r & 15) + 16 * (g >> 2)) * 16u;
    }
    const int G8 = a.K >> 3;
    const rsrc_t rbs = make_rsrc(a.bsrc, (uint32_t)((size_t)HL * G8 * a.brows * 16));
#pragma unroll
    for (int j = 0; j < NJB; j++) {
        const int c = j * PF_NT + tid;
        const int g = c / BN, col = c % BN, tok = col / HL, hl = col % HL;
        boff[j] = tok < ntok ? ((uint32_t)(hl * G8 + g) * (uint32_t)a.brows +
                                (uint32_t)(a.row_base + p0 + tok)) * 16u
                             : K3X_OOB;
    }
    const uint32_t bstep = (uint32_t)a.brows * 128u;          // 8 k-groups of B

    auto ld = [&](int slot, int st) AI {
        const bool on = st < nst;
        const uint32_t sa = (uint32_t)(st >> 1) * 4096u + (uint32_t)(st & 1) * 512u;
        uint8_t *base = sm + slot * SS;
#pragma unroll
        for (int j = 0; j < NJA; j++) {
            const int m = (j * PF_NT) / (BM * 8);            // uniform per load
            // (resource and offset through locals: the host pass of this template
            // rejects a captured array element as the builtin's operand)
            const rsrc_t r = ra[m];
            const uint32_t o = on ? aoff[j] + sa : K3X_OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (lds_void *)(base + (j * PF_NT + wave * WAVE) * 16), 16, o, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < NJB; j++) {
            // (a column past the tokens keeps an out-of-range offset: K3X_OOB plus at most
            // K/64 steps of brows*128 bytes stays below 2^32 and past the planes)
            const uint32_t o = on ? boff[j] + (uint32_t)st * bstep : K3X_OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rbs, (lds_void *)(base + SA + (j * PF_NT + wave * WAVE) * 16), 16, o, 0, 0, 0);
        }
    };

    f32x16 acc[NMAT][RW][CW];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int i = 0; i < RW; i++)
#pragma unroll
            for (int c = 0; c < CW; c++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[m][i][c][v] = 0.f;

    const int l32 = lane & 31, h = lane >> 5;
    auto compute = [&](int slot) AI {
        const uint8_t *base = sm + slot * SS;
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            const int g = 2 * s4 + h;
            bf16x8 bf[CW];
#pragma unroll
            for (int c = 0; c < CW; c++)
                bf[c] = as_bf16x8(*(const u32x4 *)(base + SA + (g * BN + (wc * CW + c) * 32 + l32) * 16));
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int i = 0; i < RW; i++) {
                    const bf16x8 av = as_bf16x8(
                        *(const u32x4 *)(base + ((m * 8 + g) * BM + (wr * RW + i) * 32 + l32) * 16));
#pragma unroll
                    for (int c = 0; c < CW; c++) acc[m][i][c] = mfma32(av, bf[c], acc[m][i][c]);
                }
        }
    };

#pragma unroll
    for (int s = 0; s < NS - 1; s++) {
        SCHED_FENCE();
        ld(s, s);
    }
    SCHED_FENCE();
    for (int st = 0; st < nst; st++) {
        meet<(NS - 2) * LPS>();
        SCHED_FENCE();
        ld((st + NS - 1) % NS, st + NS - 1);
        SCHED_FENCE();
        compute(st % NS);
    }
    // no load to LDS may still be landing when the workgroup ends
    WAIT_VMCNT_LGKM0(0);

    // ---- epilogue: lane holds column l32 of each column tile, rows 8aa + 4h + b
    const int G8o = a.R >> 3;
#pragma unroll
    for (int c = 0; c < CW; c++) {
        const int col = (wc * CW + c) * 32 + l32;
        const int tl = col / HL;
        const bool writer = (HL == 1 || (col & 1) == 0) && tl < ntok;
        const int p = p0 + tl;
#pragma unroll
        for (int i = 0; i < RW; i++)
#pragma unroll
            for (int aa = 0; aa < 4; aa++) {
                const int r0 = rb * BM + (wr * RW + i) * 32 + 8 * aa + 4 * h;
                float v0[4], v1[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    v0[b] = acc[0][i][c][4 * aa + b];
                    if (HL == 2) v0[b] += __shfl_xor(v0[b], 1);
                    if (NMAT == 2) {
                        v1[b] = acc[NMAT - 1][i][c][4 * aa + b];
                        if (HL == 2) v1[b] += __shfl_xor(v1[b], 1);
                    }
                }
                if (!writer || r0 >= a.R) continue;
                if (GU) {
                    uint32_t hi[4], lo[4];
#pragma unroll
                    for (int b = 0; b < 4; b++) split_bf16(situ(v0[b], v1[b], a.b1, a.b2), hi[b], lo[b]);
                    const size_t o = ((size_t)(r0 >> 3) * a.arows + (size_t)(a.out_base + p)) * 8 + (r0 & 7);
                    const size_t plane = (size_t)G8o * a.arows * 8;
                    *(u32x2 *)(a.act + o) = (u32x2){hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
                    *(u32x2 *)(a.act + plane + o) = (u32x2){lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
                } else {
                    float *dst = a.y + (size_t)(a.out_base + p) * (a.ldy ? a.ldy : a.R) + r0;
                    *(f32x4 *)dst = (f32x4){v0[0], v0[1], v0[2], v0[3]};
                }
            }
    }
}

// ------------------------------------------------------------------ grouped GEMM, 32x32
// The routed GEMMs (MXFP4 weights) on v_mfma_f32_32x32x16_bf16.  A workgroup computes
// NW*RT32*32 weight rows (NMAT matrices: gate and up together) by CT32 column tiles of 32
// B columns (HL columns per token: hi, or hi and lo); a wave owns RT32 row tiles of 32
// rows (two 16-row tiles of the fp4 layout), its weights held in registers through a
// ring of 4 quads of 128 k, and the waves share each quad's B block in LDS.
//
// K order.  Within a quad, lane L (row R = L%32, h = L/32) loads two 16-byte scale
// groups of row R: group kq = h (load 0) and kq = 2 + h (load 1).  Dword d of load g
// feeds the MFMA of step (g, d) with k = 64g + 32h + 8d .. +7, so one 32x32x16 step
// multiplies k-slots {64g + 8d .. +7} (lanes 0-31) and {64g + 32 + 8d .. +7} (lanes
// 32-63).  The B block in LDS is laid out to match: entry ((g*4 + d)*2 + h)*NCOL + col
// holds those 8 k of column col.  Every product of the quad is formed exactly once;
// only the order of the fp32 additions differs from the 16x16 form.
template <bool EXACT, int NMAT, int RT32, int CT32, int HL, bool GU, int NW>
__global__ void __launch_bounds__(NW * WAVE) pf_gemm32(PfGemmArgs a)
{
    constexpr int NTH = NW * WAVE;
    constexpr int NCOL = CT32 * 32;
    constexpr int TPB = NCOL / HL;
    constexpr int RPB = NW * RT32 * 32;
    constexpr int QB = NCOL * 128 * 2;
    constexpr int NJ = QB / (NTH * 16);
    constexpr int RING = 4;
    // vector loads a quad issues per wave: 2 code loads per 32 rows and the B pieces, plus
    // (the first quad of a super-quad) 2 scale dwords per 32 rows, which hold the scale
    // bytes of the super-quad's four quads
    constexpr int LPI = NMAT * RT32 * 2 + NJ;
    constexpr int LPS = LPI + NMAT * RT32 * 2;
    static_assert(NJ * NTH * 16 == QB, "B quad must split evenly");
    static_assert(LPI + LPS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) uint8_t sB[RING * QB];

    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int nrb = (a.R + RPB - 1) / RPB;
    int g = 0, rb, ntok, p0;
    {
        // Workgroups are dealt to the 8 XCDs round-robin; tiles are dealt to them in
        // contiguous runs instead (XCD x takes tiles x*per .. x*per + per-1 in order), so
        // the column blocks of one weight row block run back to back on one XCD and
        // re-read the weights from its L2.  The grid is a multiple of 8.
        // the descriptor words are read into scalar registers (readfirstlane): the
        // weight resources built from them must be wave-uniform, or every buffer load
        // becomes a loop over distinct descriptors
        const int ntiles = a.desc ? __builtin_amdgcn_readfirstlane(*a.ntile)
                                  : nrb * ((a.n0 + TPB - 1) / TPB);
        const int per = (ntiles + 7) >> 3;
        const int k = blockIdx.x >> 3, tile = (blockIdx.x & 7) * per + k;
        if (k >= per || tile >= ntiles) return;
        if (a.desc) {
            const int4 d = a.desc[(a.dbase ? __builtin_amdgcn_readfirstlane(*a.dbase) : 0) + tile];
            g = __builtin_amdgcn_readfirstlane(d.x); rb = __builtin_amdgcn_readfirstlane(d.y);
            p0 = __builtin_amdgcn_readfirstlane(d.z); ntok = __builtin_amdgcn_readfirstlane(d.w);
        } else {
            const int nc = (a.n0 + TPB - 1) / TPB;
            rb = tile / nc;
            const int cb = tile % nc;
            p0 = cb * TPB;
            ntok = min(TPB, a.n0 - p0);
        }
    }
    const int nQ = a.K >> 7;

    // ---- weights: row tile pair i = 16-row tiles 2*tp, 2*tp+1 of this wave
    const uint32_t tbytes = (uint32_t)fp4_tile_bytes(a.K);
    const int R16 = a.R >> 4;
    const int Rl = lane & 31, h = lane >> 5;
    rsrc_t ra[NMAT][RT32];
    int tp16[RT32];
#pragma unroll
    for (int i = 0; i < RT32; i++) {
        const int t16 = ((rb * NW + wave) * RT32 + i) * 2;
        tp16[i] = t16;
        // readfirstlane: the clamp is a VALU med3, whose result would make the weight
        // resource a vector operand
        const int ntl = __builtin_amdgcn_readfirstlane(R16 - t16 < 0 ? 0 : (R16 - t16 > 2 ? 2 : R16 - t16));
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            ra[m][i] = make_rsrc(a.wm[m] + (size_t)g * a.gstride + (size_t)t16 * tbytes,
                                 (uint32_t)ntl * tbytes);
    }
    // this lane's offsets inside a pair: its 16-row tile, row, and group h (load 0)
    const uint32_t lc = (uint32_t)(Rl >> 4) * tbytes + (uint32_t)((Rl & 15) + 16 * h) * 16u;
    const uint32_t ls = (uint32_t)(Rl >> 4) * tbytes + 4096u + (uint32_t)((Rl & 15) + 16 * h) * 4u;

    // ---- B pieces: entry e = (wave*NJ + j)*64 + lane; e = gdh*NCOL + col,
    // gdh = (g*4 + d)*2 + h -> k-group 8g + 4h + d of the quad
    const int G8 = a.K >> 3;
    const rsrc_t rbs = make_rsrc(a.bsrc, (uint32_t)((size_t)2 * G8 * a.brows * 16));
    const uint32_t qstep = (uint32_t)a.brows * 256u;
    uint32_t boff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e = (wave * NJ + j) * WAVE + lane;
        const int gdh = e / NCOL, col = e % NCOL;
        const int gg = gdh >> 3, dd = (gdh >> 1) & 3, hh = gdh & 1;
        const int tok = col / HL, hl = col % HL;
        if (tok < ntok) {
            const int row = a.perm ? a.perm[p0 + tok] : a.row_base + p0 + tok;
            boff[j] = ((uint32_t)(hl * G8 + 8 * gg + 4 * hh + dd) * (uint32_t)a.brows + (uint32_t)row) * 16u;
        } else {
            boff[j] = K3X_OOB;
        }
    }

    struct AQ {
        u32x4    c[NMAT][RT32][2];
    };
    AQ A[RING];
    // scale dwords: sn is loaded with the first quad of a super-quad (slot 0: quad q is
    // always computed from slot q % 4), and copied to sc before that quad is computed,
    // while the three other quads of the previous super-quad still read sc
    uint32_t sn[NMAT][RT32][2], sc[NMAT][RT32][2];
    auto ld = [&](int slot, int q) AI {
        const bool on = q < nQ;
        const uint32_t qc = (uint32_t)(q >> 2) * 4352u + (uint32_t)(q & 3) * 1024u;
        const uint32_t qs = (uint32_t)(q >> 2) * 4352u;
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int i = 0; i < RT32; i++)
#pragma unroll
                for (int gl = 0; gl < 2; gl++) {
                    A[slot].c[m][i][gl] = wld16(ra[m][i], on ? lc + qc + 512u * gl : K3X_OOB);
                    if (slot == 0) sn[m][i][gl] = wld4(ra[m][i], on ? ls + qs + 128u * gl : K3X_OOB);
                }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t o = boff[j] + (uint32_t)q * qstep;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rbs, (lds_void *)(sB + slot * QB + (wave * NJ + j) * 1024), 16, o, 0, 0, 0);
        }
    };

    f32x16 acc[NMAT][RT32][CT32];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int i = 0; i < RT32; i++)
#pragma unroll
            for (int c = 0; c < CT32; c++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[m][i][c][v] = 0.f;

    auto compute = [&](int slot, int q) AI {
        const uint8_t *bb = sB + slot * QB;
        const int sh = 8 * (q & 3);
        if (slot == 0) {
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int i = 0; i < RT32; i++)
#pragma unroll
                    for (int gl = 0; gl < 2; gl++) sc[m][i][gl] = sn[m][i][gl];
        }
#pragma unroll
        for (int gl = 0; gl < 2; gl++)
#pragma unroll
            for (int d = 0; d < 4; d++) {
                bf16x8 bf[CT32];
#pragma unroll
                for (int c = 0; c < CT32; c++)
                    bf[c] = as_bf16x8(*(const u32x4 *)(bb + (((gl * 4 + d) * 2 + h) * NCOL + c * 32 + Rl) * 16));
#pragma unroll
                for (int m = 0; m < NMAT; m++)
#pragma unroll
                    for (int i = 0; i < RT32; i++) {
                        const uint32_t sb = (sc[m][i][gl] >> sh) & 255u;
                        const bf16x8 av = EXACT ? dq8_exact(A[slot].c[m][i][gl][d], sb)
                                                : dq8(A[slot].c[m][i][gl][d], e8m0_scale(sb));
#pragma unroll
                        for (int c = 0; c < CT32; c++) acc[m][i][c] = mfma32(av, bf[c], acc[m][i][c]);
                    }
            }
    };

#pragma unroll
    for (int s = 0; s < RING - 1; s++) {
        SCHED_FENCE();
        ld(s, s);
    }
    SCHED_FENCE();
    int q = 0;
    // meet quad q + s once the loads issued after its own are all that remain: those of
    // quads q + s + 1 and q + s + 2, of which q + 4 (the next super-quad's first) also
    // loads the scale dwords
    static_assert(RING == 4, "written for a ring of 4");
    for (; q + RING <= nQ; q += RING) {
        meet<2 * LPI>();       SCHED_FENCE(); ld(3, q + 3); SCHED_FENCE(); compute(0, q);
        meet<2 * LPI>();       SCHED_FENCE(); ld(0, q + 4); SCHED_FENCE(); compute(1, q + 1);
        meet<LPI + LPS>();     SCHED_FENCE(); ld(1, q + 5); SCHED_FENCE(); compute(2, q + 2);
        meet<LPS + LPI>();     SCHED_FENCE(); ld(2, q + 6); SCHED_FENCE(); compute(3, q + 3);
    }
    if (q < nQ)     { meet<2 * LPI>(); compute(0, q); }
    if (q + 1 < nQ) { meet<LPI>();     compute(1, q + 1); }
    if (q + 2 < nQ) { meet<0>();       compute(2, q + 2); }
    WAIT_VMCNT_LGKM0(0);

    // ---- epilogue: lane holds column Rl of each column tile, rows 8a + 4h + b
    const int G8o = a.R >> 3;
#pragma unroll
    for (int c = 0; c < CT32; c++) {
        const int col = c * 32 + Rl;
        const int tl = col / HL;
        const bool writer = (HL == 1 || (col & 1) == 0) && tl < ntok;
        const int p = p0 + tl;
#pragma unroll
        for (int i = 0; i < RT32; i++)
#pragma unroll
            for (int aa = 0; aa < 4; aa++) {
                const int r0 = tp16[i] * 16 + 8 * aa + 4 * h;
                float v0[4], v1[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    v0[b] = acc[0][i][c][4 * aa + b];
                    if (HL == 2) v0[b] += __shfl_xor(v0[b], 1);
                    if (NMAT == 2) {
                        v1[b] = acc[NMAT - 1][i][c][4 * aa + b];
                        if (HL == 2) v1[b] += __shfl_xor(v1[b], 1);
                    }
                }
                if (!writer || r0 >= a.R) continue;
                if (GU) {
                    const float w = a.pw ? a.pw[p] : 1.0f;
                    uint32_t hi[4], lo[4];
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const float yv = (w == 0.0f) ? 0.0f : w * situ(v0[b], v1[b], a.b1, a.b2);
                        split_bf16(yv, hi[b], lo[b]);
                    }
                    const size_t o = ((size_t)(r0 >> 3) * a.arows + (size_t)(a.out_base + p)) * 8 + (r0 & 7);
                    const size_t plane = (size_t)G8o * a.arows * 8;
                    *(u32x2 *)(a.act + o) = (u32x2){hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
                    *(u32x2 *)(a.act + plane + o) = (u32x2){lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
                } else {
                    float *dst = a.y + (size_t)(a.out_base + p) * (a.ldy ? a.ldy : a.R) + r0;
                    *(f32x4 *)dst = (f32x4){v0[0], v0[1], v0[2], v0[3]};
                }
            }
    }
}

// ------------------------------------------------------------------ MXFP8 mode
// The opt-in prefill mode K3X_PREFILL_MXFP8: the routed expert products on the scaled
// matrix cores (v_mfma_scale_f32_32x32x64_f8f6f4), the weights as stored (E2M1 codes,
// E8M0 scale per 32 k, applied by the matrix core), the activations quantised to MXFP8:
// blocks of 32 k sharing an E8M0 scale 2^X, X the least integer with max|v| <= 448 * 2^X
// over the block's finite values (clamped to [-127, 127]; -127 for a block with no
// non-zero finite value), each finite value v * 2^-X rounded to the nearest E4M3 (FN
// encoding) value, ties to the even code, a non-finite one the NaN code.  The gate/up
// input is the token's row (x, or z in a LatentMoE layer); the down input is the
// gate/up output w * SiTU(gate, up), quantised in the gate/up epilogue.

typedef int i32x8 __attribute__((ext_vector_type(8)));

// E8M0 byte of a block whose largest finite magnitude is m
__device__ __forceinline__ int mx8_scale(float m)
{
    if (!(m > 0.0f)) return 0;
    const uint32_t b = __float_as_uint(m);
    int X = (int)((b >> 23) & 255u) - 127 - 8 + ((b & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    X = X < -127 ? -127 : (X > 127 ? 127 : X);
    return X + 127;
}

// v (finite, |v| <= 448) to its E4M3 code, nearest value, ties to the even code
__device__ __forceinline__ uint32_t e4m3_rne(float v)
{
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (a < 0x1p-6f) return sign | (uint32_t)rintf(a * 512.0f);     // steps of 2^-9
    const int E = (int)((__float_as_uint(a) >> 23) & 255u) - 127;     // -6 .. 8
    const uint32_t m = (uint32_t)rintf(a * __uint_as_float((uint32_t)(127 + 3 - E) << 23));
    return sign | (m == 16u ? (uint32_t)(E + 8) << 3 : ((uint32_t)(E + 7) << 3) | (m - 8u));
}

// SiTU out of line: its inlined expansion over the sixteen values of a quantisation block
// would take the registers the accumulators need
__device__ __attribute__((noinline)) float situ_call(float g, float u, float b1, float b2)
{
    return situ(g, u, b1, b2);
}

// the code of v in a block of scale byte sb (inv = 2^-X)
__device__ __forceinline__ uint32_t mx8_code(float v, float inv)
{
    if (!isfinite(v)) return ((__float_as_uint(v) >> 24) & 0x80u) | 0x7Fu;
    return e4m3_rne(v * inv);
}

__device__ __forceinline__ float mx8_inv(int sb) { return __uint_as_float((uint32_t)(254 - sb) << 23); }

// The routed experts' MXFP8 input in permuted order: src row perm_tok[p] (bf16 or fp32,
// rows ld elements apart), X elements -> codes [X/16][TK][16], scales [X/128][TK] dwords.
// A workgroup takes MX_R rows by one 128-k quad, one thread per (row, 32-k block); the
// codes go through LDS so that the stores run along the rows of a k16-group (1 KB
// contiguous) and each row's four scale bytes are one dword.
#define MX_R 64

static inline unsigned pf_mx8_grid(int TK, int X) { return (unsigned)(((TK + MX_R - 1) / MX_R) * (X / 128)); }

__global__ void __launch_bounds__(PF_NT) pf_mx8_rows(const void *src, int bf16, int ld, int X,
                                                     const int *perm_tok, int TK,
                                                     uint8_t *codes, uint8_t *scales)
{
    static_assert(MX_R * 4 == PF_NT, "a thread per (row, block)");
    __shared__ u32x4 sc[8][MX_R + 1];          // [k16-group of the quad][row]
    __shared__ uint32_t ss[MX_R];
    const int nq = X / 128;
    const int q = blockIdx.x % nq, p0 = (blockIdx.x / nq) * MX_R;
    const int r = threadIdx.x >> 2, b = threadIdx.x & 3, p = p0 + r;
    uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    int sb = 0;
    if (p < TK) {
        const size_t base = (size_t)perm_tok[p] * ld + (size_t)q * 128 + (size_t)b * 32;
        float v[4][8];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            load_x8(src, bf16, base + 8 * j, v[j]);
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (isfinite(v[j][e])) m = fmaxf(m, fabsf(v[j][e]));
        }
        sb = mx8_scale(m);
        const float inv = mx8_inv(sb);
#pragma unroll
        for (int d = 0; d < 8; d++) {
            uint32_t c = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) c |= mx8_code(v[d / 2][(d % 2) * 4 + e], inv) << (8 * e);
            w[d] = c;
        }
    }
    sc[2 * b][r] = (u32x4){w[0], w[1], w[2], w[3]};
    sc[2 * b + 1][r] = (u32x4){w[4], w[5], w[6], w[7]};
    // the row's four scale bytes, block b at byte b, gathered by its lane group of four
    uint32_t sw = (uint32_t)sb << (8 * b);
    sw |= __shfl_xor(sw, 1);
    sw |= __shfl_xor(sw, 2);
    if (b == 0) ss[r] = sw;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int i = j * PF_NT + threadIdx.x, g = i / MX_R, rr = i % MX_R, pp = p0 + rr;
        if (pp < TK) *(u32x4 *)(codes + ((size_t)(8 * q + g) * TK + pp) * 16) = sc[g][rr];
    }
    if (threadIdx.x < MX_R && p0 + (int)threadIdx.x < TK)
        *(uint32_t *)(scales + ((size_t)q * TK + p0 + threadIdx.x) * 4) = ss[threadIdx.x];
}

// Grouped GEMM on v_mfma_scale_f32_32x32x64_f8f6f4 (A fp4, B fp8 E4M3).  Operand layout
// of the instruction (64 k a step): A lane l holds row l%32, k = 32*(l/32) .. +31 (16
// bytes, low nibble first) with that 32-k group's scale byte; B lane l holds column l%32,
// bytes 0-15 = k 16*(l/32) .. +15 and bytes 16-31 = k 32 + 16*(l/32) .. +15, and lane
// (j + 32b) gives column j's scale of 32-k group b; D as the 32x32x16 bf16 form.  A quad
// of 128 k is two steps whose A operands are pf_gemm32's two code loads and scale dwords
// (k groups 2*step + h).  Tile lists, XCD dealing, ring and barrier protocol as
// pf_gemm32; the B block in LDS: entry gq*NCOL + col = k16-group gq of the quad, column
// col; each lane keeps its column's scale dword per quad in registers.  The gate/up
// epilogue forms w * SiTU(gate, up) and quantises each 32-row block of a column (16
// values in each of two lanes) to MXFP8 codes and a scale byte.
template <int NMAT, int RT32, int CT, bool GU, int NW>
__global__ void __launch_bounds__(NW * WAVE) pf_gemm_mx(PfGemmArgs a)
{
    constexpr int NTH = NW * WAVE;
    constexpr int NCOL = CT * 32;
    constexpr int RPB = NW * RT32 * 32;
    constexpr int QB = 8 * NCOL * 16;
    constexpr int NJ = QB / (NTH * 16);
    constexpr int RING = 4;
    // loads a quad issues per wave (as pf_gemm32's, plus a scale dword per column tile)
    constexpr int LPI = NMAT * RT32 * 2 + NJ + CT;
    constexpr int LPS = LPI + NMAT * RT32 * 2;
    static_assert(NJ * NTH * 16 == QB, "B quad must split evenly");
    static_assert(LPI + LPS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) uint8_t sB[RING * QB];

    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int nrb = (a.R + RPB - 1) / RPB;
    int g = 0, rb, ntok, p0;
    {
        const int ntiles = a.desc ? __builtin_amdgcn_readfirstlane(*a.ntile)
                                  : nrb * ((a.n0 + NCOL - 1) / NCOL);
        const int per = (ntiles + 7) >> 3;
        const int k = blockIdx.x >> 3, tile = (blockIdx.x & 7) * per + k;
        if (k >= per || tile >= ntiles) return;
        if (a.desc) {
            const int4 d = a.desc[(a.dbase ? __builtin_amdgcn_readfirstlane(*a.dbase) : 0) + tile];
            g = __builtin_amdgcn_readfirstlane(d.x); rb = __builtin_amdgcn_readfirstlane(d.y);
            p0 = __builtin_amdgcn_readfirstlane(d.z); ntok = __builtin_amdgcn_readfirstlane(d.w);
        } else {
            const int nc = (a.n0 + NCOL - 1) / NCOL;
            rb = tile / nc;
            p0 = (tile % nc) * NCOL;
            ntok = min(NCOL, a.n0 - p0);
        }
    }
    const int nQ = a.K >> 7;

    const uint32_t tbytes = (uint32_t)fp4_tile_bytes(a.K);
    const int R16 = a.R >> 4;
    const int Rl = lane & 31, h = lane >> 5;
    rsrc_t ra[NMAT][RT32];
    int tp16[RT32];
#pragma unroll
    for (int i = 0; i < RT32; i++) {
        const int t16 = ((rb * NW + wave) * RT32 + i) * 2;
        tp16[i] = t16;
        const int ntl = __builtin_amdgcn_readfirstlane(R16 - t16 < 0 ? 0 : (R16 - t16 > 2 ? 2 : R16 - t16));
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            ra[m][i] = make_rsrc(a.wm[m] + (size_t)g * a.gstride + (size_t)t16 * tbytes,
                                 (uint32_t)ntl * tbytes);
    }
    const uint32_t lc = (uint32_t)(Rl >> 4) * tbytes + (uint32_t)((Rl & 15) + 16 * h) * 16u;
    const uint32_t ls = (uint32_t)(Rl >> 4) * tbytes + 4096u + (uint32_t)((Rl & 15) + 16 * h) * 4u;

    // ---- B: entry e = (wave*NJ + j)*64 + lane = gq*NCOL + col
    const rsrc_t rbc = make_rsrc(a.b8, (uint32_t)((size_t)a.K * a.brows));
    const rsrc_t rbsc = make_rsrc(a.b8s, (uint32_t)((size_t)(a.K >> 7) * a.brows * 4));
    const uint32_t qstep = (uint32_t)a.brows * 128u, sstep = (uint32_t)a.brows * 4u;
    uint32_t boff[NJ], soff[CT];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e = (wave * NJ + j) * WAVE + lane;
        const int gq = e / NCOL, col = e % NCOL;
        boff[j] = col < ntok ? ((uint32_t)gq * (uint32_t)a.brows + (uint32_t)(a.row_base + p0 + col)) * 16u
                             : K3X_OOB;
    }
#pragma unroll
    for (int c = 0; c < CT; c++) {
        const int col = c * 32 + Rl;
        soff[c] = col < ntok ? (uint32_t)(a.row_base + p0 + col) * 4u : K3X_OOB;
    }

    struct AQ {
        u32x4    c[NMAT][RT32][2];
        uint32_t bs[CT];
    };
    AQ A[RING];
    uint32_t sn[NMAT][RT32][2], sc[NMAT][RT32][2];     // as in pf_gemm32
    auto ld = [&](int slot, int q) AI {
        const bool on = q < nQ;
        const uint32_t qc = (uint32_t)(q >> 2) * 4352u + (uint32_t)(q & 3) * 1024u;
        const uint32_t qs = (uint32_t)(q >> 2) * 4352u;
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int i = 0; i < RT32; i++)
#pragma unroll
                for (int gl = 0; gl < 2; gl++) {
                    A[slot].c[m][i][gl] = wld16(ra[m][i], on ? lc + qc + 512u * gl : K3X_OOB);
                    if (slot == 0) sn[m][i][gl] = wld4(ra[m][i], on ? ls + qs + 128u * gl : K3X_OOB);
                }
#pragma unroll
        for (int c = 0; c < CT; c++)
            A[slot].bs[c] = __builtin_amdgcn_raw_buffer_load_b32(
                rbsc, (!on | (soff[c] == K3X_OOB)) ? K3X_OOB : soff[c] + (uint32_t)q * sstep, 0, 0);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            // (bitwise, not short-circuit: a branch on the uniform `on` would split the
            // step into blocks, and the MFMAs would then sink past the next barriers)
            const uint32_t o = ((boff[j] == K3X_OOB) | !on) ? K3X_OOB : boff[j] + (uint32_t)q * qstep;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rbc, (lds_void *)(sB + slot * QB + (wave * NJ + j) * 1024), 16, o, 0, 0, 0);
        }
    };

    f32x16 acc[NMAT][RT32][CT];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int i = 0; i < RT32; i++)
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[m][i][c][v] = 0.f;

    auto compute = [&](int slot, int q) AI {
        const uint8_t *bb = sB + slot * QB;
        const int sh = 8 * (q & 3);
        if (slot == 0) {
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int i = 0; i < RT32; i++)
#pragma unroll
                    for (int gl = 0; gl < 2; gl++) sc[m][i][gl] = sn[m][i][gl];
        }
#pragma unroll
        for (int st = 0; st < 2; st++) {
            i32x8 bv[CT];
            int sbv[CT];
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const u32x4 b0 = *(const u32x4 *)(bb + ((4 * st + h) * NCOL + c * 32 + Rl) * 16);
                const u32x4 b1 = *(const u32x4 *)(bb + ((4 * st + 2 + h) * NCOL + c * 32 + Rl) * 16);
                bv[c] = (i32x8){(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                                (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
                sbv[c] = (int)((A[slot].bs[c] >> (8 * (2 * st + h))) & 255u);
            }
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int i = 0; i < RT32; i++) {
                    const u32x4 cw = A[slot].c[m][i][st];
                    const i32x8 av = {(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3], 0, 0, 0, 0};
                    const int sa = (int)((sc[m][i][st] >> sh) & 255u);
#pragma unroll
                    for (int c = 0; c < CT; c++)
                        acc[m][i][c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            av, bv[c], acc[m][i][c], 4, 0, 0, sa, 0, sbv[c]);
                }
        }
    };

#pragma unroll
    for (int s = 0; s < RING - 1; s++) {
        SCHED_FENCE();
        ld(s, s);
    }
    SCHED_FENCE();
    int q = 0;
    // meet quad q + s once the loads issued after its own are all that remain: those of
    // quads q + s + 1 and q + s + 2, of which q + 4 (the next super-quad's first) also
    // loads the scale dwords
    static_assert(RING == 4, "written for a ring of 4");
    for (; q + RING <= nQ; q += RING) {
        meet<2 * LPI>();       SCHED_FENCE(); ld(3, q + 3); SCHED_FENCE(); compute(0, q);
        meet<2 * LPI>();       SCHED_FENCE(); ld(0, q + 4); SCHED_FENCE(); compute(1, q + 1);
        meet<LPI + LPS>();     SCHED_FENCE(); ld(1, q + 5); SCHED_FENCE(); compute(2, q + 2);
        meet<LPS + LPI>();     SCHED_FENCE(); ld(2, q + 6); SCHED_FENCE(); compute(3, q + 3);
    }
    if (q < nQ)     { meet<2 * LPI>(); compute(0, q); }
    if (q + 1 < nQ) { meet<LPI>();     compute(1, q + 1); }
    if (q + 2 < nQ) { meet<0>();       compute(2, q + 2); }
    WAIT_VMCNT_LGKM0(0);

    // ---- epilogue: lane holds column Rl of each column tile, rows 8a + 4h + b
#pragma unroll
    for (int c = 0; c < CT; c++) {
        const int tl = c * 32 + Rl;
        const bool writer = tl < ntok;
        const int p = p0 + tl;
#pragma unroll
        for (int i = 0; i < RT32; i++) {
            const int rt = tp16[i] * 16;              // first row of the 32-row tile
            if (GU) {
                const float w = writer && a.pw ? a.pw[p] : 1.0f;
                float yv[16];
                float m = 0.0f;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    yv[v] = (w == 0.0f) ? 0.0f : w * situ_call(acc[0][i][c][v], acc[NMAT - 1][i][c][v], a.b1, a.b2);
                    if (isfinite(yv[v])) m = fmaxf(m, fabsf(yv[v]));
                }
                m = fmaxf(m, __shfl_xor(m, 32));
                if (!writer || rt >= a.R) continue;
                const int sb = mx8_scale(m);
                const float inv = mx8_inv(sb);
#pragma unroll
                for (int aa = 0; aa < 4; aa++) {
                    const int r0 = rt + 8 * aa + 4 * h;
                    uint32_t wd = 0;
#pragma unroll
                    for (int b = 0; b < 4; b++) wd |= mx8_code(yv[4 * aa + b], inv) << (8 * b);
                    *(uint32_t *)(a.o8 + ((size_t)(r0 >> 4) * a.arows + (size_t)(a.out_base + p)) * 16 + (r0 & 15)) = wd;
                }
                if (h == 0) {
                    const int r32 = rt >> 5;
                    a.o8s[((size_t)(r32 >> 2) * a.arows + (size_t)(a.out_base + p)) * 4 + (r32 & 3)] = (uint8_t)sb;
                }
            } else {
                if (!writer) continue;
#pragma unroll
                for (int aa = 0; aa < 4; aa++) {
                    const int r0 = rt + 8 * aa + 4 * h;
                    if (r0 >= a.R) continue;
                    float *dst = a.y + (size_t)(a.out_base + p) * (a.ldy ? a.ldy : a.R) + r0;
                    *(f32x4 *)dst = (f32x4){acc[0][i][c][4 * aa], acc[0][i][c][4 * aa + 1],
                                            acc[0][i][c][4 * aa + 2], acc[0][i][c][4 * aa + 3]};
                }
            }
        }
    }
}

// ------------------------------------------------------------------ latent norm
// The latent form's aggregates (agg [T][X], one workgroup per token): RMSNorm with the
// latent norm weights (k3_rmsnorm, k3_ops.c:132-140 and :1946; double sum of squares, inv
// rounded to float, w*x*inv), or none when nw is NULL, then the hi and lo parts for the
// up projection: planes [2][X/8][T][8] (pf_split's layout) for the dense kernel, or with
// rows set, rows [2][T][X] for the library GEMMs.
__global__ void __launch_bounds__(PF_NT) pf_latnorm(const float *agg, const float *nw, float eps,
                                                    int T, int X, uint16_t *hl, int rows)
{
    __shared__ double red[PF_NT / WAVE];
    __shared__ float s_inv;
    const int t = blockIdx.x, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const float *row = agg + (size_t)t * X;
    if (nw) {
        double ss = 0.0;
        for (int i = threadIdx.x; i < X; i += PF_NT) ss += (double)row[i] * (double)row[i];
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        if (threadIdx.x == 0) {
            double tot = 0.0;
            for (int w = 0; w < PF_NT / WAVE; w++) tot += red[w];
            s_inv = (float)(1.0 / sqrt(tot / (double)X + (double)eps));
        }
        __syncthreads();
    }
    const int G8 = X >> 3;
    for (int gi = threadIdx.x; gi < G8; gi += PF_NT) {
        float v[8];
        load_x8(row, 0, (size_t)gi * 8, v);
        if (nw) {
            float w[8];
            load_x8(nw, 0, (size_t)gi * 8, w);
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = w[j] * v[j] * s_inv;
        }
        uint32_t hi[8], lo[8];
#pragma unroll
        for (int j = 0; j < 8; j++) split_bf16(v[j], hi[j], lo[j]);
        u32x4 h, l;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            h[j] = hi[2 * j] | (hi[2 * j + 1] << 16);
            l[j] = lo[2 * j] | (lo[2 * j + 1] << 16);
        }
        if (rows) {
            *(u32x4 *)(hl + (size_t)t * X + (size_t)gi * 8) = h;
            *(u32x4 *)(hl + ((size_t)T + t) * X + (size_t)gi * 8) = l;
        } else {
            *(u32x4 *)(hl + ((size_t)gi * T + t) * 8) = h;
            *(u32x4 *)(hl + ((size_t)(G8 + gi) * T + t) * 8) = l;
        }
    }
}

// ------------------------------------------------------------------ combine
// out[t] = ((y[pos(t,0)] + y[pos(t,1)]) + ... ) + y_shared[t], then + resid (pos_of
// NULL: K = 1 and row t).
__global__ void __launch_bounds__(PF_NT) pf_combine(const float *y, const int *pos_of, int T, int K,
                                                    int H, int sh_row0, const float *resid,
                                                    float *out)
{
    const size_t i = (size_t)blockIdx.x * PF_NT + threadIdx.x;
    const int h4 = H >> 2;
    if (i >= (size_t)T * h4) return;
    const int t = (int)(i / h4), h = (int)(i % h4) * 4;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < K; j++) {
        const size_t row = pos_of ? (size_t)pos_of[(size_t)t * K + j] : (size_t)t;
        s += *(const f32x4 *)(y + row * H + h);
    }
    if (sh_row0 >= 0) s += *(const f32x4 *)(y + (size_t)(sh_row0 + t) * H + h);
    const size_t o = (size_t)t * H + h;
    if (resid) s += *(const f32x4 *)(resid + o);
    *(f32x4 *)(out + o) = s;
}

// ------------------------------------------------------------------ launcher
static inline int launch_ok(void) { return hipGetLastError() == hipSuccess ? 0 : K3X_E_HIP; }

static inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

template <int NE>
static void launch_topk(const PfTopkArgs &a, hipStream_t s)
{
    hipLaunchKernelGGL(pf_topk<NE>, dim3(cdiv(a.T, TK_W)), dim3(TK_W * WAVE), 0, s, a);
}

// Launch shapes of the routed GEMMs (pf_gemm32): NW waves of RT32 32-row tiles per
// workgroup and CT32 32-column tiles; a small shape for experts of at most one small
// column block of tokens (little padding, more workgroups per CU) and a large one for the
// others (fewer re-reads of their weights and activations).
#define NW_GS     4
#define NW_DS     4
#define NW_B      8
#define GU_RT32   1
#define GU_RT32_S 2
#define GU_CT32_S 1
#define GU_CT32_B 3
#define DN_RT32   2
#define DN_RT32_S 2
#define DN_CT32_S 2
#define DN_CT32_B 3
// The small class of a gate/up over hi and lo columns (fp32 input, or z in the latent
// form): 32 tokens in two column tiles, eight waves of one 32-row tile (256 rows).  With
// the single 16-token column tile of the bf16 shape, the K3 chunk's experts of 17 to 32
// tokens (656 of 896) fell to the large class, one 96-KB-LDS workgroup a CU: 8.07 to 8.13
// ms per chunk now against 8.39 to 8.49 (four waves of 128 rows: the same; four waves of
// 256 rows, one wave a SIMD: 8.57 to 8.64).
#ifndef NW_GS2
#define NW_GS2    8
#endif
#ifndef GU_RT32_S2
#define GU_RT32_S2 1
#endif
#ifndef GU_CT32_S2
#define GU_CT32_S2 2
#endif

template <bool EXACT, int HL, int CT32, int NW, int RT32 = GU_RT32>
static void launch_gu(const PfGemmArgs &a, unsigned grid, hipStream_t s)
{
    hipLaunchKernelGGL((pf_gemm32<EXACT, 2, RT32, CT32, HL, true, NW>), dim3(grid),
                       dim3(NW * WAVE), 0, s, a);
}

template <bool EXACT, int CT32, int NW, int RT32 = DN_RT32>
static void launch_dn(const PfGemmArgs &a, unsigned grid, hipStream_t s)
{
    hipLaunchKernelGGL((pf_gemm32<EXACT, 1, RT32, CT32, 2, false, NW>), dim3(grid),
                       dim3(NW * WAVE), 0, s, a);
}

// MXFP8 mode tiles: small class 32 tokens, large class 64; four waves a workgroup, gate/up
// 128 rows (one 32-row tile a wave), down 256 (two)
#define MX_CT_S 1
#define MX_CT_B 2
#define MX_NW   4
#ifndef MX_GU_RT32_S
#define MX_GU_RT32_S 1     // 32-row tiles a wave, small-class gate/up
#endif
#ifndef MX_DN_RT32_S
#define MX_DN_RT32_S 2     // the same, small-class down
#endif

static inline unsigned round8(size_t n) { return (unsigned)((n + 7) & ~(size_t)7); }

// stages of the dense GEMM's LDS ring (32 KB each): two, so that two workgroups share a
// CU (measured at 2048 x 7168 x 7168: 325 us, against 371 with three stages and 365 with
// four, one workgroup a CU)
#define DENSE_NS 2
// wave tiles (32 x 32 MFMA tiles per wave, four waves as 2 x 2): the gate/up products,
// and the single-matrix ones
#define DENSE_GU_RW 1
#define DENSE_GU_CW 2
#define DENSE_RW    2
#define DENSE_CW    2

// A dense product on pf_dense: NMAT matrices of R rows over a.n0 B rows, HL B columns per
// row (1: bf16 activations, 2: hi and lo parts of fp32 ones)
template <int NMAT, int RW, int CW, bool GU>
static void launch_dense(const PfGemmArgs &a, int HL, hipStream_t s)
{
    const int BM = 2 * RW * 32, BN = 2 * CW * 32;
    const unsigned grid = round8((size_t)cdiv(a.R, BM) * cdiv(a.n0, BN / HL));
    if (HL == 1)
        hipLaunchKernelGGL((pf_dense<NMAT, RW, CW, 1, GU, DENSE_NS>), dim3(grid), dim3(PF_NT), 0, s, a);
    else
        hipLaunchKernelGGL((pf_dense<NMAT, RW, CW, 2, GU, DENSE_NS>), dim3(grid), dim3(PF_NT), 0, s, a);
}

static int pf_chunk(k3x_moe_layer *L, const k3x_prefill_buf *B, float *out, const void *x,
                    int x_dtype, int T, const float *resid, int *uidx, float *uwt,
                    hipStream_t s)
{
    const k3x_cfg *c = &L->cfg;
    const int H = c->hidden, E = c->n_experts, K = c->topk, I = c->moe_inter, SI = L->SI;
    const int X = L->XL;                                 // the routed experts' width
    const int TK = T * K;
    const int x_bf16 = (x_dtype == K3X_BF16);
    const int HLg = x_bf16 ? 1 : 2;                      // B columns per token of x
    const int HLr = L->lat ? 2 : HLg;                    // of the routed gate/up input
    int rc;

    hipLaunchKernelGGL(pf_split, dim3(pf_split_grid(T, H)), dim3(PF_NT), 0, s,
                       x, x_bf16, T, H, H, B->xhl, B->counts, E);
    if ((rc = launch_ok())) return rc;

    // The shared expert (bf16 weights, every token) needs only the split activations: its
    // gate/up and down run on the layer's side stream, forked right after the split, beside
    // the router, the dispatch and the routed GEMMs on s (measured against forking after
    // the dispatch, after the large experts' gate/up or after all routed gate/up: 3.83
    // against 3.83, 3.88 and 3.91 ms at 2048 tokens).  Its T rows follow the TK routed rows
    // in y, which nothing on s writes.
    bool forked = false;
    // The library path (bf16 rows, 2*SI <= H, a kernel for each shape): the gate/up product
    // into fp32 rows [T][2*SI] held in the shared rows of y (nothing else writes them before
    // the down product, which overwrites them), SiTU into bf16 hi and lo rows [T][SI] (in
    // act_sh), then the down product as two GEMMs, hi then lo accumulated, into the shared
    // rows of y.
    const bool lib = L->blas && !B->no_lib;
    const bool sh_blas = SI > 0 && lib && L->sh_gu_rm && x_bf16 &&
                         k3x_blas_ready(L->device, H, 2 * SI, T, 0) == 0 &&
                         k3x_blas_ready(L->device, SI, H, T, 0) == 0 &&
                         k3x_blas_ready(L->device, SI, H, T, 1) == 0;
    auto fork_shared = [&]() -> int {
        if (SI <= 0) return 0;
        hipStream_t side = (hipStream_t)L->pf_side;
        if (hipEventRecord((hipEvent_t)L->pf_ev[0], s) != hipSuccess ||
            hipStreamWaitEvent(side, (hipEvent_t)L->pf_ev[0], 0) != hipSuccess)
            return K3X_E_HIP;
        if (sh_blas) {
            float *ysh = B->y + (size_t)TK * H;
            uint16_t *ahi = B->act_sh, *alo = B->act_sh + (size_t)T * SI;
            int r = k3x_blas_gemm_bf16(L->device, L->sh_gu_rm, H, 2 * SI, ysh, 2 * SI,
                                       (const uint16_t *)x, H, T, 0, side);
            if (!r) r = k3x_dev_glu_rows(ysh, T, SI, L->b1, L->b2, ahi, alo, side);
            if (!r) r = k3x_blas_gemm_bf16(L->device, L->sh_down_rm, SI, H, ysh, H, ahi, SI, T, 0,
                                           side);
            if (!r) r = k3x_blas_gemm_bf16(L->device, L->sh_down_rm, SI, H, ysh, H, alo, SI, T, 1,
                                           side);
            if (hipEventRecord((hipEvent_t)L->pf_ev[1], side) != hipSuccess) return K3X_E_HIP;
            if (r) {
                (void)hipStreamWaitEvent(s, (hipEvent_t)L->pf_ev[1], 0);
                return r;
            }
            forked = true;
            return 0;
        }
        PfGemmArgs sg;
        memset(&sg, 0, sizeof sg);
        sg.wm[0] = (const uint8_t *)L->sh_gate; sg.wm[1] = (const uint8_t *)L->sh_up;
        sg.R = SI; sg.K = H; sg.n0 = T;
        sg.bsrc = B->xhl; sg.brows = T; sg.row_base = 0;
        sg.act = B->act_sh; sg.arows = T; sg.out_base = 0;
        sg.b1 = L->b1; sg.b2 = L->b2;
        launch_dense<2, DENSE_GU_RW, DENSE_GU_CW, true>(sg, HLg, side);
        int r = launch_ok();
        PfGemmArgs sd;
        memset(&sd, 0, sizeof sd);
        sd.wm[0] = (const uint8_t *)L->sh_down; sd.R = H; sd.K = SI; sd.n0 = T;
        sd.bsrc = B->act_sh; sd.brows = T; sd.row_base = 0;
        sd.y = B->y; sd.out_base = TK;
        if (!r) {
            launch_dense<1, DENSE_RW, DENSE_CW, false>(sd, 2, side);
            r = launch_ok();
        }
        // recorded even after a failed launch, so that s can always join the side stream
        if (hipEventRecord((hipEvent_t)L->pf_ev[1], side) != hipSuccess) return K3X_E_HIP;
        if (r) {
            (void)hipStreamWaitEvent(s, (hipEvent_t)L->pf_ev[1], 0);
            return r;
        }
        forked = true;
        return 0;
    };
    // from the fork on, a failed launch joins the side stream before it returns
#define PF_RET(e) do { const int e_ = (e); \
        if (forked) (void)hipStreamWaitEvent(s, (hipEvent_t)L->pf_ev[1], 0); return e_; } while (0)
    if ((rc = fork_shared())) return rc;

    PfRouterArgs ar;
    ar.x = x; ar.x_bf16 = x_bf16; ar.W = L->router; ar.bias = L->bias;
    ar.T = T; ar.H = H; ar.E = E; ar.score = B->score; ar.choice = B->choice;
    hipLaunchKernelGGL(pf_router, dim3(cdiv(T, RM_T) * cdiv(E, RM_E)), dim3(RM_NT), 0, s, ar);
    if ((rc = launch_ok())) PF_RET(rc);

    PfTopkArgs at;
    at.score = B->score; at.choice = B->choice; at.T = T; at.E = E; at.K = K;
    at.renorm = c->moe_renorm; at.routed_scale = c->routed_scale;
    at.idx = B->idx; at.wt = B->wt; at.uidx = uidx; at.uwt = uwt; at.counts = B->counts;
    if (E <= 128)      launch_topk<2>(at, s);
    else if (E <= 256) launch_topk<4>(at, s);
    else if (E <= 384) launch_topk<6>(at, s);
    else if (E <= 512) launch_topk<8>(at, s);
    else               launch_topk<16>(at, s);
    if ((rc = launch_ok())) PF_RET(rc);

    PfScanArgs sa;
    sa.counts = B->counts; sa.E = E; sa.offsets = B->offsets; sa.cursor = B->cursor;
    sa.tb[0] = B->tb_gu; sa.tb[1] = B->tb_dn;
    const bool mx = L->pf_mode == K3X_PREFILL_MXFP8;
    sa.tpb_s[0] = mx ? MX_CT_S * 32 : (HLr == 1 ? GU_CT32_S : GU_CT32_S2) * 32 / HLr;
    sa.tpb_b[0] = mx ? MX_CT_B * 32 : GU_CT32_B * 32 / HLr;
    sa.nrb_s[0] = cdiv(I, mx ? MX_NW * MX_GU_RT32_S * 32
                             : (HLr == 1 ? NW_GS * GU_RT32_S : NW_GS2 * GU_RT32_S2) * 32);
    sa.nrb_b[0] = cdiv(I, (mx ? MX_NW : NW_B) * GU_RT32 * 32);
    sa.tpb_s[1] = mx ? MX_CT_S * 32 : DN_CT32_S * 32 / 2;
    sa.tpb_b[1] = mx ? MX_CT_B * 32 : DN_CT32_B * 32 / 2;
    sa.nrb_s[1] = cdiv(X, mx ? MX_NW * MX_DN_RT32_S * 32 : NW_DS * DN_RT32_S * 32);
    sa.nrb_b[1] = cdiv(X, (mx ? MX_NW : NW_B) * DN_RT32 * 32);
    hipLaunchKernelGGL(pf_scan, dim3(1), dim3(1024), 0, s, sa);
    if ((rc = launch_ok())) PF_RET(rc);
    hipLaunchKernelGGL(pf_scatter, dim3(cdiv(TK, PF_NT)), dim3(PF_NT), 0, s, B->idx, B->wt, TK, K,
                       E, B->offsets, B->cursor, B->perm_tok, B->perm_w, B->pos_of);
    if ((rc = launch_ok())) PF_RET(rc);
    hipLaunchKernelGGL(pf_tiles, dim3(E), dim3(PF_NT), 0, s, B->counts, B->offsets, sa,
                       (int4 *)B->desc_gu, (int4 *)B->desc_dn);
    if ((rc = launch_ok())) PF_RET(rc);
    if (L->lat) {
        // z = down . x for every token (k3_mmw_batch, k3_ops.c:1871): a plain product, on
        // the library where it serves the shape (bf16 rows), else the dense kernel
        if (lib && x_bf16 && k3x_blas_ready(L->device, H, X, T, 0) == 0) {
            if ((rc = k3x_blas_gemm_bf16(L->device, L->ldown_rm, H, X, B->zf, X,
                                         (const uint16_t *)x, H, T, 0, s)))
                PF_RET(rc);
        } else {
            PfGemmArgs zg;
            memset(&zg, 0, sizeof zg);
            zg.wm[0] = (const uint8_t *)L->ldown; zg.R = X; zg.K = H; zg.n0 = T;
            zg.bsrc = B->xhl; zg.brows = T; zg.row_base = 0;
            zg.y = B->zf; zg.out_base = 0;
            launch_dense<1, DENSE_RW, DENSE_CW, false>(zg, HLg, s);
            if ((rc = launch_ok())) PF_RET(rc);
        }
    }
    // MXFP8 mode: the routed input quantised in permuted order, codes then scales in xp;
    // the gate/up output's codes then scales in act
    uint8_t *xq8 = (uint8_t *)B->xp, *xs8 = xq8 + (((size_t)TK * X + 255) & ~(size_t)255);
    uint8_t *aq8 = (uint8_t *)B->act, *as8 = aq8 + (((size_t)TK * I + 255) & ~(size_t)255);
    if (mx) {
        const void *src = L->lat ? (const void *)B->zf : x;
        hipLaunchKernelGGL(pf_mx8_rows, dim3(pf_mx8_grid(TK, X)), dim3(PF_NT), 0, s,
                           src, L->lat ? 0 : x_bf16, X, X, B->perm_tok, TK, xq8, xs8);
    } else {
        // the routed input's planes in permuted order, from x's rows (z's in the latent
        // form), so that one k-group of an expert's segment is contiguous
        const void *src = L->lat ? (const void *)B->zf : x;
        hipLaunchKernelGGL(pf_gather, dim3(pf_gather_grid(TK, X)), dim3(PF_NT), 0, s,
                           src, L->lat ? 0 : x_bf16, TK, X, X, B->xp, B->perm_tok);
    }
    if ((rc = launch_ok())) PF_RET(rc);

    // grids: upper bounds of each list (a small expert has one column block; large ones
    // number at most TK / (tpb_s + 1)); surplus workgroups leave at once
    unsigned grid_s[2], grid_b[2];
    for (int m = 0; m < 2; m++) {
        const size_t nbig = (size_t)TK / (sa.tpb_s[m] + 1);
        grid_s[m] = round8((size_t)sa.nrb_s[m] * E);
        grid_b[m] = round8((size_t)sa.nrb_b[m] * (cdiv(TK, sa.tpb_b[m]) + (nbig < (size_t)E ? nbig : (size_t)E)));
    }
    if (grid_s[0] + grid_b[0] > (unsigned)B->ndesc_gu || grid_s[1] + grid_b[1] > (unsigned)B->ndesc_dn)
        PF_RET(K3X_E_SHAPE);

    // routed gate/up: B rows are the permuted activation rows
    PfGemmArgs g;
    memset(&g, 0, sizeof g);
    g.wm[0] = L->experts + L->gate_off; g.wm[1] = L->experts + L->up_off;
    g.gstride = L->expert_bytes;
    g.R = I; g.K = X; g.desc = (const int4 *)B->desc_gu;
    g.bsrc = B->xp; g.brows = TK; g.perm = NULL; g.row_base = 0;
    g.pw = B->perm_w; g.act = B->act; g.arows = TK; g.out_base = 0;
    g.b1 = L->b1; g.b2 = L->b2;
    const bool ex_gu = (L->special & 3) != 0;
    if (mx) {
        g.b8 = xq8; g.b8s = (const uint32_t *)xs8; g.o8 = aq8; g.o8s = as8;
    }
    PfGemmArgs gb = g;
    g.ntile = B->tb_gu + E;
    gb.ntile = B->tb_gu + 2 * E + 1; gb.dbase = B->tb_gu + E;
    // the large-expert tiles on s.  In the exact mode the small ones run on the side
    // stream after the shared expert (forked here, after the routed input is written),
    // beside the large ones, and join before the combine: 3.56 to 3.58 against 3.61 ms
    // per 2048-token chunk; the MXFP8 products measured slower that way (2.92 against
    // 2.80 ms) and stay on s.
    hipStream_t ss = s;
    const bool split = forked && !mx;
    if (split) {
        if (hipEventRecord((hipEvent_t)L->pf_ev[0], s) != hipSuccess ||
            hipStreamWaitEvent((hipStream_t)L->pf_side, (hipEvent_t)L->pf_ev[0], 0) != hipSuccess)
            PF_RET(K3X_E_HIP);
        ss = (hipStream_t)L->pf_side;
    }
    if (mx) {
        hipLaunchKernelGGL((pf_gemm_mx<2, GU_RT32, MX_CT_B, true, MX_NW>), dim3(grid_b[0]), dim3(MX_NW * WAVE), 0, s, gb);
    } else if (ex_gu) {
        if (HLr == 1) launch_gu<true, 1, GU_CT32_B, NW_B>(gb, grid_b[0], s);
        else          launch_gu<true, 2, GU_CT32_B, NW_B>(gb, grid_b[0], s);
    } else {
        if (HLr == 1) launch_gu<false, 1, GU_CT32_B, NW_B>(gb, grid_b[0], s);
        else          launch_gu<false, 2, GU_CT32_B, NW_B>(gb, grid_b[0], s);
    }
    if ((rc = launch_ok())) PF_RET(rc);

    // routed down: B rows are the activation rows, in permuted order
    PfGemmArgs d;
    memset(&d, 0, sizeof d);
    d.wm[0] = L->experts + L->down_off; d.gstride = L->expert_bytes;
    d.R = X; d.K = I; d.desc = (const int4 *)B->desc_dn;
    d.bsrc = B->act; d.brows = TK; d.perm = NULL; d.row_base = 0;
    d.y = B->y; d.out_base = 0;
    if (mx) { d.b8 = aq8; d.b8s = (const uint32_t *)as8; }
    PfGemmArgs db = d;
    d.ntile = B->tb_dn + E;
    db.ntile = B->tb_dn + 2 * E + 1; db.dbase = B->tb_dn + E;
    if (mx) {
        hipLaunchKernelGGL((pf_gemm_mx<2, MX_GU_RT32_S, MX_CT_S, true, MX_NW>), dim3(grid_s[0]), dim3(MX_NW * WAVE), 0, ss, g);
    } else if (ex_gu) {
        if (HLr == 1) launch_gu<true, 1, GU_CT32_S, NW_GS, GU_RT32_S>(g, grid_s[0], ss);
        else          launch_gu<true, 2, GU_CT32_S2, NW_GS2, GU_RT32_S2>(g, grid_s[0], ss);
    } else {
        if (HLr == 1) launch_gu<false, 1, GU_CT32_S, NW_GS, GU_RT32_S>(g, grid_s[0], ss);
        else          launch_gu<false, 2, GU_CT32_S2, NW_GS2, GU_RT32_S2>(g, grid_s[0], ss);
    }
    rc = launch_ok();
    if (!rc) {
        if (mx) hipLaunchKernelGGL((pf_gemm_mx<1, MX_DN_RT32_S, MX_CT_S, false, MX_NW>), dim3(grid_s[1]), dim3(MX_NW * WAVE), 0, ss, d);
        else if (L->special & 4) launch_dn<true, DN_CT32_S, NW_DS, DN_RT32_S>(d, grid_s[1], ss);
        else                     launch_dn<false, DN_CT32_S, NW_DS, DN_RT32_S>(d, grid_s[1], ss);
        rc = launch_ok();
    }
    // recorded even after a failed launch, so that s can always join the side stream
    if (split && hipEventRecord((hipEvent_t)L->pf_ev[1], ss) != hipSuccess && !rc) rc = K3X_E_HIP;
    if (rc) PF_RET(rc);
    if (mx) hipLaunchKernelGGL((pf_gemm_mx<1, DN_RT32, MX_CT_B, false, MX_NW>), dim3(grid_b[1]), dim3(MX_NW * WAVE), 0, s, db);
    else if (L->special & 4) launch_dn<true, DN_CT32_B, NW_B>(db, grid_b[1], s);
    else                     launch_dn<false, DN_CT32_B, NW_B>(db, grid_b[1], s);
    if ((rc = launch_ok())) PF_RET(rc);
    // the small experts' rows are in y: join the side stream
    if (split && hipStreamWaitEvent(s, (hipEvent_t)L->pf_ev[1], 0) != hipSuccess) return K3X_E_HIP;

    int sh_row0 = -1;
    const int *pos = B->pos_of;
    int KC = K;
    if (L->lat) {
        // the routed aggregates in top-k order (:1941-1942), their RMSNorm and hi/lo
        // planes (:1946), then the up projection (:1950) into y rows 0 .. T-1
        hipLaunchKernelGGL(pf_combine, dim3(cdiv((size_t)T * (X / 4), PF_NT)), dim3(PF_NT), 0, s,
                           B->y, B->pos_of, T, K, X, -1, (const float *)NULL, B->zf);
        if ((rc = launch_ok())) PF_RET(rc);
        // the up projection: a plain product over the normalised aggregates' hi and lo
        // parts, on the library where it serves the shapes (rows [T][X] of each part),
        // else the dense kernel (k-group planes)
        const bool up_blas = lib && k3x_blas_ready(L->device, X, H, T, 0) == 0 &&
                             k3x_blas_ready(L->device, X, H, T, 1) == 0;
        hipLaunchKernelGGL(pf_latnorm, dim3(T), dim3(PF_NT), 0, s, B->zf,
                           c->latent_norm ? L->lnw : (const float *)NULL, c->rms_eps, T, X, B->zhl,
                           up_blas ? 1 : 0);
        if ((rc = launch_ok())) PF_RET(rc);
        if (up_blas) {
            if ((rc = k3x_blas_gemm_bf16(L->device, L->lup_rm, X, H, B->y, H, B->zhl, X, T, 0,
                                         s)) ||
                (rc = k3x_blas_gemm_bf16(L->device, L->lup_rm, X, H, B->y, H,
                                         B->zhl + (size_t)T * X, X, T, 1, s)))
                PF_RET(rc);
        } else {
            PfGemmArgs ug;
            memset(&ug, 0, sizeof ug);
            ug.wm[0] = (const uint8_t *)L->lup; ug.R = H; ug.K = X; ug.n0 = T;
            ug.bsrc = B->zhl; ug.brows = T; ug.row_base = 0;
            ug.y = B->y; ug.out_base = 0;
            launch_dense<1, DENSE_RW, DENSE_CW, false>(ug, 2, s);
            if ((rc = launch_ok())) PF_RET(rc);
        }
        pos = NULL;
        KC = 1;
    }
    if (forked) {
        // the shared rows are in y: join the shared stream
        if (hipStreamWaitEvent(s, (hipEvent_t)L->pf_ev[1], 0) != hipSuccess) return K3X_E_HIP;
        sh_row0 = TK;
    }

    hipLaunchKernelGGL(pf_combine, dim3(cdiv((size_t)T * (H / 4), PF_NT)), dim3(PF_NT), 0, s,
                       B->y, pos, T, KC, H, sh_row0, resid, out);
    return launch_ok();
}
#undef PF_RET

// Prefill: the pipeline over chunks of up to K3X_PF_CHUNK tokens.  Each token's result
// depends only on its own routing, so the chunking changes no result.
extern "C" int k3x_dev_prefill(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                               int T, const float *resid, int *idx, float *wt, void *stream)
{
    const int H = L->cfg.hidden, K = L->cfg.topk;
    const size_t es = (x_dtype == K3X_BF16) ? 2 : 4;
    const int chunk = k3x_pf_chunk_tokens(L);
    int rc = k3x_pf_reserve(L, T, stream);
    if (rc) return rc;
    for (int t0 = 0; t0 < T; t0 += chunk) {
        const int n = T - t0 < chunk ? T - t0 : chunk;
        rc = pf_chunk(L, &L->pf, out + (size_t)t0 * H, (const char *)x + (size_t)t0 * H * es, x_dtype, n,
                      resid ? resid + (size_t)t0 * H : NULL, idx ? idx + (size_t)t0 * K : NULL,
                      wt ? wt + (size_t)t0 * K : NULL, (hipStream_t)stream);
        if (rc) return rc;
    }
    return 0;
}

// The router alone (k3x_moe_route): per chunk, every (token, expert) logit as the
// reference's chain (pf_router) and each token's top-k into the caller's arrays (pf_topk,
// no histogram).
extern "C" int k3x_dev_route(k3x_moe_layer *L, int *idx, float *wt, const void *x, int x_dtype,
                             int T, void *stream)
{
    const k3x_cfg *c = &L->cfg;
    const int H = c->hidden, E = c->n_experts, K = c->topk;
    const size_t es = (x_dtype == K3X_BF16) ? 2 : 4;
    const int chunk = k3x_pf_chunk_tokens(L);
    hipStream_t s = (hipStream_t)stream;
    int rc = k3x_pf_reserve(L, T, stream);
    if (rc) return rc;
    for (int t0 = 0; t0 < T; t0 += chunk) {
        const int n = T - t0 < chunk ? T - t0 : chunk;
        PfRouterArgs ar;
        ar.x = (const char *)x + (size_t)t0 * H * es; ar.x_bf16 = x_dtype == K3X_BF16;
        ar.W = L->router; ar.bias = L->bias; ar.T = n; ar.H = H; ar.E = E;
        ar.score = L->pf.score; ar.choice = L->pf.choice;
        hipLaunchKernelGGL(pf_router, dim3(cdiv(n, RM_T) * cdiv(E, RM_E)), dim3(RM_NT), 0, s, ar);
        if ((rc = launch_ok())) return rc;
        PfTopkArgs at;
        at.score = L->pf.score; at.choice = L->pf.choice; at.T = n; at.E = E; at.K = K;
        at.renorm = c->moe_renorm; at.routed_scale = c->routed_scale;
        at.idx = idx + (size_t)t0 * K; at.wt = wt + (size_t)t0 * K;
        at.uidx = NULL; at.uwt = NULL; at.counts = NULL;
        if (E <= 128)      launch_topk<2>(at, s);
        else if (E <= 256) launch_topk<4>(at, s);
        else if (E <= 384) launch_topk<6>(at, s);
        else if (E <= 512) launch_topk<8>(at, s);
        else               launch_topk<16>(at, s);
        if ((rc = launch_ok())) return rc;
    }
    return 0;
}

// ------------------------------------------------------------------ without allocation
// The prefill pipeline for callers that cannot allocate (graph capture, serving loops):
// its working buffers come from this static device array instead of the layer's. Each
// device holds its own copy at its own address, found once per device by
// hipGetSymbolAddress; host code uses that address, never the array's name.  Every call
// on a device shares the device's copy (calls that overlap on one device race); no
// kernel needs it to start cleared (the histogram is zeroed by pf_split each run).
static __device__ __align__(256) uint8_t scratch[K3X_NOALLOC_BYTES];

#define K3X_MAX_DEVICES 64
static void *g_scratch[K3X_MAX_DEVICES];
static std::mutex g_scratch_mu;

static void *scratch_ptr(int device)
{
    if (device < 0 || device >= K3X_MAX_DEVICES) return NULL;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
        void *p = NULL;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "k3x: hipGetSymbolAddress(scratch) on device %d failed: %s\n",
                    device, hipGetErrorString(e));
            return NULL;
        }
        g_scratch[device] = p;
    }
    return g_scratch[device];
}

extern "C" int k3x_dev_prefill_noalloc(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                                       int T, const float *resid, int *idx, float *wt,
                                       void *stream)
{
    const int chunk = k3x_pf_chunk_tokens(L);
    const size_t need = k3x_pf_layout(L, T, NULL, NULL);
    if (T > chunk || need > K3X_NOALLOC_BYTES) {
        fprintf(stderr, "k3x: a prefill of %d tokens needs %zu bytes of working memory; the "
                        "static array holds %u (and one run at most %d tokens)\n",
                T, need, K3X_NOALLOC_BYTES, chunk);
        return K3X_E_SHAPE;
    }
    if (hipSetDevice(L->device) != hipSuccess) return K3X_E_HIP;
    void *p = scratch_ptr(L->device);
    if (!p) return K3X_E_HIP;
    k3x_prefill_buf B;
    memset(&B, 0, sizeof B);
    k3x_pf_layout(L, T, (char *)p, &B);
    B.no_lib = 1;
    return pf_chunk(L, &B, out, x, x_dtype, T, resid, idx, wt, (hipStream_t)stream);
}

// ------------------------------------------------------------------ trunk products
// Y[t*ldy + o] = W[o] . X[t*ldx] for T activation rows (k3_mmw_batch_ld): X's hi/lo
// planes into `planes` (T * in * 4 bytes), then the dense bf16 GEMM.
extern "C" int k3x_dev_trunk_gemm(const uint16_t *W, int in, int out, float *y, int ldy,
                                  const void *x, int x_dtype, int ldx, int T, uint16_t *planes,
                                  void *stream)
{
    hipStream_t s = (hipStream_t)stream;
    const int x_bf16 = (x_dtype == K3X_BF16), HL = x_bf16 ? 1 : 2;
    hipLaunchKernelGGL(pf_split, dim3(pf_split_grid(T, in)), dim3(PF_NT), 0, s,
                       x, x_bf16, T, in, ldx, planes, (int *)NULL, 0);
    int rc = launch_ok();
    if (rc) return rc;
    PfGemmArgs g;
    memset(&g, 0, sizeof g);
    g.wm[0] = (const uint8_t *)W; g.R = out; g.K = in; g.n0 = T;
    g.bsrc = planes; g.brows = T; g.row_base = 0;
    g.y = y; g.out_base = 0; g.ldy = ldy;
    launch_dense<1, DENSE_RW, DENSE_CW, false>(g, HL, s);
    return launch_ok();
}
