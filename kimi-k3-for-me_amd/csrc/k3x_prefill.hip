// k3x_prefill.hip - the prefill path of the MoE block (more than 8 tokens per call):
//
//   pf_split    activations to bf16 hi/lo rows (the GEMMs' B source); clears the histogram
//   pf_router   router logits of every (token, expert) in double, one sequential chain per
//               pair in the reference's order (k3_router, k3_ops.c:1666-1688), so they
//               are the reference's logits bit for bit; sigmoid, + bias (:1691-1692)
//   pf_topk     each token's top-k by one wave (:1700-1716) and the per-expert histogram
//   pf_scan     per-expert offsets (prefix sum) and the GEMM tile lists
//   pf_scatter  each (token, slot) to its row in its expert's segment
//   pf_gemm     grouped GEMMs: gate/up of every expert segment with SwiGLU and the
//               routing weight (k3_matmul_mxfp4 :3323-3776, k3_situ_glu :148-161), then
//               down; the shared expert (bf16, :1848-1860) through the same kernel
//   pf_combine  per token, the K expert rows summed in top-k order (:1941-1942), plus
//               the shared row (:1951), plus an optional residual
//
// The GEMMs run on v_mfma_f32_16x16x32_bf16 with MXFP4 weights dequantised exactly in
// registers; the activations are bf16 hi + lo pairs (hi only when the input is bf16,
// whose lo part is zero), so products are exact and only the fp32 accumulation rounds.
#include "k3x_device.h"
#include "k3x_topk.h"

#include <string.h>

#define PF_NT 256
#define PF_CHUNK 4096          // tokens per pipeline run

// ------------------------------------------------------------------ split
// x [T][H] (bf16 or fp32) -> xhl [T][H/8][2][8] bf16: per 8 elements the hi halves, then
// the lo halves.  Block 0 also clears the expert histogram.
__global__ void __launch_bounds__(PF_NT) pf_split(const void *x, int x_bf16, int T, int H,
                                                  uint16_t *xhl, int *counts, int E)
{
    if (blockIdx.x == 0)
        for (int e = threadIdx.x; e < E; e += PF_NT) counts[e] = 0;
    const size_t g = (size_t)blockIdx.x * PF_NT + threadIdx.x;
    if (g >= (size_t)T * (H >> 3)) return;
    float v[8];
    load_x8(x, x_bf16, g * 8, v);
    uint32_t hi[8], lo[8];
#pragma unroll
    for (int j = 0; j < 8; j++) split_bf16(v[j], hi[j], lo[j]);
    u32x4 h, l;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        h[j] = hi[2 * j] | (hi[2 * j + 1] << 16);
        l[j] = lo[2 * j] | (lo[2 * j + 1] << 16);
    }
    *(u32x4 *)(xhl + g * 16) = h;
    *(u32x4 *)(xhl + g * 16 + 8) = l;
}

// ------------------------------------------------------------------ router
// Logits of a 64-token x 32-expert tile; each thread owns 4 tokens x 2 experts and runs
// their chains in double over i = 0 .. H-1 in order (a product of two floats is exact in
// double, so the chain equals the reference's fma-free loop).  K is staged 32 at a time
// in LDS as double.
#define RT_TOK 64
#define RT_EXP 32
#define RT_KC  32

struct PfRouterArgs {
    const void  *x;
    int          x_bf16;
    const float *W, *bias;
    int          T, H, E;
    float       *score, *choice;
};

__global__ void __launch_bounds__(PF_NT) pf_router(PfRouterArgs a)
{
    __shared__ double xs[RT_KC][RT_TOK];
    __shared__ double ws[RT_KC][RT_EXP];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int tok0 = blockIdx.x * RT_TOK, e0 = blockIdx.y * RT_EXP;
    double acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i][0] = acc[i][1] = 0.0;
    for (int k0 = 0; k0 < a.H; k0 += RT_KC) {
        // x tile: 64 tokens x 32 k, 8 per thread; W tile: 32 experts x 32 k, 4 per thread
        for (int f = threadIdx.x; f < RT_TOK * RT_KC / 4; f += PF_NT) {
            const int t = f / (RT_KC / 4), kk = (f % (RT_KC / 4)) * 4;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (tok0 + t < a.T) load_x4(a.x, a.x_bf16, (size_t)(tok0 + t) * a.H + k0 + kk, v);
#pragma unroll
            for (int j = 0; j < 4; j++) xs[kk + j][t] = (double)v[j];
        }
        for (int f = threadIdx.x; f < RT_EXP * RT_KC / 4; f += PF_NT) {
            const int e = f / (RT_KC / 4), kk = (f % (RT_KC / 4)) * 4;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (e0 + e < a.E) v = *(const f32x4 *)(a.W + (size_t)(e0 + e) * a.H + k0 + kk);
#pragma unroll
            for (int j = 0; j < 4; j++) ws[kk + j][e] = (double)v[j];
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < RT_KC; k++) {
            double xv[4], wv[2];
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = xs[k][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 2; j++) wv[j] = ws[k][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = __fma_rn(xv[i], wv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int t = tok0 + ty + 16 * i, e = e0 + tx + 16 * j;
            if (t < a.T && e < a.E) {
                const float sc = sigmoid_ref((float)acc[i][j]);
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

template <int NE>
__global__ void __launch_bounds__(PF_NT) pf_topk(PfTopkArgs a)
{
    __shared__ int      s_idx[PF_NT / WAVE][K3X_MAX_TOPK];
    __shared__ float    s_w[PF_NT / WAVE][K3X_MAX_TOPK];
    __shared__ uint64_t s_key[PF_NT / WAVE][K3X_MAX_TOPK];
    __shared__ int      s_e[PF_NT / WAVE][K3X_MAX_TOPK];
    __shared__ float    s_sc[PF_NT / WAVE][K3X_MAX_TOPK];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int t = blockIdx.x * (PF_NT / WAVE) + wave;
    if (t >= a.T) return;
    const rsrc_t cr = make_rsrc(a.choice, (uint32_t)((size_t)a.T * a.E * 4));
    const rsrc_t sr = make_rsrc(a.score, (uint32_t)((size_t)a.T * a.E * 4));
    wave_topk<NE>(cr, sr, (uint32_t)((size_t)t * a.E * 4), a.E, a.K, a.renorm, a.routed_scale,
                  s_idx[wave], s_w[wave], s_key[wave], s_e[wave], s_sc[wave], lane);
    if (lane < a.K) {
        const size_t o = (size_t)t * a.K + lane;
        const int e = s_idx[wave][lane];
        a.idx[o] = e;
        a.wt[o] = s_w[wave][lane];
        if (a.uidx) { a.uidx[o] = e; a.uwt[o] = s_w[wave][lane]; }
        atomicAdd(&a.counts[e], 1);
    }
}

// ------------------------------------------------------------------ scan
// One workgroup: offsets[e] = sum of counts below e; tile bases of the two routed GEMMs
// (expert e gets nrb x ceil(count/tpb) tiles); cursors cleared.
__global__ void __launch_bounds__(1024) pf_scan(const int *counts, int E, int *offsets,
                                                int *cursor, int *tb_gu, int tpb_gu, int nrb_gu,
                                                int *tb_dn, int tpb_dn, int nrb_dn)
{
    __shared__ int s_c[1024];
    for (int e = threadIdx.x; e < E; e += 1024) {
        s_c[e] = counts[e];
        cursor[e] = 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int o = 0, g = 0, d = 0;
        for (int e = 0; e < E; e++) {
            const int c = s_c[e];
            offsets[e] = o; tb_gu[e] = g; tb_dn[e] = d;
            o += c;
            g += nrb_gu * ((c + tpb_gu - 1) / tpb_gu);
            d += nrb_dn * ((c + tpb_dn - 1) / tpb_dn);
        }
        offsets[E] = o; tb_gu[E] = g; tb_dn[E] = d;
    }
}

// ------------------------------------------------------------------ scatter
__global__ void __launch_bounds__(PF_NT) pf_scatter(const int *idx, const float *wt, int TK, int K,
                                                    const int *offsets, int *cursor,
                                                    int *perm_tok, float *perm_w, int *pos_of)
{
    const int i = blockIdx.x * PF_NT + threadIdx.x;
    if (i >= TK) return;
    const int e = idx[i];
    const int p = offsets[e] + atomicAdd(&cursor[e], 1);
    perm_tok[p] = i / K;
    perm_w[p] = wt[i];
    pos_of[i] = p;
}

// ------------------------------------------------------------------ grouped GEMM
// Y[p][r] = sum_k W_g[r][k] B[p][k] over the permuted rows p of group g (an expert's
// segment, or all tokens for the shared expert).  A workgroup computes a tile of
// NW*RT*16 weight rows (NMAT matrices: gate and up together) by one column block of
// CT*16 B columns (TPB tokens; HL columns per token: hi, or hi and lo); its four waves
// own RT row tiles each and share the column block, staged in LDS one 128-wide quad at
// a time (double buffered).  Each thread keeps three quads of loads in flight (weights
// for its row tiles, its share of the next B quads), issued in quad order so that one
// wait per quad, before the LDS store of the next B quad, releases exactly one quad.
struct PfGemmArgs {
    const uint8_t  *wm[2];      // group 0's matrices (gate, up) or (down), tiled
    size_t          gstride;    // bytes between groups' records
    int             R, K;       // rows and inner dimension of each matrix
    int             G;          // groups
    const int      *gcount;     // [G] rows per group, or NULL: n0 rows in group 0
    const int      *goff;       // [G] first permuted row of each group
    const int      *tbase;      // [G+1] first tile of each group
    int             n0;
    const uint16_t *bsrc;       // B source rows [*][K/8][2][8] bf16
    uint32_t        bsrc_bytes;
    const int      *perm;       // B source row of permuted row p, or NULL: row_base + p
    int             row_base;
    const float    *pw;         // weight of permuted row p (gate/up epilogue), or NULL: 1
    uint16_t       *act;        // gate/up: output rows [*][R/8][2][8] bf16 hi/lo
    float          *y;          // down: output rows [*][R] fp32
    int             out_base;   // output row = out_base + p
};

template <bool FP4, int NMAT, int RT>
struct AQuad;

template <int NMAT, int RT>
struct AQuad<true, NMAT, RT> {              // fp4: 16 code bytes + the scale dword per tile
    u32x4    c[NMAT][RT];
    uint32_t s[NMAT][RT];
};

template <int NMAT, int RT>
struct AQuad<false, NMAT, RT> {             // bf16: 4 x 16 bytes per tile
    u32x4 c[NMAT][RT][4];
};

template <bool FP4, bool EXACT, int NMAT, int RT, int CT, int HL, bool GU>
__global__ void __launch_bounds__(PF_NT, 2) pf_gemm(PfGemmArgs a)
{
    constexpr int NW = PF_NT / WAVE;
    constexpr int NCOL = CT * 16;
    constexpr int TPB = NCOL / HL;
    constexpr int RPB = NW * RT * 16;
    constexpr int QB = NCOL * 128 * 2;             // B bytes per quad
    constexpr int NST = QB / (PF_NT * 16);         // B pieces per thread per quad
    constexpr int RING = 3;
    static_assert(NST * PF_NT * 16 == QB, "B quad must split evenly");
    __shared__ __attribute__((aligned(16))) uint8_t sB[2 * QB];

    const int wave = wave_id(), lane = threadIdx.x % WAVE;
    const int nrb = (a.R + RPB - 1) / RPB;
    // ---- which tile
    int g = 0, cnt = a.n0, off = 0, t0 = 0;
    const int tile = blockIdx.x;
    if (a.gcount) {
        if (tile >= a.tbase[a.G]) return;
        int lo = 0, hi = a.G - 1;                  // the last group whose first tile <= tile
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.tbase[mid] <= tile) lo = mid; else hi = mid - 1;
        }
        g = lo; cnt = a.gcount[g]; off = a.goff[g]; t0 = a.tbase[g];
    } else if (tile >= nrb * ((cnt + TPB - 1) / TPB)) {
        return;
    }
    const int nc = (cnt + TPB - 1) / TPB;
    const int rel = tile - t0, rb = rel / nc, cb = rel % nc;
    const int ntok = min(TPB, cnt - cb * TPB);
    const int p0 = off + cb * TPB;
    const int nQ = a.K >> 7;

    // ---- this wave's weight tiles
    const uint32_t tbytes = FP4 ? (uint32_t)fp4_tile_bytes(a.K) : (uint32_t)a.K * 32u;
    rsrc_t ra[NMAT][RT];
    bool rvalid[RT];
#pragma unroll
    for (int i = 0; i < RT; i++) {
        const int rt = (rb * NW + wave) * RT + i;
        rvalid[i] = rt < (a.R >> 4);
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            ra[m][i] = make_rsrc(a.wm[m] + (size_t)g * a.gstride + (size_t)rt * tbytes,
                                 rvalid[i] ? tbytes : 0u);
    }
    // ---- this thread's B pieces: piece f = (n*16 + g8)*HL + hl of each quad
    const rsrc_t rb_src = make_rsrc(a.bsrc, a.bsrc_bytes);
    uint32_t soff[NST], doff[NST];
#pragma unroll
    for (int s = 0; s < NST; s++) {
        const int f = threadIdx.x + PF_NT * s;
        const int n = f / (16 * HL), r2 = f % (16 * HL), g8 = r2 / HL, hl = r2 % HL;
        const int kq = g8 >> 2, t = g8 & 3;
        doff[s] = (uint32_t)(((t * 4 + kq) * NCOL + n * HL + hl) * 16);
        if (n < ntok) {
            const int row = a.perm ? a.perm[p0 + n] : a.row_base + p0 + n;
            soff[s] = (uint32_t)row * (uint32_t)(a.K * 4) + (uint32_t)(g8 * 32 + hl * 16);
        } else {
            soff[s] = K3X_OOB;
        }
    }

    AQuad<FP4, NMAT, RT> A[RING];
    u32x4 Bq[RING][NST];
    auto ld = [&](int slot, int q) AI {
        const bool on = q < nQ;
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int i = 0; i < RT; i++) {
                if constexpr (FP4) {
                    const uint32_t sq = (uint32_t)(q >> 2) * 4352u;
                    const uint32_t oc = on ? sq + (uint32_t)(q & 3) * 1024u + lane * 16u : K3X_OOB;
                    const uint32_t os = on ? sq + 4096u + lane * 4u : K3X_OOB;
                    A[slot].c[m][i] = wld16(ra[m][i], oc);
                    A[slot].s[m][i] = wld4(ra[m][i], os);
                } else {
                    const uint32_t o = on ? (uint32_t)q * 4096u + lane * 16u : K3X_OOB;
#pragma unroll
                    for (int t = 0; t < 4; t++) A[slot].c[m][i][t] = wld16(ra[m][i], o + 1024u * t);
                }
            }
#pragma unroll
        for (int s = 0; s < NST; s++)
            Bq[slot][s] = bload16(rb_src, on && soff[s] != K3X_OOB ? soff[s] + (uint32_t)q * 512u : K3X_OOB);
    };
    auto stage = [&](int slot, int buf) AI {
#pragma unroll
        for (int s = 0; s < NST; s++) *(u32x4 *)(sB + buf * QB + doff[s]) = Bq[slot][s];
    };

    f32x4 acc[NMAT][RT][CT];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
            for (int c = 0; c < CT; c++) acc[m][i][c] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int n16 = lane & 15, kq = lane >> 4;
    auto compute = [&](int slot, int q, int buf) AI {
        const uint8_t *bb = sB + buf * QB;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            bf16x8 bf[CT];
#pragma unroll
            for (int c = 0; c < CT; c++)
                bf[c] = as_bf16x8(*(const u32x4 *)(bb + ((t * 4 + kq) * NCOL + c * 16 + n16) * 16));
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
                for (int i = 0; i < RT; i++) {
                    bf16x8 av;
                    if constexpr (FP4) {
                        const uint32_t sb = (A[slot].s[m][i] >> (8 * (q & 3))) & 255u;
                        av = EXACT ? dq8_exact(A[slot].c[m][i][t], sb)
                                   : dq8(A[slot].c[m][i][t], e8m0_scale(sb));
                    } else {
                        av = as_bf16x8(A[slot].c[m][i][t]);
                    }
#pragma unroll
                    for (int c = 0; c < CT; c++) acc[m][i][c] = mfma(av, bf[c], acc[m][i][c]);
                }
        }
    };

#pragma unroll
    for (int s = 0; s < RING; s++) {
        SCHED_FENCE();
        ld(s, s);
    }
    SCHED_FENCE();
    stage(0, 0);
    __syncthreads();
    int q = 0;
    for (; q + RING <= nQ; q += RING) {
#pragma unroll
        for (int s = 0; s < RING; s++) {
            compute(s, q + s, (q + s) & 1);
            SCHED_FENCE();
            ld(s, q + s + RING);
            SCHED_FENCE();
            stage((s + 1) % RING, (q + s + 1) & 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int s = 0; s < RING - 1; s++) {
        if (q + s < nQ) {
            compute(s, q + s, (q + s) & 1);
            stage((s + 1) % RING, (q + s + 1) & 1);
            __syncthreads();
        }
    }

    // ---- epilogue: lane (n16, kq) holds rows 4*kq .. 4*kq+3 of each row tile, column n16
#pragma unroll
    for (int c = 0; c < CT; c++) {
        const int col = c * 16 + n16;
        const int tl = col / HL;
        const bool writer = (HL == 1 || (col & 1) == 0) && tl < ntok;
        const int p = p0 + tl;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const int r0 = ((rb * NW + wave) * RT + i) * 16 + 4 * kq;
            float v0[4], v1[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v0[j] = acc[0][i][c][j];
                if (HL == 2) v0[j] += __shfl_xor(v0[j], 1);
                if (NMAT == 2) {
                    v1[j] = acc[NMAT - 1][i][c][j];
                    if (HL == 2) v1[j] += __shfl_xor(v1[j], 1);
                }
            }
            if (!writer || !rvalid[i]) continue;
            if (GU) {
                const float w = a.pw ? a.pw[p] : 1.0f;
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float yv = (w == 0.0f) ? 0.0f : w * swiglu(v0[j], v1[j]);
                    split_bf16(yv, hi[j], lo[j]);
                }
                uint16_t *dst = a.act + (size_t)(a.out_base + p) * (size_t)(a.R * 2) +
                                (size_t)(r0 >> 3) * 16 + (r0 & 7);
                *(u32x2 *)dst = (u32x2){hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
                *(u32x2 *)(dst + 8) = (u32x2){lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
            } else {
                float *dst = a.y + (size_t)(a.out_base + p) * a.R + r0;
                *(f32x4 *)dst = (f32x4){v0[0], v0[1], v0[2], v0[3]};
            }
        }
    }
}

// ------------------------------------------------------------------ combine
// out[t] = ((y[pos(t,0)] + y[pos(t,1)]) + ... ) + y_shared[t], then + resid.
__global__ void __launch_bounds__(PF_NT) pf_combine(const float *y, const int *pos_of, int T, int K,
                                                    int H, int sh_row0, const float *resid,
                                                    float *out)
{
    const size_t i = (size_t)blockIdx.x * PF_NT + threadIdx.x;
    const int h4 = H >> 2;
    if (i >= (size_t)T * h4) return;
    const int t = (int)(i / h4), h = (int)(i % h4) * 4;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < K; j++) s += *(const f32x4 *)(y + (size_t)pos_of[(size_t)t * K + j] * H + h);
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
    hipLaunchKernelGGL(pf_topk<NE>, dim3(cdiv(a.T, PF_NT / WAVE)), dim3(PF_NT), 0, s, a);
}

// gate/up and down launch shapes of the routed GEMMs
#define GU_RT 2
#define GU_CT 4
#define DN_RT 4
#define DN_CT 4

template <bool EXACT, int HL>
static void launch_gu_fp4(const PfGemmArgs &a, unsigned grid, hipStream_t s)
{
    hipLaunchKernelGGL((pf_gemm<true, EXACT, 2, GU_RT, GU_CT, HL, true>), dim3(grid), dim3(PF_NT), 0, s, a);
}

static int pf_chunk(k3x_moe_layer *L, float *out, const void *x, int x_dtype, int T,
                    const float *resid, int *uidx, float *uwt, hipStream_t s)
{
    const k3x_cfg *c = &L->cfg;
    k3x_prefill_buf *B = &L->pf;
    const int H = c->hidden, E = c->n_experts, K = c->topk, I = c->moe_inter, SI = L->SI;
    const int TK = T * K;
    const int x_bf16 = (x_dtype == K3X_BF16);
    const int HLg = x_bf16 ? 1 : 2;                      // B columns per token, gate/up
    int rc;

    hipLaunchKernelGGL(pf_split, dim3(cdiv((size_t)T * (H / 8), PF_NT)), dim3(PF_NT), 0, s,
                       x, x_bf16, T, H, B->xhl, B->counts, E);
    if ((rc = launch_ok())) return rc;

    PfRouterArgs ar;
    ar.x = x; ar.x_bf16 = x_bf16; ar.W = L->router; ar.bias = L->bias;
    ar.T = T; ar.H = H; ar.E = E; ar.score = B->score; ar.choice = B->choice;
    hipLaunchKernelGGL(pf_router, dim3(cdiv(T, RT_TOK), cdiv(E, RT_EXP)), dim3(PF_NT), 0, s, ar);
    if ((rc = launch_ok())) return rc;

    PfTopkArgs at;
    at.score = B->score; at.choice = B->choice; at.T = T; at.E = E; at.K = K;
    at.renorm = c->moe_renorm; at.routed_scale = c->routed_scale;
    at.idx = B->idx; at.wt = B->wt; at.uidx = uidx; at.uwt = uwt; at.counts = B->counts;
    if (E <= 128)      launch_topk<2>(at, s);
    else if (E <= 256) launch_topk<4>(at, s);
    else if (E <= 384) launch_topk<6>(at, s);
    else if (E <= 512) launch_topk<8>(at, s);
    else               launch_topk<16>(at, s);
    if ((rc = launch_ok())) return rc;

    const int tpb_gu = GU_CT * 16 / HLg, nrb_gu = cdiv(I, (PF_NT / WAVE) * GU_RT * 16);
    const int tpb_dn = DN_CT * 16 / 2, nrb_dn = cdiv(H, (PF_NT / WAVE) * DN_RT * 16);
    hipLaunchKernelGGL(pf_scan, dim3(1), dim3(1024), 0, s, B->counts, E, B->offsets, B->cursor,
                       B->tb_gu, tpb_gu, nrb_gu, B->tb_dn, tpb_dn, nrb_dn);
    if ((rc = launch_ok())) return rc;
    hipLaunchKernelGGL(pf_scatter, dim3(cdiv(TK, PF_NT)), dim3(PF_NT), 0, s, B->idx, B->wt, TK, K,
                       B->offsets, B->cursor, B->perm_tok, B->perm_w, B->pos_of);
    if ((rc = launch_ok())) return rc;

    const size_t act_row = (size_t)I * 4, ash_row = (size_t)SI * 4;   // bytes per hi/lo row
    // routed gate/up: B rows are tokens of xhl through perm_tok
    PfGemmArgs g;
    memset(&g, 0, sizeof g);
    g.wm[0] = L->experts + L->gate_off; g.wm[1] = L->experts + L->up_off;
    g.gstride = L->expert_bytes;
    g.R = I; g.K = H; g.G = E; g.gcount = B->counts; g.goff = B->offsets; g.tbase = B->tb_gu;
    g.bsrc = B->xhl; g.bsrc_bytes = (uint32_t)((size_t)T * H * 4); g.perm = B->perm_tok;
    g.pw = B->perm_w; g.act = B->act; g.out_base = 0;
    const unsigned grid_gu = nrb_gu * (cdiv(TK, tpb_gu) + (unsigned)(E < TK ? E : TK));
    const bool ex_gu = (L->special & 3) != 0;
    if (ex_gu) { if (HLg == 1) launch_gu_fp4<true, 1>(g, grid_gu, s); else launch_gu_fp4<true, 2>(g, grid_gu, s); }
    else       { if (HLg == 1) launch_gu_fp4<false, 1>(g, grid_gu, s); else launch_gu_fp4<false, 2>(g, grid_gu, s); }
    if ((rc = launch_ok())) return rc;

    // routed down: B rows are the activation rows, in permuted order
    PfGemmArgs d;
    memset(&d, 0, sizeof d);
    d.wm[0] = L->experts + L->down_off; d.gstride = L->expert_bytes;
    d.R = H; d.K = I; d.G = E; d.gcount = B->counts; d.goff = B->offsets; d.tbase = B->tb_dn;
    d.bsrc = B->act; d.bsrc_bytes = (uint32_t)(TK * act_row); d.perm = NULL; d.row_base = 0;
    d.y = B->y; d.out_base = 0;
    const unsigned grid_dn = nrb_dn * (cdiv(TK, tpb_dn) + (unsigned)(E < TK ? E : TK));
    if (L->special & 4)
        hipLaunchKernelGGL((pf_gemm<true, true, 1, DN_RT, DN_CT, 2, false>), dim3(grid_dn), dim3(PF_NT), 0, s, d);
    else
        hipLaunchKernelGGL((pf_gemm<true, false, 1, DN_RT, DN_CT, 2, false>), dim3(grid_dn), dim3(PF_NT), 0, s, d);
    if ((rc = launch_ok())) return rc;

    int sh_row0 = -1;
    if (SI > 0) {
        // shared gate/up over every token (bf16 weights), then down; its output rows follow
        // the routed ones in y
        PfGemmArgs sg;
        memset(&sg, 0, sizeof sg);
        sg.wm[0] = (const uint8_t *)L->sh_gate; sg.wm[1] = (const uint8_t *)L->sh_up;
        sg.R = SI; sg.K = H; sg.G = 1; sg.n0 = T;
        sg.bsrc = B->xhl; sg.bsrc_bytes = (uint32_t)((size_t)T * H * 4); sg.row_base = 0;
        sg.act = B->act_sh; sg.out_base = 0;
        const int tpb_sg = 4 * 16 / HLg, nrb_sg = cdiv(SI, (PF_NT / WAVE) * 1 * 16);
        const unsigned grid_sg = nrb_sg * cdiv(T, tpb_sg);
        if (HLg == 1)
            hipLaunchKernelGGL((pf_gemm<false, false, 2, 1, 4, 1, true>), dim3(grid_sg), dim3(PF_NT), 0, s, sg);
        else
            hipLaunchKernelGGL((pf_gemm<false, false, 2, 1, 4, 2, true>), dim3(grid_sg), dim3(PF_NT), 0, s, sg);
        if ((rc = launch_ok())) return rc;
        PfGemmArgs sd;
        memset(&sd, 0, sizeof sd);
        sd.wm[0] = (const uint8_t *)L->sh_down; sd.R = H; sd.K = SI; sd.G = 1; sd.n0 = T;
        sd.bsrc = B->act_sh; sd.bsrc_bytes = (uint32_t)(T * ash_row); sd.row_base = 0;
        sd.y = B->y; sd.out_base = TK;
        const int nrb_sd = cdiv(H, (PF_NT / WAVE) * 2 * 16);
        const unsigned grid_sd = nrb_sd * cdiv(T, 32);
        hipLaunchKernelGGL((pf_gemm<false, false, 1, 2, 4, 2, false>), dim3(grid_sd), dim3(PF_NT), 0, s, sd);
        if ((rc = launch_ok())) return rc;
        sh_row0 = TK;
    }

    hipLaunchKernelGGL(pf_combine, dim3(cdiv((size_t)T * (H / 4), PF_NT)), dim3(PF_NT), 0, s,
                       B->y, B->pos_of, T, K, H, sh_row0, resid, out);
    return launch_ok();
}

// Prefill: the pipeline over chunks of up to PF_CHUNK tokens.  Each token's result
// depends only on its own routing, so the chunking changes no result.
extern "C" int k3x_dev_prefill(k3x_moe_layer *L, float *out, const void *x, int x_dtype,
                               int T, const float *resid, int *idx, float *wt, void *stream)
{
    const int H = L->cfg.hidden, K = L->cfg.topk;
    const size_t es = (x_dtype == K3X_BF16) ? 2 : 4;
    int rc = k3x_pf_reserve(L, T < PF_CHUNK ? T : PF_CHUNK);
    if (rc) return rc;
    for (int t0 = 0; t0 < T; t0 += PF_CHUNK) {
        const int n = T - t0 < PF_CHUNK ? T - t0 : PF_CHUNK;
        rc = pf_chunk(L, out + (size_t)t0 * H, (const char *)x + (size_t)t0 * H * es, x_dtype, n,
                      resid ? resid + (size_t)t0 * H : NULL, idx ? idx + (size_t)t0 * K : NULL,
                      wt ? wt + (size_t)t0 * K : NULL, (hipStream_t)stream);
        if (rc) return rc;
    }
    return 0;
}
