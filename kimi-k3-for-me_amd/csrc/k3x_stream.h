// k3x_stream.h - the streaming pieces the decode kernels share: load rings, LDS staging,
// B-fragment views, fp4 super-quads and bf16 quads with their products, B sets of raw
// activations, per-token epilogues and the per-workgroup trace.
#ifndef K3X_STREAM_H
#define K3X_STREAM_H

#include "k3x_device.h"

#define SQ_BYTES 4352u     // an fp4 super-quad of a 16-row tile

extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];

// Items 0 .. cnt-1 through a ring of R slots: ld(slot, k) issues item k's loads (any k;
// k >= cnt must load nothing), use(slot, k) consumes item k.  ring_prime issues the
// first R items; ring_loop runs the rest, refilling a slot right after it is used.
// Scheduling barriers keep each slot's loads together and in slot order, in the prime
// as in the loop: the wait counts of the loop body are derived from both orders.
template <int R, class LD>
__device__ __forceinline__ void ring_prime(LD ld)
{
#pragma unroll
    for (int i = 0; i < R; i++) {
        SCHED_FENCE();
        ld(i, i);
    }
    SCHED_FENCE();
}

template <int R, class LD, class USE>
__device__ __forceinline__ void ring_loop(int cnt, LD ld, USE use)
{
    int k = 0;
    for (; k + R <= cnt; k += R) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            use(i, k + i);
            SCHED_FENCE();
            ld(i, k + i + R);
            SCHED_FENCE();
        }
    }
#pragma unroll
    for (int i = 0; i < R - 1; i++)
        if (k + i < cnt) use(i, k + i);
}

// ------------------------------------------------------------------ LDS staging
// Copy `bytes` (a multiple of 16) of global memory to dynamic LDS (at lds_off).  issue()
// loads up to MAXR 16-byte pieces per thread into registers; commit() stores them and
// copies what is left.  Issued before the weight loads, the staging loads come back
// first, so commit's wait leaves the weights in flight.
template <int MAXR>
struct Stage {
    u32x4    v[MAXR];
    rsrc_t   r;
    uint32_t bytes;

    __device__ __forceinline__ void issue(const void *src, uint32_t nbytes, int nthreads)
    {
        bytes = nbytes;
        r = make_rsrc(src, nbytes);
        const uint32_t step = (uint32_t)nthreads * 16u;
#pragma unroll
        for (int i = 0; i < MAXR; i++) v[i] = bload16(r, threadIdx.x * 16u + i * step);
    }
    __device__ __forceinline__ void commit(int nthreads, uint32_t lds_off = 0u)
    {
        const uint32_t step = (uint32_t)nthreads * 16u;
#pragma unroll
        for (int i = 0; i < MAXR; i++) {
            const uint32_t o = threadIdx.x * 16u + i * step;
            if (o < bytes) *(u32x4 *)(dyn_lds + lds_off + o) = v[i];
        }
        for (uint32_t o = threadIdx.x * 16u + MAXR * step; o < bytes; o += step)
            *(u32x4 *)(dyn_lds + lds_off + o) = bload16(r, o);
    }
};

// ------------------------------------------------------------------ B fragments
// A lane's view of a compact B set of NC columns, in LDS (staged at offset 0) or in
// global memory.  Lane (n, kq) reads entry ((q*4 + t)*4 + kq)*NC + n of quad q.  A lane
// whose column holds no token (n >= NC) reads column 0's entry instead: a B column only
// reaches the same column of the product, which is discarded.
template <bool LDSB>
struct BFrag {
    rsrc_t   r;
    uint32_t off;
    int      NC;

    __device__ __forceinline__ void init(const void *gsrc, uint32_t bytes, int NC_, int lane)
    {
        NC = NC_;
        const int n = lane & 15, kq = lane >> 4;
        off = (uint32_t)((kq * NC + (n < NC ? n : 0)) * 16);
        if (!LDSB) r = make_rsrc(gsrc, bytes);
    }
    // product t of quad q of the set `sbase` bytes in (wave-uniform)
    __device__ __forceinline__ u32x4 get(uint32_t sbase, int q, int t) const
    {
        const uint32_t o = off + (uint32_t)(q * 256 * NC + t * 64 * NC);
        if (LDSB) return *(const u32x4 *)(dyn_lds + sbase + o);
        return __builtin_amdgcn_raw_buffer_load_b128(r, o, sbase, 0);
    }
};

// ------------------------------------------------------------------ fp4 super-quads
// A super-quad of a tiled fp4 matrix for this lane: four 16-byte code groups (one scale
// group each) and the scale dword (byte j for quad j).
struct SQ {
    u32x4    c[4];
    uint32_t s;
};

// base: the super-quad's byte offset in the tile, or K3X_OOB (loads nothing)
__device__ __forceinline__ void sq_load(SQ &a, rsrc_t r, uint32_t base, int lane)
{
    const uint32_t o = base + (uint32_t)lane * 16u;
    a.c[0] = wld16(r, o);
    a.c[1] = wld16(r, o + 1024u);
    a.c[2] = wld16(r, o + 2048u);
    a.c[3] = wld16(r, o + 3072u);
    a.s = wld4(r, base + 4096u + (uint32_t)lane * 4u);
}

// A operand of product t of quad j.  EXACT takes the reference's float product for any
// scale byte; the fast path needs bytes 1..252.
template <bool EXACT>
__device__ __forceinline__ bf16x8 sq_a(const SQ &a, int j, int t)
{
    const uint32_t sb = (a.s >> (8 * j)) & 255u;
    if (EXACT) return dq8_exact(a.c[j][t], sb);
    return dq8(a.c[j][t], e8m0_scale(sb));
}

// d += dequant(a) x B over super-quad S (quads 4S .. 4S+3)
template <bool EXACT, bool LDSB>
__device__ __forceinline__ void sq_mfma(f32x4 &d, const SQ &a, const BFrag<LDSB> &b,
                                        uint32_t sbase, int S)
{
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int t = 0; t < 4; t++)
            d = mfma(sq_a<EXACT>(a, j, t), as_bf16x8(b.get(sbase, 4 * S + j, t)), d);
}

// gate and up over the same B
template <bool EXACT, bool LDSB>
__device__ __forceinline__ void sq_mfma2(f32x4 &dg, f32x4 &du, const SQ &g, const SQ &u,
                                         const BFrag<LDSB> &b, int S)
{
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const bf16x8 bv = as_bf16x8(b.get(0u, 4 * S + j, t));
            dg = mfma(sq_a<EXACT>(g, j, t), bv, dg);
            du = mfma(sq_a<EXACT>(u, j, t), bv, du);
        }
}

// ------------------------------------------------------------------ bf16 quads
// One quad of a tiled bf16 matrix for this lane: four 16-byte A fragments.
struct QB {
    u32x4 a[4];
};

__device__ __forceinline__ void qb_load(QB &a, rsrc_t r, uint32_t base, int lane)
{
    const uint32_t o = base + (uint32_t)lane * 16u;
#pragma unroll
    for (int t = 0; t < 4; t++) a.a[t] = wld16(r, o + 1024u * t);
}

__device__ __forceinline__ void qb_mfma(f32x4 &d, const QB &a, const u32x4 (&b)[4])
{
#pragma unroll
    for (int t = 0; t < 4; t++) d = mfma(as_bf16x8(a.a[t]), as_bf16x8(b[t]), d);
}

// B fragments of quad q straight from activations x [T][H] (no staging): bf16 x is its
// own hi column (lo = 0); fp32 x is split here.
__device__ __forceinline__ void bx_load(u32x4 (&b)[4], const void *x, int x_bf16, rsrc_t xr,
                                        int H, int NC, int q, int lane)
{
    const int n0 = lane & 15, kq = lane >> 4;
    const int n = n0 < NC ? n0 : 0, tok = n >> 1, hl = n & 1;
    if (x_bf16) {
        const uint32_t off = (uint32_t)(((size_t)tok * H + (size_t)q * 128 + kq * 32) * 2);
#pragma unroll
        for (int t = 0; t < 4; t++) b[t] = bload16(xr, hl ? K3X_OOB : off + 16u * t);
    } else {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float xv[8];
            load_x8(x, 0, (size_t)tok * H + (size_t)q * 128 + kq * 32 + t * 8, xv);
            b[t] = bfrag_of(xv, hl);
        }
    }
}

// Compact B fragments of x [T][H] (NC = 2T columns) over nq quads (quads from H/128 on
// are zeros), written by `nthreads` threads.  With nw, of the normalised rows
// nw[i] * x[i] * inv[token] instead (fp32 x).
__device__ __forceinline__ void x_to_bset(uint8_t *dst, const void *x, int x_bf16, int H, int NC,
                                          int nq, int tid, int nthreads,
                                          const float *nw = nullptr, const float *inv = nullptr)
{
    const int nQ = H >> 7, ne = nq * 16 * NC;
    for (int f = tid; f < ne; f += nthreads) {
        const int n = f % NC, kq = (f / NC) & 3, t = (f / (NC * 4)) & 3, q = f / (NC * 16);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (q < nQ) {
            float xv[8];
            load_x8(x, x_bf16, (size_t)(n >> 1) * H + (size_t)q * 128 + kq * 32 + t * 8, xv);
            if (nw) {
                float wv[8];
                load_x8(nw, 0, (size_t)q * 128 + kq * 32 + t * 8, wv);
#pragma unroll
                for (int j = 0; j < 8; j++) xv[j] = wv[j] * xv[j] * inv[n >> 1];
            }
            v = bfrag_of(xv, n & 1);
        }
        *(u32x4 *)(dst + (size_t)f * 16) = v;
    }
}

// hi + lo columns of a product summed per token (lanes n, n^1), then
// f(row0, token, values) on the even lanes of live columns: wave 0's rows row0 + i.
template <int NV, class F>
__device__ __forceinline__ void per_token(const float (&acc)[NV], int NC, int lane, F f)
{
    const int n = lane & 15, kq = lane >> 4;
    float v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = acc[i] + __shfl_xor(acc[i], 1);
    if ((n & 1) == 0 && n < NC) f(4 * kq, n >> 1, v);
}

// ------------------------------------------------------------------ diagnostics
// Optional per-workgroup trace (a layer made with K3X_TRACE=1): thread 0 writes
// {workgroup | XCD << 28 | hardware ids << 32, start, end} (100 MHz clock) at rec.
struct WgTrace {
    unsigned long long *rec;       // [grid][3] for this launch, or NULL
    uint64_t            t0;
    __device__ __forceinline__ void start(unsigned long long *r)
    {
        rec = r;
        if (rec && threadIdx.x == 0) t0 = __builtin_amdgcn_s_memrealtime();
    }
    __device__ __forceinline__ void end()
    {
        if (!rec || threadIdx.x != 0) return;
        const uint32_t hw = __builtin_amdgcn_s_getreg((4) | (0 << 6) | (31 << 11));   // HW_ID
        const uint32_t xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11));  // XCC_ID
        unsigned long long *p = rec + (size_t)blockIdx.x * 3;
        p[0] = (unsigned long long)blockIdx.x | ((unsigned long long)hw << 32) |
               ((unsigned long long)(xcc & 15) << 28);
        p[1] = t0;
        p[2] = __builtin_amdgcn_s_memrealtime();
    }
};

#endif
