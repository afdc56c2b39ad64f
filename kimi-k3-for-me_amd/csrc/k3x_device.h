// k3x_device.h - device helpers shared by the gfx950 kernels: bf16 rounding, the
// reference's sigmoid and SwiGLU, MXFP4 dequantisation into matrix-core operands, the
// bf16 MFMA, range-checked buffer loads and the tiled-layout offsets (k3x_internal.h
// describes the layouts).
#ifndef K3X_DEVICE_H
#define K3X_DEVICE_H

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "k3x_internal.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((__vector_size__(2 * sizeof(double)))) double f64x2;

#define WAVE 64

// ------------------------------------------------------------------ rounding
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

// ------------------------------------------------------------------ reference math
// ------------------------------------------------------------------ exact sums
// The reference sums n products p_i, each exact in double (a product of two floats), in
// one chain i = 0 .. n-1.  A kernel that adds them in another order, each product taking
// part in at most n/128 + 16 additions (a thread's run of at most n/256 + 4 of them, a
// wave's shuffle tree, a few wave partials), differs from that chain by at most
// (n + n/128 + 16) 2^-53 sum |p_i| in total (Higham, Accuracy and Stability of Numerical
// Algorithms, 2nd ed., eq. 4.4, applied to both sums); the factor 1 + 2^-16 covers the
// bound's own second-order terms.  chain_gap takes sum |p_i| as asum, an upper bound.
__device__ __forceinline__ double chain_gap(double asum, int n)
{
    return ((double)n + (double)(n >> 7) + 16.0) * 0x1p-53 * (1.0 + 0x1p-16) * asum;
}

// An upper bound of sum |p_i| from a float sum of the |p_i| formed like the products'
// (at most n/128 + 16 roundings of 2^-24 each on a product's way) with products below
// float's range flushed: widened by (n + 64) 2^-23 and n 2^-126.
__device__ __forceinline__ double abs_bound(float fsum, int n)
{
    return (double)fsum * (1.0 + ((double)n + 64.0) * 0x1p-23) + (double)n * 0x1p-126;
}

// The reference's RMSNorm scale from a sum of squares (k3_ops.c:137).
__device__ __forceinline__ float rms_inv(double ss, int n, float eps)
{
    return (float)(1.0 / sqrt(ss / (double)n + (double)eps));
}

// Whether rms_inv of a sum of squares ss formed in another order (as chain_gap describes)
// is the reference's: its chain lies in [ss - d, ss + d] (the terms are non-negative, so
// ss itself bounds their sum within the gap's slack), and rms_inv is monotonic (each step
// is a correctly rounded monotonic operation), so the two ends rounding alike proves it.
__device__ __forceinline__ bool rms_inv_proven(double ss, int n, float eps)
{
    const double d = chain_gap(ss, n);
    return rms_inv(ss - d, n, eps) == rms_inv(ss + d, n, eps);
}

// Whether (float)v of a sum v formed in another order is the float of the reference's
// chain, given the gap bound d: the chain is a double in [v - d, v + d], and rounding is
// monotonic.
__device__ __forceinline__ bool float_proven(double v, double d)
{
    const float f = (float)v;
    return (float)(v - d) == f && (float)(v + d) == f;
}

// The reference's chain sum_i (double)(a[i] * s) * (double)b[i] for i = 0 .. n-1 in order
// (s = 1: sum_i a[i] b[i]; a = b: the sum of squares of k3_ops.c:135-136), worked out by
// a workgroup of nt threads: chunks of C elements of a and b staged in buf (2C floats of
// LDS), thread 0 adds them.  Every thread calls; the value in thread 0.  For the rare
// sums whose float result another order does not prove.
__device__ double wg_dot_chain(const float *a, float s, const float *b, int n, float *buf, int C,
                               int nt)
{
    double acc = 0.0;
    for (int i0 = 0; i0 < n; i0 += C) {
        const int m = n - i0 < C ? n - i0 : C;
        for (int i = threadIdx.x; i < m; i += nt) {
            buf[i] = a[i0 + i];
            buf[C + i] = b[i0 + i];
        }
        __syncthreads();
        if (threadIdx.x == 0)
            for (int i = 0; i < m; i++) acc += (double)(buf[i] * s) * (double)buf[C + i];
        __syncthreads();
    }
    return acc;
}

// The reference's sigmoid, 1/(1+expf(-x)) in float (k3_ops.c:143).  exp is evaluated in
// double and rounded once: the correctly rounded expf(-x) except within ~2^-29
// relative of a float rounding midpoint.
__device__ __forceinline__ float sigmoid_ref(float x)
{
    const float e = (float)exp(-(double)x);
    return 1.0f / (1.0f + e);
}

// The GLU epilogues' functions in float, as k3_situ_glu computes them (k3_ops.c:143-161),
// with the device library's tanhf and expf: both within 1 ulp of the correctly rounded
// value (measured over 2^24 points of each of [-87, 88], [-10, 10], [-1, 1] and
// [-0.01, 0.01] on gfx950), as the reference's calls into the host's libm are not
// correctly rounded either.  The router's scores keep sigmoid_ref, whose exp is rounded
// once from double: the top-k compares them bit for bit.  (The double forms cost the
// K3-shape prefill 2.3 ms of its 10.9 ms chunk, in the gate/up epilogues.)
__device__ __forceinline__ float glu_sigmoid(float g)
{
    return 1.0f / (1.0f + expf(-g));
}

// SwiGLU as k3_situ_glu computes it at 2^64 betas: a = g*sigmoid(g), y = a*u, in float.
__device__ __forceinline__ float swiglu(float g, float u)
{
    const float a = g * glu_sigmoid(g);
    return a * u;
}

// SiTU-GLU as k3_situ_glu computes it (k3_ops.c:148-161): a = b1*tanh(g/b1) * sigmoid(g)
// (the sigmoid takes the UNCAPPED gate), u' = b2*tanh(u/b2), y = a*u', in float.  A beta
// of 0 leaves its half uncapped, as a beta of 2^64 does in the reference, so betas 0 and
// 0 give swiglu() exactly.
__device__ __forceinline__ float situ(float g, float u, float b1, float b2)
{
    const float gc = b1 != 0.0f ? b1 * tanhf(g / b1) : g;
    const float uc = b2 != 0.0f ? b2 * tanhf(u / b2) : u;
    const float a = gc * glu_sigmoid(g);
    return a * uc;
}

// ------------------------------------------------------------------ MXFP4 -> bf16
// 8 E2M1 codes (one dword, low nibble = lower column) times 2^(s-127) -> 8 bf16, exact
// for scale bytes 1..252 (v_cvt_scalef32_pk_bf16_fp4 takes the scale as an fp32 power
// of two; from byte 253 on, 6 x 2^(s-127) overflows bf16).  Other bytes take dq8_exact.
__device__ __forceinline__ bf16x8 dq8(uint32_t codes, float scale)
{
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 0);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 1);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 2);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes, scale, 3);
    bf16x8 r = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    return r;
}

__device__ __forceinline__ float e8m0_scale(uint32_t b) { return __uint_as_float(b << 23); }

// Any E8M0 byte, the reference's way (k3_ops.c:3125-3132, :3427-3433): the weight is the
// float product E2M1[c] * 2^(b-127) (2^-127 subnormal for byte 0, zero for 255, inf on
// overflow), rounded to bf16 (exact except where that float is below bf16's range).
__device__ __attribute__((noinline)) bf16x8 dq8_exact(uint32_t codes, uint32_t b)
{
    const float sc = (b == 255u) ? 0.0f : (b == 0u ? __uint_as_float(0x00400000u)
                                                   : __uint_as_float(b << 23));
    uint32_t h[8];
    for (int j = 0; j < 8; j++) {
        const uint32_t c = (codes >> (4 * j)) & 15u;
        const uint32_t m = c & 7u;
        const float mag = m == 0 ? 0.0f : (m == 1 ? 0.5f : (float)(2 + (m & 1)) * (float)(1u << ((m >> 1) - 1)) * 0.5f);
        const float v = (c & 8u) ? -mag : mag;
        h[j] = f2bf(v * sc);
    }
    u32x4 r = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// 32x32x16: A lane l = row l%32, k-slots 8*(l/32) .. +7; B lane l = column l%32, same
// k-slots; D lane l holds column l%32, rows 8a + 4*(l/32) + b in element 4a + b.  Twice
// the 16x16x32 form's throughput on gfx950 for the same operand registers.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

// Weights are streamed once per call: non-temporal loads keep them from displacing
// reused data (activations, B fragments) in the caches.
__device__ __forceinline__ u32x4 ldw16(const void *p)
{
    return __builtin_nontemporal_load((const u32x4 *)p);
}
__device__ __forceinline__ uint32_t ldw4(const void *p)
{
    return __builtin_nontemporal_load((const uint32_t *)p);
}

// ------------------------------------------------------------------ buffer loads
// Range-checked loads: an offset at or beyond the buffer's size returns zeros without a
// memory access (used for B-fragment lanes whose column holds no token).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#define K3X_OOB 0x80000000u   /* beyond any buffer here, with room for offsets */

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// ------------------------------------------------------------------ waves
#define AI __attribute__((always_inline))

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE); }

// Number of items w, w + st, ... below n.
__device__ __forceinline__ int strided_count(int w, int st, int n) { return w < n ? (n - 1 - w) / st + 1 : 0; }

// ------------------------------------------------------------------ weight loads
// Weights: range-checked buffer loads with the non-temporal cache policy (they are read
// once per call and should not displace the activations).
#define CPOL_NT 2
// device-coherent read (sc1): served from the level every XCD writes through to, never
// from a line another XCD's L2 may hold stale
#define CPOL_SC1 16
__device__ __forceinline__ u32x4 wld16(rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_NT);
}
__device__ __forceinline__ uint32_t wld4(rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_NT);
}

#define SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(n) lgkmcnt(0) (expcnt left at its maximum), gfx9 encoding
#define WAIT_VMCNT_LGKM0(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4))

// Meet the other waves once this wave's loads of a stage are in (N = vector loads issued
// after the stage's; exact, since the wait is what makes LDS data written by loads
// straight to LDS safe to read) and its LDS reads of the previous stage are done.  A bare
// s_barrier: __syncthreads' release fence would wait for every load in flight; the empty
// asm keeps the compiler from moving LDS accesses across it.
template <int N>
__device__ __forceinline__ void meet()
{
    WAIT_VMCNT_LGKM0(N);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ------------------------------------------------------------------ layout offsets
__device__ __forceinline__ size_t fp4_tile_bytes(int K)
{
    return (size_t)(((K >> 7) + 3) >> 2) * 4352;
}

// COMPACT B FRAGMENTS of NC = 2T live columns: entry (q, t, kq, n) holds the 8 bf16 of
// column n at K-indices 128q + 32kq + 8t .. +7, stored at entry index
// ((q*4 + t)*4 + kq)*NC + n, 16 bytes each; K*NC*2 bytes for a K-long set.
// Element offset (bf16 units) of K-index r, column n:
__device__ __forceinline__ size_t bfrag_off(int r, int n, int NC)
{
    const int q = r >> 7, kq = (r & 127) >> 5, t = (r & 31) >> 3, j = r & 7;
    return ((((size_t)q * 4 + t) * 4 + kq) * NC + n) * 8 + j;
}

// ------------------------------------------------------------------ activations
// 4 / 8 consecutive activations (base a multiple of 4 / 8), widened to float.
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

// One B fragment (8 bf16 of the hi or the lo column) from 8 activations.
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

// Cross-wave sum of per-lane accumulators through LDS; wave 0 ends with the total.
template <int NV, int NW>
__device__ __forceinline__ void wave_sum_lds(float (&acc)[NV], float *lds, int wave, int lane)
{
    if (wave != 0)
        for (int v = 0; v < NV; v++) lds[((wave - 1) * NV + v) * WAVE + lane] = acc[v];
    __syncthreads();
    if (wave == 0)
        for (int w = 1; w < NW; w++)
            for (int v = 0; v < NV; v++) acc[v] += lds[((w - 1) * NV + v) * WAVE + lane];
}

#endif
