// k3x_layout.hip - moving weights into the layer's HBM layouts (k3x_internal.h): the
// tiled MXFP4 and bf16 formats, their inverse, the synthetic-layer generator (writing
// tiled bytes directly), and the device RMSNorm (k3_rmsnorm, k3_ops.c:132-140).
#include <string.h>

#include "k3x_device.h"

#define NT 256

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
        for (int j = 0; j < 4; j++) {
            const int q = 4 * S + j;
            const uint8_t *src = packed + (size_t)row * (K / 2) + (size_t)(128 * q + 32 * kq) / 2;
            for (int b = 0; b < 16; b++) so[j * 1024 + l * 16 + b] = j < nq ? src[b] : 0;
            if (j < nq) sw |= (uint32_t)scales[(size_t)row * (K / 32) + 4 * q + kq] << (8 * j);
        }
        *(uint32_t *)(so + 4096 + l * 4) = sw;
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
        const uint32_t sw = *(const uint32_t *)(so + 4096 + l * 4);
        for (int j = 0; j < nq; j++) {
            const int q = 4 * S + j;
            uint8_t *d = packed + (size_t)row * (K / 2) + (size_t)(128 * q + 32 * kq) / 2;
            for (int b = 0; b < 16; b++) d[b] = so[j * 1024 + l * 16 + b];
            scales[(size_t)row * (K / 32) + 4 * q + kq] = (uint8_t)(sw >> (8 * j));
        }
    }
}

// A tiled fp4 matrix dequantised to fp32 rows (k3_mxfp4_dequant, k3_ops.c:3778-3808)
// through the product kernels' own conversion: each lane's dword t of quad j goes
// through dq8 (scale bytes 1..252) or, when the layer takes the exact path for this
// matrix, dq8_exact, and the 8 bf16 results are widened.
__global__ void dequant_fp4_kernel(float *out, const uint8_t *src, int R, int K, int exact)
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
        const uint32_t sw = *(const uint32_t *)(so + 4096 + l * 4);
        for (int j = 0; j < nq; j++) {
            const u32x4 c = *(const u32x4 *)(so + j * 1024 + l * 16);
            const uint32_t sb = (sw >> (8 * j)) & 255u;
            for (int t = 0; t < 4; t++) {
                const bf16x8 v = exact ? dq8_exact(c[t], sb) : dq8(c[t], e8m0_scale(sb));
                const u32x4 u = __builtin_bit_cast(u32x4, v);
                float *d = out + (size_t)row * K + 128 * (4 * S + j) + 32 * kq + 8 * t;
                for (int i = 0; i < 4; i++) {
                    d[2 * i] = bf2f(u[i] & 0xFFFFu);
                    d[2 * i + 1] = bf2f(u[i] >> 16);
                }
            }
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
        for (int j = 0; j < 4; j++) {
            const int q = 4 * S + j;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (j < nq) {
                const uint64_t i0 = (uint64_t)row * (K / 2) + (uint64_t)(128 * q + 32 * kq) / 2;
                // i0 is a multiple of 16, so the 16 bytes are two whole draws
                const uint64_t d0 = draw(ck, i0 >> 3), d1 = draw(ck, (i0 >> 3) + 1);
                v = (u32x4){(uint32_t)d0, (uint32_t)(d0 >> 32), (uint32_t)d1, (uint32_t)(d1 >> 32)};
                const uint64_t si = (uint64_t)row * (K / 32) + 4 * q + kq;
                sw |= (uint32_t)(lo + (int)((draw(sk, si) >> 32) % span)) << (8 * j);
            }
            *(u32x4 *)(so + j * 1024 + l * 16) = v;
        }
        *(uint32_t *)(so + 4096 + l * 4) = sw;
    }
}

// ------------------------------------------------------------------ RMSNorm
// RMSNorm of one row per workgroup (k3_rmsnorm, k3_ops.c:132-140): the sum of squares in
// double (each product exact; the additions in a tree rather than the reference's
// chain), inv rounded to float, then y = w * x * inv in float in the reference's order.
// Where the tree's sum does not prove the float inv to be the reference's
// (rms_inv_proven), the squares are summed again as the reference's chain, so inv is the
// reference's on every row.
// Rows of up to RN_MAX * NT * 4 floats (16-byte aligned) are loaded once, x and w
// together with every load issued before the first use, and kept in registers between
// the two passes; other rows take the plain loop.
#define RN_MAX 8
__global__ void __launch_bounds__(NT) rmsnorm_kernel(float *y, const float *x, const float *w,
                                                      int n, float eps)
{
    __shared__ double red[NT / WAVE];
    __shared__ float buf[2 * 512];
    __shared__ double s_ss;
    const float *xr = x + (size_t)blockIdx.x * n;
    float *yr = y + (size_t)blockIdx.x * n;
    const bool vec = (n & 3) == 0 && n <= RN_MAX * NT * 4 &&
                     (((uintptr_t)xr | (uintptr_t)yr | (uintptr_t)w) & 15) == 0;
    const int n4 = n >> 2;
    f32x4 xv[RN_MAX], wv[RN_MAX];
    double ss = 0.0;
    if (vec) {
#pragma unroll
        for (int r = 0; r < RN_MAX; r++) {
            const int i = threadIdx.x + r * NT;
            xv[r] = i < n4 ? ((const f32x4 *)xr)[i] : (f32x4){0.f, 0.f, 0.f, 0.f};
            wv[r] = i < n4 ? ((const f32x4 *)w)[i] : (f32x4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int r = 0; r < RN_MAX; r++)
#pragma unroll
            for (int k = 0; k < 4; k++) ss += (double)xv[r][k] * (double)xv[r][k];
    } else {
        for (int i = threadIdx.x; i < n; i += NT) ss += (double)xr[i] * (double)xr[i];
    }
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / WAVE] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int i = 0; i < NT / WAVE; i++) tot += red[i];
    if (!rms_inv_proven(tot, n, eps)) {          // uniform; rare
        // the squares summed again as the reference's chain
        const double ss = wg_dot_chain(xr, 1.0f, xr, n, buf, 512, NT);
        if (threadIdx.x == 0) s_ss = ss;
        __syncthreads();
        tot = s_ss;
    }
    const float inv = rms_inv(tot, n, eps);
    if (vec) {
#pragma unroll
        for (int r = 0; r < RN_MAX; r++) {
            const int i = threadIdx.x + r * NT;
            if (i < n4) {
                f32x4 o;
#pragma unroll
                for (int k = 0; k < 4; k++) o[k] = wv[r][k] * xv[r][k] * inv;
                ((f32x4 *)yr)[i] = o;
            }
        }
    } else {
        for (int i = threadIdx.x; i < n; i += NT) yr[i] = w[i] * xr[i] * inv;
    }
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

extern "C" int k3x_dev_dequant_fp4(float *out, const uint8_t *src, int R, int K, int exact,
                                   void *stream)
{
    const long total = (long)(R >> 4) * (((K >> 7) + 3) >> 2) * 64;
    hipLaunchKernelGGL(dequant_fp4_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       (hipStream_t)stream, out, src, R, K, exact);
    return launch_ok();
}

// fp32 rows -> bf16 hi and lo rows (the GEMM operands of fp32 activations), eight
// elements a thread: two 16-byte reads, two 16-byte writes
__global__ void split_rows_kernel(const float *x, int ldx, int T, int n, uint16_t *hi,
                                  uint16_t *lo)
{
    const int n8 = n >> 3;
    const long total = (long)T * n8;
    for (long f = blockIdx.x * (long)blockDim.x + threadIdx.x; f < total;
         f += (long)gridDim.x * blockDim.x) {
        const int t = (int)(f / n8), c = (int)(f % n8) * 8;
        const float *src = x + (size_t)t * ldx + c;
        const f32x4 a = *(const f32x4 *)src, b = *(const f32x4 *)(src + 4);
        uint32_t h[8], l[8];
        for (int k = 0; k < 4; k++) {
            split_bf16(a[k], h[k], l[k]);
            split_bf16(b[k], h[4 + k], l[4 + k]);
        }
        u32x4 hv, lv;
        for (int k = 0; k < 4; k++) {
            hv[k] = h[2 * k] | (h[2 * k + 1] << 16);
            lv[k] = l[2 * k] | (l[2 * k + 1] << 16);
        }
        *(u32x4 *)(hi + (size_t)t * n + c) = hv;
        *(u32x4 *)(lo + (size_t)t * n + c) = lv;
    }
}

// The shared expert's activation from its gate/up product rows: ygu [T][2*SI] fp32 (gate
// columns 0 .. SI-1, up columns SI .. 2*SI-1) -> SiTU (as k3_situ_glu, k3_ops.c:148-161)
// split into bf16 hi and lo rows [T][SI], four elements a thread
__global__ void glu_rows_kernel(const float *ygu, int T, int SI, float b1, float b2,
                                uint16_t *hi, uint16_t *lo)
{
    const int n4 = SI >> 2;
    const long total = (long)T * n4;
    for (long f = blockIdx.x * (long)blockDim.x + threadIdx.x; f < total;
         f += (long)gridDim.x * blockDim.x) {
        const int t = (int)(f / n4), c = (int)(f % n4) * 4;
        const float *row = ygu + (size_t)t * 2 * SI;
        const f32x4 g = *(const f32x4 *)(row + c), u = *(const f32x4 *)(row + SI + c);
        uint32_t h[4], l[4];
        for (int k = 0; k < 4; k++) split_bf16(situ(g[k], u[k], b1, b2), h[k], l[k]);
        *(u32x2 *)(hi + (size_t)t * SI + c) = (u32x2){h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        *(u32x2 *)(lo + (size_t)t * SI + c) = (u32x2){l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
    }
}

extern "C" int k3x_dev_glu_rows(const float *ygu, int T, int SI, float b1, float b2,
                                uint16_t *hi, uint16_t *lo, void *stream)
{
    const long total = (long)T * (SI >> 2);
    hipLaunchKernelGGL(glu_rows_kernel, dim3(grid_for(total, NT)), dim3(NT), 0,
                       (hipStream_t)stream, ygu, T, SI, b1, b2, hi, lo);
    return launch_ok();
}

extern "C" int k3x_dev_split_rows(const float *x, int ldx, int T, int n, uint16_t *hi,
                                  uint16_t *lo, void *stream)
{
    const long total = (long)T * (n >> 3);
    hipLaunchKernelGGL(split_rows_kernel, dim3(grid_for(total, NT)), dim3(NT), 0,
                       (hipStream_t)stream, x, ldx, T, n, hi, lo);
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

