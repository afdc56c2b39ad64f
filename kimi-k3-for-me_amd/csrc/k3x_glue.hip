// k3x_glue.hip - the decoder layer's glue around the MoE block: the block attention-
// residual aggregation (k3_attn_res, k3_ops.c:1722-1753, with a block count per call or
// per row as k3_decoder_layer_core takes them, :2481-2493) and a float row copy.
#include "k3x_device.h"

#define AR_NT 256
#define AR_MAXSRC 64

__device__ __forceinline__ const float *ar_src(const float *blocks, int maxb, int nb,
                                               const float *pref, int n, int t, int s)
{
    return s < nb ? blocks + ((size_t)t * maxb + s) * n : pref + (size_t)t * n;
}

// Double sum of a per-thread partial over the workgroup (every thread gets it).
__device__ __forceinline__ double ar_sum(double v, double *red)
{
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < AR_NT / WAVE; w++) tot += red[w];
    return tot;
}

// One workgroup per row t: the sources are blocks[t][0 .. nb-1] then pref[t], nb = row
// t's block count: nbv[t * nbs] when nbv is given (device memory; nbs 0 for one count
// shared by every row, 1 for a count per row: K3_NB(t), k3_ops.c:2481-2483, 2493), else
// nb0.  Each source's key is its RMS-normalised row (inv rounded to float, v*inv in
// float) dotted with fold in double, the two double sums formed in a tree; where the
// tree does not prove the float result (inv, or the key rounded to float) to be the
// reference's chain's, that sum is formed again as the chain (rms_inv_proven,
// float_proven, wg_dot_chain); softmax with exp evaluated in double and rounded to
// float (the reference's expf), the double sum z; p = (float)(e/z); h = sum_s p_s v_s in
// float, in source order from 0 (the raw rows are the values).  A device count outside
// 0 .. min(maxb, AR_MAXSRC - 1) (or above 0 without blocks) fills row t with quiet NaNs
// instead: the reference reads past its stack there.
__global__ void __launch_bounds__(AR_NT) attn_res_kernel(float *h, const float *blocks, int maxb,
                                                         int nb0, const int *nbv, int nbs,
                                                         const float *pref,
                                                         const float *fold, int n, float eps)
{
    __shared__ double red[AR_NT / WAVE];
    __shared__ float p[AR_MAXSRC];
    __shared__ float sc[AR_MAXSRC];
    __shared__ float buf[2 * 512];
    __shared__ double s_ss;
    const int t = blockIdx.x;
    const int nb = nbv ? nbv[(size_t)t * nbs] : nb0;
    if (nb < 0 || nb > maxb || nb + 1 > AR_MAXSRC || (nb > 0 && !blocks)) {
        for (int i = threadIdx.x; i < n; i += AR_NT) h[(size_t)t * n + i] = __int_as_float(0x7FC00000);
        return;
    }
    const int nsrc = nb + 1;
    for (int s = 0; s < nsrc; s++) {
        const float *v = ar_src(blocks, maxb, nb, pref, n, t, s);
        double ss = 0.0;
        for (int i = threadIdx.x; i < n; i += AR_NT) ss += (double)v[i] * (double)v[i];
        ss = ar_sum(ss, red);
        if (!rms_inv_proven(ss, n, eps)) {             // uniform; rare
            const double c = wg_dot_chain(v, 1.0f, v, n, buf, 512, AR_NT);
            if (threadIdx.x == 0) s_ss = c;
            __syncthreads();
            ss = s_ss;
        }
        const float inv = rms_inv(ss, n, eps);
        double acc = 0.0;
        float aa = 0.0f;                               // sum |v*inv| |fold|, for the gap
        for (int i = threadIdx.x; i < n; i += AR_NT) {
            const float vi = v[i] * inv;
            acc += (double)vi * (double)fold[i];
            aa = fmaf(fabsf(vi), fabsf(fold[i]), aa);
        }
        acc = ar_sum(acc, red);
        const double asum = ar_sum((double)aa, red);
        if (!float_proven(acc, chain_gap(abs_bound((float)asum, n), n)))   // uniform; rare
            acc = wg_dot_chain(v, inv, fold, n, buf, 512, AR_NT);          // thread 0's
        if (threadIdx.x == 0) sc[s] = (float)acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = sc[0];
        for (int s = 1; s < nsrc; s++) m = sc[s] > m ? sc[s] : m;
        double z = 0.0;
        for (int s = 0; s < nsrc; s++) {
            sc[s] = (float)exp((double)(sc[s] - m));
            z += sc[s];
        }
        for (int s = 0; s < nsrc; s++) p[s] = (float)(sc[s] / z);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += AR_NT) {
        float o = 0.0f;
        for (int s = 0; s < nsrc; s++) o += p[s] * ar_src(blocks, maxb, nb, pref, n, t, s)[i];
        h[(size_t)t * n + i] = o;
    }
}

__global__ void __launch_bounds__(AR_NT) copy_f32x4(float *dst, const float *src, size_t n4)
{
    const size_t i = (size_t)blockIdx.x * AR_NT + threadIdx.x;
    if (i < n4) ((f32x4 *)dst)[i] = ((const f32x4 *)src)[i];
}

// nbv == NULL: the count nb for every row (checked here); else the rows' counts are read
// on the device from nbv[t * nbs] (nb unused).
extern "C" int k3x_dev_attn_res(float *h, const float *blocks, int maxb, int nb, const int *nbv,
                                int nbs, const float *pref, const float *fold, int n, int T,
                                float eps, void *stream)
{
    if (!nbv && nb + 1 > AR_MAXSRC) return K3X_E_SHAPE;
    hipLaunchKernelGGL(attn_res_kernel, dim3(T), dim3(AR_NT), 0, (hipStream_t)stream, h, blocks,
                       maxb, nb, nbv, nbs, pref, fold, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : K3X_E_HIP;
}

// dst = src, n floats (n a multiple of 4, both 16-byte aligned): a kernel rather than a
// memcpy node, so that a captured sequence holds kernels only.
extern "C" int k3x_dev_copy_f32(float *dst, const float *src, size_t n, void *stream)
{
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(copy_f32x4, dim3((unsigned)((n4 + AR_NT - 1) / AR_NT)), dim3(AR_NT), 0,
                       (hipStream_t)stream, dst, src, n4);
    return hipGetLastError() == hipSuccess ? 0 : K3X_E_HIP;
}
