// k3x_blas.cpp - plain bf16 GEMMs on hipBLASLt: the trunk products of more than eight
// rows (k3_mmw_batch_ld, k3.h:457-478) and the prefill shared expert's products
// (moe_shared, k3_ops.c:1848-1860), Y[t*ldy + o] = sum_k W[o][k] X[t*ldx + k] with W and X
// bf16, Y fp32, accumulated in fp32 on the matrix cores.  These products carry no fused
// epilogue (the shared expert's SiTU runs as its own small kernel between them), so the
// library's tuned GEMMs serve them: about 1.2 PFLOP/s at 2048 x 7168 x 7168 on gfx950,
// against 0.77 for the hand-written dense kernel, which keeps the products whose
// epilogues feed the routed GEMMs' layouts.
//
// One handle per device, created with the first matrix uploaded to it.  The algorithm of
// a shape (in, out, T, accumulate) is chosen once, for packed rows, among those that need
// no workspace (no split-K reduction buffers, so no atomics and no allocation), and kept:
// every later call of that shape, with any row strides, runs the same kernel, so equal
// inputs give equal bits, and a call under graph capture does no host-side selection
// after the first.
#include <hip/hip_runtime_api.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "k3x_internal.h"

namespace {

constexpr int kMaxDevices = 64;

struct Shape {
    hipblasLtMatmulAlgo_t algo;
    bool                  ok;
};

struct Dev {
    hipblasLtHandle_t                              h = nullptr;
    std::map<std::tuple<int, int, int, int>, Shape> shapes;
};

std::mutex g_mu;
Dev        g_dev[kMaxDevices];

// C (column-major out x T, ld ldy) = A^T B: A is W, row-major [out][in], seen as
// column-major in x out (ld in); B is X, row-major [T][ldx], seen as column-major in x T.
struct Desc {
    hipblasLtMatmulDesc_t   md = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    bool make(int in, int out, int T, int ldx, int ldy)
    {
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        return hipblasLtMatmulDescCreate(&md, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatmulDescSetAttribute(md, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) ==
                   HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatmulDescSetAttribute(md, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) ==
                   HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatrixLayoutCreate(&la, HIP_R_16BF, in, out, in) == HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatrixLayoutCreate(&lb, HIP_R_16BF, in, T, ldx) == HIPBLAS_STATUS_SUCCESS &&
               hipblasLtMatrixLayoutCreate(&lc, HIP_R_32F, out, T, ldy) == HIPBLAS_STATUS_SUCCESS;
    }
    ~Desc()
    {
        if (lc) hipblasLtMatrixLayoutDestroy(lc);
        if (lb) hipblasLtMatrixLayoutDestroy(lb);
        if (la) hipblasLtMatrixLayoutDestroy(la);
        if (md) hipblasLtMatmulDescDestroy(md);
    }
};

} // namespace

extern "C" int k3x_blas_init(int device)
{
    if (device < 0 || device >= kMaxDevices) return K3X_E_ARG;
    std::lock_guard<std::mutex> g(g_mu);
    Dev &d = g_dev[device];
    if (d.h) return 0;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(device) != hipSuccess) return K3X_E_HIP;
    const hipblasStatus_t st = hipblasLtCreate(&d.h);
    (void)hipSetDevice(cur);
    if (st != HIPBLAS_STATUS_SUCCESS) {
        d.h = nullptr;
        return K3X_E_HIP;
    }
    return 0;
}

// The kept kernel of a shape, chosen at its first use (g_mu held)
static const Shape *shape_of(Dev &d, int in, int out, int T, int accumulate)
{
    const auto key = std::make_tuple(in, out, T, accumulate ? 1 : 0);
    auto it = d.shapes.find(key);
    if (it == d.shapes.end()) {
        Shape sh{};
        sh.ok = false;
        Desc pk;
        hipblasLtMatmulPreference_t pref = nullptr;
        const uint64_t ws = 0;
        if (pk.make(in, out, T, in, out) &&
            hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                  &ws, sizeof ws) == HIPBLAS_STATUS_SUCCESS) {
            hipblasLtMatmulHeuristicResult_t res;
            int n = 0;
            if (hipblasLtMatmulAlgoGetHeuristic(d.h, pk.md, pk.la, pk.lb, pk.lc, pk.lc, pref, 1,
                                                &res, &n) == HIPBLAS_STATUS_SUCCESS &&
                n > 0) {
                sh.algo = res.algo;
                sh.ok = true;
            }
        }
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        it = d.shapes.emplace(key, sh).first;
    }
    return &it->second;
}

extern "C" int k3x_blas_ready(int device, int in, int out, int T, int accumulate)
{
    if (device < 0 || device >= kMaxDevices) return K3X_E_ARG;
    std::lock_guard<std::mutex> g(g_mu);
    Dev &d = g_dev[device];
    if (!d.h) return K3X_E_HIP;
    return shape_of(d, in, out, T, accumulate)->ok ? 0 : K3X_E_HIP;
}

extern "C" int k3x_blas_gemm_bf16(int device, const uint16_t *W, int in, int out, float *Y,
                                  int ldy, const uint16_t *X, int ldx, int T, int accumulate,
                                  void *stream)
{
    if (device < 0 || device >= kMaxDevices) return K3X_E_ARG;
    std::lock_guard<std::mutex> g(g_mu);
    Dev &d = g_dev[device];
    if (!d.h) return K3X_E_HIP;
    const Shape *sh = shape_of(d, in, out, T, accumulate);
    if (!sh->ok) return K3X_E_HIP;
    Desc dc;
    if (!dc.make(in, out, T, ldx, ldy)) return K3X_E_HIP;
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    const hipblasStatus_t st =
        hipblasLtMatmul(d.h, dc.md, &alpha, W, dc.la, X, dc.lb, &beta, Y, dc.lc, Y, dc.lc,
                        &sh->algo, nullptr, 0, (hipStream_t)stream);
    return st == HIPBLAS_STATUS_SUCCESS ? 0 : K3X_E_HIP;
}
