/* k3x_trunk.h - the trunk's bf16 matrix products on the device.
 *
 * The reference applies every trunk matrix (attention projections, the shared experts,
 * the latent down/up projections) through
 *
 *     void k3_mmw_batch_ld(float *Y, int ldy, const float *X, int ldx, const void *W,
 *                          int wdt, int in, int out, int T);           k3.h:457-478
 *     void k3_mmw_batch(float *Y, const float *X, const void *W, int wdt, int in,
 *                       int out, int T);                              k3.h:480-484
 *
 * Y[t*ldy + o] = W[o] . X[t*ldx] for t < T, W bf16 [out][in] (K3_WBF16).  Here a matrix
 * is uploaded once and applied on the device: T <= 8 rows stream it once through a GEMV
 * on the matrix cores (over a copy re-laid out for them), larger T run a plain GEMM on
 * hipBLASLt (over the row-major copy; fp32 X as two bf16 GEMMs, its hi parts, then its lo
 * parts accumulated), or the library's absence, the hand-written dense GEMM.  The handle
 * holds both copies (4 bytes per weight).  Products are exact (bf16 weights, X split into
 * hi + lo bf16), accumulation is fp32 (the reference accumulates in double), so results
 * agree with the reference to fp32 rounding rather than bit for bit; a call repeats its
 * bits exactly (one kernel per shape, chosen at the shape's first call).
 */
#ifndef K3X_TRUNK_H
#define K3X_TRUNK_H

#include <stddef.h>
#include <stdint.h>

#include "k3x_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct k3x_trunk k3x_trunk;

/* Upload W, bf16 [out][in] row-major in host memory, to `device`: in a multiple of 128,
 * out a multiple of 16 (else K3X_E_SHAPE). */
int  k3x_trunk_create(const uint16_t *W, int in, int out, int device, k3x_trunk **t);
void k3x_trunk_destroy(k3x_trunk *t);

/* Y[t*ldy + o] = W[o] . X[t*ldx] for t < T (k3_mmw_batch_ld), device pointers, X fp32
 * (K3X_F32) or bf16 (K3X_BF16), ldx >= in, ldy >= out, X 16-byte aligned with ldx a
 * multiple of 8; asynchronous on `stream`.  T > 8 uses a workspace of T*in*4 bytes held
 * by the handle, grown (an allocation, at least doubling) when a larger T arrives; two
 * calls on one handle must be ordered on one stream.
 * Graph capture: a call may be captured once the workspace covers its T (reserve first
 * with k3x_trunk_reserve); a call that would grow it on a stream under capture returns
 * K3X_E_SHAPE and enqueues nothing.  An outgrown workspace is kept until
 * k3x_trunk_destroy (a graph captured over it stays valid); after 16 growths a further
 * one returns K3X_E_NOMEM. */
int  k3x_trunk_apply(k3x_trunk *t, float *Y, int ldy, const void *X, int x_dtype, int ldx,
                     int T, void *stream);

/* Grow the workspace for calls of up to max_T rows now (outside capture).  No
 * counterpart in the reference, whose products need no workspace. */
int  k3x_trunk_reserve(k3x_trunk *t, int max_T);

/* The host-pointer form with k3_mmw_batch's semantics (synchronous): Y [T][out] and
 * X [T][in] fp32 in host memory. */
int  k3x_trunk_apply_host(k3x_trunk *t, float *Y, const float *X, int T);

#ifdef __cplusplus
}
#endif
#endif
