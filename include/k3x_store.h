/* k3x_store.h - the checkpoint side of the MoE block: safetensors shards indexed by
 * tensor name, routed experts resolved and read as whole byte runs, and a layer's experts
 * streamed from the shards straight into its HBM arena.
 *
 * The reference reads its Kimi K3 checkpoint through
 *
 *     int  k3_st_open(K3St *s, const char *dir);                        k3_st.h:69
 *     const K3Tensor *k3_st_find(const K3St *s, const char *name);      k3_st.h:75
 *     int64_t k3_st_read(const K3St *s, const K3Tensor *t, void *buf);  k3_st.h:78
 *     int  k3_expert_ref(const K3St *s, int layer, int expert, K3ExpertRef *r);
 *     int64_t k3_expert_load(const K3St *s, const K3ExpertRef *r, unsigned char *buf);
 *                                                                       k3_load.h:47-52
 *
 * and hands experts to the MoE block through a K3ExpertSrc (k3.h:521-544).  This header
 * gives the same operations (plain C: pointers, sizes, status codes) plus the supplier
 * over a store and a whole-layer upload from it.
 *
 * Format (safetensors): [8-byte little-endian header length N][N bytes of JSON][data];
 * each JSON entry {"dtype", "shape", "data_offsets": [begin, end]} with offsets relative
 * to the end of the header; "__metadata__" is skipped.  Every *.safetensors file of the
 * directory is a shard, numbered in byte order of the file names.
 *
 * Expert tensors are named "language_model.model.layers.L.block_sparse_moe.experts.E.wM.
 * weight_packed" / ".weight_scale" (M = 1 gate, 2 down, 3 up; k3_load.c:11), U8, 2-D,
 * packed [rows][width/2], scales [rows][width/32].  When an expert's six tensors tile one
 * contiguous span of a shard (w1 packed, w1 scale, w2 packed, ... in the released
 * checkpoint, k3_load.h:3-22) the expert is read with one pread; otherwise six.
 */
#ifndef K3X_STORE_H
#define K3X_STORE_H

#include <stddef.h>
#include <stdint.h>

#include "k3x_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct k3x_store k3x_store;

/* dtypes of K3Dtype (k3_st.h:34-35) the reader accepts */
enum { K3X_DT_UNKNOWN = 0, K3X_DT_U8 = 1, K3X_DT_BF16 = 2, K3X_DT_F16 = 3, K3X_DT_F32 = 4 };

/* One tensor, as K3Tensor (k3_st.h:37-45): off is the ABSOLUTE byte offset in its shard. */
typedef struct k3x_tensor_info {
    int     shard;
    int     dtype;
    int     ndim;
    int64_t shape[4];
    int64_t off;
    int64_t nbytes;
} k3x_tensor_info;

/* Open and index every *.safetensors file of dir (k3_st_open).  Fails with K3X_E_ARG on a
 * malformed header, an unsupported dtype, a tensor whose byte count does not match its
 * shape or whose span leaves the file, or a name seen twice. */
int  k3x_store_open(const char *dir, k3x_store **out);
void k3x_store_close(k3x_store *s);
int  k3x_store_count(const k3x_store *s);                 /* tensors indexed */
int  k3x_store_shards(const k3x_store *s);                /* shard files     */

/* O(1) lookup by name (k3_st_find): 0 and *info, or K3X_E_ARG when absent. */
int  k3x_store_find(const k3x_store *s, const char *name, k3x_tensor_info *info);

/* The raw bytes of a tensor (k3_st_read) into buf (cap bytes): the byte count, or a
 * negative status (K3X_E_ARG: absent or cap too small; K3X_E_HIP is never returned). */
int64_t k3x_store_read(const k3x_store *s, const char *name, void *buf, int64_t cap);

/* One quantised matrix inside an expert's byte run (K3QMat, k3_load.h:30-35). */
typedef struct k3x_qmat {
    int64_t p_off, p_bytes;   /* packed nibbles, offset within the run */
    int64_t s_off, s_bytes;   /* E8M0 scales, offset within the run    */
    int     rows, pcols;      /* packed [rows][pcols]; width = 2 * pcols */
    int     scols;            /* scales [rows][scols], scols = width / 32 */
} k3x_qmat;

/* An expert's six tensors (K3ExpertRef, k3_load.h:37-45): m[0] w1 (gate), m[1] w2
 * (down), m[2] w3 (up). */
typedef struct k3x_expert_ref {
    int     layer, expert, shard;
    int64_t off;              /* absolute offset of the run (contiguous) */
    int64_t nbytes;           /* bytes of the run / of the packed buffer */
    int     contiguous;       /* 1: one read                             */
    k3x_qmat m[3];
} k3x_expert_ref;

/* Resolve and validate an expert (k3_expert_ref, k3_load.c:15-105): all six tensors
 * present, U8, 2-D, packed and scale rows equal, 32 elements per scale, one shard.
 * 0, or K3X_E_ARG (with the reason on stderr, as the reference). */
int  k3x_store_expert_ref(const k3x_store *s, int layer, int expert, k3x_expert_ref *r);

/* The expert's bytes into buf (r->nbytes): one read when contiguous, else six into the
 * same layout (k3_expert_load, k3_load.c:107-135).  Bytes read, or a negative status. */
int64_t k3x_store_expert_load(const k3x_store *s, const k3x_expert_ref *r, unsigned char *buf);

/* A supplier over the store (the K3ExpertSrc seam): get(layer, expert) reads the expert
 * into a buffer the supplier owns and points the k3x_expert_q into it (valid until the
 * next get).  Its getmany() only advises the kernel to read the experts' ranges ahead and
 * returns 0 (none made resident: get() still reads each).  k3x_store_src_fetches()
 * counts the reads. */
int  k3x_store_src_create(k3x_store *s, k3x_expert_src **out);
/* The same supplier for a layer whose experts are gate/up [moe_inter][width] and down
 * [width][moe_inter] (width: the latent width, or hidden): get() fails, so the layer
 * counts a drop, for an expert of any other shape instead of handing out arrays shorter
 * than the upload reads.  (The plain supplier checks only that an expert's three
 * matrices agree with one another.) */
int  k3x_store_src_create_for(k3x_store *s, int moe_inter, int width, k3x_expert_src **out);
void k3x_store_src_destroy(k3x_expert_src *src);
long k3x_store_src_fetches(const k3x_expert_src *src);

/* A layer with its routed experts streamed from the store into HBM (no counterpart in
 * the reference, which keeps experts on disk and reads them per token, k3_ops.c:1905-1931):
 * each expert's run is read into one of two pinned host buffers, copied to the device
 * and re-laid out there while the next run is read.  w supplies the router, bias, shared,
 * latent weights as for k3x_moe_layer_create (w->src and w->bank are ignored).  Expert
 * shapes are checked against c: w1/w3 [moe_inter][X], w2 [X][moe_inter], X the latent
 * width (or hidden).  A missing or malformed expert counts in k3x_expert_drops and fails
 * with K3X_E_DROP. */
int  k3x_moe_layer_create_from_store(const k3x_cfg *c, const k3x_moe_w *w, k3x_store *s,
                                     int layer, int device, k3x_moe_layer **out);

/* ---- expert cache: a layer with only part of its experts resident in HBM ----
 *
 * The reference streams its 1.45 TB of routed experts through a host-RAM cache
 * (K3Cache, k3_cache.h:46-113; k3_cache_init :115, k3_cache_pin :121, stats :137-138)
 * whose supplier k3_moe pulls from per token (k3_cache.c:394-563).  Here the arena is
 * in HBM: a layer made by k3x_moe_layer_create_cached holds nslot experts; each decode
 * call (k3x_moe_forward with T <= 8) first runs the selection, then makes the experts it
 * names resident, reading a miss's run from the store (pinned buffer, copy, re-layout
 * into the least recently used unpinned slot the call does not name), then runs the
 * expert products through the slot table.  The results are those of a layer with every
 * expert resident.  Cached layers run a prefill call as decode-path calls of 8 tokens
 * (k3x_moe_prefill_noalloc and the stacked graph return K3X_E_ARG), and a call whose
 * tokens name more experts than there are slots returns K3X_E_SHAPE.  The misses of a
 * call are read together (as k3x_cache_getmany).  A miss that cannot be read counts in
 * k3x_expert_drops and fails the call with K3X_E_DROP. */
typedef struct k3x_cache_stat {
    int                nslot;        /* slots in the arena                         */
    int                resident;     /* slots holding an expert                    */
    unsigned long long hits;         /* named experts found resident               */
    unsigned long long misses;       /* named experts read from the store          */
    unsigned long long evictions;    /* residents replaced                          */
    unsigned long long bytes_read;   /* bytes of expert runs read from the store   */
} k3x_cache_stat;

/* nslot in [topk + 1, n_experts] (k3_cache_init refuses fewer than topk + 1 slots);
 * w supplies the router, bias, shared and latent weights as for k3x_moe_layer_create;
 * the cache starts empty. */
int  k3x_moe_layer_create_cached(const k3x_cfg *c, const k3x_moe_w *w, k3x_store *s,
                                 int layer, int nslot, int device, k3x_moe_layer **out);
/* The same cache with its misses fetched through the layer's supplier w->src instead of
 * a store (the reference's K3ExpertSrc behind a binding): for each batch of a call's
 * misses, the supplier's getmany() when it has one, then get() one expert at a time, its
 * arrays (the layer's shapes) copied into a pinned buffer.  A failed get() counts in
 * k3x_expert_drops and fails the call with K3X_E_DROP.  The supplier must outlive the
 * layer. */
int  k3x_moe_layer_create_cached_src(const k3x_cfg *c, const k3x_moe_w *w, int nslot,
                                     int device, k3x_moe_layer **out);
/* Expert slots that fit in `fraction` (0 < fraction <= 1) of the device's free memory
 * beside one layer's other weights of shape c (at most n_experts): the nslot to give a
 * cache when the whole layer does not fit. */
int  k3x_cache_slots_fit(const k3x_cfg *c, int device, double fraction);
int  k3x_cache_stats(const k3x_moe_layer *L, k3x_cache_stat *st);
/* pin = 1: make the expert resident (a miss) and never evict it; 0: release it.  At
 * least topk slots stay unpinned (K3X_E_SHAPE otherwise). */
int  k3x_cache_pin(k3x_moe_layer *L, int expert, int pin);
/* cache_getmany's counterpart (k3_cache.c:394-512): make experts[0 .. n-1] resident, the
 * misses read from the store together (up to 8 at once, each by its own thread into its
 * own pinned buffer), evicting least recently used unpinned slots that the list does not
 * name.  Returns the number of listed experts now resident, K3X_E_SHAPE when n exceeds
 * the slots, or K3X_E_DROP when a run could not be read (the others are loaded).
 * Synchronous. */
int  k3x_cache_getmany(k3x_moe_layer *L, const int *experts, int n);
/* 1 when the expert is resident in the layer's HBM (every expert of a layer made without
 * a cache), 0 when not: the resident() of the reference's supplier (k3.h:540-542). */
int  k3x_cache_resident(const k3x_moe_layer *L, int expert);

#ifdef __cplusplus
}
#endif
#endif
