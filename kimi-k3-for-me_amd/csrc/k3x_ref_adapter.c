/* k3x_ref_adapter.c - the binding a maintainer of the reference engine adds to route its
 * MoE block to libk3x.  Compiled inside the reference's build (it includes the
 * reference's k3.h); it is not part of libk3x.so.
 *
 * k3_moe_gpu / k3_moe_prefill_gpu have the signatures of k3_moe / k3_moe_prefill
 * (include/k3/k3.h:629-637) and return 0 when the call ran on the GPU, -1 when the
 * caller must run its CPU path instead (k3_ops.c:1862, :2008).  On first use of a layer
 * they upload it through the layer's own K3ExpertSrc (k3.h:521-544) and keep the handle;
 * afterwards every call runs on the GPU.
 *
 * Accepted: bf16 trunk weights (wdt == K3_WBF16) and a streamed expert source.  A layer
 * with latent == hidden whose down/up are identity matrices (the K2-class emulation) is
 * uploaded without projections; any other latent layer with its down/up projections,
 * latent norm and SiTU betas.  The upload hands the source's getmany (when it has one)
 * each batch of experts before their get() calls.  A cache-only draft (k3.h:564-568)
 * routes over the experts the source's resident() reports, asked for every expert at
 * each call (the host cache's residency, which the device copy does not share), with
 * the reference's renormalisation (k3_ops.c:1887-1896); a source without resident() is
 * refused (-1), as the reference's draft loop needs it.  An expert that cannot be
 * fetched at upload counts in k3_expert_drops (as k3_ops.c:1916-1926 counts a per-token
 * drop) and the call returns -1; a device call that fails (k3x status, including a
 * decode workgroup that gave up its wait) returns -1 without counting a drop.
 */
#include "k3.h"
#include "k3x_moe.h"
#include "k3x_store.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define K3X_ADAPTER_MAX_LAYERS 128

typedef struct {
    k3x_expert_src  base;   /* first member: the callback casts back */
    K3ExpertSrc    *src;
} adapter_src;

/* A layer is reused while the K3MoeW it was built from is the same object with the
 * same weights and shape; anything else uploads it again.  A layer kept as an HBM expert
 * cache fetches its misses through as, which lives as long as the layer. */
typedef struct {
    k3x_moe_layer *L;
    const K3MoeW  *w;
    const void    *gate, *sh1, *down, *src;
    int            hidden, n_experts, topk, moe_inter, latent;
    adapter_src    as;
} adapter_slot;

static adapter_slot g_slots[K3X_ADAPTER_MAX_LAYERS];

static int adapter_getmany(k3x_expert_src *self, int layer, const int *experts, int n)
{
    adapter_src *a = (adapter_src *)self;
    return a->src->getmany(a->src, layer, experts, n);
}

static int adapter_get(k3x_expert_src *self, int layer, int expert, k3x_expert_q *out)
{
    adapter_src *a = (adapter_src *)self;
    K3ExpertQ q;
    memset(&q, 0, sizeof q);
    if (a->src->get(a->src, layer, expert, &q) != 0) return -1;
    out->p1 = q.p1; out->s1 = q.s1;
    out->p3 = q.p3; out->s3 = q.s3;
    out->p2 = q.p2; out->s2 = q.s2;
    return 0;
}

static int gpu_form(const K3MoeW *w, const K3Cfg *c)
{
    return w->src && w->src->get && w->wdt == K3_WBF16 && w->down && w->up &&
           c->latent > 0 && (!w->cache_only || w->src->resident) && w->layer >= 0 &&
           w->layer < K3X_ADAPTER_MAX_LAYERS;
}

/* 1 when the bf16 [n][n] matrix m is the identity (1.0 = 0x3F80 on the diagonal, +0
 * elsewhere): then the projection is exact and the layer needs none. */
static int is_identity_bf16(const uint16_t *m, int n)
{
    for (size_t r = 0; r < (size_t)n; r++)
        for (size_t k = 0; k < (size_t)n; k++)
            if (m[r * n + k] != (r == k ? 0x3F80 : 0)) return 0;
    return 1;
}

static int slot_matches(const adapter_slot *s, const K3MoeW *w, const K3Cfg *c)
{
    return s->L && s->w == w && s->gate == (const void *)w->gate && s->sh1 == w->sh1 &&
           s->down == w->down && s->src == (const void *)w->src && s->hidden == c->hidden &&
           s->n_experts == c->n_experts && s->topk == c->topk &&
           s->moe_inter == c->moe_inter && s->latent == c->latent;
}

static k3x_moe_layer *layer_for(const K3MoeW *w, const K3Cfg *c)
{
    adapter_slot *s = &g_slots[w->layer];
    if (slot_matches(s, w, c)) return s->L;
    k3x_cfg kc;
    memset(&kc, 0, sizeof kc);
    kc.hidden = c->hidden;
    kc.n_experts = c->n_experts;
    kc.topk = c->topk;
    kc.moe_inter = c->moe_inter;
    kc.n_shared = c->n_shared;
    kc.moe_renorm = c->moe_renorm;
    kc.routed_scale = c->routed_scale;
    kc.group = K3_MXFP4_GROUP;
    const uint16_t *down = (const uint16_t *)w->down, *up = (const uint16_t *)w->up;
    const int plain = c->latent == c->hidden && is_identity_bf16(down, c->hidden) &&
                      is_identity_bf16(up, c->hidden);
    kc.latent = plain ? 0 : c->latent;
    kc.latent_norm = c->latent_norm;
    kc.rms_eps = c->rms_eps;
    kc.situ_b1 = c->situ_b1;
    kc.situ_b2 = c->situ_b2;
    adapter_src as;
    memset(&as, 0, sizeof as);
    as.base.get = adapter_get;
    if (w->src->getmany) as.base.getmany = adapter_getmany;
    as.src = w->src;
    if (s->L) {                 /* the old layer (and the supplier it holds) goes first */
        k3x_moe_layer_destroy(s->L);
        memset(s, 0, sizeof *s);
    }
    s->as = as;
    k3x_moe_w kw;
    memset(&kw, 0, sizeof kw);
    kw.gate = w->gate;
    kw.bias = w->bias;
    kw.sh1 = (const uint16_t *)w->sh1;
    kw.sh3 = (const uint16_t *)w->sh3;
    kw.sh2 = (const uint16_t *)w->sh2;
    kw.src = &s->as.base;
    kw.layer = w->layer;
    kw.down = plain ? NULL : down;
    kw.up = plain ? NULL : up;
    kw.latent_norm = w->latent_norm;
    k3x_moe_layer *L = NULL;
    /* the whole layer in HBM; when it does not fit (or K3X_ADAPTER_SLOTS asks for it),
     * an HBM expert cache of that many slots, or of the slots that fit in three quarters
     * of the free device memory (at least 8 * topk + 1, so that a call of 8 tokens fits),
     * whose misses come through the same source */
    const char *forced = getenv("K3X_ADAPTER_SLOTS");
    int rc = forced ? K3X_E_NOMEM : k3x_moe_layer_create(&kc, &kw, 0, &L);
    if (rc == K3X_E_NOMEM) {
        int nslot = forced ? atoi(forced) : k3x_cache_slots_fit(&kc, 0, 0.75);
        if (!forced && nslot < 8 * kc.topk + 1) nslot = 8 * kc.topk + 1;
        if (nslot < kc.topk + 1) nslot = kc.topk + 1;
        if (nslot > kc.n_experts) nslot = kc.n_experts;
        rc = k3x_moe_layer_create_cached_src(&kc, &kw, nslot, 0, &L);
    }
    if (rc) {
        /* a failed fetch was counted in k3x_expert_drops; mirror it for the CLI check
         * (k3_run.c:1027-1031) */
        if (rc == K3X_E_DROP) k3_expert_drops++;
        fprintf(stderr, "k3x: layer %d upload failed: %s\n", w->layer, k3x_strerror(rc));
        return NULL;
    }
    s->L = L;
    s->w = w;
    s->gate = w->gate; s->sh1 = w->sh1; s->down = w->down; s->src = w->src;
    s->hidden = c->hidden; s->n_experts = c->n_experts; s->topk = c->topk;
    s->moe_inter = c->moe_inter; s->latent = c->latent;
    return L;
}

static int run(int prefill, float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
               int T, int *idx, float *wt)
{
    if (!gpu_form(w, c)) return -1;
    k3x_moe_layer *L = layer_for(w, c);
    if (!L) return -1;
    int rc = 0;
    if (w->cache_only) {
        unsigned char *res = (unsigned char *)malloc((size_t)c->n_experts);
        if (!res) return -1;
        for (int e = 0; e < c->n_experts; e++)
            res[e] = w->src->resident(w->src, w->layer, e, NULL) ? 1 : 0;
        rc = k3x_moe_layer_set_cache_only(L, 1, res);
        free(res);
    }
    if (!rc)
        rc = prefill ? k3x_moe_prefill(L, out, x, T, idx, wt) : k3x_moe(L, out, x, T, idx, wt);
    if (w->cache_only) k3x_moe_layer_set_cache_only(L, 0, NULL);
    if (rc) {
        /* an expert the cache could not fetch: counted like the reference's per-token drop */
        if (rc == K3X_E_DROP) k3_expert_drops++;
        fprintf(stderr, "k3x: layer %d call failed: %s\n", w->layer, k3x_strerror(rc));
        return -1;
    }
    return 0;
}

int k3_moe_gpu(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T, int *idx,
               float *wt, float *scratch)
{
    (void)scratch;
    return run(0, out, x, w, c, T, idx, wt);
}

int k3_moe_prefill_gpu(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                       int *idx, float *wt, float *scratch)
{
    (void)scratch;
    return run(1, out, x, w, c, T, idx, wt);
}

/* k3_moe_scratch's counterpart (k3.h:574): the device path keeps its working memory in
 * the layer and needs no caller scratch, so 0 floats.  A caller still sizes the scratch
 * it passes with k3_moe_scratch, for the CPU path it runs when a call returns -1. */
size_t k3_moe_gpu_scratch(const K3Cfg *c, int T)
{
    (void)c;
    (void)T;
    return 0;
}

/* Drops every uploaded layer (a model's teardown, or before its weights are replaced in
 * place). */
void k3_moe_gpu_release(void)
{
    for (int l = 0; l < K3X_ADAPTER_MAX_LAYERS; l++) {
        if (g_slots[l].L) k3x_moe_layer_destroy(g_slots[l].L);
        memset(&g_slots[l], 0, sizeof g_slots[l]);
    }
}
