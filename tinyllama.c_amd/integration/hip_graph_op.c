/*
 * hip_graph_op.c — the executor-side shim a tinyllama.c build adds beside
 * src/backend/gpu/gpu_op.cu so that graph_op_compute (src/graph.c:1186-1207)
 * runs OP_ATTN on libtlkv.  It is compiled against the reference tree's own
 * headers (def.h: OpCtx, Graph, GraphPlan, KvCache, AttnKvCache; kvcache.h:
 * KvRadixCache) and linked with libtlkv; it is not part of libtlkv.
 *
 * Mapping, reference -> libtlkv:
 *   OpCtx (def.h:550-565): pos, n, scale, q_dim, kv_dim -> tl_attn_args
 *   node->src[0..2] (Q, K, V rows), node->data / dst   -> q, k, v, dst
 *   node->params[0] (layer), params[1] (window)         -> layer, window
 *     (graph.c:410-415)
 *   plan->cache->std[layer] (AttnKvCache, def.h:289-294) -> tl_kv_layer; its
 *     k / v hold f16 device storage of cap * n_kv * khd halves — the one
 *     ABI change (the reference's are f32)
 *   plan->radix (KvRadixCache) -> the device mirror of req.slots, uploaded
 *     by the executor after kv_cache_append (hip_graph_op_set_slots)
 * Semantics follow op_attn (src/backend/cpu/cpu_op.c:964-1064): the batch
 * rows are written through at their slots, akc->n = pos + n, then causal
 * (optionally windowed) attention over the cache.  Errors return false (the
 * executor's goto fail path), never exit.
 */
#include <stdint.h>
#include <stdio.h>

#include "def.h"
#include "kvcache.h"
#include "tlkv.h"

static const uint32_t *g_slots;   /* device mirror of radix->req.slots */
static void *g_stream;            /* hipStream_t of the executor (NULL = default) */

void hip_graph_op_set_slots(const uint32_t *d_slots) { g_slots = d_slots; }
void hip_graph_op_set_stream(void *stream) { g_stream = stream; }

bool hip_graph_op(OpCtx *c) {
    if (!c || !c->node || c->node->op != OP_ATTN) return false;   /* not handled here */
    KvCache *kc = (c->g && c->g->plan) ? c->g->plan->cache : NULL;
    if (!kc || !kc->std) return false;
    const u32 layer = c->node->params[0];
    AttnKvCache *akc = &kc->std[layer];
    if (!akc->k || !akc->v) return false;
    if (c->cfg->head_dim != c->cfg->kv_head_dim) {
        fprintf(stderr, "hip_graph_op: head_dim %u != kv_head_dim %u\n", c->cfg->head_dim,
                c->cfg->kv_head_dim);
        return false;
    }
    KvRadixCache *radix = (KvRadixCache *)c->g->plan->radix;
    if (radix && (radix->req.len < c->pos + c->n || !g_slots)) return false;

    tl_kv_layer L = {
        .k = akc->k, .v = akc->v, .cap = akc->cap,
        .n_kv_head = c->cfg->n_kv_head, .head_dim = c->cfg->kv_head_dim, .ring = 0,
    };
    tl_attn_args a = {
        .q = (const float *)c->node->src[0]->data,
        .k = (const float *)c->node->src[1]->data,
        .v = (const float *)c->node->src[2]->data,
        .dst = c->dst,
        .slots = radix ? g_slots : NULL,
        .pos = c->pos, .n = c->n, .n_head = c->cfg->n_head,
        .q_stride = c->q_dim, .kv_stride = c->kv_dim,
        .window = c->node->params[1], .scale = c->scale,
    };
    int rc = tl_attn(&L, &a, g_stream);
    if (rc) {
        fprintf(stderr, "hip_graph_op: OP_ATTN layer %u: %s\n", layer, tl_last_error());
        return false;
    }
    akc->n = c->pos + c->n;
    return true;
}
