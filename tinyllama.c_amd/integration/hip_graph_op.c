/*
 * hip_graph_op.c — the executor-side shim a tinyllama.c build adds beside
 * src/backend/gpu/gpu_op.cu so that graph_op_compute (src/graph.c:1186-1207)
 * runs the KV path on libtlkv.  It takes the device backend's dispatch slot:
 * graph_op_compute calls hip_graph_op for every BACKEND_CUDA node; OP_ATTN
 * and OP_ROPE_NORM / OP_ROPE_NEOX run here, every other op goes on to the
 * backend's own gpu_graph_op (src/backend/gpu/gpu_op.cu:968) when the build
 * links one.  It is compiled against the reference tree's own headers
 * (def.h: OpCtx, Graph, GraphNode, GraphPlan, KvCache, AttnKvCache;
 * kvcache.h: KvRadixCache) and linked with libtlkv; it is not part of libtlkv.
 *
 * Mapping, reference -> libtlkv:
 *   OpCtx (def.h:550-565): pos, n, scale, q_dim, kv_dim -> tl_attn_args
 *   node->src[0..2] (Q, K, V rows), dst                  -> q, k, v, dst
 *   node->params[0] (layer), params[1] (window)          -> layer, window
 *     (graph.c:410-415)
 *   plan->cache->std[layer] (AttnKvCache, def.h:289-294) -> tl_kv_layer; its
 *     k / v hold f16 device storage of cap * n_kv * khd halves — the one
 *     ABI change (the reference's are f32)
 *   plan->radix: a KvRadixCache made by libtlkv's kv_cache_create, whose
 *     leading fields sit at the reference's offsets (TlKvRadixHead), so
 *     radix->req and radix->ctx_size read the same here as in op_attn
 *     (src/backend/cpu/cpu_op.c:988-993).  The shim keeps a device mirror of
 *     req.slots per cache and uploads what kv_cache_append changed before
 *     each OP_ATTN (tl_slot_mirror_sync), on the executor's stream.
 * Semantics follow op_attn (src/backend/cpu/cpu_op.c:964-1064): the batch
 * rows are written through at their slots, akc->n = pos + n, then causal
 * (optionally windowed) attention over the cache.
 *
 * RoPE fusion (graph.c:410-436 builds OP_ROPE_* nodes that feed OP_ATTN): a
 * RoPE node whose only consumer is the layer's OP_ATTN, as Q (n_head heads)
 * or K (n_kv_head heads), is not run on its own; the OP_ATTN of that layer
 * then reads the RoPE inputs and rotates them in its own launch
 * (tl_attn_rope: same results as the rotation followed by the attention,
 * bit for bit).  The fused launch reads the RoPE node's source later than
 * the walk would, so a RoPE node is held back only when no node that runs
 * between it and the OP_ATTN — the OP_ATTN's own output included — holds an
 * arena slot overlapping that source: arena_plan (src/graph.c:671-724)
 * frees a slot right after its last consumer runs, and for the Q / K
 * projection that consumer is the RoPE node, so the OP_ATTN output (same
 * size as Q) is often placed on the Q projection's slot.  Other RoPE nodes
 * run out of place as op_rope_norm / op_rope_neox do (cpu_op.c:653-700):
 * copy the rows, rotate them (tl_rope).
 *
 * Errors return false (the executor's goto fail path), never exit.  Like
 * the reference's device backend, the shim keeps process-global state
 * (mirrors, deferred RoPE nodes) and relies on graph_compute's global lock
 * (src/graph.c:1340-1350).
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "def.h"
#include "kvcache.h"
#include "tlkv.h"

/* libtlkv's slot mirror (tl_session.h), declared with the reference's
 * KvRadixCache: its leading fields are laid out alike */
typedef struct tl_slot_mirror tl_slot_mirror;
int  tl_slot_mirror_create(uint32_t ctx_size, tl_slot_mirror **out);
void tl_slot_mirror_destroy(tl_slot_mirror *m);
int  tl_slot_mirror_sync(tl_slot_mirror *m, KvRadixCache *radix, void *stream,
                         const uint32_t **d_slots);

/* the device backend's own op dispatcher, when the build links it */
extern bool gpu_graph_op(OpCtx *c) __attribute__((weak));

#define SHIM_MAX_CACHES 64
#define SHIM_MAX_DEFERRED 8

static void *g_stream;   /* hipStream_t of the executor (NULL = default) */
static struct { KvRadixCache *radix; tl_slot_mirror *m; } g_mirror[SHIM_MAX_CACHES];
static struct { const GraphNode *node; u32 pos, n; } g_deferred[SHIM_MAX_DEFERRED];
static unsigned g_fused;

void hip_graph_op_set_stream(void *stream) { g_stream = stream; }

/* OP_ATTN calls that ran with their RoPE fused in (diagnostics) */
unsigned hip_graph_op_fused_count(void) { return g_fused; }

/* Drop the device mirror of a prefix cache; call before kv_cache_destroy
 * (cache_destroy, src/graph.c:899-913). */
void hip_graph_op_release(void *radix) {
    for (int i = 0; i < SHIM_MAX_CACHES; i++)
        if (g_mirror[i].radix == radix) {
            tl_slot_mirror_destroy(g_mirror[i].m);
            g_mirror[i].radix = NULL;
            g_mirror[i].m = NULL;
        }
}

static const uint32_t *device_slots(KvRadixCache *radix) {
    int free_i = -1;
    for (int i = 0; i < SHIM_MAX_CACHES; i++) {
        if (g_mirror[i].radix == radix) {
            const uint32_t *d = NULL;
            if (tl_slot_mirror_sync(g_mirror[i].m, radix, g_stream, &d)) {
                fprintf(stderr, "hip_graph_op: slot upload: %s\n", tl_last_error());
                return NULL;
            }
            return d;
        }
        if (!g_mirror[i].radix && free_i < 0) free_i = i;
    }
    if (free_i < 0) {
        fprintf(stderr, "hip_graph_op: more than %d prefix caches\n", SHIM_MAX_CACHES);
        return NULL;
    }
    if (tl_slot_mirror_create(radix->ctx_size, &g_mirror[free_i].m)) {
        fprintf(stderr, "hip_graph_op: slot mirror: %s\n", tl_last_error());
        return NULL;
    }
    g_mirror[free_i].radix = radix;
    return device_slots(radix);
}

static bool is_rope(const GraphNode *n) {
    return n && (n->op == OP_ROPE_NORM || n->op == OP_ROPE_NEOX);
}

static u32 consumers(const Graph *g, const GraphNode *x, const GraphNode **only) {
    u32 cnt = 0;
    for (const GraphNode *it = g->head; it; it = it->next)
        for (int s = 0; s < GRAPH_NODE_MAX_SRC; s++)
            if (it->src[s] == x) {
                cnt++;
                *only = it;
            }
    return cnt;
}

/* the Q and K inputs of `attn` are RoPE nodes of one kind and one rotation,
 * over the model's head counts and head_dim, each read by `attn` only */
static bool attn_rope_pair(const OpCtx *c, const GraphNode *attn) {
    const GraphNode *q = attn->src[0], *k = attn->src[1];
    if (!is_rope(q) || !is_rope(k) || q == k || q->op != k->op) return false;
    if (q->backend != attn->backend || k->backend != attn->backend) return false;
    if (q->params[0] != k->params[0] || q->params[2] != k->params[2] ||
        q->params[3] != k->params[3])
        return false;
    if (q->params[1] != c->cfg->n_head || k->params[1] != c->cfg->n_kv_head ||
        q->params[2] != c->cfg->kv_head_dim)
        return false;
    const GraphNode *only = NULL;
    if (consumers(c->g, q, &only) != 1 || only != attn) return false;
    if (consumers(c->g, k, &only) != 1 || only != attn) return false;
    return true;
}

/* bytes [a, a + an) and [b, b + bn) share at least one byte */
static bool overlaps(const void *a, size_t an, const void *b, size_t bn) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return an && bn && x < y + bn && y < x + an;
}

/* The `bytes` read from rope->src[0] stay intact until `attn` has run: no
 * node after `rope` up to and including `attn` writes an arena slot that
 * overlaps them (node->data_cap bytes at node->data, src/graph.c:753-754;
 * a node with data but no recorded size counts as overlapping). */
static bool source_outlives(const GraphNode *rope, const GraphNode *attn, size_t bytes) {
    const void *src = rope->src[0] ? rope->src[0]->data : NULL;
    if (!src) return false;
    for (const GraphNode *it = rope->next; it; it = it->next) {
        if (it->data && (!it->data_cap || overlaps(it->data, it->data_cap, src, bytes)))
            return false;
        if (it == attn) return true;
    }
    return false;   /* attn not after rope */
}

static int deferred_index(const GraphNode *node, u32 pos, u32 n) {
    for (int i = 0; i < SHIM_MAX_DEFERRED; i++)
        if (g_deferred[i].node == node && g_deferred[i].pos == pos && g_deferred[i].n == n)
            return i;
    return -1;
}

static bool defer_rope(const OpCtx *c) {
    int at = -1;
    for (int i = 0; i < SHIM_MAX_DEFERRED && at < 0; i++)
        if (!g_deferred[i].node || g_deferred[i].node == c->node) at = i;
    if (at < 0) {
        /* only entries left behind by a failed walk can fill the table */
        memset(g_deferred, 0, sizeof(g_deferred));
        at = 0;
    }
    g_deferred[at].node = c->node;
    g_deferred[at].pos = c->pos;
    g_deferred[at].n = c->n;
    return true;
}

/* op_rope_norm / op_rope_neox out of place: rows [base, base + r) of the
 * source, rotated at absolute positions pos + base + p */
static bool run_rope(const GraphNode *node, float *dst, u32 od, u32 r, u32 base, u32 pos) {
    const float *src = (const float *)node->src[0]->data;
    float theta;
    memcpy(&theta, &node->params[0], sizeof(theta));
    if (hipMemcpyAsync(dst, src + (size_t)base * od, (size_t)r * od * sizeof(float),
                       hipMemcpyDeviceToDevice, (hipStream_t)g_stream) != hipSuccess) {
        fprintf(stderr, "hip_graph_op: rope copy failed\n");
        return false;
    }
    int rc = tl_rope(dst, r, od, node->params[1], node->params[2], node->params[3], pos + base,
                     theta, node->op == OP_ROPE_NEOX, g_stream);
    if (rc) {
        fprintf(stderr, "hip_graph_op: rope: %s\n", tl_last_error());
        return false;
    }
    return true;
}

static bool op_rope(OpCtx *c) {
    const GraphNode *only = NULL;
    if (c->base == 0 && c->r == c->n && consumers(c->g, c->node, &only) == 1 &&
        only->op == OP_ATTN && attn_rope_pair(c, only) &&
        c->od == (c->node == only->src[0] ? c->q_dim : c->kv_dim) &&
        source_outlives(c->node, only, (size_t)c->n * c->od * sizeof(float)) && defer_rope(c))
        return true;   /* rotated inside that layer's OP_ATTN */
    return run_rope(c->node, c->dst, c->od, c->r, c->base, c->pos);
}

static bool op_attn(OpCtx *c) {
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
    const uint32_t *d_slots = NULL;
    if (radix) {
        if (radix->req.len < c->pos + c->n) return false;   /* kv_cache_append not run */
        if (!(d_slots = device_slots(radix))) return false;
    }
    /* RoPE inputs held back for this node: both fuse, or the held one runs now */
    const GraphNode *qn = c->node->src[0], *kn = c->node->src[1];
    const int iq = deferred_index(qn, c->pos, c->n), ik = deferred_index(kn, c->pos, c->n);
    const bool fuse = iq >= 0 && ik >= 0;
    if (!fuse) {
        if (iq >= 0 && !run_rope(qn, (float *)qn->data, c->q_dim, c->n, 0, c->pos)) return false;
        if (ik >= 0 && !run_rope(kn, (float *)kn->data, c->kv_dim, c->n, 0, c->pos)) return false;
    }
    if (iq >= 0) g_deferred[iq].node = NULL;
    if (ik >= 0) g_deferred[ik].node = NULL;

    tl_kv_layer L = {
        .k = akc->k, .v = akc->v, .cap = akc->cap,
        .n_kv_head = c->cfg->n_kv_head, .head_dim = c->cfg->kv_head_dim, .ring = 0,
    };
    tl_attn_args a = {
        .q = (const float *)(fuse ? qn->src[0]->data : qn->data),
        .k = (const float *)(fuse ? kn->src[0]->data : kn->data),
        .v = (const float *)c->node->src[2]->data,
        .dst = c->dst,
        .slots = d_slots,
        .pos = c->pos, .n = c->n, .n_head = c->cfg->n_head,
        .q_stride = c->q_dim, .kv_stride = c->kv_dim,
        .window = c->node->params[1], .scale = c->scale,
    };
    int rc;
    if (fuse) {
        float theta;
        memcpy(&theta, &qn->params[0], sizeof(theta));
        tl_rope_params rp = {
            .rope_dim = qn->params[3], .theta = theta, .neox = qn->op == OP_ROPE_NEOX,
        };
        rc = tl_attn_rope(&L, &a, &rp, g_stream);
        if (!rc) g_fused++;
    } else {
        rc = tl_attn(&L, &a, g_stream);
    }
    if (rc) {
        fprintf(stderr, "hip_graph_op: OP_ATTN layer %u: %s\n", layer, tl_last_error());
        return false;
    }
    akc->n = c->pos + c->n;
    return true;
}

bool hip_graph_op(OpCtx *c) {
    if (!c || !c->node) return false;
    switch (c->node->op) {
        case OP_ATTN:      return op_attn(c);
        case OP_ROPE_NORM:
        case OP_ROPE_NEOX: return op_rope(c);
        default:
            if (gpu_graph_op) return gpu_graph_op(c);
            fprintf(stderr, "hip_graph_op: op %d needs the device backend's gpu_graph_op\n",
                    (int)c->node->op);
            return false;
    }
}
