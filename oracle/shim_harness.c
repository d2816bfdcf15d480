/*
 * shim_harness.c — drives tinyllama.c_amd/integration/hip_graph_op.c (the
 * executor shim) with the reference's own OpCtx / Graph / GraphNode /
 * GraphPlan / KvCache structs, built as the executor builds them
 * (src/graph.c:410-436 node builders, 1250-1300 the walk: od, r = n,
 * base = 0 for non-sink nodes, scale = 1/sqrt(khd)).  The prefix cache is
 * one made by libtlkv's kv_cache_create (passed in as a handle), so the shim
 * reads radix->req through the reference's header from libtlkv's struct —
 * the binding a tinyllama.c build would use.  TEST INFRASTRUCTURE ONLY;
 * built into oracle/_ref/ where the reference tree exists.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "def.h"
#include "kvcache.h"

bool hip_graph_op(OpCtx *c);
unsigned hip_graph_op_fused_count(void);
void hip_graph_op_release(void *radix);

/* The device backend's dispatcher as the shim sees it: records the ops that
 * fell through to it. */
static int g_fallthrough_op = -1;
bool gpu_graph_op(OpCtx *c) {
    g_fallthrough_op = (int)c->node->op;
    return true;
}

typedef struct {
    ArchConfig cfg;
    AttnKvCache akc[2];
    KvCache kcache;
    GraphPlan plan;
    Graph g;
    Session *s;
} Rig;

static void rig_init(Rig *r, void *kc, void *vc, u32 cap, void *radix, u32 n_head, u32 n_kv,
                     u32 hd) {
    memset(r, 0, sizeof(*r));
    r->cfg.n_head = n_head;
    r->cfg.n_kv_head = n_kv;
    r->cfg.head_dim = hd;
    r->cfg.kv_head_dim = hd;
    r->cfg.n_layer = 2;
    r->akc[1].k = (float *)kc;       /* f16 device storage behind the f32-typed fields */
    r->akc[1].v = (float *)vc;
    r->akc[1].cap = cap;
    r->kcache.n_layer = 2;
    r->kcache.head_dim = hd;
    r->kcache.n_kv_head = n_kv;
    r->kcache.std = r->akc;
    r->plan.cache = &r->kcache;
    r->plan.radix = radix;
    r->g.plan = &r->plan;
    r->s = calloc(1, sizeof(Session));
}

static void link_nodes(Rig *r, GraphNode **nodes, u32 n_node) {
    for (u32 i = 0; i < n_node; i++) {
        nodes[i]->idx = i;
        nodes[i]->backend = BACKEND_CUDA;
        nodes[i]->next = i + 1 < n_node ? nodes[i + 1] : NULL;
    }
    r->g.head = nodes[0];
    r->g.tail = nodes[n_node - 1];
    r->g.n_node = n_node;
}

static OpCtx ctx_for(Rig *r, GraphNode *node, u32 od, u32 pos, u32 n) {
    OpCtx c = {
        .g = &r->g, .s = r->s, .cfg = &r->cfg, .node = node, .dst = (float *)node->data,
        .od = od, .r = n, .base = 0, .pos = pos, .n = n,
        .scr = NULL, .scale = 1.0f / sqrtf((float)r->cfg.kv_head_dim),
        .q_dim = r->cfg.n_head * r->cfg.head_dim, .kv_dim = r->cfg.n_kv_head * r->cfg.kv_head_dim,
    };
    return c;
}

/* One OP_ATTN node over layer 1 of a two-layer cache.  q/k/v/dst: device
 * rows; kc/vc: device f16 cache [n_kv][cap][khd]; radix: libtlkv prefix
 * cache (kv_cache_append already run for [pos, pos + n)) or NULL for the
 * contiguous path.  *n_after receives akc->n.  Returns 0 when the op ran. */
int rh_attn_shim(const float *q, const float *k, const float *v, float *dst, void *kc,
                 void *vc, u32 cap, void *radix, u32 pos, u32 n, u32 n_head, u32 n_kv,
                 u32 hd, u32 win, u32 *n_after) {
    Rig r;
    rig_init(&r, kc, vc, cap, radix, n_head, n_kv, hd);
    GraphNode nq, nk, nv, node;
    memset(&nq, 0, sizeof(nq)); memset(&nk, 0, sizeof(nk));
    memset(&nv, 0, sizeof(nv)); memset(&node, 0, sizeof(node));
    nq.op = nk.op = nv.op = OP_MATMUL;   /* producers, already computed */
    nq.data = (void *)q; nk.data = (void *)k; nv.data = (void *)v;
    node.op = OP_ATTN;
    node.src[0] = &nq; node.src[1] = &nk; node.src[2] = &nv;
    node.params[0] = 1;
    node.params[1] = win;
    node.data = dst;
    GraphNode *nodes[] = {&nq, &nk, &nv, &node};
    link_nodes(&r, nodes, 4);
    OpCtx c = ctx_for(&r, &node, n_head * hd, pos, n);
    bool ok = hip_graph_op(&c);
    free(r.s);
    if (n_after) *n_after = r.akc[1].n;
    return ok ? 0 : -1;
}

/* A layer's RoPE + attention subgraph, walked in build order as
 * graph_compute does: q_in, k_in, v (producers) -> rope(q_in), rope(k_in)
 * (graph_rope / graph_rope_norm params: theta bits, heads, head_dim,
 * rope_dim) -> OP_ATTN.  With `extra` set, one more node reads the rotated K,
 * so the shim must run the K rotation on its own.  q_rot / k_rot: device
 * buffers the RoPE nodes write when they run.  Every node records its slot
 * size in data_cap, as arena_plan does (src/graph.c:753-754); the caller may
 * pass slots that alias as arena_plan can place them (dst == q_in: the
 * OP_ATTN output on the Q projection's freed slot; k_rot == q_in: the K
 * rotation there).  *fused receives the number of OP_ATTN calls that fused
 * their RoPE. */
int rh_layer_shim(const float *q_in, const float *k_in, const float *v, float *q_rot,
                  float *k_rot, float *dst, void *kc, void *vc, u32 cap, void *radix, u32 pos,
                  u32 n, u32 n_head, u32 n_kv, u32 hd, u32 win, int neox, float theta,
                  u32 rdim, int extra, u32 *fused) {
    Rig r;
    rig_init(&r, kc, vc, cap, radix, n_head, n_kv, hd);
    GraphNode nq, nk, nv, rq, rk, at, ex;
    GraphNode *all[] = {&nq, &nk, &nv, &rq, &rk, &at, &ex};
    for (int i = 0; i < 7; i++) memset(all[i], 0, sizeof(GraphNode));
    nq.op = nk.op = nv.op = OP_MATMUL;
    nq.data = (void *)q_in; nk.data = (void *)k_in; nv.data = (void *)v;
    u32 bits;
    memcpy(&bits, &theta, sizeof(bits));
    rq.op = rk.op = neox ? OP_ROPE_NEOX : OP_ROPE_NORM;
    rq.src[0] = &nq; rk.src[0] = &nk;
    rq.params[0] = rk.params[0] = bits;
    rq.params[1] = n_head; rk.params[1] = n_kv;
    rq.params[2] = rk.params[2] = hd;
    rq.params[3] = rk.params[3] = rdim;
    rq.data = q_rot; rk.data = k_rot;
    at.op = OP_ATTN;
    at.src[0] = &rq; at.src[1] = &rk; at.src[2] = &nv;
    at.params[0] = 1;
    at.params[1] = win;
    at.data = dst;
    ex.op = OP_ADD;                     /* a second reader of the rotated K */
    ex.src[0] = &rk; ex.src[1] = &rk;
    link_nodes(&r, all, extra ? 7 : 6);
    const u32 qd = n_head * hd, kd = n_kv * hd;
    nq.data_cap = rq.data_cap = at.data_cap = (size_t)n * qd * sizeof(float);
    nk.data_cap = nv.data_cap = rk.data_cap = (size_t)n * kd * sizeof(float);
    unsigned f0 = hip_graph_op_fused_count();
    OpCtx c1 = ctx_for(&r, &rq, qd, pos, n);
    OpCtx c2 = ctx_for(&r, &rk, kd, pos, n);
    OpCtx c3 = ctx_for(&r, &at, qd, pos, n);
    bool ok = hip_graph_op(&c1) && hip_graph_op(&c2) && hip_graph_op(&c3);
    if (fused) *fused = hip_graph_op_fused_count() - f0;
    free(r.s);
    return ok ? 0 : -1;
}

/* A node of another op goes through the shim; returns the op the backend's
 * gpu_graph_op saw (-1: none) or -2 when the shim failed. */
int rh_fallthrough(int op) {
    Rig r;
    rig_init(&r, NULL, NULL, 0, NULL, 1, 1, 64);
    GraphNode node;
    memset(&node, 0, sizeof(node));
    node.op = (GraphOp)op;
    GraphNode *nodes[] = {&node};
    link_nodes(&r, nodes, 1);
    OpCtx c = ctx_for(&r, &node, 64, 0, 1);
    g_fallthrough_op = -1;
    bool ok = hip_graph_op(&c);
    free(r.s);
    return ok ? g_fallthrough_op : -2;
}

int rh_op_id(const char *name) {
    if (!strcmp(name, "OP_ADD")) return OP_ADD;
    if (!strcmp(name, "OP_SOFTMAX")) return OP_SOFTMAX;
    if (!strcmp(name, "OP_MATMUL")) return OP_MATMUL;
    return -1;
}

void rh_shim_release(void *radix) { hip_graph_op_release(radix); }
