/*
 * shim_harness.c — drives tinyllama.c_amd/integration/hip_graph_op.c (the
 * executor shim) with the reference's own OpCtx / Graph / GraphPlan /
 * KvCache / KvRadixCache structs, built as the executor builds them for
 * OP_ATTN (src/graph.c:410-415, 1270-1275; the same population as
 * ref_harness.c's rh_attn, which runs cpu_graph_op).  TEST INFRASTRUCTURE
 * ONLY; built into oracle/_ref/ where the reference tree exists.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "def.h"
#include "kvcache.h"

bool hip_graph_op(OpCtx *c);
void hip_graph_op_set_slots(const uint32_t *d_slots);

/* q/k/v/dst: device rows; kc/vc: device f16 cache [n_kv][cap][khd];
 * slots (host) != NULL -> a radix whose req.slots it is, slots_dev its
 * device mirror.  *n_after receives akc->n.  Returns 0 when the op ran. */
int rh_attn_shim(const float *q, const float *k, const float *v, float *dst,
                 void *kc, void *vc, u32 cap, u32 *slots, const u32 *slots_dev,
                 u32 pos, u32 n, u32 n_head, u32 n_kv, u32 hd, u32 win, u32 *n_after) {
    ArchConfig cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.n_head = n_head;
    cfg.n_kv_head = n_kv;
    cfg.head_dim = hd;
    cfg.kv_head_dim = hd;
    cfg.n_layer = 2;

    AttnKvCache akc[2];
    memset(akc, 0, sizeof(akc));
    akc[1].k = (float *)kc;          /* f16 device storage behind the f32-typed fields */
    akc[1].v = (float *)vc;
    akc[1].cap = cap;
    KvCache kcache;
    memset(&kcache, 0, sizeof(kcache));
    kcache.n_layer = 2;
    kcache.head_dim = hd;
    kcache.n_kv_head = n_kv;
    kcache.std = akc;

    KvRadixCache radix;
    memset(&radix, 0, sizeof(radix));
    radix.req.slots = slots;
    radix.req.len = pos + n;

    GraphPlan plan;
    memset(&plan, 0, sizeof(plan));
    plan.cache = &kcache;
    plan.radix = slots ? (void *)&radix : NULL;
    Graph g;
    memset(&g, 0, sizeof(g));
    g.plan = &plan;

    GraphNode nq, nk, nv, node;
    memset(&nq, 0, sizeof(nq)); memset(&nk, 0, sizeof(nk));
    memset(&nv, 0, sizeof(nv)); memset(&node, 0, sizeof(node));
    nq.data = (void *)q; nk.data = (void *)k; nv.data = (void *)v;
    node.op = OP_ATTN;
    node.src[0] = &nq; node.src[1] = &nk; node.src[2] = &nv;
    node.params[0] = 1;              /* layer 1 of the plan's cache */
    node.params[1] = win;
    node.data = dst;

    Session *s = calloc(1, sizeof(Session));
    OpCtx c = {
        .g = &g, .s = s, .cfg = &cfg, .node = &node, .dst = dst,
        .od = n_head * hd, .r = n, .base = 0, .pos = pos, .n = n,
        .scr = NULL, .scale = 1.0f / sqrtf((float)hd),
        .q_dim = n_head * hd, .kv_dim = n_kv * hd,
    };
    hip_graph_op_set_slots(slots_dev);
    bool ok = hip_graph_op(&c);
    free(s);
    if (n_after) *n_after = akc[1].n;
    return ok ? 0 : -1;
}
