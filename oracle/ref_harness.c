/*
 * ref_harness.c — drives the COMPILED REFERENCE (tinyllama.c sources under
 * the reference tree, built by oracle/Makefile into oracle/_ref/) through its
 * own entry points.  TEST INFRASTRUCTURE ONLY: used to pin oracle.c and the
 * product's host kvcache, never linked into the product.
 *
 *   rh_attn      -> cpu_graph_op(OP_ATTN)      src/backend/cpu/cpu_op.c:1070,964
 *   rh_attn_radix   the same over a prefix cache made by another library
 *   rh_radix_layout offsets of the reference's KvRadixCache (kvcache.h:50-57)
 *   rh_rope      -> cpu_graph_op(OP_ROPE_*)    src/backend/cpu/cpu_op.c:653,674
 *   rh_kv_*      -> kv_cache_create/match/append/destroy  src/kvcache.c:122-270
 *                   (rh_kv_lookup: a read-only raxFind walk over the same tree)
 *   rh_kvs_*     -> the same with a Session whose Graph registers one host
 *                   recurrent-state buffer (graph_state_bytes/save/load,
 *                   src/graph.c:360-408), and kv_cache_checkpoint/restore
 *                   src/kvcache.c:272-321
 *   rh_dequant_q8_0 -> gguf_dequant(GGUF_TYPE_Q8_0)  src/quants.c:640-652,368
 *
 * The structs are the reference's own (def.h / kvcache.h); only the fields
 * op_attn reads are populated (cpu_op.c:968-993).
 */
#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#include "def.h"
#include "kvcache.h"
#include "backend/cpu/cpu_op.h"
#include "quants.h"

/* --- attention ----------------------------------------------------------- */

/* kc/vc: f32 [n_kv][cap][khd] (the reference layout, graph.c:852-858).
 * slots == NULL -> no radix (contiguous path, cpu_op.c:1034-1041). */
static int attn_with(void *radix_ext, const float *q, const float *k, const float *v,
                     float *dst, float *kc, float *vc, u32 cap, u32 *slots, u32 pos,
                     u32 n, u32 n_head, u32 n_kv, u32 hd, u32 khd, u32 win);

int rh_attn(const float *q, const float *k, const float *v, float *dst,
            float *kc, float *vc, u32 cap, u32 *slots, u32 pos, u32 n,
            u32 n_head, u32 n_kv, u32 hd, u32 khd, u32 win) {
    return attn_with(NULL, q, k, v, dst, kc, vc, cap, slots, pos, n, n_head, n_kv, hd,
                     khd, win);
}

/* The same OP_ATTN with plan->radix = `radix`, a prefix cache made elsewhere
 * (libtlkv's kv_cache_create): op_attn reads its req.slots / req.len through
 * the reference's struct layout (cpu_op.c:988-993). */
int rh_attn_radix(void *radix, const float *q, const float *k, const float *v,
                  float *dst, float *kc, float *vc, u32 cap, u32 pos, u32 n,
                  u32 n_head, u32 n_kv, u32 hd, u32 win) {
    if (!radix) return -1;
    return attn_with(radix, q, k, v, dst, kc, vc, cap, NULL, pos, n, n_head, n_kv, hd, hd,
                     win);
}

/* offsetof / sizeof of the reference's KvRadixCache fields (kvcache.h:50-57) */
void rh_radix_layout(u64 *out) {
    out[0] = offsetof(KvRadixCache, tree);
    out[1] = offsetof(KvRadixCache, pool);
    out[2] = offsetof(KvRadixCache, pool.n_free);
    out[3] = offsetof(KvRadixCache, pool.free_stack);
    out[4] = offsetof(KvRadixCache, meta);
    out[5] = offsetof(KvRadixCache, req);
    out[6] = offsetof(KvRadixCache, req.len);
    out[7] = offsetof(KvRadixCache, req.shared_len);
    out[8] = offsetof(KvRadixCache, req.active);
    out[9] = offsetof(KvRadixCache, kv);
    out[10] = offsetof(KvRadixCache, n_layer);
    out[11] = offsetof(KvRadixCache, ctx_size);
    out[12] = offsetof(KvRadixCache, enabled);
    out[13] = sizeof(KvSlotMeta);
    out[14] = offsetof(KvSlotMeta, last_used);
    out[15] = offsetof(KvSlotMeta, in_tree);
}

static int attn_with(void *radix_ext, const float *q, const float *k, const float *v,
                     float *dst, float *kc, float *vc, u32 cap, u32 *slots, u32 pos,
                     u32 n, u32 n_head, u32 n_kv, u32 hd, u32 khd, u32 win) {
    ArchConfig cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.n_head = n_head;
    cfg.n_kv_head = n_kv;
    cfg.head_dim = hd;
    cfg.kv_head_dim = khd;
    cfg.n_layer = 1;

    AttnKvCache akc = { .k = kc, .v = vc, .n = 0, .cap = cap };
    KvCache kcache;
    memset(&kcache, 0, sizeof(kcache));
    kcache.n_layer = 1;
    kcache.head_dim = khd;
    kcache.n_kv_head = n_kv;
    kcache.std = &akc;

    KvRadixCache radix;
    memset(&radix, 0, sizeof(radix));
    radix.req.slots = slots;
    radix.req.len = pos + n;

    GraphPlan plan;
    memset(&plan, 0, sizeof(plan));
    plan.cache = &kcache;
    plan.radix = radix_ext ? radix_ext : slots ? (void *)&radix : NULL;

    Graph g;
    memset(&g, 0, sizeof(g));
    g.plan = &plan;

    GraphNode nq, nk, nv, node;
    memset(&nq, 0, sizeof(nq)); memset(&nk, 0, sizeof(nk));
    memset(&nv, 0, sizeof(nv)); memset(&node, 0, sizeof(node));
    nq.data = (void *)q; nk.data = (void *)k; nv.data = (void *)v;
    node.op = OP_ATTN;
    node.src[0] = &nq; node.src[1] = &nk; node.src[2] = &nv;
    node.params[0] = 0;
    node.params[1] = win;
    node.data = dst;

    Session *s = calloc(1, sizeof(Session));
    float *scr = malloc(((size_t)pos + n) * sizeof(float));
    OpCtx c = {
        .g = &g, .s = s, .cfg = &cfg, .node = &node, .dst = dst,
        .od = n_head * hd, .r = n, .base = 0, .pos = pos, .n = n,
        .scr = scr, .scale = 1.0f / sqrtf((float)khd),
        .q_dim = n_head * hd, .kv_dim = n_kv * khd,
    };
    bool ok = cpu_graph_op(&c);
    free(scr);
    free(s);
    return ok ? 0 : -1;
}

/* --- Q8_0 dequant ---------------------------------------------------------- */

/* n elements of GGUF Q8_0 blocks (34 bytes: f16 d, 32 x int8) -> f32,
 * element by element through the reference's dispatcher. */
void rh_dequant_q8_0(const u8 *blocks, u64 n, float *out) {
    TensorInfo ti;
    memset(&ti, 0, sizeof(ti));
    ti.type = GGUF_TYPE_Q8_0;
    ti.data = (void *)blocks;
    ti.n_element = n;
    for (u64 i = 0; i < n; i++) out[i] = gguf_dequant(&ti, i);
}

/* --- RoPE ---------------------------------------------------------------- */

/* neox != 0 -> OP_ROPE_NEOX else OP_ROPE_NORM.  src/dst [rows][od] f32. */
int rh_rope(int neox, const float *src, float *dst, u32 rows, u32 od,
            u32 heads, u32 hdim, u32 rdim, u32 pos, float theta) {
    ArchConfig cfg;
    memset(&cfg, 0, sizeof(cfg));
    Graph g;
    memset(&g, 0, sizeof(g));
    GraphNode ns, node;
    memset(&ns, 0, sizeof(ns));
    memset(&node, 0, sizeof(node));
    ns.data = (void *)src;
    node.op = neox ? OP_ROPE_NEOX : OP_ROPE_NORM;
    node.src[0] = &ns;
    memcpy(&node.params[0], &theta, sizeof(float));
    node.params[1] = heads;
    node.params[2] = hdim;
    node.params[3] = rdim;
    node.data = dst;
    Session *s = calloc(1, sizeof(Session));
    OpCtx c = {
        .g = &g, .s = s, .cfg = &cfg, .node = &node, .dst = dst,
        .od = od, .r = rows, .base = 0, .pos = pos, .n = rows,
    };
    bool ok = cpu_graph_op(&c);
    free(s);
    return ok ? 0 : -1;
}

/* --- kvcache ------------------------------------------------------------- */

typedef struct {
    KvCache kv;
    KvRadixCache *c;
} RhKv;

void *rh_kv_create(u32 ctx) {
    RhKv *h = calloc(1, sizeof(*h));
    h->kv.n_layer = 1;
    h->c = kv_cache_create(NULL, &h->kv, ctx);
    if (!h->c) { free(h); return NULL; }
    return h;
}

void rh_kv_destroy(void *p) {
    RhKv *h = p;
    if (!h) return;
    kv_cache_destroy(h->c);
    free(h);
}

u32 rh_kv_match(void *p, const u32 *tokens, u32 n) {
    return kv_cache_match(((RhKv *)p)->c, tokens, n);
}

int rh_kv_append(void *p, const u32 *tokens, u32 pos, u32 n) {
    return kv_cache_append(((RhKv *)p)->c, tokens, pos, n) ? 1 : 0;
}

/* Longest cached prefix of tokens[0..n), read-only: the same raxFind walk
 * kv_cache_match makes (kvcache.c:199-207: raw u32 keys of growing length,
 * an in-tree slot behind each), without its reference counts, LRU touches or
 * statistics. */
u32 rh_kv_lookup(void *p, const u32 *tokens, u32 n) {
    KvRadixCache *c = ((RhKv *)p)->c;
    u32 i = 0;
    for (; i < n; i++) {
        void *v = raxFind(c->tree, (unsigned char *)tokens, (size_t)(i + 1) * sizeof(u32));
        if (v == raxNotFound) break;
        u32 slot = (u32)((uintptr_t)v - 1);
        if (slot >= c->pool.n_slots || !c->meta[slot].in_tree) break;
    }
    return i;
}

/* req.len, req.shared_len, req.active, pool.n_free */
void rh_kv_req(void *p, u32 *out4) {
    KvRadixCache *c = ((RhKv *)p)->c;
    out4[0] = c->req.len;
    out4[1] = c->req.shared_len;
    out4[2] = c->req.active;
    out4[3] = c->pool.n_free;
}

void rh_kv_slots(void *p, u32 *out, u32 n) {
    KvRadixCache *c = ((RhKv *)p)->c;
    memcpy(out, c->req.slots, (size_t)n * sizeof(u32));
}

/* hit_tokens, computed_tokens, evictions, allocations, clock */
void rh_kv_stats(void *p, u64 *out5) {
    KvRadixCache *c = ((RhKv *)p)->c;
    out5[0] = c->stats.hit_tokens;
    out5[1] = c->stats.computed_tokens;
    out5[2] = c->stats.evictions;
    out5[3] = c->stats.allocations;
    out5[4] = c->clock;
}

/* token, parent, child_count, ref_count, in_tree, last_used(lo), last_used(hi) */
void rh_kv_meta(void *p, u32 slot, u32 *out7) {
    KvSlotMeta *m = &((RhKv *)p)->c->meta[slot];
    out7[0] = m->token;
    out7[1] = m->parent;
    out7[2] = m->child_count;
    out7[3] = m->ref_count;
    out7[4] = m->in_tree;
    out7[5] = (u32)m->last_used;
    out7[6] = (u32)(m->last_used >> 32);
}

/* --- kvcache with recurrent state ------------------------------------------ */

typedef struct {
    RhKv base;                 /* first: the rh_kv_* accessors take it */
    Session s;
    Graph g;
    void *buf[1];
    size_t size[1];
    BackendType be[1];
} RhKvS;

void *rh_kvs_create(u32 ctx, u64 state_bytes) {
    RhKvS *h = calloc(1, sizeof(*h));
    h->buf[0] = calloc(1, (size_t)state_bytes);
    h->size[0] = (size_t)state_bytes;
    h->be[0] = BACKEND_CPU;
    h->g.state = h->buf;
    h->g.state_size = h->size;
    h->g.state_backend = h->be;
    h->g.n_state = 1;
    h->g.state_cap = 1;
    h->s.graph = &h->g;
    h->base.kv.n_layer = 1;
    h->base.c = kv_cache_create(&h->s, &h->base.kv, ctx);
    if (!h->base.c) { free(h->buf[0]); free(h); return NULL; }
    return h;
}

void rh_kvs_destroy(void *p) {
    RhKvS *h = p;
    if (!h) return;
    kv_cache_destroy(h->base.c);
    free(h->buf[0]);
    free(h);
}

void rh_kvs_set_state(void *p, const u8 *src) {
    RhKvS *h = p;
    memcpy(h->buf[0], src, h->size[0]);
}

void rh_kvs_get_state(void *p, u8 *dst) {
    RhKvS *h = p;
    memcpy(dst, h->buf[0], h->size[0]);
}

u32 rh_kvs_cap_snaps(void *p) { return ((RhKvS *)p)->base.c->cap_snaps; }

int rh_kvs_checkpoint(void *p, u32 pos) {
    return kv_cache_checkpoint(((RhKvS *)p)->base.c, pos) ? 1 : 0;
}

u32 rh_kvs_restore(void *p, u32 matched, u32 n, u32 *restored) {
    bool r = false;
    u32 pos = kv_cache_restore(((RhKvS *)p)->base.c, matched, n, &r);
    *restored = r ? 1 : 0;
    return pos;
}
