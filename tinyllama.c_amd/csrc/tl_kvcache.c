/*
 * tl_kvcache.c — host-side prefix cache: logical position -> physical slot.
 *
 * Behaviour follows the reference's src/kvcache.c (cited per function); the
 * data structures are this build's own:
 *   - the prefix index is a token trie (tl_trie.c) instead of rax; a cursor at
 *     the end of the request's prefix makes each appended token one probe
 *     (the reference re-walks the whole key of every position);
 *   - eviction takes its victim from a min-heap of evictable leaves keyed by
 *     last_used instead of scanning every slot (src/kvcache.c:70-81).  The
 *     clock is unique per touch, so the minimum — and the victim — is the
 *     same.  Entries are lazily invalidated: a slot only becomes evictable in
 *     request_release (ref_count reaches 0) or when its last child is evicted,
 *     and its last_used never changes while it is evictable (every touch
 *     happens with ref_count >= 1).
 */
#include "../../include/tl_kvcache.h"
#include "tl_trie.h"

#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#define KV_SNAP_BUDGET (256ULL * 1024 * 1024)
#define KV_SNAP_MAX 16

typedef struct {
    u64 last_used;
    u32 slot;
} HeapEnt;

/* The fields up to `enabled` sit where the reference's struct puts them
 * (src/kvcache.h:50-57), so code compiled against the reference's header —
 * op_attn reading radix->req.slots / req.len (src/backend/cpu/cpu_op.c:988-993),
 * the executor shim — reads this struct correctly.  TlKvRadixHead in
 * tl_kvcache.h spells the layout; the asserts below hold the two together. */
struct KvRadixCache {
    TlTrie         *tree;        /* = &trie (the reference's `rax *tree` slot) */
    KvSlotPool      pool;
    KvSlotMeta     *meta;        /* [n_slots] */
    KvRequestState  req;
    KvCache        *kv;
    u32             n_layer;     /* 0: the KvCache is opaque to this library */
    u32             ctx_size;
    bool            enabled;
    Session        *s;
    TlTrie          trie;        /* token prefix -> slot + 1 */
    u32            *node_of;     /* [ctx_size] trie node holding each in-tree slot */
    /* cursor: trie node of the prefix cur_key[0..cur_len) */
    u32            *cur_key;     /* [ctx_size] */
    u32             cur_len;
    u32             cur_node;
    u64             cur_epoch;
    bool            cur_valid;
    /* evictable leaves */
    HeapEnt        *heap;
    u32             heap_n, heap_cap;
    /* recurrent-state snapshots */
    TlKvStateOps    ops;
    size_t          state_bytes;
    KvStateSnapshot *snaps;
    u32             cap_snaps;
    u64             clock;
    KvRequstStats   stats;
    u32             dirty_lo;
};

_Static_assert(offsetof(struct KvRadixCache, tree) == offsetof(TlKvRadixHead, tree), "layout");
_Static_assert(offsetof(struct KvRadixCache, pool) == offsetof(TlKvRadixHead, pool), "layout");
_Static_assert(offsetof(struct KvRadixCache, meta) == offsetof(TlKvRadixHead, meta), "layout");
_Static_assert(offsetof(struct KvRadixCache, req) == offsetof(TlKvRadixHead, req), "layout");
_Static_assert(offsetof(struct KvRadixCache, kv) == offsetof(TlKvRadixHead, kv), "layout");
_Static_assert(offsetof(struct KvRadixCache, n_layer) == offsetof(TlKvRadixHead, n_layer), "layout");
_Static_assert(offsetof(struct KvRadixCache, ctx_size) == offsetof(TlKvRadixHead, ctx_size), "layout");
_Static_assert(offsetof(struct KvRadixCache, enabled) == offsetof(TlKvRadixHead, enabled), "layout");

/* ---- evictable-leaf heap --------------------------------------------------- */

static bool evictable(const KvRadixCache *c, u32 slot) {
    const KvSlotMeta *m = &c->meta[slot];
    return m->in_tree && m->child_count == 0 && m->ref_count == 0;
}

static void heap_sift_up(HeapEnt *h, u32 i) {
    HeapEnt e = h[i];
    while (i > 0) {
        u32 p = (i - 1) / 2;
        if (h[p].last_used <= e.last_used) break;
        h[i] = h[p];
        i = p;
    }
    h[i] = e;
}

static void heap_sift_down(HeapEnt *h, u32 n, u32 i) {
    HeapEnt e = h[i];
    for (;;) {
        u32 l = 2 * i + 1;
        if (l >= n) break;
        u32 m = (l + 1 < n && h[l + 1].last_used < h[l].last_used) ? l + 1 : l;
        if (h[m].last_used >= e.last_used) break;
        h[i] = h[m];
        i = m;
    }
    h[i] = e;
}

static void heap_rebuild(KvRadixCache *c) {
    c->heap_n = 0;
    for (u32 i = 0; i < c->pool.n_slots; i++)
        if (evictable(c, i)) c->heap[c->heap_n++] = (HeapEnt){c->meta[i].last_used, i};
    for (u32 i = c->heap_n / 2; i-- > 0;) heap_sift_down(c->heap, c->heap_n, i);
}

/* record `slot` if it just became evictable */
static void heap_note(KvRadixCache *c, u32 slot) {
    if (!evictable(c, slot)) return;
    if (c->heap_n == c->heap_cap) {
        heap_rebuild(c);   /* drops stale entries; at most n_slots remain */
        if (c->heap_n == c->heap_cap) return;   /* already present: full set */
    }
    c->heap[c->heap_n] = (HeapEnt){c->meta[slot].last_used, slot};
    heap_sift_up(c->heap, c->heap_n++);
}

/* the evictable slot with the smallest last_used, or KV_SLOT_NONE */
static u32 heap_take(KvRadixCache *c) {
    while (c->heap_n) {
        HeapEnt top = c->heap[0];
        c->heap[0] = c->heap[--c->heap_n];
        if (c->heap_n) heap_sift_down(c->heap, c->heap_n, 0);
        if (evictable(c, top.slot) && c->meta[top.slot].last_used == top.last_used)
            return top.slot;
    }
    return KV_SLOT_NONE;
}

/* ---- snapshots (src/kvcache.c:11-37) ------------------------------------- */

/* snapshot storage: the callbacks' allocator when set, else host memory */
static void *snap_alloc(KvRadixCache *c) {
    return c->ops.alloc ? c->ops.alloc(c->s, c->state_bytes) : malloc(c->state_bytes);
}

static void snap_release(KvRadixCache *c, void *p) {
    if (!p) return;
    if (c->ops.release) c->ops.release(c->s, p);
    else free(p);
}

static void snapshot_clear(KvRadixCache *c, u32 idx) {
    if (!c->snaps || idx >= c->cap_snaps) return;
    KvStateSnapshot *sn = &c->snaps[idx];
    if (sn->valid && sn->slot < c->pool.n_slots && c->meta[sn->slot].snap == idx)
        c->meta[sn->slot].snap = KV_SLOT_NONE;
    sn->valid = false;
    sn->slot = KV_SLOT_NONE;
    sn->pos = 0;
}

static u32 snapshot_select(KvRadixCache *c) {
    if (!c->snaps || c->cap_snaps == 0) return KV_SLOT_NONE;
    for (u32 i = 0; i < c->cap_snaps; i++)
        if (!c->snaps[i].valid) return i;
    u32 victim = KV_SLOT_NONE;
    u64 oldest = UINT64_MAX;
    for (u32 i = 0; i < c->cap_snaps; i++)
        if (c->snaps[i].valid && c->snaps[i].last_used < oldest) {
            oldest = c->snaps[i].last_used;
            victim = i;
        }
    if (victim != KV_SLOT_NONE) snapshot_clear(c, victim);
    return victim;
}

/* ---- slots and requests (src/kvcache.c:44-120) ---------------------------- */

static void mark_dirty(KvRadixCache *c, u32 i) {
    if (i < c->dirty_lo) c->dirty_lo = i;
}

/* drop the request's positions [keep, len) */
static void request_release(KvRadixCache *c, u32 keep) {
    if (keep > c->req.len) keep = c->req.len;
    for (u32 i = keep; i < c->req.len; i++) {
        u32 slot = c->req.slots[i];
        if (slot < c->pool.n_slots && c->meta[slot].ref_count > 0) {
            c->meta[slot].ref_count--;
            heap_note(c, slot);
        }
        c->req.slots[i] = KV_SLOT_NONE;
    }
    if (keep < c->req.len) mark_dirty(c, keep);
    c->req.len = keep;
    if (keep == 0) {
        c->req.shared_len = 0;
        c->req.active = false;
    }
}

static void slot_free(KvRadixCache *c, u32 slot) {
    KvSlotMeta *m = &c->meta[slot];
    if (m->snap != KV_SLOT_NONE) snapshot_clear(c, m->snap);
    m->snap = KV_SLOT_NONE;
    m->in_tree = false;
    m->ref_count = 0;
    m->child_count = 0;
    m->parent = KV_SLOT_NONE;
    c->pool.free_stack[c->pool.n_free++] = slot;
}

static bool slot_evict_one(KvRadixCache *c) {
    u32 victim = heap_take(c);
    if (victim == KV_SLOT_NONE) return false;
    /* the reference rebuilds the victim's key from the parent chain and
     * removes it (src/kvcache.c:82-96); the trie node holding the victim is
     * known, so the same key is removed without re-walking it */
    tl_trie_remove_node(&c->trie, c->node_of[victim]);
    c->node_of[victim] = TL_TRIE_NONE;
    u32 parent = c->meta[victim].parent;
    slot_free(c, victim);
    if (parent != KV_SLOT_NONE && c->meta[parent].child_count > 0) {
        c->meta[parent].child_count--;
        heap_note(c, parent);
    }
    c->stats.evictions++;
    return true;
}

static u32 slot_alloc(KvRadixCache *c, u32 token, u32 parent) {
    while (c->pool.n_free == 0)
        if (!slot_evict_one(c)) return KV_SLOT_NONE;
    u32 slot = c->pool.free_stack[--c->pool.n_free];
    KvSlotMeta *m = &c->meta[slot];
    m->token = token;
    m->parent = parent;
    m->child_count = 0;
    m->ref_count = 1;
    m->last_used = ++c->clock;
    m->in_tree = false;
    c->stats.allocations++;
    return slot;
}

/* ---- create / destroy (src/kvcache.c:122-190) ---------------------------- */

void kv_cache_destroy(KvRadixCache *c) {
    if (!c) return;
    tl_trie_free(&c->trie);
    free(c->pool.free_stack);
    free(c->meta);
    free(c->req.slots);
    free(c->node_of);
    free(c->cur_key);
    free(c->heap);
    if (c->snaps) {
        for (u32 i = 0; i < c->cap_snaps; i++) snap_release(c, c->snaps[i].state);
        free(c->snaps);
    }
    free(c);
}

KvRadixCache *kv_cache_create(Session *s, KvCache *kv, u32 ctx_size) {
    if (!kv || ctx_size == 0) return NULL;
    KvRadixCache *c = (KvRadixCache *)calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->kv = kv;
    c->s = s;
    c->ctx_size = ctx_size;
    c->enabled = true;
    c->tree = &c->trie;
    c->pool.n_slots = ctx_size;
    c->pool.free_stack = (u32 *)malloc((size_t)ctx_size * sizeof(u32));
    c->meta = (KvSlotMeta *)calloc(ctx_size, sizeof(KvSlotMeta));
    c->req.slots = (u32 *)malloc((size_t)ctx_size * sizeof(u32));
    c->node_of = (u32 *)malloc((size_t)ctx_size * sizeof(u32));
    c->cur_key = (u32 *)malloc((size_t)ctx_size * sizeof(u32));
    c->heap_cap = 4 * ctx_size + 16;
    c->heap = (HeapEnt *)malloc((size_t)c->heap_cap * sizeof(HeapEnt));
    if (!c->pool.free_stack || !c->meta || !c->req.slots || !c->node_of || !c->cur_key ||
        !c->heap || !tl_trie_init(&c->trie, ctx_size)) {
        kv_cache_destroy(c);
        return NULL;
    }
    /* slot 0 is popped first */
    for (u32 i = 0; i < ctx_size; i++) c->pool.free_stack[i] = ctx_size - 1 - i;
    c->pool.n_free = ctx_size;
    for (u32 i = 0; i < ctx_size; i++) {
        c->meta[i].parent = KV_SLOT_NONE;
        c->meta[i].snap = KV_SLOT_NONE;
        c->req.slots[i] = KV_SLOT_NONE;
        c->node_of[i] = TL_TRIE_NONE;
    }
    c->dirty_lo = 0;
    return c;
}

void tl_kv_cache_set_state_ops(KvRadixCache *c, const TlKvStateOps *ops) {
    if (!c) return;
    if (c->snaps) {
        for (u32 i = 0; i < c->cap_snaps; i++) {
            snapshot_clear(c, i);
            snap_release(c, c->snaps[i].state);
        }
        free(c->snaps);
        c->snaps = NULL;
        c->cap_snaps = 0;
    }
    memset(&c->ops, 0, sizeof(c->ops));
    c->state_bytes = 0;
    if (!ops || !ops->bytes || !ops->save || !ops->load) return;
    c->ops = *ops;
    c->state_bytes = ops->bytes(c->s);
    if (!c->state_bytes) return;
    u64 max = KV_SNAP_BUDGET / (u64)c->state_bytes;   /* src/kvcache.c:155-165 */
    if (max < 1) max = 1;
    if (max > KV_SNAP_MAX) max = KV_SNAP_MAX;
    c->snaps = (KvStateSnapshot *)calloc((size_t)max, sizeof(KvStateSnapshot));
    if (!c->snaps) {
        c->state_bytes = 0;
        return;
    }
    c->cap_snaps = (u32)max;
    for (u32 i = 0; i < c->cap_snaps; i++) c->snaps[i].slot = KV_SLOT_NONE;
}

/* ---- match (src/kvcache.c:192-218) -------------------------------------- */

u32 kv_cache_match(KvRadixCache *c, const u32 *tokens, u32 n) {
    if (!c || !c->enabled || !tokens || n == 0) return 0;
    if (n > c->ctx_size) n = c->ctx_size;
    request_release(c, 0);
    u32 matched = 0;
    u32 node = TL_TRIE_ROOT;
    for (u32 i = 0; i < n; i++) {
        u32 nx = tl_trie_child(&c->trie, node, tokens[i]);
        if (nx == TL_TRIE_NONE || c->trie.nodes[nx].value == 0) break;
        u32 slot = c->trie.nodes[nx].value - 1;
        if (slot >= c->pool.n_slots || !c->meta[slot].in_tree) break;
        c->req.slots[i] = slot;
        c->meta[slot].ref_count++;
        c->meta[slot].last_used = ++c->clock;
        node = nx;
        matched = i + 1;
    }
    if (matched) mark_dirty(c, 0);
    c->req.len = matched;
    c->req.shared_len = matched;
    c->req.active = matched > 0;
    c->stats.hit_tokens += matched;
    if (n > matched) c->stats.computed_tokens += n - matched;
    /* the cursor now ends at the matched prefix */
    memcpy(c->cur_key, tokens, (size_t)matched * sizeof(u32));
    c->cur_len = matched;
    c->cur_node = node;
    c->cur_epoch = c->trie.epoch;
    c->cur_valid = true;
    return matched;
}

/* ---- append (src/kvcache.c:220-270) ------------------------------------- */

/* trie node of tokens[0..len): from the cursor when it still describes that
 * prefix, else by walking from the root (TL_TRIE_NONE if absent) */
static u32 prefix_node(KvRadixCache *c, const u32 *tokens, u32 len) {
    if (c->cur_valid && c->cur_len == len &&
        memcmp(c->cur_key, tokens, (size_t)len * sizeof(u32)) == 0) {
        if (c->cur_epoch == c->trie.epoch || len == 0) return c->cur_node;
        /* nodes were pruned since: the cursor still stands when it is the
         * node of the request's slot for position len - 1.  That slot is
         * pinned by the request (ref_count >= 1), so its key -- and the node
         * holding it -- cannot have been evicted. */
        if (len <= c->req.len) {
            const u32 s = c->req.slots[len - 1];
            if (s < c->pool.n_slots && c->meta[s].in_tree && c->meta[s].ref_count > 0 &&
                c->node_of[s] == c->cur_node)
                return c->cur_node;
        }
    }
    return tl_trie_walk(&c->trie, TL_TRIE_ROOT, tokens, len);
}

/* a node that eviction can free: not the root and not holding the key of a
 * slot some request still references */
static bool node_may_vanish(const KvRadixCache *c, u32 node) {
    if (node == TL_TRIE_ROOT || node == TL_TRIE_NONE) return false;
    u32 v = c->trie.nodes[node].value;
    return v == 0 || c->meta[v - 1].ref_count == 0;
}

bool kv_cache_append(KvRadixCache *c, const u32 *tokens, u32 pos, u32 n) {
    if (!c || !c->enabled || n == 0) return true;
    if ((u64)pos + n > c->ctx_size) return false;

    u32 node = prefix_node(c, tokens, pos);
    c->cur_valid = false;   /* set again below once the new prefix is in */
    for (u32 k = 0; k < n; k++) {
        const u32 i = pos + k;
        if (i < c->req.len) {
            u32 old = c->req.slots[i];
            if (old < c->pool.n_slots && c->meta[old].in_tree &&
                c->meta[old].token == tokens[i]) {
                c->meta[old].last_used = ++c->clock;
                node = tl_trie_child(&c->trie, node, tokens[i]);
                continue;
            }
            request_release(c, i);
        }
        if (i != c->req.len) return false;

        u32 nx = tl_trie_child(&c->trie, node, tokens[i]);
        if (nx != TL_TRIE_NONE && c->trie.nodes[nx].value) {
            u32 slot = c->trie.nodes[nx].value - 1;
            if (slot >= c->pool.n_slots || !c->meta[slot].in_tree) return false;
            c->req.slots[i] = slot;
            mark_dirty(c, i);
            c->meta[slot].ref_count++;
            c->meta[slot].last_used = ++c->clock;
            c->req.len = i + 1;
            node = nx;
            continue;
        }

        u32 parent = i > 0 ? c->req.slots[i - 1] : KV_SLOT_NONE;
        if (i > 0 && parent == KV_SLOT_NONE) return false;
        const bool fragile = node_may_vanish(c, node);
        const u64 epoch = c->trie.epoch;
        u32 slot = slot_alloc(c, tokens[i], parent);
        if (slot == KV_SLOT_NONE) return false;
        if (fragile && c->trie.epoch != epoch) node = TL_TRIE_NONE;

        c->req.slots[i] = slot;
        mark_dirty(c, i);
        if (parent != KV_SLOT_NONE) c->meta[parent].child_count++;
        /* insert key tokens[0..i] (creating the prefix path if needed) */
        if (node == TL_TRIE_NONE) {
            node = TL_TRIE_ROOT;
            for (u32 j = 0; j < i && node != TL_TRIE_NONE; j++)
                node = tl_trie_child_make(&c->trie, node, tokens[j]);
        }
        nx = tl_trie_child_make(&c->trie, node, tokens[i]);
        if (nx == TL_TRIE_NONE) {
            if (parent != KV_SLOT_NONE && c->meta[parent].child_count > 0) {
                c->meta[parent].child_count--;
                heap_note(c, parent);
            }
            slot_free(c, slot);
            return false;
        }
        c->trie.nodes[nx].value = slot + 1;
        c->node_of[slot] = nx;
        c->meta[slot].in_tree = true;
        c->req.len = i + 1;
        node = nx;
    }
    /* cursor: prefix tokens[0..pos+n) ends at `node` */
    if (node != TL_TRIE_NONE) {
        memcpy(c->cur_key, tokens, (size_t)(pos + n) * sizeof(u32));
        c->cur_len = pos + n;
        c->cur_node = node;
        c->cur_epoch = c->trie.epoch;
        c->cur_valid = true;
    }
    return true;
}

/* ---- state snapshots (src/kvcache.c:272-321) ---------------------------- */

bool kv_cache_checkpoint(KvRadixCache *c, u32 pos) {
    if (!c || !c->state_bytes || !c->snaps || pos == 0 || pos > c->req.len) return true;
    u32 slot = c->req.slots[pos - 1];
    if (slot >= c->pool.n_slots || !c->meta[slot].in_tree) return true;
    u32 idx = c->meta[slot].snap;
    if (idx < c->cap_snaps && c->snaps[idx].valid) {
        c->snaps[idx].pos = pos;
        c->snaps[idx].last_used = ++c->clock;
        return true;
    }
    idx = snapshot_select(c);
    if (idx == KV_SLOT_NONE) return true;
    KvStateSnapshot *sn = &c->snaps[idx];
    if (!sn->state) sn->state = snap_alloc(c);
    if (!sn->state || !c->ops.save(c->s, sn->state, c->state_bytes)) return false;
    sn->valid = true;
    sn->slot = slot;
    sn->pos = pos;
    sn->last_used = ++c->clock;
    c->meta[slot].snap = idx;
    return true;
}

u32 kv_cache_restore(KvRadixCache *c, u32 matched, u32 n, bool *restored) {
    if (restored) *restored = false;
    if (!c || !c->state_bytes || !c->snaps || matched == 0) return 0;
    for (u32 pos = matched; pos > 0; pos--) {
        if (pos >= n) continue;
        u32 slot = c->req.slots[pos - 1];
        if (slot >= c->pool.n_slots || !c->meta[slot].in_tree) continue;
        u32 idx = c->meta[slot].snap;
        if (idx >= c->cap_snaps || !c->snaps[idx].valid) continue;
        if (c->snaps[idx].pos != pos || !c->snaps[idx].state) continue;
        if (!c->ops.load(c->s, c->snaps[idx].state, c->state_bytes)) return 0;
        c->snaps[idx].last_used = ++c->clock;
        if (restored) *restored = true;
        return pos;
    }
    return 0;
}

/* ---- compaction and read-only lookup (no reference counterpart) ---------- */

/* Renumber the cached slots so that the n_live in-tree slots occupy
 * [0, n_live).  Every live slot s >= n_live moves to a free slot below
 * n_live, lowest to lowest; moves[i] = (src[i], dst[i]).  Slot metadata,
 * parent links, the trie's slot values, req.slots, snapshots and the
 * evictable-leaf heap follow the move; the free stack is rebuilt so that the
 * lowest free slot pops first, as after kv_cache_create.  Logical behaviour
 * (hits, evictions, the LRU order) is unchanged: eviction and matching never
 * depend on slot numbers.  Returns the number of moves, or UINT32_MAX when
 * more than `max` moves are needed (nothing changed then). */
u32 tl_kv_cache_compact(KvRadixCache *c, u32 *src, u32 *dst, u32 max) {
    if (!c) return UINT32_MAX;
    const u32 ns = c->pool.n_slots;
    u32 n_live = 0;
    for (u32 i = 0; i < ns; i++) n_live += c->meta[i].in_tree;
    u32 n_moves = 0;
    for (u32 i = n_live; i < ns; i++) n_moves += c->meta[i].in_tree;
    if (n_moves > max || (n_moves && (!src || !dst))) return UINT32_MAX;
    if (n_moves == 0) goto rebuild_free;
    {
        u32 *remap = (u32 *)malloc((size_t)ns * sizeof(u32));
        if (!remap) return UINT32_MAX;
        for (u32 i = 0; i < ns; i++) remap[i] = i;
        u32 hole = 0, k = 0;
        for (u32 s = n_live; s < ns; s++) {
            if (!c->meta[s].in_tree) continue;
            while (c->meta[hole].in_tree) hole++;
            remap[s] = hole;
            src[k] = s;
            dst[k] = hole;
            k++;
            c->meta[hole] = c->meta[s];
            c->meta[hole].in_tree = true;   /* claims the hole for the scan */
            KvSlotMeta *m = &c->meta[s];
            m->in_tree = false;
            m->ref_count = 0;
            m->child_count = 0;
            m->parent = KV_SLOT_NONE;
            m->snap = KV_SLOT_NONE;
            hole++;
        }
        for (u32 i = 0; i < n_live; i++)
            if (c->meta[i].parent != KV_SLOT_NONE) c->meta[i].parent = remap[c->meta[i].parent];
        for (u32 nd = 1; nd < c->trie.n_nodes; nd++) {
            u32 v = c->trie.nodes[nd].value;
            if (v) c->trie.nodes[nd].value = remap[v - 1] + 1;
        }
        for (u32 k2 = 0; k2 < k; k2++) {
            c->node_of[dst[k2]] = c->node_of[src[k2]];
            c->node_of[src[k2]] = TL_TRIE_NONE;
        }
        for (u32 i = 0; i < c->req.len; i++)
            if (c->req.slots[i] < ns) c->req.slots[i] = remap[c->req.slots[i]];
        if (c->req.len) mark_dirty(c, 0);
        for (u32 i = 0; i < c->cap_snaps; i++)
            if (c->snaps[i].valid && c->snaps[i].slot < ns) c->snaps[i].slot = remap[c->snaps[i].slot];
        free(remap);
        heap_rebuild(c);
    }
rebuild_free:
    c->pool.n_free = 0;
    for (u32 i = ns; i-- > 0;)
        if (!c->meta[i].in_tree) c->pool.free_stack[c->pool.n_free++] = i;
    return n_moves;
}

/* Evict least-recently-used unreferenced leaves (the victims slot_alloc
 * would take, in the same order) until at most `keep` slots are live.
 * Returns the number evicted; stops early when nothing is evictable. */
u32 tl_kv_cache_trim(KvRadixCache *c, u32 keep) {
    if (!c) return 0;
    u32 n = 0;
    while (c->pool.n_slots - c->pool.n_free > keep && slot_evict_one(c)) n++;
    return n;
}

/* Length of the longest cached prefix of tokens[0..n) and its slots, without
 * touching reference counts, the LRU clock or statistics. */
u32 tl_kv_cache_lookup(const KvRadixCache *c, const u32 *tokens, u32 n, u32 *slots) {
    if (!c || !c->enabled || !tokens || n == 0) return 0;
    if (n > c->ctx_size) n = c->ctx_size;
    u32 node = TL_TRIE_ROOT, matched = 0;
    for (u32 i = 0; i < n; i++) {
        u32 nx = tl_trie_child(&c->trie, node, tokens[i]);
        if (nx == TL_TRIE_NONE || c->trie.nodes[nx].value == 0) break;
        u32 slot = c->trie.nodes[nx].value - 1;
        if (slot >= c->pool.n_slots || !c->meta[slot].in_tree) break;
        if (slots) slots[i] = slot;
        node = nx;
        matched = i + 1;
    }
    return matched;
}

/* ---- accessors ------------------------------------------------------------ */

const KvRequestState *tl_kv_cache_req(const KvRadixCache *c) { return c ? &c->req : NULL; }
const KvRequstStats *tl_kv_cache_stats(const KvRadixCache *c) { return c ? &c->stats : NULL; }
const KvSlotMeta *tl_kv_cache_meta(const KvRadixCache *c, u32 slot) {
    return (c && slot < c->pool.n_slots) ? &c->meta[slot] : NULL;
}
u32 tl_kv_cache_n_free(const KvRadixCache *c) { return c ? c->pool.n_free : 0; }
u64 tl_kv_cache_clock(const KvRadixCache *c) { return c ? c->clock : 0; }
u32 tl_kv_cache_take_dirty(KvRadixCache *c) {
    if (!c) return KV_SLOT_NONE;
    u32 d = c->dirty_lo;
    c->dirty_lo = KV_SLOT_NONE;
    return d;
}
