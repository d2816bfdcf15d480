/*
 * tl_kvcache.h — host-side KV-cache bookkeeping: the prefix cache that maps a
 * request's logical positions to physical cache rows ("slots").
 *
 * Drop-in for the reference's src/kvcache.h:72-90 — same function names,
 * signatures and semantics:
 *   kv_cache_create      src/kvcache.c:122-174  (slot 0 pops first, all free)
 *   kv_cache_destroy     src/kvcache.c:176-190
 *   kv_cache_match       src/kvcache.c:192-218  (lock the longest cached prefix)
 *   kv_cache_append      src/kvcache.c:220-270  (map / allocate slots for
 *                        [pos, pos+n); LRU leaf eviction when the pool is empty,
 *                        src/kvcache.c:70-120)
 *   kv_cache_checkpoint  src/kvcache.c:272-300  (recurrent-state snapshots)
 *   kv_cache_restore     src/kvcache.c:302-321
 * The request map (req.slots / req.len / req.shared_len / req.active), the
 * per-slot metadata and the statistics keep the reference's field names, so
 * code that reads radix->req.slots (src/backend/cpu/cpu_op.c:988-993) reads
 * the same thing here.
 *
 * Differences that callers can observe: none in slot assignment, eviction
 * order, hit counts or return values (checked against the compiled reference
 * on random request streams).  The prefix index is a token trie instead of
 * the vendored rax; eviction picks the same victim (the in-tree leaf with
 * ref_count 0 and the smallest last_used) from a heap instead of a full scan.
 * The struct's leading fields (through req and enabled) sit at the
 * reference's offsets (TlKvRadixHead below).  Session and KvCache are opaque
 * here: kv_cache_create only keeps the pointers; state snapshots go through the callbacks set with
 * tl_kv_cache_set_state_ops (none set = no snapshots, as for a Session whose
 * graph has no recurrent state).
 */
#ifndef TL_KVCACHE_H
#define TL_KVCACHE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint32_t u32;
typedef uint64_t u64;

typedef struct Session Session;   /* opaque: passed back to the state callbacks */
typedef struct KvCache KvCache;   /* opaque: only stored */

#define KV_SLOT_NONE UINT32_MAX

typedef struct {
    u32  token;        /* token id stored in this slot */
    u32  parent;       /* slot of the previous token; KV_SLOT_NONE for root */
    u32  child_count;  /* direct children (leaf detection) */
    u32  ref_count;    /* requests currently using this slot */
    u64  last_used;    /* LRU clock value */
    u32  snap;         /* state snapshot index or KV_SLOT_NONE */
    bool in_tree;      /* attached to the prefix index */
} KvSlotMeta;

typedef struct {
    u32  n_slots;
    u32  n_free;
    u32 *free_stack;   /* LIFO of free slot indices */
} KvSlotPool;

typedef struct {
    u32 *slots;        /* [ctx_size] logical position -> physical slot */
    u32  len;
    u32  shared_len;
    bool active;
} KvRequestState;

typedef struct {
    u64 hit_tokens;
    u64 computed_tokens;
    u64 evictions;
    u64 allocations;
} KvRequstStats;       /* spelled as the reference spells it (kvcache.h:34-39) */

typedef struct {
    void *state;
    u32   slot;
    u32   pos;
    u64   last_used;
    bool  valid;
} KvStateSnapshot;

/* Recurrent-state callbacks (the reference calls graph_state_bytes/save/load,
 * src/graph.c:368-408).  alloc / release (optional) own the snapshot
 * storage: when set, a snapshot's `state` comes from alloc(s, bytes) — e.g.
 * device memory, so save/load are device-to-device copies
 * (tl_session_set_state) — and is returned with release(s, ptr); when NULL
 * it is host memory (malloc/free, as the reference's smalloc/sfree). */
typedef struct {
    size_t (*bytes)(Session *s);
    bool   (*save)(Session *s, void *dst, size_t cap);
    bool   (*load)(Session *s, const void *src, size_t len);
    void  *(*alloc)(Session *s, size_t bytes);
    void   (*release)(Session *s, void *ptr);
} TlKvStateOps;

typedef struct KvRadixCache KvRadixCache;

/* The leading fields of struct KvRadixCache, in the reference's order and at
 * its offsets (src/kvcache.h:50-57).  op_attn reads radix->req.slots and
 * radix->req.len straight from the struct (src/backend/cpu/cpu_op.c:988-993),
 * and so does any code compiled against the reference's kvcache.h, so a
 * KvRadixCache made by this library may be handed to such code as the
 * reference's own.  Fields past `enabled` are private and differ.  `tree`
 * points to this library's trie, not to a rax; `n_layer` is 0 (KvCache is
 * opaque here).  Read-only for callers: the library owns every field. */
typedef struct {
    void          *tree;
    KvSlotPool     pool;
    KvSlotMeta    *meta;
    KvRequestState req;
    KvCache       *kv;
    u32            n_layer;
    u32            ctx_size;
    bool           enabled;
} TlKvRadixHead;

KvRadixCache *kv_cache_create(Session *s, KvCache *kv, u32 ctx_size);
void kv_cache_destroy(KvRadixCache *c);
u32  kv_cache_match(KvRadixCache *c, const u32 *tokens, u32 n);
bool kv_cache_append(KvRadixCache *c, const u32 *tokens, u32 pos, u32 n);
bool kv_cache_checkpoint(KvRadixCache *c, u32 pos);
u32  kv_cache_restore(KvRadixCache *c, u32 matched, u32 n, bool *restored);

/* ---- accessors (no reference counterpart: the reference's callers read the
 *      struct fields directly) ---- */
void tl_kv_cache_set_state_ops(KvRadixCache *c, const TlKvStateOps *ops);
const KvRequestState *tl_kv_cache_req(const KvRadixCache *c);
const KvRequstStats  *tl_kv_cache_stats(const KvRadixCache *c);
const KvSlotMeta     *tl_kv_cache_meta(const KvRadixCache *c, u32 slot);
u32  tl_kv_cache_n_free(const KvRadixCache *c);
u64  tl_kv_cache_clock(const KvRadixCache *c);
/* Lowest req.slots index written since the last call (KV_SLOT_NONE if none),
 * and reset; lets a device mirror of req.slots upload only what changed. */
u32  tl_kv_cache_take_dirty(KvRadixCache *c);

/* ---- compaction and lookup (no reference counterpart: the reference never
 *      moves a cached row, src/kvcache.c:59-120) ---- */

/* Renumber cached slots so the n_live in-tree slots occupy [0, n_live).
 * Writes the moves to src[i] -> dst[i] (host arrays of at least `max`
 * entries; dst rows are always free, below every src row) and updates slot
 * metadata, the prefix index, req.slots (marked dirty from 0), snapshots and
 * the free stack (lowest free slot pops first).  The caller copies the rows
 * on the device (tl_kv_copy) before any kernel reads the new slot numbers.
 * Returns the move count, or UINT32_MAX if more than `max` are needed (then
 * nothing changed).  Hits, evictions and the LRU order are unaffected. */
u32  tl_kv_cache_compact(KvRadixCache *c, u32 *src, u32 *dst, u32 max);

/* Evict unreferenced leaves in LRU order — the victims and order of the
 * reference's on-demand eviction (src/kvcache.c:70-104) — until at most
 * `keep` slots are live.  Returns the number evicted (counted in
 * stats.evictions); stops early when nothing is evictable. */
u32  tl_kv_cache_trim(KvRadixCache *c, u32 keep);

/* Longest cached prefix of tokens[0..n) and its slots (slots may be NULL),
 * read-only: no reference counts, LRU touches or statistics change. */
u32  tl_kv_cache_lookup(const KvRadixCache *c, const u32 *tokens, u32 n, u32 *slots);

#ifdef __cplusplus
}
#endif
#endif
