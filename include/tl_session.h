/*
 * tl_session.h — the KV part of the reference's executor for one session:
 * KV storage per layer on the device, the prefix cache on the host, a device
 * mirror of the request's slot table, and the micro-batch loop that runs
 * OP_ATTN for every layer.
 *
 * Counterparts in the reference:
 *   tl_session_create     cache_build_attn_kvcache, src/graph.c:817-872
 *                         (per-layer K/V storage sized ctx_size, radix created
 *                         with kv_cache_create(s, kc, ctx_size))
 *   tl_session_kv_prepare graph_kv_prepare, src/graph.c:1423-1454: match,
 *                         reset, resume = matched < n ? matched : matched - 1
 *                         (0 when nothing matched) for stateless archs, the
 *                         snapshot restore for stateful ones
 *                         (tl_session_set_state); the caller then sets the
 *                         position to `resume` as server.c:834-837 does
 *   tl_session_set_state / tl_session_checkpoint
 *                         graph_state registration and graph_kv_checkpoint
 *                         (src/graph.c:340-408, 1456-1460) with device snapshots
 *   tl_session_execute    graph_execute, src/graph.c:1360-1421, restricted to
 *                         the KV path: n_ubatch chunks, kv_cache_append per
 *                         chunk ("KV slot allocation failed" -> TL_ERANGE),
 *                         then OP_ATTN on every layer with the chunk's rows
 *
 * The activations that the rest of the model would produce (RoPE'd Q and K,
 * V) are inputs: per layer a device array [n_tokens][stride] f32.  Output is
 * the attention result per layer, [n_tokens][q_stride] f32.
 */
#ifndef TL_SESSION_H
#define TL_SESSION_H

#include <stdint.h>
#include "tlkv.h"
#include "tl_kvcache.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tl_session tl_session;

typedef struct tl_session_cfg {
    uint32_t        n_layer;
    uint32_t        n_head;       /* q heads */
    uint32_t        n_kv_head;
    uint32_t        head_dim;     /* == kv_head_dim */
    uint32_t        ctx_size;     /* KV pool size in rows (Session.ctx_size) */
    uint32_t        n_ubatch;     /* prefill chunk (Session.n_ubatch) */
    const uint32_t *window;       /* [n_layer] sliding window (0 = full) or NULL */
    const uint32_t *ring;         /* [n_layer] ring rows for windowed layers
                                     (0 = addressed through the slot table) or NULL */
    int             use_radix;    /* 1: prefix cache maps positions to slots */
    void           *stream;       /* hipStream_t, NULL = default stream */
    int             kv_q8;        /* 1: Q8_0 cache (tl_kv_layer_q8 storage, tl_attn_q8) */
} tl_session_cfg;

int  tl_session_create(const tl_session_cfg *cfg, tl_session **out);
void tl_session_destroy(tl_session *s);

int  tl_session_kv_prepare(tl_session *s, const uint32_t *tokens, uint32_t n,
                           uint32_t *matched, uint32_t *resume);

int  tl_session_execute(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                        const float *const *q, const float *const *k,
                        const float *const *v, float *const *out,
                        uint32_t q_stride, uint32_t kv_stride);

/* tl_session_execute without the attention: the chunk loop's
 * kv_cache_append calls (per n_ubatch chunk, as graph_execute makes them),
 * then one slot upload and the K/V write-through (the part of OP_ATTN at
 * src/backend/cpu/cpu_op.c:995-1008) of the whole batch for every layer.
 * For callers that fill or extend a cache whose attention outputs they do
 * not need.  If a chunk's slot allocation fails, the rows of the chunks
 * before it are still written, the position ends after them, and TL_ERANGE
 * is returned (the reference's chunk loop stops at the same chunk). */
int  tl_session_append(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                       const float *const *k, const float *const *v, uint32_t kv_stride);

/* Prefix fork (no reference counterpart: there a prefix cached by another
 * -np slot's Session is recomputed, src/server.c:1464-1478).  Runs
 * tl_session_kv_prepare's match on `s`; when `donor` caches a longer prefix
 * of tokens[0..n), rows for the difference are allocated in `s`
 * (kv_cache_append) and copied from the donor's pool on the device
 * (tl_kv_copy_between, on s's stream: the donor's rows must be complete in
 * that stream's order).  *matched counts both; *forked = rows copied.  The
 * resume rule is the same as tl_session_kv_prepare's. */
int  tl_session_kv_prepare_from(tl_session *s, tl_session *donor, const uint32_t *tokens,
                                uint32_t n, uint32_t *matched, uint32_t *resume,
                                uint32_t *forked);

/* Eviction compaction (no reference counterpart): evict LRU leaves until at
 * most `keep` rows are live (tl_kv_cache_trim; UINT32_MAX = no eviction),
 * then renumber the pool so the live rows occupy slots [0, n_live)
 * (tl_kv_cache_compact) and move their K/V rows on the device, all layers in
 * one launch.  Rows [n_live, ctx_size) are then free as one block.
 * *evicted / *moved (may be NULL) = rows evicted / moved. */
int  tl_session_compact(tl_session *s, uint32_t keep, uint32_t *evicted, uint32_t *moved);

/* Recurrent state of a stateful arch (hybrid Gated DeltaNet / SSM layers):
 * register the session's device state buffers (graph_state(),
 * src/graph.c:340-366; NULL / 0 = stateless).  The prefix cache then keeps
 * snapshots of them in device memory (kv_cache_checkpoint / restore with
 * device-to-device copies, tl_state_copy, on the session's stream), and
 * tl_session_kv_prepare follows graph_kv_prepare's stateful rule
 * (src/graph.c:1427-1449): a pure continuation keeps the state, anything else
 * zeroes it and resumes at the deepest restored snapshot (0 when none).
 * Re-registering drops the existing snapshots. */
int  tl_session_set_state(tl_session *s, const tl_state_seg *segs, uint32_t n_seg);

/* graph_kv_checkpoint (src/graph.c:1456-1460): snapshot the state at the
 * current position (no-op without radix or state). */
int  tl_session_checkpoint(tl_session *s);

/* accessors */
uint32_t           tl_session_pos(const tl_session *s);        /* Session.n_tokens */
void               tl_session_set_pos(tl_session *s, uint32_t pos);
KvRadixCache      *tl_session_radix(tl_session *s);            /* NULL without radix */
const tl_kv_layer *tl_session_layer(const tl_session *s, uint32_t layer);   /* NULL if kv_q8 */
const tl_kv_layer_q8 *tl_session_layer_q8(const tl_session *s, uint32_t layer); /* NULL if f16 */
const uint32_t    *tl_session_device_slots(const tl_session *s);  /* device [ctx_size] */

/* ---- device mirror of a prefix cache's request map, for executors that run
 * OP_ATTN node by node (the reference's graph_execute, src/graph.c:1395-1413,
 * calls kv_cache_append per chunk and then graph_compute; op_attn reads
 * radix->req.slots, src/backend/cpu/cpu_op.c:988-993).  No reference
 * counterpart: the reference's device backend has no slot table.
 *
 * tl_slot_mirror_sync uploads the part of req.slots[0, req.len) that changed
 * since the previous sync of the same cache (all of it for a cache the mirror
 * has not seen), in `stream` order, and returns the device table in
 * *d_slots.  It consumes the cache's change mark (tl_kv_cache_take_dirty), so
 * one cache feeds one mirror.  Fails with TL_ERANGE for a slot outside the
 * mirror's ctx_size.  A sync that uploads on another stream than the
 * previous upload first synchronises that stream (its queued copies and
 * readers of the map must finish before the map is overwritten). */
typedef struct tl_slot_mirror tl_slot_mirror;
int  tl_slot_mirror_create(uint32_t ctx_size, tl_slot_mirror **out);
void tl_slot_mirror_destroy(tl_slot_mirror *m);
int  tl_slot_mirror_sync(tl_slot_mirror *m, KvRadixCache *radix, void *stream,
                         const uint32_t **d_slots);

#ifdef __cplusplus
}
#endif
#endif
