/*
 * tl_session.c — one session's KV path: device storage per layer, the host
 * prefix cache, the device mirror of req.slots, and the micro-batch loop
 * (reference: src/graph.c:817-872, 1360-1454).
 */
#include "../../include/tl_session.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int tl_set_error(int code, const char *msg);

#define STAGE_WORDS (1u << 20)   /* pinned staging ring for slot uploads */

struct tl_session {
    tl_session_cfg cfg;
    uint32_t      *window;      /* [n_layer] */
    tl_kv_layer   *layers;      /* [n_layer] f16 storage, or NULL */
    tl_kv_layer_q8 *layers8;    /* [n_layer] Q8_0 storage (cfg.kv_q8), or NULL */
    KvRadixCache  *radix;
    uint32_t      *tokens;      /* [ctx_size] host token history (Session.tokens) */
    uint32_t       n_tokens;    /* Session.n_tokens */
    uint32_t      *d_slots;     /* device mirror of req.slots */
    uint32_t      *d_moves;     /* device [2 * ctx_size]: n copy sources, then n destinations */
    uint32_t      *h_moves;     /* host   [2 * ctx_size] */
    uint32_t      *stage;       /* pinned */
    uint32_t       stage_pos;
    float          scale;
    int            has_ring;    /* some layer keeps only a window of rows */
    uint32_t       min_ring;    /* smallest ring of those layers (0: none) */
    tl_state_seg  *state;       /* registered recurrent-state buffers (device) */
    uint32_t       n_state;
    size_t         state_bytes; /* their total (graph_state_bytes) */
};

static int fail(int code, const char *msg) { return tl_set_error(code, msg); }

void tl_session_destroy(tl_session *s) {
    if (!s) return;
    if (s->layers)
        for (uint32_t l = 0; l < s->cfg.n_layer; l++) tl_kv_layer_free(&s->layers[l]);
    if (s->layers8)
        for (uint32_t l = 0; l < s->cfg.n_layer; l++) tl_kv_layer_free_q8(&s->layers8[l]);
    free(s->layers);
    free(s->layers8);
    free(s->window);
    kv_cache_destroy(s->radix);
    free(s->tokens);
    free(s->state);
    if (s->d_slots) (void)hipFree(s->d_slots);
    if (s->d_moves) (void)hipFree(s->d_moves);
    free(s->h_moves);
    if (s->stage) (void)hipHostFree(s->stage);
    free(s);
}

int tl_session_create(const tl_session_cfg *cfg, tl_session **out) {
    if (!cfg || !out || cfg->n_layer == 0 || cfg->ctx_size == 0 || cfg->n_ubatch == 0 ||
        cfg->n_kv_head == 0 || cfg->n_head % cfg->n_kv_head)
        return fail(TL_EINVAL, "session: bad configuration");
    *out = NULL;
    tl_session *s = (tl_session *)calloc(1, sizeof(*s));
    if (!s) return fail(TL_ENOMEM, "session: host allocation");
    s->cfg = *cfg;
    s->cfg.window = NULL;
    s->cfg.ring = NULL;
    s->window = (uint32_t *)calloc(cfg->n_layer, sizeof(uint32_t));
    if (cfg->kv_q8)
        s->layers8 = (tl_kv_layer_q8 *)calloc(cfg->n_layer, sizeof(tl_kv_layer_q8));
    else
        s->layers = (tl_kv_layer *)calloc(cfg->n_layer, sizeof(tl_kv_layer));
    s->tokens = (uint32_t *)calloc(cfg->ctx_size, sizeof(uint32_t));
    if (!s->window || (!s->layers && !s->layers8) || !s->tokens) {
        tl_session_destroy(s);
        return fail(TL_ENOMEM, "session: host allocation");
    }
    for (uint32_t l = 0; l < cfg->n_layer; l++) {
        s->window[l] = cfg->window ? cfg->window[l] : 0;
        uint32_t ring = cfg->ring ? cfg->ring[l] : 0;
        if (ring) {
            s->has_ring = 1;
            if (!s->min_ring || ring < s->min_ring) s->min_ring = ring;
        }
        if (ring && (!s->window[l] || ring < s->window[l] + cfg->n_ubatch - 1)) {
            tl_session_destroy(s);
            return fail(TL_EINVAL, "session: a ring needs window + n_ubatch - 1 rows");
        }
        const uint32_t rows = ring ? ring : cfg->ctx_size;
        int rc = cfg->kv_q8
                     ? tl_kv_layer_alloc_q8(&s->layers8[l], rows, cfg->n_kv_head, cfg->head_dim, ring)
                     : tl_kv_layer_alloc(&s->layers[l], rows, cfg->n_kv_head, cfg->head_dim, ring);
        if (rc) {
            tl_session_destroy(s);
            return rc;
        }
    }
    if (cfg->use_radix) {
        /* the prefix cache only stores the KvCache pointer; the session is
         * handed back to the state callbacks */
        s->radix = kv_cache_create((Session *)s,
                                   s->layers8 ? (KvCache *)s->layers8 : (KvCache *)s->layers,
                                   cfg->ctx_size);
        if (!s->radix) {
            tl_session_destroy(s);
            return fail(TL_ENOMEM, "session: kv_cache_create failed");
        }
        s->h_moves = (uint32_t *)malloc((size_t)cfg->ctx_size * 2 * sizeof(uint32_t));
        if (!s->h_moves ||
            hipMalloc((void **)&s->d_slots, (size_t)cfg->ctx_size * sizeof(uint32_t)) != hipSuccess ||
            hipMalloc((void **)&s->d_moves, (size_t)cfg->ctx_size * 2 * sizeof(uint32_t)) != hipSuccess ||
            hipHostMalloc((void **)&s->stage, STAGE_WORDS * sizeof(uint32_t), 0) != hipSuccess) {
            s->stage = NULL;
            tl_session_destroy(s);
            return fail(TL_ENOMEM, "session: slot table allocation");
        }
    }
    s->scale = 1.0f / sqrtf((float)cfg->head_dim);   /* src/graph.c:1275 */
    *out = s;
    return TL_OK;
}

/* copy host words to device memory in stream order through a pinned ring of
 * STAGE_WORDS words (*pos = next free word) */
static int stage_upload(uint32_t *stage, uint32_t *pos, hipStream_t st, uint32_t *d_dst,
                        const uint32_t *src, uint32_t n_words) {
    while (n_words) {
        uint32_t n = n_words;
        if (n > STAGE_WORDS) n = STAGE_WORDS;
        if (*pos + n > STAGE_WORDS) {
            /* staged words may still be read by queued copies */
            if (hipStreamSynchronize(st) != hipSuccess) return fail(TL_EHIP, "upload: sync");
            *pos = 0;
        }
        uint32_t *stg = stage + *pos;
        memcpy(stg, src, (size_t)n * sizeof(uint32_t));
        if (hipMemcpyAsync(d_dst, stg, (size_t)n * sizeof(uint32_t), hipMemcpyHostToDevice,
                           st) != hipSuccess)
            return fail(TL_EHIP, "upload: copy");
        *pos += n;
        d_dst += n;
        src += n;
        n_words -= n;
    }
    return TL_OK;
}

static int upload_words(tl_session *s, uint32_t *d_dst, const uint32_t *src, uint32_t n_words) {
    return stage_upload(s->stage, &s->stage_pos, (hipStream_t)s->cfg.stream, d_dst, src,
                        n_words);
}

/* upload req.slots[lo..hi) to the device mirror */
static int upload_slots(tl_session *s, uint32_t lo, uint32_t hi) {
    if (hi <= lo) return TL_OK;
    const KvRequestState *req = tl_kv_cache_req(s->radix);
    for (uint32_t i = lo; i < hi; i++)
        if (req->slots[i] >= s->cfg.ctx_size) return fail(TL_ERANGE, "session: slot outside the cache");
    return upload_words(s, s->d_slots + lo, req->slots + lo, hi - lo);
}

/* upload whatever part of req.slots changed since the last upload */
static int sync_slots(tl_session *s) {
    uint32_t lo = tl_kv_cache_take_dirty(s->radix);
    uint32_t len = tl_kv_cache_req(s->radix)->len;
    if (lo == KV_SLOT_NONE || lo >= len) return TL_OK;
    return upload_slots(s, lo, len);
}

int tl_session_kv_prepare(tl_session *s, const uint32_t *tokens, uint32_t n,
                          uint32_t *matched, uint32_t *resume) {
    if (matched) *matched = 0;
    if (resume) *resume = 0;
    if (!s || !tokens || n == 0) return TL_OK;
    uint32_t m = 0;
    if (s->radix) {
        m = kv_cache_match(s->radix, tokens, n);
    } else if (s->n_tokens) {   /* no prefix cache: common prefix with history */
        uint32_t limit = s->n_tokens < n ? s->n_tokens : n;
        while (m < limit && s->tokens[m] == tokens[m]) m++;
    }
    uint32_t r;
    if (s->state_bytes && m == s->n_tokens && n > m) {
        /* stateful continuation: keep the state, resume at the match
         * (src/graph.c:1439-1443) */
        if (matched) *matched = m;
        if (resume) *resume = m;
        return TL_OK;
    }
    if (s->state_bytes) {
        /* reset (zero the state), then restore the deepest snapshot at or
         * below the match (src/graph.c:1445-1449, kvcache.c:303-321); ring
         * layers cannot resume, so they take no snapshot either */
        int rc = tl_state_copy(s->state, s->n_state, NULL, TL_STATE_ZERO, s->cfg.stream);
        if (rc) return rc;
        r = (s->radix && !s->has_ring) ? kv_cache_restore(s->radix, m, n, NULL) : 0;
    } else {
        r = m == 0 ? 0 : (m < n ? m : m - 1);
        /* ring layers hold only the last window + n_ubatch - 1 rows of the
         * previous request: a prefix hit cannot be resumed on them */
        if (s->has_ring) r = 0;
    }
    s->n_tokens = r;   /* reset, then resume (src/graph.c:1443-1452, server.c:837) */
    if (r) memcpy(s->tokens, tokens, (size_t)r * sizeof(uint32_t));
    if (matched) *matched = m;
    if (resume) *resume = r;
    return TL_OK;
}

/* write-through of rows [pos, pos + n) of every layer: launches cover up to 64
 * layers (the library splits them per 16), and on sessions with ring layers
 * no launch spans more rows than the smallest ring, so positions p and p + R
 * never land on one physical row within a launch (stream order then keeps
 * the later row) */
static int write_rows(tl_session *s, const float *const *k, const float *const *v,
                      uint32_t kv_stride, uint32_t pos, uint32_t n) {
    const uint32_t *sl = s->radix ? s->d_slots : NULL;
    const uint32_t piece = s->min_ring ? s->min_ring : n;
    for (uint32_t r0 = 0; r0 < n; r0 += piece) {
        const uint32_t nr = n - r0 < piece ? n - r0 : piece;
        for (uint32_t l0 = 0; l0 < s->cfg.n_layer; l0 += 64) {
            const uint32_t nl = s->cfg.n_layer - l0 < 64 ? s->cfg.n_layer - l0 : 64;
            const float *kk[64], *vv[64];
            for (uint32_t j = 0; j < nl; j++) {
                kk[j] = k[l0 + j] + (size_t)r0 * kv_stride;
                vv[j] = v[l0 + j] + (size_t)r0 * kv_stride;
            }
            int rc = s->layers8
                         ? tl_kv_append_layers_q8(&s->layers8[l0], nl, kk, vv, kv_stride, sl,
                                                  pos + r0, nr, s->cfg.stream)
                         : tl_kv_append_layers(&s->layers[l0], nl, kk, vv, kv_stride, sl,
                                               pos + r0, nr, s->cfg.stream);
            if (rc) return rc;
        }
    }
    return TL_OK;
}

/* K/V write-through only (no attention): the prefix cache takes every
 * n_ubatch chunk of the batch first -- the same kv_cache_append calls, in the
 * same order, as the chunk loop below makes -- then one slot-table upload and
 * the write-through of the whole batch (write_rows).  No chunk's rows can be
 * evicted by a later chunk: the request pins its slots.  If a chunk's slot
 * allocation fails, the rows of the chunks before it are still written (as
 * the reference's chunk loop would have written them) and the session
 * position ends after them. */
static int append_only(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                       const float *const *k, const float *const *v, uint32_t kv_stride) {
    const uint32_t pos = s->n_tokens;
    if ((uint64_t)pos + n_tokens > s->cfg.ctx_size)
        return fail(TL_ERANGE, "append: batch exceeds ctx_size");
    memcpy(s->tokens + pos, tokens, (size_t)n_tokens * sizeof(uint32_t));
    uint32_t done = n_tokens;
    int err = TL_OK;
    if (s->radix) {
        for (done = 0; done < n_tokens;) {
            uint32_t chunk = n_tokens - done;
            if (chunk > s->cfg.n_ubatch) chunk = s->cfg.n_ubatch;
            if (!kv_cache_append(s->radix, s->tokens, pos + done, chunk)) {
                err = TL_ERANGE;
                break;
            }
            done += chunk;
        }
        const KvRequestState *req = tl_kv_cache_req(s->radix);
        if (req->len < pos + done) return fail(TL_ERANGE, "append: request map too short");
        /* everything mapped so far, also positions a failed chunk mapped
         * before failing: the change mark is consumed here */
        uint32_t lo = tl_kv_cache_take_dirty(s->radix);
        if (lo != KV_SLOT_NONE && lo < req->len) {
            int rc = upload_slots(s, lo, req->len);
            if (rc) return rc;
        }
    }
    if (done) {
        int rc = write_rows(s, k, v, kv_stride, pos, done);
        if (rc) return rc;
    }
    s->n_tokens = pos + done;
    return err ? fail(err, "KV slot allocation failed") : TL_OK;
}

/* The chunk loop of graph_execute (src/graph.c:1395-1413). */
static int run_chunks(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                      const float *const *q, const float *const *k,
                      const float *const *v, float *const *out,
                      uint32_t q_stride, uint32_t kv_stride) {
    const uint32_t pos = s->n_tokens;
    if ((uint64_t)pos + n_tokens > s->cfg.ctx_size)
        return fail(TL_ERANGE, "execute: batch exceeds ctx_size");
    uint32_t done = 0;
    while (done < n_tokens) {
        uint32_t chunk = n_tokens - done;
        if (chunk > s->cfg.n_ubatch) chunk = s->cfg.n_ubatch;
        const uint32_t p0 = pos + done;
        memcpy(s->tokens + p0, tokens + done, (size_t)chunk * sizeof(uint32_t));
        if (s->radix) {
            if (!kv_cache_append(s->radix, s->tokens, p0, chunk))
                return fail(TL_ERANGE, "KV slot allocation failed");
            const KvRequestState *req = tl_kv_cache_req(s->radix);
            if (req->len < p0 + chunk) return fail(TL_ERANGE, "execute: request map too short");
            uint32_t lo = tl_kv_cache_take_dirty(s->radix);
            if (lo != KV_SLOT_NONE && lo < req->len) {
                int rc = upload_slots(s, lo, req->len);
                if (rc) return rc;
            }
        }
        for (uint32_t l = 0; l < s->cfg.n_layer; l++) {
            tl_attn_args a;
            memset(&a, 0, sizeof(a));
            a.q = q[l] + (size_t)done * q_stride;
            a.k = k[l] + (size_t)done * kv_stride;
            a.v = v[l] + (size_t)done * kv_stride;
            a.dst = out[l] + (size_t)done * q_stride;
            a.slots = s->radix ? s->d_slots : NULL;
            a.pos = p0;
            a.n = chunk;
            a.n_head = s->cfg.n_head;
            a.q_stride = q_stride;
            a.kv_stride = kv_stride;
            a.window = s->window[l];
            a.scale = s->scale;
            int rc = s->layers8 ? tl_attn_q8(&s->layers8[l], &a, s->cfg.stream)
                                : tl_attn(&s->layers[l], &a, s->cfg.stream);
            if (rc) return rc;
        }
        done += chunk;
    }
    s->n_tokens = pos + n_tokens;
    return TL_OK;
}

int tl_session_execute(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                       const float *const *q, const float *const *k,
                       const float *const *v, float *const *out,
                       uint32_t q_stride, uint32_t kv_stride) {
    if (!s || !tokens || n_tokens == 0) return fail(TL_EINVAL, "execute: missing tokens");
    if (!q || !k || !v || !out) return fail(TL_EINVAL, "execute: missing activations");
    return run_chunks(s, tokens, n_tokens, q, k, v, out, q_stride, kv_stride);
}

int tl_session_append(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                      const float *const *k, const float *const *v, uint32_t kv_stride) {
    if (!s || !tokens || n_tokens == 0) return fail(TL_EINVAL, "append: missing tokens");
    if (!k || !v) return fail(TL_EINVAL, "append: missing activations");
    return append_only(s, tokens, n_tokens, k, v, kv_stride);
}

/* Compaction: optional LRU trim, then renumber the pool so live rows occupy
 * [0, n_live), moving the rows on the device in one copy launch. */
int tl_session_compact(tl_session *s, uint32_t keep, uint32_t *evicted, uint32_t *moved) {
    if (moved) *moved = 0;
    if (evicted) *evicted = 0;
    if (!s) return fail(TL_EINVAL, "compact: no session");
    if (!s->radix) return TL_OK;
    uint32_t ev = tl_kv_cache_trim(s->radix, keep);
    if (evicted) *evicted = ev;
    const uint32_t ctx = s->cfg.ctx_size;
    uint32_t *src = s->h_moves, *dst = s->h_moves + ctx;
    uint32_t n = tl_kv_cache_compact(s->radix, src, dst, ctx);
    if (n == UINT32_MAX) return fail(TL_ERANGE, "compact: move list overflow");
    if (n) {
        /* sources then destinations, packed: one upload */
        memmove(src + n, dst, (size_t)n * sizeof(uint32_t));
        int rc = upload_words(s, s->d_moves, src, 2 * n);
        if (!rc)
            rc = s->layers8 ? tl_kv_copy_q8(s->layers8, s->cfg.n_layer, s->d_moves,
                                            s->d_moves + n, n, s->cfg.stream)
                            : tl_kv_copy(s->layers, s->cfg.n_layer, s->d_moves, s->d_moves + n,
                                         n, s->cfg.stream);
        if (!rc) rc = sync_slots(s);
        if (rc) return rc;
    }
    if (moved) *moved = n;
    return TL_OK;
}

/* Prefix fork: like tl_session_kv_prepare, but a longer prefix cached in
 * `donor` is first copied into this session's pool (rows allocated through
 * kv_cache_append, copied on the device), so it need not be recomputed. */
int tl_session_kv_prepare_from(tl_session *s, tl_session *donor, const uint32_t *tokens,
                               uint32_t n, uint32_t *matched, uint32_t *resume,
                               uint32_t *forked) {
    if (forked) *forked = 0;
    /* no fork without two prefix caches, or for a stateful session (forked
     * K/V rows come without the recurrent state at their end) */
    if (!donor || donor == s || !s || !s->radix || !donor->radix || s->state_bytes)
        return tl_session_kv_prepare(s, tokens, n, matched, resume);
    if (matched) *matched = 0;
    if (resume) *resume = 0;
    if (!tokens || n == 0) return TL_OK;
    if (s->has_ring || donor->has_ring) return fail(TL_EINVAL, "fork: ring layers hold no slot rows");
    if (donor->cfg.n_layer != s->cfg.n_layer || donor->cfg.n_kv_head != s->cfg.n_kv_head ||
        donor->cfg.head_dim != s->cfg.head_dim || !donor->layers8 != !s->layers8)
        return fail(TL_EINVAL, "fork: sessions differ in shape or cache type");
    const uint32_t ctx = s->cfg.ctx_size;
    uint32_t m = kv_cache_match(s->radix, tokens, n);
    uint32_t *src = s->h_moves;
    uint32_t lim = n < ctx ? n : ctx;
    uint32_t md = tl_kv_cache_lookup(donor->radix, tokens, lim, src);
    if (md > m) {
        const uint32_t nc = md - m;
        if (!kv_cache_append(s->radix, tokens, m, nc)) return fail(TL_ERANGE, "fork: KV slot allocation failed");
        const KvRequestState *req = tl_kv_cache_req(s->radix);
        if (req->len < md) return fail(TL_ERANGE, "fork: request map too short");
        /* sources (donor rows) then destinations, packed at the front of
         * h_moves ([0, 2 nc), nc <= ctx): one upload */
        memmove(src, src + m, (size_t)nc * sizeof(uint32_t));
        memcpy(src + nc, req->slots + m, (size_t)nc * sizeof(uint32_t));
        int rc = upload_words(s, s->d_moves, src, 2 * nc);
        if (!rc)
            rc = s->layers8 ? tl_kv_copy_between_q8(s->layers8, donor->layers8, s->cfg.n_layer,
                                                    s->d_moves, s->d_moves + nc, nc, s->cfg.stream)
                            : tl_kv_copy_between(s->layers, donor->layers, s->cfg.n_layer,
                                                 s->d_moves, s->d_moves + nc, nc, s->cfg.stream);
        if (!rc) rc = sync_slots(s);
        if (rc) return rc;
        if (forked) *forked = nc;
        m = md;
    }
    uint32_t r = m == 0 ? 0 : (m < n ? m : m - 1);
    s->n_tokens = r;
    if (r) memcpy(s->tokens, tokens, (size_t)r * sizeof(uint32_t));
    if (matched) *matched = m;
    if (resume) *resume = r;
    return TL_OK;
}

/* ---- recurrent state (device snapshots) ---------------------------------- */

static size_t state_bytes_cb(Session *ss) { return ((tl_session *)ss)->state_bytes; }

static bool state_save_cb(Session *ss, void *dst, size_t cap) {
    tl_session *s = (tl_session *)ss;
    if (cap < s->state_bytes) return false;
    return tl_state_copy(s->state, s->n_state, dst, TL_STATE_SAVE, s->cfg.stream) == TL_OK;
}

static bool state_load_cb(Session *ss, const void *src, size_t len) {
    tl_session *s = (tl_session *)ss;
    if (len < s->state_bytes) return false;
    return tl_state_copy(s->state, s->n_state, (void *)src, TL_STATE_LOAD, s->cfg.stream) == TL_OK;
}

static void *state_alloc_cb(Session *ss, size_t bytes) {
    (void)ss;
    void *p = NULL;
    return hipMalloc(&p, bytes) == hipSuccess ? p : NULL;
}

static void state_release_cb(Session *ss, void *p) {
    tl_session *s = (tl_session *)ss;
    /* a save or load in flight on the session's stream may still use it */
    (void)hipStreamSynchronize((hipStream_t)s->cfg.stream);
    (void)hipFree(p);
}

int tl_session_set_state(tl_session *s, const tl_state_seg *segs, uint32_t n_seg) {
    if (!s || (n_seg && !segs)) return fail(TL_EINVAL, "set_state: bad arguments");
    tl_state_seg *copy = NULL;
    size_t total = 0;
    if (n_seg) {
        copy = (tl_state_seg *)malloc((size_t)n_seg * sizeof(*copy));
        if (!copy) return fail(TL_ENOMEM, "set_state: host allocation");
        for (uint32_t i = 0; i < n_seg; i++) {
            if (segs[i].bytes && !segs[i].ptr) {
                free(copy);
                return fail(TL_EINVAL, "set_state: null buffer");
            }
            copy[i] = segs[i];
            total += segs[i].bytes;
        }
    }
    /* drop the old snapshots (with the old buffers' callbacks) first */
    if (s->radix) tl_kv_cache_set_state_ops(s->radix, NULL);
    free(s->state);
    s->state = copy;
    s->n_state = n_seg;
    s->state_bytes = total;
    if (s->radix && total) {
        TlKvStateOps ops = {state_bytes_cb, state_save_cb, state_load_cb, state_alloc_cb,
                            state_release_cb};
        tl_kv_cache_set_state_ops(s->radix, &ops);
    }
    return TL_OK;
}

int tl_session_checkpoint(tl_session *s) {
    if (!s) return fail(TL_EINVAL, "checkpoint: null session");
    if (!s->radix || !s->state_bytes) return TL_OK;
    if (!kv_cache_checkpoint(s->radix, s->n_tokens))
        return fail(TL_ENOMEM, "checkpoint: snapshot allocation or copy failed");
    return TL_OK;
}

uint32_t tl_session_pos(const tl_session *s) { return s ? s->n_tokens : 0; }
void tl_session_set_pos(tl_session *s, uint32_t pos) {
    if (s && pos <= s->cfg.ctx_size) s->n_tokens = pos;
}
KvRadixCache *tl_session_radix(tl_session *s) { return s ? s->radix : NULL; }
const tl_kv_layer_q8 *tl_session_layer_q8(const tl_session *s, uint32_t layer) {
    return (s && s->layers8 && layer < s->cfg.n_layer) ? &s->layers8[layer] : NULL;
}
const tl_kv_layer *tl_session_layer(const tl_session *s, uint32_t layer) {
    return (s && s->layers && layer < s->cfg.n_layer) ? &s->layers[layer] : NULL;
}
const uint32_t *tl_session_device_slots(const tl_session *s) { return s ? s->d_slots : NULL; }

/* ---- slot mirror ---------------------------------------------------------- */

struct tl_slot_mirror {
    uint32_t      ctx_size;
    uint32_t     *d_slots;     /* device [ctx_size] */
    uint32_t     *stage;       /* pinned [STAGE_WORDS] */
    uint32_t      stage_pos;
    KvRadixCache *seen;        /* the cache whose change marks the mirror follows */
    void         *last;        /* stream of the last sync that queued work */
    int           queued;      /* some sync has queued work on `last` */
};

int tl_slot_mirror_create(uint32_t ctx_size, tl_slot_mirror **out) {
    if (!out || ctx_size == 0) return fail(TL_EINVAL, "slot mirror: bad arguments");
    *out = NULL;
    tl_slot_mirror *m = (tl_slot_mirror *)calloc(1, sizeof(*m));
    if (!m) return fail(TL_ENOMEM, "slot mirror: host allocation");
    m->ctx_size = ctx_size;
    if (hipMalloc((void **)&m->d_slots, (size_t)ctx_size * sizeof(uint32_t)) != hipSuccess ||
        hipHostMalloc((void **)&m->stage, STAGE_WORDS * sizeof(uint32_t), 0) != hipSuccess) {
        m->stage = NULL;
        tl_slot_mirror_destroy(m);
        return fail(TL_ENOMEM, "slot mirror: allocation");
    }
    *out = m;
    return TL_OK;
}

void tl_slot_mirror_destroy(tl_slot_mirror *m) {
    if (!m) return;
    if (m->d_slots) (void)hipFree(m->d_slots);
    if (m->stage) (void)hipHostFree(m->stage);
    free(m);
}

int tl_slot_mirror_sync(tl_slot_mirror *m, KvRadixCache *radix, void *stream,
                        const uint32_t **d_slots) {
    if (d_slots) *d_slots = NULL;
    if (!m || !radix) return fail(TL_EINVAL, "slot mirror: missing mirror or cache");
    const KvRequestState *req = tl_kv_cache_req(radix);
    uint32_t lo = tl_kv_cache_take_dirty(radix);
    if (m->seen != radix) {
        lo = 0;   /* a cache this mirror has not followed: upload the whole map */
        m->seen = radix;
    }
    const uint32_t len = req->len;
    if (len > m->ctx_size) {
        m->seen = NULL;
        return fail(TL_ERANGE, "slot mirror: request longer than the mirror");
    }
    if (lo != KV_SLOT_NONE && lo < len) {
        for (uint32_t i = lo; i < len; i++)
            if (req->slots[i] >= m->ctx_size) {
                m->seen = NULL;   /* re-upload everything next time */
                return fail(TL_ERANGE, "slot mirror: slot outside the cache");
            }
        /* A sync on another stream than the last one: the copies (and the
         * kernels reading the mirror) queued there may still read the staged
         * words and the device map this upload overwrites, so let them
         * finish first; uploads on one stream are ordered by the stream. */
        if (m->queued && m->last != stream) {
            if (hipStreamSynchronize((hipStream_t)m->last) != hipSuccess) {
                m->seen = NULL;
                return fail(TL_EHIP, "slot mirror: sync of the previous stream");
            }
            m->queued = 0;
        }
        m->last = stream;
        m->queued = 1;
        int rc = stage_upload(m->stage, &m->stage_pos, (hipStream_t)stream, m->d_slots + lo,
                              req->slots + lo, len - lo);
        if (rc) {
            m->seen = NULL;
            return rc;
        }
    }
    if (d_slots) *d_slots = m->d_slots;
    return TL_OK;
}
