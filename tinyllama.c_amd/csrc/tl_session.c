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
    tl_kv_layer   *layers;      /* [n_layer] */
    KvRadixCache  *radix;
    uint32_t      *tokens;      /* [ctx_size] host token history (Session.tokens) */
    uint32_t       n_tokens;    /* Session.n_tokens */
    uint32_t      *d_slots;     /* device mirror of req.slots */
    uint32_t      *stage;       /* pinned */
    uint32_t       stage_pos;
    float          scale;
    int            has_ring;    /* some layer keeps only a window of rows */
};

static int fail(int code, const char *msg) { return tl_set_error(code, msg); }

void tl_session_destroy(tl_session *s) {
    if (!s) return;
    if (s->layers)
        for (uint32_t l = 0; l < s->cfg.n_layer; l++) tl_kv_layer_free(&s->layers[l]);
    free(s->layers);
    free(s->window);
    kv_cache_destroy(s->radix);
    free(s->tokens);
    if (s->d_slots) (void)hipFree(s->d_slots);
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
    s->layers = (tl_kv_layer *)calloc(cfg->n_layer, sizeof(tl_kv_layer));
    s->tokens = (uint32_t *)calloc(cfg->ctx_size, sizeof(uint32_t));
    if (!s->window || !s->layers || !s->tokens) {
        tl_session_destroy(s);
        return fail(TL_ENOMEM, "session: host allocation");
    }
    for (uint32_t l = 0; l < cfg->n_layer; l++) {
        s->window[l] = cfg->window ? cfg->window[l] : 0;
        uint32_t ring = cfg->ring ? cfg->ring[l] : 0;
        if (ring) s->has_ring = 1;
        if (ring && (!s->window[l] || ring < s->window[l] + cfg->n_ubatch - 1)) {
            tl_session_destroy(s);
            return fail(TL_EINVAL, "session: a ring needs window + n_ubatch - 1 rows");
        }
        int rc = tl_kv_layer_alloc(&s->layers[l], ring ? ring : cfg->ctx_size,
                                   cfg->n_kv_head, cfg->head_dim, ring);
        if (rc) {
            tl_session_destroy(s);
            return rc;
        }
    }
    if (cfg->use_radix) {
        /* the prefix cache only stores the KvCache pointer */
        s->radix = kv_cache_create(NULL, (KvCache *)s->layers, cfg->ctx_size);
        if (!s->radix) {
            tl_session_destroy(s);
            return fail(TL_ENOMEM, "session: kv_cache_create failed");
        }
        if (hipMalloc((void **)&s->d_slots, (size_t)cfg->ctx_size * sizeof(uint32_t)) != hipSuccess ||
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

/* upload req.slots[lo..hi) to the device mirror, in stream order */
static int upload_slots(tl_session *s, uint32_t lo, uint32_t hi) {
    hipStream_t st = (hipStream_t)s->cfg.stream;
    const KvRequestState *req = tl_kv_cache_req(s->radix);
    while (lo < hi) {
        uint32_t n = hi - lo;
        if (n > STAGE_WORDS) n = STAGE_WORDS;
        if (s->stage_pos + n > STAGE_WORDS) {
            /* staged words may still be read by queued copies */
            if (hipStreamSynchronize(st) != hipSuccess) return fail(TL_EHIP, "session: sync");
            s->stage_pos = 0;
        }
        uint32_t *dst = s->stage + s->stage_pos;
        memcpy(dst, req->slots + lo, (size_t)n * sizeof(uint32_t));
        if (hipMemcpyAsync(s->d_slots + lo, dst, (size_t)n * sizeof(uint32_t),
                           hipMemcpyHostToDevice, st) != hipSuccess)
            return fail(TL_EHIP, "session: slot upload");
        s->stage_pos += n;
        lo += n;
    }
    return TL_OK;
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
    uint32_t r = m == 0 ? 0 : (m < n ? m : m - 1);
    /* ring layers hold only the last window + n_ubatch - 1 rows of the
     * previous request: a prefix hit cannot be resumed on them */
    if (s->has_ring) r = 0;
    s->n_tokens = r;   /* reset, then resume (src/graph.c:1443-1452, server.c:837) */
    if (r) memcpy(s->tokens, tokens, (size_t)r * sizeof(uint32_t));
    if (matched) *matched = m;
    if (resume) *resume = r;
    return TL_OK;
}

int tl_session_execute(tl_session *s, const uint32_t *tokens, uint32_t n_tokens,
                       const float *const *q, const float *const *k,
                       const float *const *v, float *const *out,
                       uint32_t q_stride, uint32_t kv_stride) {
    if (!s || !tokens || n_tokens == 0) return fail(TL_EINVAL, "execute: missing tokens");
    if (!q || !k || !v || !out) return fail(TL_EINVAL, "execute: missing activations");
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
            if (lo != KV_SLOT_NONE && lo < p0 + chunk) {
                for (uint32_t i = lo; i < p0 + chunk; i++)
                    if (req->slots[i] >= s->cfg.ctx_size)
                        return fail(TL_ERANGE, "execute: slot outside the cache");
                int rc = upload_slots(s, lo, p0 + chunk);
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
            int rc = tl_attn(&s->layers[l], &a, s->cfg.stream);
            if (rc) return rc;
        }
        done += chunk;
    }
    s->n_tokens = pos + n_tokens;
    return TL_OK;
}

uint32_t tl_session_pos(const tl_session *s) { return s ? s->n_tokens : 0; }
void tl_session_set_pos(tl_session *s, uint32_t pos) {
    if (s && pos <= s->cfg.ctx_size) s->n_tokens = pos;
}
KvRadixCache *tl_session_radix(tl_session *s) { return s ? s->radix : NULL; }
const tl_kv_layer *tl_session_layer(const tl_session *s, uint32_t layer) {
    return (s && layer < s->cfg.n_layer) ? &s->layers[layer] : NULL;
}
const uint32_t *tl_session_device_slots(const tl_session *s) { return s ? s->d_slots : NULL; }
