/*
 * tl_kv.hip — gfx950 kernels and C ABI for the KV-cache hot path.
 *
 *   kv_append_kernel    OP_ATTN's K/V write-through (reference:
 *                       src/backend/cpu/cpu_op.c:995-1008), f32 -> f16 RNE,
 *                       one 16-byte store per 8 elements.
 *   kv_gather_kernel    read rows by slot.
 *   kv_copy_kernel      row copies across all layers (fork / compaction).
 *   rope_kernel         OP_ROPE_NORM / OP_ROPE_NEOX (cpu_op.c:632-700).
 *   The decode attention (tl_decode.hip, attn_decode_ring_kernel) is
 *   split-K ("flash-decoding") attention over the slot table, one workgroup
 *   per (split, kv-head, row) serving all q-heads of the GQA group; math of
 *   cpu_op.c:1011-1062.
 * The MFMA chunked-prefill kernel lives in tl_prefill.hip, the Q8_0 cache's
 * storage / append / gather / copies in tl_q8.hip, the recurrent-state
 * snapshot copies in tl_state.hip.
 */
#include "tl_common.h"
#include "tl_internal.h"
#include "../../include/tlkv.h"

#include <atomic>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* errors                                                                    */
/* ------------------------------------------------------------------------ */

static thread_local char g_err[512] = "";

int tl_fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

extern "C" const char *tl_last_error(void) { return g_err; }


/* ------------------------------------------------------------------------ */
/* split-K workspace, one per (device, stream)                               */
/* ------------------------------------------------------------------------ */

/* Each stream that launches split attention gets its own partials and merge
 * counters, so launches queued on different streams (two sessions, each on
 * its own stream) never share them; launches on one stream run in order.
 * The table holds TL_WS_STREAMS streams per device; a further stream takes
 * the least recently used entry (its buffers are freed, which waits for the
 * device). */
#define TL_MAX_DEV 16
#define TL_WS_STREAMS 16
struct WsSlot {
    hipStream_t st;
    bool live;
    u64 used;
    TlWorkspace w;
};
static WsSlot g_ws[TL_MAX_DEV][TL_WS_STREAMS];
static u64 g_ws_clock;
static std::mutex g_ws_mu;
static thread_local TlWorkspace *g_ws_fixed;   /* set by TlWsFixed */

TlWsFixed::TlWsFixed(TlWorkspace *w) : prev(g_ws_fixed) { g_ws_fixed = w; }
TlWsFixed::~TlWsFixed() { g_ws_fixed = prev; }
size_t tl_workspace_fixed_acc(void) { return g_ws_fixed ? g_ws_fixed->acc_cap : 0; }

static void ws_release(TlWorkspace *w) {
    if (w->acc) (void)hipFree(w->acc);
    if (w->ml) (void)hipFree(w->ml);
    if (w->cnt) (void)hipFree(w->cnt);
    memset(w, 0, sizeof(*w));
}

static int ws_grow(TlWorkspace *w, size_t acc_floats, size_t ml_pairs, size_t counters) {
    if (acc_floats > w->acc_cap) {
        if (w->acc) HIP_TRY(hipFree(w->acc));
        w->acc = NULL;
        w->acc_cap = 0;
        size_t cap = acc_floats + acc_floats / 4 + 1024;
        if (hipMalloc((void **)&w->acc, cap * sizeof(float)) != hipSuccess)
            return tl_fail(TL_ENOMEM, "workspace: %zu floats", cap);
        HIP_TRY(hipMemset(w->acc, 0, cap * sizeof(float)));
        w->acc_cap = cap;
    }
    if (ml_pairs > w->ml_cap) {
        if (w->ml) HIP_TRY(hipFree(w->ml));
        w->ml = NULL;
        w->ml_cap = 0;
        size_t cap = ml_pairs + ml_pairs / 4 + 256;
        if (hipMalloc((void **)&w->ml, cap * sizeof(float2)) != hipSuccess)
            return tl_fail(TL_ENOMEM, "workspace: %zu pairs", cap);
        /* zero: the in-launch merge reads epoch-tagged records here, which
         * must not match by chance what an earlier owner of the memory (a
         * workspace of another stream, with its own launch counter) left */
        HIP_TRY(hipMemset(w->ml, 0, cap * sizeof(float2)));
        HIP_TRY(hipDeviceSynchronize());
        w->ml_cap = cap;
    }
    if (counters > w->cnt_cap) {
        if (w->cnt) HIP_TRY(hipFree(w->cnt));
        w->cnt = NULL;
        w->cnt_cap = 0;
        size_t cap = counters + 256;
        if (hipMalloc((void **)&w->cnt, cap * sizeof(u32)) != hipSuccess)
            return tl_fail(TL_ENOMEM, "workspace: %zu counters", cap);
        /* The merge state starts at zero; launches keep it consistent
         * from then on (tl_internal.h). */
        HIP_TRY(hipMemset(w->cnt, 0, cap * sizeof(u32)));
        HIP_TRY(hipDeviceSynchronize());
        w->cnt_cap = cap;
    }
    return TL_OK;
}

int tl_workspace_get(hipStream_t st, size_t acc_floats, size_t ml_pairs, size_t counters,
                     TlWorkspace **out) {
    if (g_ws_fixed) {
        /* a no-allocation call: the caller's fixed region or nothing */
        TlWorkspace *w = g_ws_fixed;
        if (acc_floats > w->acc_cap || ml_pairs > w->ml_cap || counters > w->cnt_cap)
            return tl_fail(TL_ERANGE,
                           "scratch: %zu partial floats, %zu pairs, %zu counters exceed "
                           "%zu / %zu / %zu",
                           acc_floats, ml_pairs, counters, w->acc_cap, w->ml_cap, w->cnt_cap);
        *out = w;
        return TL_OK;
    }
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= TL_MAX_DEV) return tl_fail(TL_EINVAL, "device %d", dev);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    WsSlot *tab = g_ws[dev], *hit = nullptr;
    for (int i = 0; i < TL_WS_STREAMS && !hit; i++)
        if (tab[i].live && tab[i].st == st) hit = &tab[i];
    if (!hit) {
        /* a free entry, else the least recently used one */
        for (int i = 0; i < TL_WS_STREAMS; i++)
            if (!hit || (hit->live && (!tab[i].live || tab[i].used < hit->used))) hit = &tab[i];
        if (hit->live) ws_release(&hit->w);
        hit->live = true;
        hit->st = st;
    }
    hit->used = ++g_ws_clock;
    int rc = ws_grow(&hit->w, acc_floats, ml_pairs, counters);
    if (rc) return rc;
    *out = &hit->w;
    return TL_OK;
}

/* ------------------------------------------------------------------------ */
/* fixed scratch for the no-allocation entry point (tl_attn_noalloc)         */
/* ------------------------------------------------------------------------ */

/* One region per GPU for the whole process: split partials, (max, sum)
 * pairs and merge counters of tl_attn_noalloc.  Host code never uses the
 * symbol's name as an address: each device's copy sits at the address
 * hipGetSymbolAddress returns with that device current (g_scratch_ws). */
#define TL_SCRATCH_ACC_FLOATS (28u << 18)   /* 28 MiB of partials */
#define TL_SCRATCH_ML_PAIRS (1u << 17)      /* 1 MiB of (max, sum) pairs */
#define TL_SCRATCH_COUNTERS (3u << 18)      /* 3 MiB of merge counters */
static_assert(TL_SCRATCH_COUNTERS >= TL_MERGE_CNT_WORDS, "scratch counters");
#define TL_SCRATCH_BYTES                                                      \
    ((size_t)TL_SCRATCH_ACC_FLOATS * 4 + (size_t)TL_SCRATCH_ML_PAIRS * 8 +   \
     (size_t)TL_SCRATCH_COUNTERS * 4)
static __device__ __align__(256) unsigned char scratch[TL_SCRATCH_BYTES];
static TlWorkspace g_scratch_ws[TL_MAX_DEV];   /* views of each device's region */
static std::mutex g_scratch_mu;

/* the calling thread's device's scratch region, set up on first use: its
 * address (hipGetSymbolAddress with the device current) and zeroed merge
 * counters (launches keep them consistent from then on) */
static int scratch_setup(int dev, TlWorkspace **out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    TlWorkspace *w = &g_scratch_ws[dev];
    if (!w->acc) {
        void *ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return tl_fail(TL_EHIP, "scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
        unsigned char *base = (unsigned char *)ptr;
        u32 *cnt = (u32 *)(base + (size_t)TL_SCRATCH_ACC_FLOATS * 4 +
                           (size_t)TL_SCRATCH_ML_PAIRS * 8);
        HIP_TRY(hipMemset(base, 0, TL_SCRATCH_BYTES));
        HIP_TRY(hipDeviceSynchronize());
        w->acc = (float *)base;
        w->ml = (float *)(base + (size_t)TL_SCRATCH_ACC_FLOATS * 4);
        w->cnt = cnt;
        w->acc_cap = TL_SCRATCH_ACC_FLOATS;
        w->ml_cap = TL_SCRATCH_ML_PAIRS;
        w->cnt_cap = TL_SCRATCH_COUNTERS;
    }
    *out = w;
    return TL_OK;
}

extern "C" int tl_init(int device) {
    HIP_TRY(hipSetDevice(device));
    if (device < 0 || device >= TL_MAX_DEV) return tl_fail(TL_EINVAL, "device %d", device);
    TlWorkspace *sc;
    int rc = scratch_setup(device, &sc);
    if (rc) return rc;
    TlWorkspace *w;
    return tl_workspace_get(nullptr, 1 << 20, 1 << 14, 4096, &w);
}

/* launch-shape overrides: seeded once from the environment, then only
 * tl_set_tuning writes them (relaxed atomics: a launch reads a consistent
 * word, and callers that change them between launches order the change
 * themselves) */
static std::atomic<u32> g_tune[TL_TUNE_COUNT];
static std::once_flag g_tune_once;

static void tune_seed() {
    static const char *const names[TL_TUNE_COUNT] = {
        "TL_DECODE_WGS", "TL_DECODE_MIN_KEYS", "TL_DECODE_MERGE_KERNEL", "TL_PREFILL_SPLITS",
        "TL_NO_PREFILL", "TL_DECODE_SINGLE_MERGE", "TL_DECODE_MERGE_POLLS",
        "TL_PREFILL_APPEND_POLLS", "TL_PREFILL_SEPARATE_APPEND", "TL_DECODE_MFMA", "TL_DECODE_ROWS"};
    for (int i = 0; i < TL_TUNE_COUNT; i++) {
        const char *e = getenv(names[i]);
        g_tune[i].store(e && *e ? (u32)strtoul(e, NULL, 10) : 0u, std::memory_order_relaxed);
    }
}

uint32_t tl_tune(int key) {
    std::call_once(g_tune_once, tune_seed);
    return (key >= 0 && key < TL_TUNE_COUNT) ? g_tune[key].load(std::memory_order_relaxed) : 0u;
}

extern "C" int tl_set_tuning(int key, uint32_t value) {
    if (key < 0 || key >= TL_TUNE_COUNT) return tl_fail(TL_EINVAL, "tuning key %d", key);
    std::call_once(g_tune_once, tune_seed);
    g_tune[key].store(value, std::memory_order_relaxed);
    return TL_OK;
}

extern "C" uint32_t tl_get_tuning(int key) { return tl_tune(key); }

/* ------------------------------------------------------------------------ */
/* layer storage                                                             */
/* ------------------------------------------------------------------------ */

static int check_layer(const tl_kv_layer *L) {
    if (!L || !L->k || !L->v) return tl_fail(TL_EINVAL, "layer: null storage");
    if (L->head_dim != 64 && L->head_dim != 128 && L->head_dim != 256)
        return tl_fail(TL_EINVAL, "head_dim %u unsupported (64/128/256)", L->head_dim);
    if (L->n_kv_head == 0 || L->cap == 0)
        return tl_fail(TL_EINVAL, "layer: empty shape");
    if (L->ring > L->cap) return tl_fail(TL_EINVAL, "ring %u > cap %u", L->ring, L->cap);
    /* kernels address one kv-head's rows with 32-bit byte offsets */
    if ((u64)L->cap * L->head_dim * sizeof(u16) > 0xFFFFFFFFull)
        return tl_fail(TL_ERANGE, "layer: %u rows of head_dim %u exceed 4 GiB per kv-head",
                       L->cap, L->head_dim);
    if (((uintptr_t)L->k | (uintptr_t)L->v) & 15)
        return tl_fail(TL_EINVAL, "cache storage not 16-byte aligned");
    return TL_OK;
}

extern "C" int tl_kv_layer_alloc(tl_kv_layer *L, uint32_t cap, uint32_t n_kv_head,
                                 uint32_t head_dim, uint32_t ring) {
    if (!L) return tl_fail(TL_EINVAL, "null layer");
    memset(L, 0, sizeof(*L));
    size_t bytes = (size_t)cap * n_kv_head * head_dim * sizeof(u16);
    if (bytes == 0) return tl_fail(TL_EINVAL, "empty layer");
    /* shape rules first, so a rejected layer holds no memory */
    {
        tl_kv_layer probe = {(void *)16, (void *)16, cap, n_kv_head, head_dim, ring};
        int rc = check_layer(&probe);
        if (rc) return rc;
    }
    if (hipMalloc(&L->k, bytes) != hipSuccess) {
        L->k = NULL;
        return tl_fail(TL_ENOMEM, "layer K: %zu bytes", bytes);
    }
    if (hipMalloc(&L->v, bytes) != hipSuccess) {
        (void)hipFree(L->k);
        L->k = NULL;
        L->v = NULL;
        return tl_fail(TL_ENOMEM, "layer V: %zu bytes", bytes);
    }
    L->cap = cap;
    L->n_kv_head = n_kv_head;
    L->head_dim = head_dim;
    L->ring = ring;
    if (hipMemset(L->k, 0, bytes) != hipSuccess || hipMemset(L->v, 0, bytes) != hipSuccess) {
        tl_kv_layer_free(L);
        return tl_fail(TL_EHIP, "layer: clearing %zu bytes failed", bytes);
    }
    return TL_OK;
}

extern "C" int tl_kv_layer_free(tl_kv_layer *L) {
    if (!L) return TL_OK;
    if (L->k) HIP_TRY(hipFree(L->k));
    if (L->v) HIP_TRY(hipFree(L->v));
    L->k = L->v = NULL;
    return TL_OK;
}

/* ------------------------------------------------------------------------ */
/* append / gather / copy                                                    */
/* ------------------------------------------------------------------------ */

TL_DEV u32 phys_row(u32 p, u32 ring, const u32 *slots) {
    return ring ? p % ring : (slots ? slots[p] : p);
}

TL_DEV uint4 cvt8(const float *src) {
    float4 a = *(const float4 *)src;
    float4 b = *(const float4 *)(src + 4);
    uint4 o;
    o.x = pack_f16x2(a.x, a.y);
    o.y = pack_f16x2(a.z, a.w);
    o.z = pack_f16x2(b.x, b.y);
    o.w = pack_f16x2(b.z, b.w);
    return o;
}


/* grid: (blocks, n_seg).  One thread per 8-element vector of one row of one
 * head; consecutive threads cover consecutive 16-byte pieces of a row. */
template <bool ROPE, int NS>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendParamsN<NS> p) {
    const AppendSeg &sg = p.seg[blockIdx.y];
    const u32 vpr = sg.head_dim >> 3;
    const u64 total = (u64)sg.n * sg.n_kv * vpr;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        u32 c = (u32)(idx % vpr);
        u64 t = idx / vpr;
        u32 h = (u32)(t % sg.n_kv);
        u32 i = (u32)(t / sg.n_kv);
        u32 slot = phys_row(sg.pos + i, sg.ring, sg.slots);
        if (slot >= sg.cap) continue;
        u64 src = (u64)i * sg.kv_stride + (u64)h * sg.head_dim + c * 8;
        u64 dst = ((u64)h * sg.cap + slot) * sg.head_dim + c * 8;
        if constexpr (ROPE)
            *(uint4 *)(sg.kc + dst) = cvt8_rope(sg.k + (src - c * 8), c * 8, sg.pos + i,
                                                p.rope.rdim, p.rope.theta, p.rope.neox);
        else
            *(uint4 *)(sg.kc + dst) = cvt8(sg.k + src);
        *(uint4 *)(sg.vc + dst) = cvt8(sg.v + src);
    }
}

int tl_launch_append(const AppendParams &p, u32 n_seg, hipStream_t stream) {
    u64 most = 0;
    for (u32 s = 0; s < n_seg; s++) {
        u64 t = (u64)p.seg[s].n * p.seg[s].n_kv * (p.seg[s].head_dim >> 3);
        if (t > most) most = t;
    }
    if (most == 0) return TL_OK;
    u64 blocks = (most + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (n_seg == 1) {
        AppendParamsN<1> p1;
        p1.seg[0] = p.seg[0];
        p1.rope = p.rope;
        if (p.rope.rdim)
            hipLaunchKernelGGL((kv_append_kernel<true, 1>), dim3((u32)blocks, 1), dim3(256), 0,
                               stream, p1);
        else
            hipLaunchKernelGGL((kv_append_kernel<false, 1>), dim3((u32)blocks, 1), dim3(256), 0,
                               stream, p1);
    } else if (p.rope.rdim) {
        hipLaunchKernelGGL((kv_append_kernel<true, TL_MAX_BATCH_SEQ>), dim3((u32)blocks, n_seg),
                           dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL((kv_append_kernel<false, TL_MAX_BATCH_SEQ>), dim3((u32)blocks, n_seg),
                           dim3(256), 0, stream, p);
    }
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

static int fill_seg(AppendSeg &sg, const tl_kv_layer *L, const float *k,
                    const float *v, u32 kv_stride, const u32 *slots, u32 pos,
                    u32 n) {
    if (!k || !v) return tl_fail(TL_EINVAL, "append: null rows");
    if (kv_stride < L->n_kv_head * L->head_dim || (kv_stride & 3) ||
        (((uintptr_t)k | (uintptr_t)v) & 15))
        return tl_fail(TL_EINVAL, "append: rows must be 16-byte aligned, stride %u", kv_stride);
    sg.kc = (u16 *)L->k;
    sg.vc = (u16 *)L->v;
    sg.k = k;
    sg.v = v;
    sg.slots = slots;
    sg.cap = L->cap;
    sg.ring = L->ring;
    sg.n_kv = L->n_kv_head;
    sg.head_dim = L->head_dim;
    sg.kv_stride = kv_stride;
    sg.pos = pos;
    sg.n = n;
    return TL_OK;
}

extern "C" int tl_kv_append(const tl_kv_layer *L, const float *k, const float *v,
                            uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                            uint32_t n, void *stream) {
    int rc = check_layer(L);
    if (rc) return rc;
    if (n == 0) return TL_OK;
    AppendParams p;
    memset(&p, 0, sizeof(p));
    rc = fill_seg(p.seg[0], L, k, v, kv_stride, slots, pos, n);
    if (rc) return rc;
    return tl_launch_append(p, 1, (hipStream_t)stream);
}

int tl_rope_cfg(uint32_t head_dim, const tl_rope_params *r, RopeCfg &c) {
    c.rdim = 0;
    c.theta = 0.f;
    c.neox = 0;
    if (!r) return TL_OK;
    if (r->rope_dim > head_dim || (r->rope_dim & 1) || !(r->theta > 0.f))
        return tl_fail(TL_EINVAL, "rope: dim %u theta %g", r->rope_dim, (double)r->theta);
    c.rdim = r->rope_dim;
    c.theta = r->theta;
    c.neox = r->neox ? 1 : 0;
    return TL_OK;
}

extern "C" int tl_kv_append_layers(const tl_kv_layer *layers, uint32_t n_layer,
                                   const float *const *k, const float *const *v,
                                   uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                                   uint32_t n, void *stream) {
    if (n == 0 || n_layer == 0) return TL_OK;
    if (!layers || !k || !v) return tl_fail(TL_EINVAL, "append_layers: null pointer");
    for (u32 l0 = 0; l0 < n_layer; l0 += TL_MAX_BATCH_SEQ) {
        const u32 nl = n_layer - l0 < TL_MAX_BATCH_SEQ ? n_layer - l0 : TL_MAX_BATCH_SEQ;
        AppendParams p;
        memset(&p, 0, sizeof(p));
        for (u32 j = 0; j < nl; j++) {
            const tl_kv_layer *L = &layers[l0 + j];
            int rc = check_layer(L);
            if (!rc) rc = fill_seg(p.seg[j], L, k[l0 + j], v[l0 + j], kv_stride, slots, pos, n);
            if (rc) return rc;
        }
        int rc = tl_launch_append(p, nl, (hipStream_t)stream);
        if (rc) return rc;
    }
    return TL_OK;
}

static int rope_cfg(const tl_kv_layer *L, const tl_rope_params *r, RopeCfg &c) {
    return tl_rope_cfg(L->head_dim, r, c);
}

extern "C" int tl_kv_append_rope(const tl_kv_layer *L, const float *k, const float *v,
                                 uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                                 uint32_t n, const tl_rope_params *rope, void *stream) {
    int rc = check_layer(L);
    if (rc) return rc;
    if (n == 0) return TL_OK;
    AppendParams p;
    memset(&p, 0, sizeof(p));
    rc = fill_seg(p.seg[0], L, k, v, kv_stride, slots, pos, n);
    if (!rc) rc = rope_cfg(L, rope, p.rope);
    if (rc) return rc;
    return tl_launch_append(p, 1, (hipStream_t)stream);
}

__global__ __launch_bounds__(256) void kv_gather_kernel(
    const u16 *kc, const u16 *vc, u32 cap, u32 n_kv, u32 head_dim,
    const u32 *slots, u32 n, u16 *ko, u16 *vo) {
    const u32 vpr = head_dim >> 3;
    const u64 total = (u64)n * n_kv * vpr;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        u32 c = (u32)(idx % vpr);
        u64 t = idx / vpr;
        u32 h = (u32)(t % n_kv);
        u32 i = (u32)(t / n_kv);
        u32 slot = slots[i];
        uint4 kk = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
        if (slot < cap) {
            u64 src = ((u64)h * cap + slot) * head_dim + c * 8;
            kk = *(const uint4 *)(kc + src);
            vv = *(const uint4 *)(vc + src);
        }
        u64 dst = ((u64)i * n_kv + h) * head_dim + c * 8;
        *(uint4 *)(ko + dst) = kk;
        *(uint4 *)(vo + dst) = vv;
    }
}

extern "C" int tl_kv_gather(const tl_kv_layer *L, const uint32_t *slots, uint32_t n,
                            uint16_t *k_out, uint16_t *v_out, void *stream) {
    int rc = check_layer(L);
    if (rc) return rc;
    if (n == 0) return TL_OK;
    if (!slots || !k_out || !v_out) return tl_fail(TL_EINVAL, "gather: null pointer");
    if (((uintptr_t)k_out | (uintptr_t)v_out) & 15)
        return tl_fail(TL_EINVAL, "gather: outputs not 16-byte aligned");
    u64 total = (u64)n * L->n_kv_head * (L->head_dim >> 3);
    u64 blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(kv_gather_kernel, dim3((u32)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const u16 *)L->k, (const u16 *)L->v,
                       L->cap, L->n_kv_head, L->head_dim, slots, n, k_out, v_out);
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

/* grid: (blocks, layers-in-batch).  Copies one 16-byte vector of K and of V
 * per thread and grid-stride step. */
__global__ __launch_bounds__(256) void kv_copy_kernel(const CopyParams p,
                                                      const u32 *src, const u32 *dst,
                                                      u32 n) {
    const u32 l = blockIdx.y;
    u16 *kd = p.k[l];
    u16 *vd = p.v[l];
    const u16 *ks = p.ks[l];
    const u16 *vs = p.vs[l];
    const u32 vpr = p.head_dim >> 3;
    const u64 total = (u64)n * p.n_kv * vpr;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        u32 c = (u32)(idx % vpr);
        u64 t = idx / vpr;
        u32 h = (u32)(t % p.n_kv);
        u32 i = (u32)(t / p.n_kv);
        u32 s = src[i], d = dst[i];
        if (s >= p.src_cap || d >= p.cap) continue;
        u64 so = ((u64)h * p.src_cap + s) * p.head_dim + c * 8;
        u64 dof = ((u64)h * p.cap + d) * p.head_dim + c * 8;
        *(uint4 *)(kd + dof) = *(const uint4 *)(ks + so);
        *(uint4 *)(vd + dof) = *(const uint4 *)(vs + so);
    }
}

static int copy_rows(const tl_kv_layer *dl, const tl_kv_layer *sl, uint32_t n_layer,
                     const uint32_t *src, const uint32_t *dst, uint32_t n, void *stream) {
    if (n == 0 || n_layer == 0) return TL_OK;
    if (!dl || !sl || !src || !dst) return tl_fail(TL_EINVAL, "copy: null pointer");
    for (u32 l0 = 0; l0 < n_layer; l0 += TL_COPY_MAX_LAYERS) {
        u32 nl = n_layer - l0 < TL_COPY_MAX_LAYERS ? n_layer - l0 : TL_COPY_MAX_LAYERS;
        CopyParams p;
        memset(&p, 0, sizeof(p));
        for (u32 j = 0; j < nl; j++) {
            const tl_kv_layer *D = &dl[l0 + j], *S = &sl[l0 + j];
            int rc = check_layer(D);
            if (!rc) rc = check_layer(S);
            if (rc) return rc;
            if (D->ring || S->ring) return tl_fail(TL_EINVAL, "copy: ring layers hold no slot rows");
            if (S->n_kv_head != D->n_kv_head || S->head_dim != D->head_dim)
                return tl_fail(TL_EINVAL, "copy: source and destination differ in shape");
            if (j == 0) {
                p.cap = D->cap;
                p.src_cap = S->cap;
                p.n_kv = D->n_kv_head;
                p.head_dim = D->head_dim;
            } else if (D->cap != p.cap || S->cap != p.src_cap || D->n_kv_head != p.n_kv ||
                       D->head_dim != p.head_dim) {
                return tl_fail(TL_EINVAL, "copy: layers differ in shape");
            }
            p.k[j] = (u16 *)D->k;
            p.v[j] = (u16 *)D->v;
            p.ks[j] = (const u16 *)S->k;
            p.vs[j] = (const u16 *)S->v;
        }
        u64 total = (u64)n * p.n_kv * (p.head_dim >> 3);
        u64 blocks = (total + 255) / 256;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL(kv_copy_kernel, dim3((u32)blocks, nl), dim3(256), 0,
                           (hipStream_t)stream, p, src, dst, n);
        HIP_TRY(hipGetLastError());
    }
    return TL_OK;
}

extern "C" int tl_kv_copy(const tl_kv_layer *layers, uint32_t n_layer,
                          const uint32_t *src, const uint32_t *dst, uint32_t n,
                          void *stream) {
    return copy_rows(layers, layers, n_layer, src, dst, n, stream);
}

extern "C" int tl_kv_copy_between(const tl_kv_layer *dst_layers, const tl_kv_layer *src_layers,
                                  uint32_t n_layer, const uint32_t *src, const uint32_t *dst,
                                  uint32_t n, void *stream) {
    return copy_rows(dst_layers, src_layers, n_layer, src, dst, n, stream);
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                      */
/* ------------------------------------------------------------------------ */

/* One thread per rotated pair.  theta_i and the angle are formed in f32 as
 * in the reference: NORM t = 1/powf(base, i/rdim) for even i, NEOX
 * t = 1/powf(base, 2i/rdim); angle = (float)pos * t. */
__global__ __launch_bounds__(256) void rope_kernel(float *x, u32 rows, u32 row_stride,
                                                  u32 heads, u32 hdim, u32 rdim,
                                                  u32 pos, float base, int neox) {
    const u32 pairs = rdim >> 1;
    const u64 total = (u64)rows * heads * pairs;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        u32 i = (u32)(idx % pairs);
        u64 t = idx / pairs;
        u32 h = (u32)(t % heads);
        u32 r = (u32)(t / heads);
        float *bh = x + (u64)r * row_stride + (u64)h * hdim;
        const u32 ia = neox ? i : 2 * i, ib = neox ? i + pairs : 2 * i + 1;
        float c, s, nx, ny;
        rope_cs(i, rdim, base, pos + r, c, s);
        rope_rot(bh[ia], bh[ib], c, s, nx, ny);
        bh[ia] = nx;
        bh[ib] = ny;
    }
}

extern "C" int tl_rope(float *x, uint32_t rows, uint32_t row_stride, uint32_t heads,
                       uint32_t head_dim, uint32_t rope_dim, uint32_t pos, float theta,
                       int neox, void *stream) {
    if (rows == 0) return TL_OK;
    if (!x || rope_dim > head_dim || (rope_dim & 1) || row_stride < heads * head_dim)
        return tl_fail(TL_EINVAL, "rope: bad shape");
    u64 total = (u64)rows * heads * (rope_dim >> 1);
    u64 blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(rope_kernel, dim3((u32)blocks), dim3(256), 0, (hipStream_t)stream,
                       x, rows, row_stride, heads, head_dim, rope_dim, pos, theta, neox);
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

/* ------------------------------------------------------------------------ */
/* OP_ATTN entry points                                                      */
/* ------------------------------------------------------------------------ */

LayerView tl_view(const tl_kv_layer *L) {
    LayerView v;
    v.k = L->k;
    v.v = L->v;
    v.ks = v.vs = nullptr;
    v.cap = L->cap;
    v.n_kv_head = L->n_kv_head;
    v.head_dim = L->head_dim;
    v.ring = L->ring;
    v.q8 = false;
    return v;
}

/* OP_ATTN argument rules shared by the f16 and Q8_0 caches (the layer
 * itself has been checked) */
int tl_check_attn_args(const LayerView &L, const tl_attn_args *a) {
    if (!a || !a->q || !a->dst) return tl_fail(TL_EINVAL, "attn: null q/dst");
    if (a->n_head == 0 || a->n_head % L.n_kv_head)
        return tl_fail(TL_EINVAL, "attn: n_head %u not a multiple of n_kv %u",
                       a->n_head, L.n_kv_head);
    if (a->n_head / L.n_kv_head > 8)
        return tl_fail(TL_EINVAL, "attn: gqa ratio %u > 8", a->n_head / L.n_kv_head);
    if (a->q_stride < a->n_head * L.head_dim || (a->q_stride & 3) ||
        (((uintptr_t)a->q | (uintptr_t)a->dst) & 15))
        return tl_fail(TL_EINVAL, "attn: q/dst rows must be 16-byte aligned");
    if (L.ring) {
        if (!a->window || L.ring < a->window + a->n - 1)
            return tl_fail(TL_EINVAL, "attn: ring %u too small for window %u and %u rows",
                           L.ring, a->window, a->n);
    } else if (!a->slots && (u64)a->pos + a->n > L.cap) {
        return tl_fail(TL_ERANGE, "attn: pos %u + n %u exceeds cap %u", a->pos, a->n, L.cap);
    }
    return TL_OK;
}

static int check_args(const tl_kv_layer *L, const tl_attn_args *a) {
    int rc = check_layer(L);
    if (rc) return rc;
    return tl_check_attn_args(tl_view(L), a);
}

/* append (when `append`) + attention.  Decode-sized batches run as one
 * fused launch (the decode kernel writes the new rows itself); prefill-sized
 * ones append first and then run the MFMA kernel. */
static int attn_core(const tl_kv_layer *L, const tl_attn_args *a, bool append,
                     const RopeCfg &rope, hipStream_t st) {
    const LayerView lv = tl_view(L);
    if (tl_use_prefill(lv, a)) {
        bool fused = false;
        if (append) {
            AppendParams ap;
            memset(&ap, 0, sizeof(ap));
            int rc = fill_seg(ap.seg[0], L, a->k, a->v, a->kv_stride, a->slots, a->pos, a->n);
            if (rc) return rc;
            /* the prefill launch writes the rows itself (its stores address
             * the whole layer through one 2 GB buffer resource) */
            fused = !tl_tune(TL_TUNE_PREFILL_SEPARATE_APPEND) &&
                    (u64)L->n_kv_head * L->cap * L->head_dim * 2 < 0x7ffffff0ull;
            if (!fused) {
                ap.rope = rope;
                rc = tl_launch_append(ap, 1, st);
                if (rc) return rc;
            }
        }
        return tl_launch_prefill(lv, a, rope, st, fused);
    }
    DecParams p;
    memset(&p, 0, sizeof(p));
    if (append && a->n > TL_DEC_MAX_NEW) {
        /* more new rows than a decode launch stages: append first */
        AppendParams ap;
        memset(&ap, 0, sizeof(ap));
        int rc = fill_seg(ap.seg[0], L, a->k, a->v, a->kv_stride, a->slots, a->pos, a->n);
        if (rc) return rc;
        ap.rope = rope;
        rc = tl_launch_append(ap, 1, st);
        if (rc) return rc;
    } else if (append) {
        AppendSeg chk;
        int rc = fill_seg(chk, L, a->k, a->v, a->kv_stride, a->slots, a->pos, a->n);
        if (rc) return rc;
        p.seq[0].kin = a->k;
        p.seq[0].vin = a->v;
        p.seq[0].kv_stride = a->kv_stride;
    }
    p.seq[0].k = (const u16 *)L->k;
    p.seq[0].v = (const u16 *)L->v;
    p.seq[0].slots = a->slots;
    p.seq[0].q = a->q;
    p.seq[0].dst = a->dst;
    p.seq[0].cap = L->cap;
    p.seq[0].ring = L->ring;
    p.seq[0].pos = a->pos;
    p.rows_per_seq = a->n;
    p.n_kv = L->n_kv_head;
    p.n_head = a->n_head;
    p.q_stride = a->q_stride;
    p.window = a->window;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.rope = rope;
    u32 max_keys = a->pos + a->n;
    u32 max_vis = (a->window && max_keys > a->window) ? a->window : max_keys;
    return tl_launch_decode(p, a->n, L->head_dim, a->n_head / L->n_kv_head, max_vis, st);
}

extern "C" int tl_attn(const tl_kv_layer *L, const tl_attn_args *a, void *stream) {
    int rc = check_args(L, a);
    if (rc) return rc;
    if (a->n == 0) return TL_OK;
    RopeCfg rc0;
    rope_cfg(L, nullptr, rc0);
    return attn_core(L, a, true, rc0, (hipStream_t)stream);
}

extern "C" int tl_attn_rope(const tl_kv_layer *L, const tl_attn_args *a,
                            const tl_rope_params *rope, void *stream) {
    int rc = check_args(L, a);
    if (rc) return rc;
    if (a->n == 0) return TL_OK;
    RopeCfg c;
    rc = rope_cfg(L, rope, c);
    if (rc) return rc;
    return attn_core(L, a, true, c, (hipStream_t)stream);
}

extern "C" int tl_attn_noappend(const tl_kv_layer *L, const tl_attn_args *a, void *stream) {
    int rc = check_args(L, a);
    if (rc) return rc;
    if (a->n == 0) return TL_OK;
    RopeCfg rc0;
    rope_cfg(L, nullptr, rc0);
    return attn_core(L, a, false, rc0, (hipStream_t)stream);
}

/* Guards of the fixed region: one call inside tl_attn_noalloc per device at
 * a time, and the stream and completion event of the last uncaptured call,
 * so that a call on another stream while that one's work is still queued or
 * running is refused instead of racing on the region. */
static std::atomic<int> g_scratch_busy[TL_MAX_DEV];
static hipStream_t g_scratch_last[TL_MAX_DEV];
static hipEvent_t g_scratch_done[TL_MAX_DEV];

extern "C" int tl_attn_noalloc(const tl_kv_layer *L, const tl_attn_args *a, void *stream) {
    int rc = check_args(L, a);
    if (rc) return rc;
    if (a->n == 0) return TL_OK;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= TL_MAX_DEV) return tl_fail(TL_EINVAL, "device %d", dev);
    const hipStream_t st = (hipStream_t)stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(st, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    int idle = 0;
    if (!g_scratch_busy[dev].compare_exchange_strong(idle, 1, std::memory_order_acquire))
        return tl_fail(TL_EBUSY, "noalloc: another call on device %d is in progress", dev);
    struct Release {
        int d;
        ~Release() { g_scratch_busy[d].store(0, std::memory_order_release); }
    } release{dev};
    TlWorkspace *w = &g_scratch_ws[dev];
    if (!w->acc) {
        if (capturing)
            return tl_fail(TL_EINVAL, "noalloc: call tl_init(%d) before capturing", dev);
        rc = scratch_setup(dev, &w);
        if (rc) return rc;
    }
    hipEvent_t &done = g_scratch_done[dev];
    if (!capturing) {
        if (!done) HIP_TRY(hipEventCreateWithFlags(&done, hipEventDisableTiming));
        else if (g_scratch_last[dev] != st) {
            const hipError_t q = hipEventQuery(done);
            if (q == hipErrorNotReady)
                return tl_fail(TL_EBUSY,
                               "noalloc: the previous call's work on another stream has not "
                               "finished");
            if (q != hipSuccess) HIP_TRY(q);
        }
    }
    {
        TlWsFixed scope(w);
        RopeCfg rc0;
        rope_cfg(L, nullptr, rc0);
        rc = attn_core(L, a, true, rc0, st);
    }
    if (!rc && !capturing) {
        HIP_TRY(hipEventRecord(done, st));
        g_scratch_last[dev] = st;
    }
    return rc;
}

static int decode_batch(const tl_decode_seq *seqs, uint32_t n_seq, uint32_t n_head,
                        uint32_t window, float scale, const tl_rope_params *rope,
                        void *stream);

extern "C" int tl_attn_decode_batch(const tl_decode_seq *seqs, uint32_t n_seq,
                                    uint32_t n_head, uint32_t window, float scale,
                                    void *stream) {
    return decode_batch(seqs, n_seq, n_head, window, scale, nullptr, stream);
}

extern "C" int tl_attn_decode_batch_rope(const tl_decode_seq *seqs, uint32_t n_seq,
                                         uint32_t n_head, uint32_t window, float scale,
                                         const tl_rope_params *rope, void *stream) {
    return decode_batch(seqs, n_seq, n_head, window, scale, rope, stream);
}

static int decode_batch(const tl_decode_seq *seqs, uint32_t n_seq, uint32_t n_head,
                        uint32_t window, float scale, const tl_rope_params *rope,
                        void *stream) {
    if (n_seq == 0) return TL_OK;
    if (!seqs || n_seq > TL_MAX_BATCH_SEQ)
        return tl_fail(TL_EINVAL, "decode_batch: 1..%d sessions", TL_MAX_BATCH_SEQ);
    const tl_kv_layer *L0 = &seqs[0].layer;
    DecParams p;
    memset(&p, 0, sizeof(p));
    u32 max_vis = 1;
    for (u32 i = 0; i < n_seq; i++) {
        const tl_decode_seq *s = &seqs[i];
        tl_attn_args a;
        memset(&a, 0, sizeof(a));
        a.q = s->q; a.k = s->k; a.v = s->v; a.dst = s->dst; a.slots = s->slots;
        a.pos = s->pos; a.n = 1; a.n_head = n_head;
        a.q_stride = n_head * s->layer.head_dim;
        a.kv_stride = s->layer.n_kv_head * s->layer.head_dim;
        a.window = window; a.scale = scale;
        int rc = check_args(&s->layer, &a);
        if (rc) return rc;
        if (s->layer.n_kv_head != L0->n_kv_head || s->layer.head_dim != L0->head_dim)
            return tl_fail(TL_EINVAL, "decode_batch: sessions differ in shape");
        AppendSeg chk;
        rc = fill_seg(chk, &s->layer, s->k, s->v, a.kv_stride, s->slots, s->pos, 1);
        if (rc) return rc;
        p.seq[i].kin = s->k;
        p.seq[i].vin = s->v;
        p.seq[i].kv_stride = a.kv_stride;
        p.seq[i].k = (const u16 *)s->layer.k;
        p.seq[i].v = (const u16 *)s->layer.v;
        p.seq[i].slots = s->slots;
        p.seq[i].q = s->q;
        p.seq[i].dst = s->dst;
        p.seq[i].cap = s->layer.cap;
        p.seq[i].ring = s->layer.ring;
        p.seq[i].pos = s->pos;
        u32 nk = s->pos + 1;
        u32 vis = (window && nk > window) ? window : nk;
        if (vis > max_vis) max_vis = vis;
    }
    p.rows_per_seq = 1;
    p.n_kv = L0->n_kv_head;
    p.n_head = n_head;
    p.q_stride = n_head * L0->head_dim;
    p.window = window;
    p.scale_log2 = scale * 1.4426950408889634f;
    int rc = rope_cfg(L0, rope, p.rope);
    if (rc) return rc;
    return tl_launch_decode(p, n_seq, L0->head_dim, n_head / L0->n_kv_head, max_vis,
                            (hipStream_t)stream);
}

/* ------------------------------------------------------------------------ */
/* HBM read-bandwidth probe (measurement aid)                                */
/* ------------------------------------------------------------------------ */

/* Streams `bytes` from src with 16-byte loads, `depth` independent loads in
 * flight per lane, and writes one word per thread so the loads stay live. */
template <int DEPTH>
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4 *src, u64 n16, u32 *sink) {
    u32 acc = 0;
    const u64 stride = (u64)gridDim.x * blockDim.x;
    u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (DEPTH - 1) * stride < n16; i += DEPTH * stride) {
        uint4 v[DEPTH];
#pragma unroll
        for (int k = 0; k < DEPTH; k++) v[k] = src[i + k * stride];
#pragma unroll
        for (int k = 0; k < DEPTH; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += stride) {
        uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    sink[(u64)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

extern "C" int tl_probe_read(const void *src, uint64_t bytes, uint32_t *sink,
                             uint32_t blocks, uint32_t depth, void *stream) {
    if (!src || !sink || (bytes & 15) || blocks == 0)
        return tl_fail(TL_EINVAL, "probe: bad arguments");
    const u64 n16 = bytes / 16;
    switch (depth) {
    case 1: hipLaunchKernelGGL(read_probe_kernel<1>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4 *)src, n16, sink); break;
    case 4: hipLaunchKernelGGL(read_probe_kernel<4>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4 *)src, n16, sink); break;
    case 8: hipLaunchKernelGGL(read_probe_kernel<8>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4 *)src, n16, sink); break;
    case 16: hipLaunchKernelGGL(read_probe_kernel<16>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4 *)src, n16, sink); break;
    default: return tl_fail(TL_EINVAL, "probe: depth 1/4/8/16");
    }
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

/* Error reporting for the C translation units of the library. */
extern "C" int tl_set_error(int code, const char *msg) { return tl_fail(code, "%s", msg); }
