/* tl_internal.h — launch parameter blocks shared by the .hip translation units. */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/tlkv.h"

#define TL_COPY_MAX_LAYERS 64
#define TL_PREFILL_MIN_ROWS 16
#define TL_PREFILL_MIN_WORK 262144  /* rows x visible keys up to which the decode kernel runs */
#define TL_PREFILL_MIN_WORK_Q8 163840  /* the same over a Q8_0 cache */
#define TL_DEC_FOLD_MAX_ROWS 64     /* most rows of a decode-kernel batch */
#define TL_DEC_MAX_NEW 16          /* new rows of one fused decode launch (< TL_PREFILL_MIN_ROWS) */
#define TL_DEC_Q8_ROPE_NEW 4       /* ... into a Q8_0 cache with RoPE (f32 staging of rotated K) */

/* One segment of an append launch: n rows of one layer of one session. */
/* RoPE applied on the fly (rdim == 0: none).  Same math as rope_kernel. */
struct RopeCfg {
    uint32_t rdim;
    float theta;
    int32_t neox;
};

struct AppendSeg {
    uint16_t *kc, *vc;
    const float *k, *v;
    const uint32_t *slots;
    uint32_t cap, ring, n_kv, head_dim, kv_stride, pos, n;
};
/* NS segments per launch; single-segment launches use NS = 1, because the
 * kernel arguments are copied per launch (measured: a 512-row append takes
 * 4.6 us with one segment's arguments, 5.5 us with TL_MAX_BATCH_SEQ) */
template <int NS>
struct AppendParamsN {
    AppendSeg seg[NS];
    RopeCfg rope;            /* applied to K before the conversion */
};
typedef AppendParamsN<TL_MAX_BATCH_SEQ> AppendParams;

struct CopyParams {
    uint16_t *k[TL_COPY_MAX_LAYERS];          /* destination pool */
    uint16_t *v[TL_COPY_MAX_LAYERS];
    const uint16_t *ks[TL_COPY_MAX_LAYERS];   /* source pool (== k, v within a pool) */
    const uint16_t *vs[TL_COPY_MAX_LAYERS];
    uint32_t cap, src_cap, n_kv, head_dim;
};

/* One sequence of a decode launch (rows_per_seq rows at positions pos..). */
struct DecSeq {
    const uint16_t *k, *v;    /* f16 rows, or int8 rows of a Q8_0 cache */
    const uint16_t *ks, *vs;  /* Q8_0 scales (f16 [n_kv][cap][D/32]), else NULL */
    const uint32_t *slots;
    const float *q;
    float *dst;
    const float *kin, *vin;   /* new rows (f32) to append in the same launch, or NULL */
    uint32_t cap, ring, pos, kv_stride;
};
struct DecParams {
    DecSeq seq[TL_MAX_BATCH_SEQ];
    uint32_t rows_per_seq;
    uint32_t n_kv, n_head, q_stride, window;
    float scale_log2;
    uint32_t chunk, n_split;
    float *ws_acc;           /* split partials: [rows][n_head][n_split][D] */
    float2 *ws_ml;           /* split (max, sum): [rows][n_head][n_split] */
    RopeCfg rope;            /* applied to q and to new K rows */
    uint32_t *counters;      /* merge counters (TL_MERGE_CNT_WORDS, layout below);
                                NULL = partials are merged by attn_merge_kernel */
    uint32_t dist;           /* 1: every split merges its own slice of the output */
    uint32_t polls;          /* most polls per bounded wait of the split merge */
    uint32_t rows_per_wg;    /* matrix-core tile: batch rows per workgroup group (their
                                heads side by side as the MFMA columns); 0 or 1: one */
};

/* In-launch split merge state, per workspace (u32 words, zero at start):
 *   [0, TL_MERGE_MAX_GROUPS * TL_MERGE_PAD): the arrival count of each
 *     (row, kv-head) group, alone in a 128-byte line; the last split to
 *     arrive sets it back to zero;
 *   then TL_MERGE_MAX_SPLIT_DIST claim tags per group;
 *   then the launch counter (its own line): every group's last split adds
 *   one when a launch merges slices in every split (dist), and such a
 *   launch reads it first: epoch = counter + 1 marks that launch's partial
 *   records and claim tags.  Epochs never repeat on a workspace, also when
 *   a captured graph replays the same launches. */
#define TL_MERGE_MAX_GROUPS 4096
#define TL_MERGE_PAD 32
#define TL_MERGE_MAX_SPLIT_DIST 64
#define TL_MERGE_TAGS (TL_MERGE_MAX_GROUPS * TL_MERGE_PAD)
#define TL_MERGE_LAUNCHES (TL_MERGE_TAGS + TL_MERGE_MAX_SPLIT_DIST * TL_MERGE_MAX_GROUPS)
/* groups of the current launch whose closer has run (dist merge): the last
 * one resets it and advances TL_MERGE_LAUNCHES, so the launch counter moves
 * once per launch, after every workgroup of the launch has read it */
#define TL_MERGE_CLOSED (TL_MERGE_LAUNCHES + TL_MERGE_PAD / 2)
#define TL_MERGE_CNT_WORDS (TL_MERGE_LAUNCHES + TL_MERGE_PAD)

/* Chunked-prefill launch (one OP_ATTN batch of one session). */
struct PrefParams {
    const uint16_t *k, *v;    /* f16 rows, or int8 rows of a Q8_0 cache */
    const uint16_t *ks, *vs;  /* Q8_0 scales, else NULL */
    const uint32_t *slots;
    uint32_t cap, ring;
    const float *q;
    float *dst;
    uint32_t q_stride, pos, n, n_head, n_kv, window;
    float scale_log2;
    uint32_t n_split;
    float *ws_acc;
    float2 *ws_ml;
    RopeCfg rope;            /* applied to q rows (and to appended K rows) */
    /* fused append (f16 cache; kin NULL: none): the batch's K/V rows, f32
     * [n][kv_stride], converted and written by the launch's own workgroups
     * in units of 16 rows of one kv-head; flags[kvh * units + u] = epoch once
     * a unit is in the cache; ctr[0] = launch counter (epoch - 1), ctr[1] =
     * workgroups finished in this launch */
    const float *kin, *vin;
    uint32_t kv_stride, polls;
    uint32_t *flags, *ctr;
};
/* the fused append's counters sit past the decode merge's in a workspace */
#define TL_PF_CTR_WORDS 64
#define TL_PF_ROWS 16

struct TlWorkspace {
    float *acc;
    float *ml;
    uint32_t *cnt;
    size_t acc_cap, ml_cap, cnt_cap;
};

/* A layer's storage as the attention launches read it: an f16 cache
 * (tl_kv_layer) or a Q8_0 cache (tl_kv_layer_q8, q8 = true). */
struct LayerView {
    const void *k, *v;
    const uint16_t *ks, *vs;
    uint32_t cap, n_kv_head, head_dim, ring;
    bool q8;
};
LayerView tl_view(const tl_kv_layer *L);
int tl_check_attn_args(const LayerView &L, const tl_attn_args *a);
int tl_rope_cfg(uint32_t head_dim, const tl_rope_params *r, RopeCfg &c);

int tl_fail(int code, const char *fmt, ...);

/* launch-shape override `key` (TL_TUNE_*), 0 = automatic */
uint32_t tl_tune(int key);

#define HIP_TRY(expr)                                                         \
    do {                                                                      \
        hipError_t e_ = (expr);                                               \
        if (e_ != hipSuccess)                                                 \
            return tl_fail(TL_EHIP, "%s: %s", #expr, hipGetErrorString(e_));  \
    } while (0)

/* Most keys one decode workgroup handles (its slot indices are staged in LDS). */
#define TL_DEC_MAX_CHUNK 2048
#define TL_DEC_MAX_CHUNK16 4096   /* ... staged as u16 (pools of at most 65536 rows) */
/* split partials for a launch on `st`: the stream's own workspace (grown on
 * demand), or inside a TlWsFixed scope the fixed region (TL_ERANGE when it
 * is too small; nothing is allocated) */
int tl_workspace_get(hipStream_t st, size_t acc_floats, size_t ml_pairs, size_t counters,
                     TlWorkspace **out);
/* Scope in which this thread's launches take their partials from `w`. */
struct TlWsFixed {
    explicit TlWsFixed(TlWorkspace *w);
    ~TlWsFixed();
    TlWorkspace *prev;
};
/* partial floats of the fixed region in scope, 0 outside one */
size_t tl_workspace_fixed_acc(void);
int tl_launch_append(const AppendParams &p, uint32_t n_seg, hipStream_t stream);
/* q8: the seq[] rows are a Q8_0 cache (no fused append: kin must be NULL) */
int tl_launch_decode(DecParams &p, uint32_t n_rows_total, uint32_t head_dim, uint32_t G,
                     uint32_t max_vis, hipStream_t st, bool q8 = false);
/* combine n_split partial rows (ws_acc / ws_ml) into seq[..].dst */
int tl_launch_merge(const DecParams &p, uint32_t n_rows_total, uint32_t head_dim, hipStream_t st);

/* MFMA chunked-prefill attention (tl_prefill.hip). */
bool tl_prefill_supported(const LayerView &L, const tl_attn_args *a);
/* the batch runs on the prefill kernel (else on the decode kernel) */
bool tl_use_prefill(const LayerView &L, const tl_attn_args *a);
int tl_launch_prefill(const LayerView &L, const tl_attn_args *a, const RopeCfg &rope,
                      hipStream_t st, bool append = false);
