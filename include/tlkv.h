/*
 * tlkv.h — C ABI of the MI355X (gfx950) KV-cache device library.
 *
 * Plain C: pointers, sizes and a stream handle.  All pointers named "device"
 * are HIP device addresses; `stream` is a hipStream_t passed as void* (NULL =
 * the default stream).  Every entry point returns 0 on success or a negative
 * TL_E* code; tl_last_error() gives the message of the calling thread's last
 * failure.  No entry point aborts the process (the reference's CUDA backend
 * exits on API errors, src/backend/gpu/gpu.h:41-50; here they are returned,
 * the same way kvcache.c returns false).
 *
 * Reference interfaces replaced (paths relative to the tinyllama.c tree):
 *   tl_kv_append      the K/V write-through of OP_ATTN:
 *                     src/backend/cpu/cpu_op.c:995-1008 (slot-indexed) and
 *                     src/backend/gpu/gpu_op.cu:632-644,947-951 (k_kv_write)
 *   tl_attn           OP_ATTN as a whole: cpu_op.c:964-1064 (op_attn) and
 *                     gpu_op.cu:925-962 (gpu_op_attn) — append, then causal
 *                     GQA attention over the slot table with the optional
 *                     sliding window (cpu_op.c:1019-1022)
 *   tl_attn_decode_batch  one-token OP_ATTN for several sessions in one
 *                     launch (the -np slots of src/server.c:1464-1478 are
 *                     independent Sessions, each with its own KvCache)
 *   tl_kv_gather      read view of the cache rows (the rows op_attn reads at
 *                     cpu_op.c:1024-1033,1045-1052)
 *   tl_kv_copy        slot-row copy across all layers: prefix fork and
 *                     eviction compaction (no counterpart: the reference shares
 *                     slots in place, src/kvcache.c:192-218)
 *   tl_rope           OP_ROPE_NORM / OP_ROPE_NEOX, cpu_op.c:632-700,
 *                     gpu_op.cu:300-355
 *
 * Cache layout (per layer, per K and V): f16 bits [n_kv_head][cap][head_dim],
 * the reference's head-major layout (src/graph.c:852-858, AttnKvCache in
 * src/def.h:289-294) with binary16 elements instead of f32.  The f16 value of
 * a row element is the IEEE round-to-nearest-even of the f32 input; NaN maps
 * to a quiet NaN that keeps the sign and the top 9 payload bits.
 */
#ifndef TLKV_H
#define TLKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TL_OK        = 0,
    TL_EINVAL    = -1,   /* bad argument / shape the kernels do not support */
    TL_ERANGE    = -2,   /* slot or position outside the cache */
    TL_EHIP      = -3,   /* HIP runtime error */
    TL_ENOMEM    = -4,   /* device allocation failed */
    TL_EBUSY     = -5,   /* a shared resource is in use by an overlapping call */
};

/* One layer of the KV cache (the device twin of AttnKvCache). */
typedef struct tl_kv_layer {
    void     *k;          /* device, f16 [n_kv_head][cap][head_dim] */
    void     *v;          /* device, f16 [n_kv_head][cap][head_dim] */
    uint32_t  cap;        /* rows per head */
    uint32_t  n_kv_head;
    uint32_t  head_dim;   /* kv_head_dim: 64, 128 or 256 */
    uint32_t  ring;       /* 0: rows addressed through the slot table;
                             R > 0: physical row of position p is p % R
                             (sliding-window layers; R <= cap) */
} tl_kv_layer;

/* Arguments of one OP_ATTN call (the fields of OpCtx, src/def.h:550-565,
 * that op_attn reads). */
typedef struct tl_attn_args {
    const float    *q;        /* device [n][q_stride] f32, RoPE'd */
    const float    *k;        /* device [n][kv_stride] f32, RoPE'd new rows */
    const float    *v;        /* device [n][kv_stride] f32 new rows */
    float          *dst;      /* device [n][q_stride] f32 */
    const uint32_t *slots;    /* device slot table, logical pos -> row, at
                                 least pos+n entries; NULL = identity */
    uint32_t        pos;      /* absolute position of batch row 0 */
    uint32_t        n;        /* batch rows */
    uint32_t        n_head;   /* q heads (multiple of n_kv_head, ratio <= 8) */
    uint32_t        q_stride; /* floats between q / dst rows (>= n_head*head_dim) */
    uint32_t        kv_stride;/* floats between k / v rows (>= n_kv*head_dim) */
    uint32_t        window;   /* sliding window, 0 = full causal */
    float           scale;    /* 1/sqrt(kv_head_dim) in the reference (graph.c:1275) */
} tl_attn_args;

/* One session of a batched one-token decode. */
typedef struct tl_decode_seq {
    tl_kv_layer     layer;
    const uint32_t *slots;    /* device slot table of this session, or NULL */
    uint32_t        pos;      /* position of the new token */
    uint32_t        pad_;
    const float    *q;        /* device [n_head*head_dim] f32 */
    const float    *k;        /* device [n_kv*head_dim] f32 */
    const float    *v;        /* device [n_kv*head_dim] f32 */
    float          *dst;      /* device [n_head*head_dim] f32 */
} tl_decode_seq;

#define TL_MAX_BATCH_SEQ 16

/* RoPE applied inside a fused entry point (the reference's OP_ROPE_NORM /
 * OP_ROPE_NEOX, src/backend/cpu/cpu_op.c:632-700, on Q and K before OP_ATTN).
 * Pair i of each head rotates by angle pos * theta^(-2i/rope_dim); NORM
 * (neox = 0) pairs elements (2i, 2i+1), NEOX pairs (i, i + rope_dim/2). */
typedef struct tl_rope_params {
    uint32_t rope_dim;        /* rotated elements per head (even, <= head_dim) */
    float    theta;           /* base */
    int32_t  neox;
} tl_rope_params;

const char *tl_last_error(void);

/* Select the device for the calling thread and set up library state. */
int tl_init(int device);

/* Launch-shape overrides (measurement and testing aid; no reference
 * counterpart).  Every value defaults to 0 = automatic; the first library
 * call reads the environment variable of the same name once (e.g.
 * TL_DECODE_WGS=512), after which only tl_set_tuning changes them.
 * Results do not depend on them beyond floating-point summation order. */
#define TL_TUNE_DECODE_WGS          0   /* decode workgroups per launch */
#define TL_TUNE_DECODE_MIN_KEYS     1   /* fewest keys per decode split */
#define TL_TUNE_DECODE_MERGE_KERNEL 2   /* 1: merge decode splits in a separate launch */
#define TL_TUNE_PREFILL_SPLITS      3   /* key splits of the prefill kernel */
#define TL_TUNE_NO_PREFILL          4   /* 1: run every batch on the decode kernel, 2: every
                                           batch of at least 16 rows on the prefill kernel */
#define TL_TUNE_DECODE_SINGLE_MERGE 5   /* 1: the last split of a group merges all of it */
#define TL_TUNE_DECODE_MERGE_POLLS  6   /* n: at most n - 1 polls per wait of the split merge */
#define TL_TUNE_PREFILL_APPEND_POLLS 7  /* n: at most n - 1 polls per wait for the fused append */
#define TL_TUNE_PREFILL_SEPARATE_APPEND 8 /* 1: prefill batches append in a launch of their own */
#define TL_TUNE_DECODE_MFMA         9   /* 1: decode tiles on the vector ALUs, 2: on the matrix cores */
#define TL_TUNE_DECODE_ROWS        10   /* n: batch rows per matrix-core decode group (1: one) */
#define TL_TUNE_COUNT               11
int tl_set_tuning(int key, uint32_t value);
uint32_t tl_get_tuning(int key);

/* Allocate / free one layer's K and V storage (hipMalloc, contents zero). */
int tl_kv_layer_alloc(tl_kv_layer *L, uint32_t cap, uint32_t n_kv_head,
                      uint32_t head_dim, uint32_t ring);
int tl_kv_layer_free(tl_kv_layer *L);

/* Write n rows of K and V (f32 -> f16 RNE) at slots[pos+i] (or pos+i when
 * slots is NULL, or (pos+i) % ring on ring layers).  Rows whose slot is
 * outside the cache are skipped on the device; callers validate slots on the
 * host (the session layer does). */
int tl_kv_append(const tl_kv_layer *L, const float *k, const float *v,
                 uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                 uint32_t n, void *stream);

/* Copy rows slots[i] of every head to k_out/v_out [n][n_kv_head][head_dim]
 * f16 (device).  slots: device [n]. */
int tl_kv_gather(const tl_kv_layer *L, const uint32_t *slots, uint32_t n,
                 uint16_t *k_out, uint16_t *v_out, void *stream);

/* For every layer in layers[0..n_layer) (host array) copy row src[i] to row
 * dst[i] in K and V, all heads.  src/dst: device [n].  The destination rows
 * must not be source rows of the same call. */
int tl_kv_copy(const tl_kv_layer *layers, uint32_t n_layer,
               const uint32_t *src, const uint32_t *dst, uint32_t n,
               void *stream);

/* The same across two pools of equal row shape (capacities may differ): row
 * src[i] of src_layers[l] -> row dst[i] of dst_layers[l].  Used to fork a
 * cached prefix from one session into another (the reference's -np slots are
 * separate Sessions with separate caches, src/server.c:1464-1478, and a hit
 * in another slot's cache is recomputed there). */
int tl_kv_copy_between(const tl_kv_layer *dst_layers, const tl_kv_layer *src_layers,
                       uint32_t n_layer, const uint32_t *src, const uint32_t *dst,
                       uint32_t n, void *stream);

/* Fused RoPE + OP_ATTN (the reference's own to-do, REMEMBER.md:20; the
 * reference runs OP_ROPE on Q and K, cpu_op.c:637-700, then OP_ATTN,
 * cpu_op.c:964-1064).  Same results as tl_rope(q rows at pos..), tl_rope(k
 * rows at pos..) then tl_attn, bit for bit, in one launch for decode batches
 * (two for prefill batches: append+RoPE, then attention).  q and k are read,
 * not rotated in place. */
int tl_attn_rope(const tl_kv_layer *L, const tl_attn_args *a, const tl_rope_params *rope,
                 void *stream);

/* The write-through of one token batch into several layers in one launch
 * per 16 layers (no reference counterpart: the reference writes a layer's
 * rows inside that layer's OP_ATTN, cpu_op.c:995-1008).  For callers that
 * hold every layer's rows at once — restoring or extending a cache without
 * attention (tl_session_append).  Layer l takes k[l], v[l]; all layers share
 * kv_stride, slots, pos and n.  Same bytes as n_layer tl_kv_append calls. */
int tl_kv_append_layers(const tl_kv_layer *layers, uint32_t n_layer, const float *const *k,
                        const float *const *v, uint32_t kv_stride, const uint32_t *slots,
                        uint32_t pos, uint32_t n, void *stream);

/* tl_kv_append with RoPE applied to K on the way (same bits as tl_rope then
 * tl_kv_append; k is not modified). */
int tl_kv_append_rope(const tl_kv_layer *L, const float *k, const float *v,
                      uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                      uint32_t n, const tl_rope_params *rope, void *stream);

/* OP_ATTN: append the batch rows, then attend.  Decode-sized batches use the
 * split-K LDS kernel, larger ones the MFMA chunked-prefill kernel. */
int tl_attn(const tl_kv_layer *L, const tl_attn_args *a, void *stream);

/* tl_attn that allocates nothing.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops).  The split partials and merge counters live in one
 * fixed region per GPU (32 MiB, held until the process ends; set up by
 * tl_init or the first call on a device).  Calls needing more than it holds
 * fail with TL_ERANGE (prefill batches take fewer key splits to fit).  All
 * calls on one GPU share the region, so calls must not overlap on one GPU;
 * the overlaps the library can see fail with TL_EBUSY instead of racing: a
 * call while another thread's call is inside the function, and a call on
 * another stream than the previous call's while that call's work has not
 * finished.  Under HIP graph capture, call tl_init(device) first (setting the
 * region up synchronises the device), and keep replays of captured calls
 * from overlapping other calls: the library cannot see those. */
int tl_attn_noalloc(const tl_kv_layer *L, const tl_attn_args *a, void *stream);

/* Attention only (no append): the rows at positions < pos+n are assumed
 * already in the cache. */
int tl_attn_noappend(const tl_kv_layer *L, const tl_attn_args *a, void *stream);

/* One-token OP_ATTN (append + attention) for n_seq sessions in one launch.
 * All sessions share n_kv_head, head_dim and n_head. */
int tl_attn_decode_batch(const tl_decode_seq *seqs, uint32_t n_seq,
                         uint32_t n_head, uint32_t window, float scale,
                         void *stream);

/* tl_attn_decode_batch with RoPE on every session's q and new k row (each at
 * its own position), as tl_attn_rope. */
int tl_attn_decode_batch_rope(const tl_decode_seq *seqs, uint32_t n_seq, uint32_t n_head,
                              uint32_t window, float scale, const tl_rope_params *rope,
                              void *stream);

/* OP_ROPE_NORM (neox = 0) / OP_ROPE_NEOX (neox = 1) in place on x
 * [rows][row_stride] f32, row p at position pos+p. */
int tl_rope(float *x, uint32_t rows, uint32_t row_stride, uint32_t heads,
            uint32_t head_dim, uint32_t rope_dim, uint32_t pos, float theta,
            int neox, void *stream);

/* ---- recurrent-state snapshots on the device ------------------------------
 * graph_state_save / graph_state_load (src/graph.c:368-408) copy every
 * registered state buffer to / from one host snapshot with a cudaMemcpy per
 * buffer.  tl_state_copy does the same between device buffers and a device
 * snapshot in one launch: dir TL_STATE_SAVE concatenates segs[0..n_seg) into
 * snap (in order, each seg's bytes), TL_STATE_LOAD splits snap back into
 * them, TL_STATE_ZERO clears the segments (snap unused; the reset a
 * stateful arch does before a restore, src/graph.c:1443).  Any sizes and
 * alignments; 16-byte aligned segments move 16 bytes per lane. */
#define TL_STATE_SAVE 0
#define TL_STATE_LOAD 1
#define TL_STATE_ZERO 2
typedef struct tl_state_seg {
    void     *ptr;        /* device */
    uint64_t  bytes;
} tl_state_seg;

int tl_state_copy(const tl_state_seg *segs, uint32_t n_seg, void *snap, int dir,
                  void *stream);

/* ---- Q8_0 cache ------------------------------------------------------------
 * A quantized KV cache (the reference's cache is f32, and its notes list a
 * quantized KV cache as missing, REMEMBER.md:18).  Each row of each head is
 * cut into blocks of 32 elements stored in the GGUF Q8_0 form the reference
 * dequantizes (src/quants.c:368-373: value = q * d, q int8, d binary16),
 * with the values and the scales in two planes so every row stays 16-byte
 * aligned:
 *   k, v    int8 [n_kv_head][cap][head_dim]
 *   ks, vs  f16  [n_kv_head][cap][head_dim / 32]
 * Quantization of a block x[32] is the reference's Q8_0 quantizer
 * (src/backend/gpu/gpu.cu:1077-1086): amax = max |x_j|, d = amax / 127,
 * q_j = rint(x_j * (d > 0 ? 1/d : 0)) (ties to even), d stored RNE as
 * binary16.  Inputs are expected finite.  Attention over a Q8_0 cache
 * equals attention over the dequantized values q * d.  No counterpart in
 * the reference's KV API (an added format). */
typedef struct tl_kv_layer_q8 {
    void     *k;          /* device, int8 [n_kv_head][cap][head_dim] */
    void     *v;
    void     *ks;         /* device, f16 [n_kv_head][cap][head_dim/32] */
    void     *vs;
    uint32_t  cap;
    uint32_t  n_kv_head;
    uint32_t  head_dim;   /* 64, 128 or 256 */
    uint32_t  ring;       /* as tl_kv_layer.ring */
} tl_kv_layer_q8;

int tl_kv_layer_alloc_q8(tl_kv_layer_q8 *L, uint32_t cap, uint32_t n_kv_head,
                         uint32_t head_dim, uint32_t ring);
int tl_kv_layer_free_q8(tl_kv_layer_q8 *L);

/* Quantize and write n rows of K and V at slots[pos+i] (as tl_kv_append). */
int tl_kv_append_q8(const tl_kv_layer_q8 *L, const float *k, const float *v,
                    uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                    uint32_t n, void *stream);

/* tl_kv_append_layers over Q8_0 layers (same bytes as per-layer
 * tl_kv_append_q8 calls). */
int tl_kv_append_layers_q8(const tl_kv_layer_q8 *layers, uint32_t n_layer,
                           const float *const *k, const float *const *v, uint32_t kv_stride,
                           const uint32_t *slots, uint32_t pos, uint32_t n, void *stream);

/* Read rows slots[i] of every head: values to k_out/v_out
 * [n][n_kv_head][head_dim] int8, scales to ks_out/vs_out
 * [n][n_kv_head][head_dim/32] f16 bits (device). */
int tl_kv_gather_q8(const tl_kv_layer_q8 *L, const uint32_t *slots, uint32_t n,
                    int8_t *k_out, uint16_t *ks_out, int8_t *v_out, uint16_t *vs_out,
                    void *stream);

/* One session of a batched one-token decode over Q8_0 caches. */
typedef struct tl_decode_seq_q8 {
    tl_kv_layer_q8  layer;
    const uint32_t *slots;    /* device slot table of this session, or NULL */
    uint32_t        pos;      /* position of the new token */
    uint32_t        pad_;
    const float    *q;        /* device [n_head*head_dim] f32 */
    const float    *k;        /* device [n_kv*head_dim] f32 */
    const float    *v;        /* device [n_kv*head_dim] f32 */
    float          *dst;      /* device [n_head*head_dim] f32 */
} tl_decode_seq_q8;

/* tl_attn_decode_batch over Q8_0 caches: one quantizing append launch for
 * every session's new row, then one decode launch for all sessions. */
int tl_attn_decode_batch_q8(const tl_decode_seq_q8 *seqs, uint32_t n_seq, uint32_t n_head,
                            uint32_t window, float scale, void *stream);

/* Row copies across layers (prefix fork / compaction, as tl_kv_copy and
 * tl_kv_copy_between): values and scales of rows src[i] -> dst[i]. */
int tl_kv_copy_q8(const tl_kv_layer_q8 *layers, uint32_t n_layer, const uint32_t *src,
                  const uint32_t *dst, uint32_t n, void *stream);
int tl_kv_copy_between_q8(const tl_kv_layer_q8 *dst_layers, const tl_kv_layer_q8 *src_layers,
                          uint32_t n_layer, const uint32_t *src, const uint32_t *dst,
                          uint32_t n, void *stream);

/* OP_ATTN over a Q8_0 cache: quantize-append the batch rows, then attend
 * (decode-sized batches: the split-K kernel reading the int8 rows; larger
 * ones: the MFMA kernel, which dequantizes its K/V tiles to f16 in LDS). */
int tl_attn_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a, void *stream);
int tl_attn_noappend_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a, void *stream);

/* Fused RoPE over a Q8_0 cache (as tl_attn_rope / tl_kv_append_rope): K is
 * rotated before it is quantized, q as it is staged; the same bits as
 * tl_rope on q and k followed by tl_attn_q8 / tl_kv_append_q8. */
int tl_attn_rope_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a,
                    const tl_rope_params *rope, void *stream);
int tl_kv_append_rope_q8(const tl_kv_layer_q8 *L, const float *k, const float *v,
                         uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                         uint32_t n, const tl_rope_params *rope, void *stream);

/* Measurement aid (no reference counterpart): stream `bytes` of device
 * memory with 16-byte loads, `depth` (1/4/8/16) in flight per lane, over
 * `blocks` workgroups of 256; sink receives blocks*256 words.  Gives the
 * achievable HBM read ceiling the decode roofline is compared with. */
int tl_probe_read(const void *src, uint64_t bytes, uint32_t *sink,
                  uint32_t blocks, uint32_t depth, void *stream);

/* Measurement aid (no reference counterpart): `blocks` workgroups of 256
 * threads, each wave running `iters` x 4 v_mfma_f32_32x32x16_f16 (32768 flops
 * each) on register operands; sink receives blocks*256 floats.  Gives the
 * achievable dense f16 MFMA rate the prefill roofline is compared with. */
int tl_probe_mfma(uint64_t iters, uint32_t blocks, float *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif
