/*
 * tl_prefill.hip — chunked-prefill attention on MFMA (gfx950).
 *
 * Math of op_attn (reference src/backend/cpu/cpu_op.c:1011-1062) for a batch
 * of n rows at positions pos..pos+n-1: row i attends to keys
 * [start_i, pos+i] (causal, start_i = pos+i+1-window when windowed) through
 * the slot table; out = softmax(q.K^T * scale) V.
 *
 * Work decomposition:
 *   A workgroup owns one kv-head, a block of 32*QB query rows and one split
 *   of the key range; its W = G*QB waves each own one q-head of the GQA group
 *   and 32 query rows, so every K/V tile staged in LDS serves G*QB*32 rows.
 *   Per tile of BN keys (64 at head_dim <= 128, 32 at 256):
 *     S^T[key][row] = K . Q^T      v_mfma_f32_32x32x16_f16 per 32-key block,
 *                                  A = K rows from LDS, B = Q (registers, f16,
 *                                  pre-scaled by scale*log2 e); each lane ends
 *                                  up owning one query row and 16 keys of the
 *                                  block, so the row max / sum need one shuffle
 *                                  between the two half-waves.
 *     online softmax in f32 (exp2); mask arithmetic only on tiles that cross
 *                                  the causal diagonal, the window edge or the
 *                                  range end.  Each row's reference mu moves
 *                                  only when a tile's max passes it by more
 *                                  than 2^8 (then O and the sum are rescaled);
 *                                  -mu seeds the QK accumulators, so S - mu
 *                                  leaves the MFMA as is.  P^T is packed to
 *                                  f16 straight from the accumulator
 *                                  registers; the row sum is a dot2 of the
 *                                  packed P with (1, 1).
 *     O^T[d][row] += V^T . P^T     v_mfma_f32_32x32x16_f16 per 16 keys,
 *                                  A = V^T read from the row-major V tile with
 *                                  ds_read_b64_tr_b16 (a 4x16 -> 16x4 transpose
 *                                  per 16-lane group), B = P^T.  The MFMA's
 *                                  reduction index k is mapped to the keys each
 *                                  lane already holds, so P^T never goes
 *                                  through LDS and V is stored as loaded.
 *   K/V tiles are double-buffered in LDS (one barrier per tile): the next
 *   tile's rows are loaded into registers while the current one is computed
 *   and written to the other buffer afterwards.  Key splits (when the grid
 *   would not fill the chip) write partial (O, max, sum) rows that
 *   attn_merge_kernel combines.
 */
#include "tl_prefill_kernels.h"

TL_PREFILL_PICKER(tl_prefill_fn, false, false)

/* ------------------------------------------------------------------------ */

bool tl_prefill_supported(const LayerView &L, const tl_attn_args *a) {
    if (tl_tune(TL_TUNE_NO_PREFILL) == 1) return false;
    const u32 G = a->n_head / L.n_kv_head;
    return (L.head_dim == 64 || L.head_dim == 128 || L.head_dim == 256) && G >= 1 && G <= 8;
}

/* The prefill kernel for batches of at least TL_PREFILL_MIN_ROWS rows whose
 * rows x visible keys exceed TL_PREFILL_MIN_WORK (or of more than
 * TL_DEC_FOLD_MAX_ROWS rows); smaller ones run on the decode kernel, whose
 * matrix tile folds the rows into its columns.  Measured (f16, 8 or 4
 * kv-heads, head_dim 64-256, us per launch, decode vs prefill kernel): 64
 * rows at 1K keys 16.0 vs 25.6, at 2K 21.0 vs 27.9; 32 rows at 4K 21.4 vs
 * 26.3; 16 rows at 8K 19.5 vs 26.2, 24 rows 27.4 vs 27.0; 32 rows at 8K
 * 46.9 vs 28.0; 16 rows at 16K 49.3 vs 31.8.  The Q8_0 cache's decode tile
 * is dearer per key: 32 rows at 4K 27.1 vs 29.1, 48 rows 56.0 vs 32.4; 16
 * rows at 8K 28.4 vs 30.4, 24 rows 37.5 vs 32.2. */
bool tl_use_prefill(const LayerView &L, const tl_attn_args *a) {
    if (a->n < TL_PREFILL_MIN_ROWS || !tl_prefill_supported(L, a)) return false;
    if (tl_tune(TL_TUNE_NO_PREFILL) == 2) return true;
    const u64 keys = (u64)a->pos + a->n;
    const u64 vis = (a->window && keys > a->window) ? a->window : keys;
    const u64 work = L.q8 ? TL_PREFILL_MIN_WORK_Q8 : TL_PREFILL_MIN_WORK;
    return a->n > TL_DEC_FOLD_MAX_ROWS || (u64)a->n * vis > work;
}

/* query blocks (one 32-row block per wave and q-head) per workgroup: PCfg::QB */
static u32 qblocks(u32 D, u32 G) {
    const u32 wmax = D <= 128 ? 8 : 4;
    return wmax / G ? wmax / G : 1;
}

int tl_launch_prefill(const LayerView &L, const tl_attn_args *a, const RopeCfg &rope,
                      hipStream_t st, bool append) {
    if (append && L.q8) return tl_fail(TL_EINVAL, "prefill: no fused append into a Q8_0 cache");
    const u32 D = L.head_dim, G = a->n_head / L.n_kv_head;
    if (L.q8 && (!L.ks || !L.vs)) return tl_fail(TL_EINVAL, "prefill: a Q8_0 cache needs scales");
    PrefParams p;
    memset(&p, 0, sizeof(p));
    p.k = (const u16 *)L.k;
    p.v = (const u16 *)L.v;
    p.ks = L.ks;
    p.vs = L.vs;
    p.slots = a->slots;
    p.cap = L.cap;
    p.ring = L.ring;
    p.q = a->q;
    p.dst = a->dst;
    p.q_stride = a->q_stride;
    p.pos = a->pos;
    p.n = a->n;
    p.n_head = a->n_head;
    p.n_kv = L.n_kv_head;
    p.window = a->window;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.rope = rope;

    const u32 rows = 32 * qblocks(D, G);
    const u32 nqb = (a->n + rows - 1) / rows;
    int cus = 256;
    {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
    }
    const u32 base = nqb * L.n_kv_head;
    const u32 span = a->pos + a->n;        /* most keys any workgroup sees */
    u32 ns = (u32)((cus + base - 1) / base);
    const u32 max_ns = (span + 511) / 512;  /* keep >= 512 keys per split */
    if (ns > max_ns) ns = max_ns;
    if (ns < 1) ns = 1;
    if (const u32 t = tl_tune(TL_TUNE_PREFILL_SPLITS)) ns = t;
    if (const size_t fixed = tl_workspace_fixed_acc()) {
        /* no-allocation call: as many key splits as the fixed region holds */
        const size_t per_split = (size_t)a->n * a->n_head * D;
        if ((size_t)ns * per_split > fixed) ns = (u32)(fixed / per_split);
        if (ns < 1) ns = 1;
    }
    p.n_split = ns;
    const size_t units = (size_t)L.n_kv_head * ((a->n + TL_PF_ROWS - 1) / TL_PF_ROWS);
    if (ns > 1 || append) {
        TlWorkspace *w;
        size_t parts = ns > 1 ? (size_t)a->n * a->n_head * ns : 0;
        /* fused append: launch counter and unit flags past the decode
         * merge's counters */
        int rc = tl_workspace_get(st, parts * D, parts,
                                  append ? TL_MERGE_CNT_WORDS + TL_PF_CTR_WORDS + units : 0, &w);
        if (rc) return rc;
        if (ns > 1) {
            p.ws_acc = w->acc;
            p.ws_ml = (float2 *)w->ml;
        }
        if (append) {
            p.kin = a->k;
            p.vin = a->v;
            p.kv_stride = a->kv_stride;
            p.ctr = w->cnt + TL_MERGE_CNT_WORDS;
            p.flags = p.ctr + TL_PF_CTR_WORDS;
            const u32 polls = tl_tune(TL_TUNE_PREFILL_APPEND_POLLS);
            p.polls = polls ? polls - 1 : 4096;
        }
    }
    const u32 blocks = base * ns;
    const bool rope_on = rope.rdim != 0;
    const void *fn = L.q8 ? (rope_on ? tl_prefill_fn_q8_rope(D, G) : tl_prefill_fn_q8(D, G))
                          : (rope_on ? tl_prefill_fn_rope(D, G) : tl_prefill_fn(D, G));
    if (!fn) return tl_fail(TL_EINVAL, "prefill: head_dim %u gqa %u", D, G);
    void *args[] = {(void *)&p};
    HIP_TRY(hipLaunchKernel(fn, dim3(blocks), dim3(64 * G * qblocks(D, G)), args, 0, st));
    if (ns == 1) return TL_OK;
    /* combine the key splits (same partial layout as the decode kernel) */
    DecParams mp;
    memset(&mp, 0, sizeof(mp));
    mp.seq[0].dst = a->dst;
    mp.rows_per_seq = a->n;
    mp.n_kv = L.n_kv_head;
    mp.n_head = a->n_head;
    mp.q_stride = a->q_stride;
    mp.n_split = ns;
    mp.ws_acc = p.ws_acc;
    mp.ws_ml = p.ws_ml;
    return tl_launch_merge(mp, a->n, D, st);
}

/* ------------------------------------------------------------------------ */

/* MFMA ceiling probe: every wave runs `iters` rounds of 4 independent
 * v_mfma_f32_32x32x16_f16 chains on register operands (no memory traffic),
 * then folds its accumulators into one word of `sink` so nothing is dead. */
__global__ __launch_bounds__(256) void mfma_probe_kernel(u64 iters, float *sink) {
    const int tid = threadIdx.x;
    half8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)((float)((tid + i) & 7) * 0.125f);
        b[i] = (_Float16)((float)((tid * 3 + i) & 7) * 0.0625f);
    }
    floatx16_t c[4] = {};
    for (u64 it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) s += c[j][e];
    sink[(u64)blockIdx.x * blockDim.x + tid] = s;
}

extern "C" int tl_probe_mfma(uint64_t iters, uint32_t blocks, float *sink, void *stream) {
    if (!sink || blocks == 0 || iters == 0) return tl_fail(TL_EINVAL, "probe: bad arguments");
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (u64)iters,
                       sink);
    HIP_TRY(hipGetLastError());
    return TL_OK;
}
