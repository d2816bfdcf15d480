/*
 * tl_decode.hip — split-K decode attention over the slot-indexed f16 or
 * Q8_0 cache.
 *
 * Math of op_attn (reference src/backend/cpu/cpu_op.c:1011-1062): for each
 * q-head h and batch row r, n_keys = pos + r + 1, visible keys
 * [start, n_keys) with start = n_keys - window when window > 0 and
 * n_keys > window (cpu_op.c:1019-1022); s_t = (K[h/gqa][slot_t] . q) * scale;
 * out = softmax(s) @ V.
 *
 * Work decomposition (gfx950, wave64): attn_decode_ring_kernel.
 *   grid = n_split x (rows x n_kv_head) workgroups of 8 waves, one per CU,
 *   mapped so that all splits of one (row, kv-head) group run on one XCD.  A
 *   workgroup streams one contiguous chunk of keys of one kv-head and serves
 *   every q-head of the GQA group from the same K/V bytes, so each cache byte
 *   is read from HBM once per step instead of gqa times.  The chunk's slot
 *   indices and q are staged in LDS first.
 *   Each wave owns every 8th tile (4 KB of K + 4 KB of V) and streams it
 *   through a 2-stage LDS ring filled by non-temporal LDS-direct loads.
 *   Scores: v_dot2_f32_f16 of the f16 K row with q (pre-scaled by
 *   scale*log2(e), rounded to f16), reduced over the key's lanes with DPP;
 *   each lane group keeps its own (l, acc) against a wave-uniform running
 *   max that moves only when a score exceeds it by 2^8; p is rounded to f16
 *   and PV runs as v_dot2 over key pairs of V (head_dim 256, Q8_0).  Up to
 *   head_dim 128 the tile runs on the matrix cores instead (mfma_tile:
 *   S^T = K.Q^T and O^T += V^T.P^T as v_mfma 16x16 tiles, the GQA heads as
 *   the columns, one head column's softmax state per lane).
 *   States merge across waves through LDS and across splits in the last
 *   workgroup of the group to finish (partials written with device-coherent
 *   stores, a per-group atomic counter that this workgroup resets), or in a
 *   separate merge launch when the partials exceed that workgroup's LDS.
 *   The fused append of decode rows: the split-0 workgroup of row 0 writes
 *   the new K/V rows; workgroups that need a new key convert it from the f32
 *   input into LDS.
 *   Q8_0 instance (Q8): int8 rows and their f16 block scales stream through
 *   a 4-stage ring in the same LDS (values as loaded, scales by 32-lane
 *   dword loads); int8 -> f16 by byte permutes (exact), scores scaled per
 *   key block in f32, V dequantized to f16 for the PV v_dot2 (ring_tile_q8);
 *   no fused append (the quantizing append is its own launch).
 */
#include "tl_decode_kernels.h"

#include <atomic>
#include <mutex>

template <int D>
static DecKernel pick_kernel(int G, bool rope, bool q8, bool mf) {
    if (q8) return tl_pick_decode_q8(D, G, rope, mf);   /* tl_decode_q8.hip */
    constexpr int NT = 64 * TL_RING_WAVES;
    switch (G) {
#define TL_CASE(g)                                                                            \
    case g:                                                                                   \
        if (mf) {                                                                             \
            if (rope) return {(const void *)attn_decode_ring_kernel<D, g, true, false, true>, 4096, NT}; \
            return {(const void *)attn_decode_ring_kernel<D, g, false, false, true>, 4096, NT};         \
        }                                                                                     \
        if (rope) return {(const void *)attn_decode_ring_kernel<D, g, true, false, false>, 4096, NT};  \
        return {(const void *)attn_decode_ring_kernel<D, g, false, false, false>, 4096, NT};
        TL_CASE(1) TL_CASE(2) TL_CASE(3) TL_CASE(4)
        TL_CASE(5) TL_CASE(6) TL_CASE(7) TL_CASE(8)
#undef TL_CASE
    default:
        return {nullptr, 0, 0};
    }
}

/* override `key` when set, else the automatic value */
static u32 tuned(int key, u32 dflt) {
    const u32 v = tl_tune(key);
    return v ? v : dflt;
}

/* CUs of the current device (cached per device; launches from several host
 * threads may fill the cache at once and store the same value) */
static int cu_count() {
    static std::atomic<int> cus[16];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

/* resident workgroups per CU of a kernel (cached per entry point, under a
 * lock: several host threads may launch at once) */
static int resident_per_cu(const void *fn, int threads) {
    static std::mutex mu;
    static const void *keys[64];
    static int vals[64];
    static int n = 0;
    {
        std::lock_guard<std::mutex> lk(mu);
        for (int i = 0; i < n; i++)
            if (keys[i] == fn) return vals[i];
    }
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, threads, 0) != hipSuccess || b < 1) b = 1;
    std::lock_guard<std::mutex> lk(mu);
    if (n < 64) {
        keys[n] = fn;
        vals[n++] = b;
    }
    return b;
}

/* Pick the kernel, the split count and launch.  max_vis = most visible keys
 * of any row.  The grid is one full wave of resident workgroups (every CU
 * gets the same number of equal key chunks).  The partials of a split group
 * are merged by the group's last workgroup when they fit its LDS, else by
 * attn_merge_kernel. */
static int launch_decode(DecParams &p, u32 n_rows_total, u32 head_dim, u32 G, u32 max_vis,
                         hipStream_t st, bool q8, bool fold_rows) {
    if (q8 && p.rope.rdim && p.rows_per_seq > TL_DEC_Q8_ROPE_NEW) {
        for (u32 i = 0; i < TL_MAX_BATCH_SEQ; i++)
            if (p.seq[i].kin)
                return tl_fail(TL_EINVAL, "decode: fused append with RoPE into a Q8_0 cache: "
                                          "at most %d rows", TL_DEC_Q8_ROPE_NEW);
    }
    DecKernel K;
    /* tiles on the matrix cores where measured faster (8 kv-heads, 1K and
     * 32K keys, gqa 1-8): the f16 cache at head_dim 64 and 128 from gqa 2
     * (gqa 8: 16.3 vs 38.3 us at 32K keys; gqa 1 even); the Q8_0 cache at
     * head_dim 64 from gqa 2 and at 128 from gqa 4 (gqa 8: 26.9 vs 57.9 us;
     * with two ring tiles per softmax chain the matrix tile takes 24.3 vs
     * 24.65 us at gqa 4 and 8 kv-heads, 16.4 vs 17.9 at 4 kv-heads; gqa 1
     * stays on the vector tile: 17.7 vs 25.9 us).  At head_dim 256 (8-key
     * tiles, half of each 16-key block padding) the vector tile is faster
     * (config 5, gqa 2: 13.1 vs 13.4 us per launch). */
    const u32 tile_sel = tl_tune(TL_TUNE_DECODE_MFMA);
    /* with several batch rows the matrix tile folds up to 16 / gqa of them
     * (8 / gqa at head_dim 256) into its columns and reads K/V once for all,
     * where the vector tile reads them once per row: folding wins at every
     * head_dim and cache type (measured at 32K keys: MHA head_dim 128, 8
     * rows: 26.7 vs 128.6 us; Q8_0 head_dim 128, gqa 1, 4 rows: 24.7 vs
     * 46.2 us; head_dim 256, gqa 4, 2 rows: 28.4 vs 45.9 us), so any fold
     * takes the matrix tile */
    const u32 rows_in = p.rows_per_seq ? p.rows_per_seq : 1u;
    const u32 rmax = (head_dim == 256 ? 8u : 16u) / G;
    const bool can_fold = fold_rows && rows_in > 1 && rmax > 1 &&
                          !tl_tune(TL_TUNE_DECODE_MERGE_KERNEL) && tl_tune(TL_TUNE_DECODE_ROWS) != 1;
    const bool mf_auto = can_fold ||
                         (head_dim == 64 ? G >= 2 : head_dim == 128 ? G >= (q8 ? 4u : 2u) : false);
    const bool mf = tile_sel == 2 || (tile_sel != 1 && mf_auto);
    switch (head_dim) {
    case 64: K = pick_kernel<64>((int)G, p.rope.rdim != 0, q8, mf); break;
    case 128: K = pick_kernel<128>((int)G, p.rope.rdim != 0, q8, mf); break;
    case 256: K = pick_kernel<256>((int)G, p.rope.rdim != 0, q8, mf); break;
    default: return tl_fail(TL_EINVAL, "head_dim %u", head_dim);
    }
    if (!K.fn) return tl_fail(TL_EINVAL, "gqa ratio %u unsupported (1..8)", G);
    const u32 tk = (u32)K.tile_bytes / (2 * head_dim);   /* keys per wave tile */
    /* two workgroups per CU: measured best on MI355X for both tile sizes
     * (one resident wave of workgroups; more per CU only shortens chunks) */
    int per_cu = resident_per_cu(K.fn, K.threads);
    if (per_cu > 2) per_cu = 2;
    const u32 target = tuned(TL_TUNE_DECODE_WGS, (u32)(per_cu * cu_count()));
    /* matrix-core tile: R batch rows of a session share each workgroup
     * group (their heads side by side as MFMA columns, R x gqa <= 16, 8 at
     * head_dim 256), so the rows read each K/V byte once instead of R
     * times; their partials are merged inside the launch */
    const u32 rows = p.rows_per_seq ? p.rows_per_seq : 1u;
    u32 R = 1;
    if (fold_rows && mf && rows > 1 && !tl_tune(TL_TUNE_DECODE_MERGE_KERNEL)) {
        const u32 most = (head_dim == 256 ? 8u : 16u) / G;
        R = tuned(TL_TUNE_DECODE_ROWS, most);
        if (R > most) R = most;
        if (R > rows) R = rows;
        if (R < 1) R = 1;
    }
    if (R > 1 && p.window) max_vis += R - 1;   /* the rows' windows start apart */
    u64 n_groups = (u64)(n_rows_total / rows) * ((rows + R - 1) / R) * p.n_kv;
    /* splits per group: as many as fill the resident workgroups, never more
     * (a grid a few workgroups past one resident wave runs a second round
     * for them) */
    u32 n_split = n_groups < target ? (u32)(target / n_groups) : 1u;
    const u32 waves = (u32)K.threads / 64;
    /* fewest keys per split: a tile for every wave at head_dim 128, for half
     * of them at 64 and 256, at most 128 keys (measured: head_dim 64, P =
     * 700: 128 keys per split 8.8 us vs 9.5 us at 256, and fewer make the
     * merge dearer than the shorter chunks save; head_dim 256, the 1024-key
     * window of config 5's local layers: 32 keys 12.1 us per launch on
     * average vs 12.55 at 64) */
    const u32 min_tiles = head_dim == 128 ? waves : waves / 2;
    const u32 min_keys = tuned(TL_TUNE_DECODE_MIN_KEYS, min_tiles * tk < 128 ? min_tiles * tk : 128);
    const u32 max_split = (max_vis + min_keys - 1) / min_keys;
    /* keys per workgroup: limited by the slot-table staging only (u32
     * indices, or u16 ones in the matrix-core f16 instances when every
     * staged pool has at most 65536 rows); launches without a slot table
     * stage nothing */
    bool any_staged = false, s16_ok = mf && !q8;
    for (u32 i = 0; i < n_rows_total / rows && i < TL_MAX_BATCH_SEQ; i++)
        if (p.seq[i].slots && !p.seq[i].ring) {
            any_staged = true;
            if (p.seq[i].cap > 65536u) s16_ok = false;
        }
    const u32 max_chunk = !any_staged ? 0xffffffffu : s16_ok ? TL_DEC_MAX_CHUNK16 : TL_DEC_MAX_CHUNK;
    const u32 min_split = (u32)(((u64)max_vis + max_chunk - 1) / max_chunk);
    if (n_split > max_split) n_split = max_split;
    if (n_split < min_split) {
        /* the chunk limit needs more workgroups than one resident round:
         * fill whole rounds evenly instead of leaving a partial last round
         * of full-length chunks */
        n_split = min_split;
        const u64 wgs = (u64)n_split * n_groups;
        if (wgs > target) {
            const u64 rounds = (wgs + target - 1) / target;
            const u64 even = rounds * target / n_groups;
            if (even > n_split) n_split = (u32)(even < max_split ? even : max_split);
        }
    }
    if (n_split < 1) n_split = 1;
    const u32 chunk = (max_vis + n_split - 1) / n_split;
    n_split = (max_vis + chunk - 1) / chunk;
    if (n_split > TL_MERGE_MAX_SPLIT)
        return tl_fail(TL_EINVAL, "decode: %u keys need %u splits", max_vis, n_split);
    p.chunk = chunk;
    p.n_split = n_split;
    if (any_staged && chunk > TL_DEC_MAX_CHUNK) {
        /* measured: the u16 staging chosen at run time cost every launch
         * 0.4 us, so it is an instance of its own */
        K = tl_pick_decode_s16((int)head_dim, (int)G, p.rope.rdim != 0);
        if (!K.fn) return tl_fail(TL_EINVAL, "decode: no u16-slot instance for gqa %u", G);
    }
    p.counters = nullptr;
    p.dist = 0;
    const bool in_kernel_merge = n_split > 1 && R * G * n_split <= 2048 &&
                                 n_groups <= TL_MERGE_MAX_GROUPS &&
                                 !tl_tune(TL_TUNE_DECODE_MERGE_KERNEL);
    if (R > 1 && n_split > 1 && !in_kernel_merge) {
        /* the separate merge launch reads one row per group: plan again */
        if (p.window) max_vis -= R - 1;
        return launch_decode(p, n_rows_total, head_dim, G, max_vis, st, q8, false);
    }
    p.rows_per_wg = R;
    if (n_split > 1) {
        /* every split merges a slice of the output (dist) when there are
         * enough splits to share the merge (measured: with 8 or fewer the
         * last split alone is faster) and all of the grid is resident at
         * once (a split waits, bounded, for the rest of its group) */
        const u64 resident = (u64)resident_per_cu(K.fn, K.threads) * cu_count();
        p.dist = in_kernel_merge && n_split >= 12 && n_split <= TL_MERGE_MAX_SPLIT_DIST &&
                 (u64)n_split * n_groups <= resident && !tl_tune(TL_TUNE_DECODE_SINGLE_MERGE);
        TlWorkspace *w;
        size_t parts = (size_t)n_groups * R * G * n_split;
        /* dist: one (m, l, epoch, ~epoch) record of 16 bytes per partial */
        int rc = tl_workspace_get(st, parts * head_dim, p.dist ? 2 * parts : parts,
                                  in_kernel_merge ? TL_MERGE_CNT_WORDS : 0, &w);
        if (rc) return rc;
        p.ws_acc = w->acc;
        p.ws_ml = (float2 *)w->ml;
        if (in_kernel_merge) {
            p.counters = w->cnt;
            const u32 polls = tl_tune(TL_TUNE_DECODE_MERGE_POLLS);
            p.polls = polls ? polls - 1 : TL_MERGE_SPIN;
        }
    }
    void *args[] = {(void *)&p};
    HIP_TRY(hipLaunchKernel(K.fn, dim3(n_split * (u32)n_groups), dim3(K.threads), args, 0, st));
    if (n_split == 1 || in_kernel_merge) return TL_OK;
    return tl_launch_merge(p, n_rows_total, head_dim, st);
}

int tl_launch_decode(DecParams &p, u32 n_rows_total, u32 head_dim, u32 G,
                     u32 max_vis, hipStream_t st, bool q8) {
    return launch_decode(p, n_rows_total, head_dim, G, max_vis, st, q8, true);
}

int tl_launch_merge(const DecParams &p, u32 n_rows_total, u32 head_dim, hipStream_t st) {
    if (p.n_split > TL_MERGE_MAX_SPLIT) return tl_fail(TL_EINVAL, "merge: %u splits", p.n_split);
    const u32 n_out = n_rows_total * p.n_head;
    const dim3 mg((u32)(((u64)n_out * (head_dim / 4) + 255) / 256));
    MergeParams m;
    for (u32 i = 0; i < TL_MAX_BATCH_SEQ; i++) m.dst[i] = p.seq[i].dst;
    m.rows_per_seq = p.rows_per_seq;
    m.n_head = p.n_head;
    m.q_stride = p.q_stride;
    m.n_split = p.n_split;
    m.ws_acc = p.ws_acc;
    m.ws_ml = p.ws_ml;
    switch (head_dim) {
    case 64: hipLaunchKernelGGL(attn_merge_kernel<64>, mg, dim3(256), 0, st, m, n_out); break;
    case 128: hipLaunchKernelGGL(attn_merge_kernel<128>, mg, dim3(256), 0, st, m, n_out); break;
    case 256: hipLaunchKernelGGL(attn_merge_kernel<256>, mg, dim3(256), 0, st, m, n_out); break;
    default: return tl_fail(TL_EINVAL, "merge: head_dim %u", head_dim);
    }
    HIP_TRY(hipGetLastError());
    return TL_OK;
}
