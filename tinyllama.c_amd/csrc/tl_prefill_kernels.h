/* tl_prefill_kernels.h — the chunked-prefill MFMA kernel (template) and its
 * device helpers, shared by the translation units that instantiate it:
 * tl_prefill.hip (f16 cache, launch code) and tl_prefill_rope.hip,
 * tl_prefill_q8.hip, tl_prefill_q8_rope.hip (one (RoPE, Q8_0) variant each,
 * so the instances build in parallel).  The design is described in
 * tl_prefill.hip. */
#pragma once
#include "tl_common.h"
#include "tl_internal.h"

#include <stdlib.h>
#include <string.h>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

template <int D, int G>
struct PCfg {
    static constexpr int WMAX = (D <= 128) ? 8 : 4;
    static constexpr int QB = (WMAX / G) > 0 ? (WMAX / G) : 1;   /* 32-row query blocks */
    static constexpr int W = G * QB;                              /* waves */
    static constexpr int ROWS = 32 * QB;                          /* query rows per WG */
    static constexpr int BN = (D <= 128) ? 64 : 32;               /* keys per tile */
};

#define TL_PF_VPAD 32      /* V row padding in halves: a transpose read's 16-lane
                              group hits 4 rows x 32 B at row steps of 16 (or 48)
                              banks, and the group 32 B to its right fills the
                              gaps, so two groups cover all 64 banks once
                              (16 halves: 2-way conflicts, 4% slower) */

TL_DEV half8_t h8_from_u4(uint4 v) { return __builtin_bit_cast(half8_t, v); }

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef u32 pf_u2v __attribute__((vector_size(8)));
TL_DEV half2_t pf_h2(u32 v) { return __builtin_bit_cast(half2_t, v); }

#define TL_PF_RESCALE 8.0f /* lazy rescale threshold of the running max (log2) */

TL_DEV u32 pack2(float a, float b) { return pack_f16x2_fast(a, b); }

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

/* ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
 * (i & 3) of the 4-half vector addressed by lane 4e + (i >> 2), for e = 0..3.
 * With lane j addressing row (j >> 2), column 4 (j & 3) of a 4 x 16 block,
 * lane i receives column i of rows 0..3: a 4x16 -> 16x4 transpose. */
TL_DEV uint2 ld_tr16(const _Float16 *lds_ptr) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t *)(lds_ptr));
    const u32 lo = (u32)(u16)v.x | ((u32)(u16)v.y << 16);
    const u32 hi = (u32)(u16)v.z | ((u32)(u16)v.w << 16);
    return make_uint2(lo, hi);
}

template <int D, int G, bool ROPE, bool Q8>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * PCfg<D, G>::W, 64 * PCfg<D, G>::W))) void attn_prefill_kernel(const PrefParams p) {
    using C = PCfg<D, G>;
    constexpr int W = C::W, ROWS = C::ROWS, BN = C::BN;
    constexpr int T = 64 * W;
    constexpr int CPR = D / 8;           /* 16-byte chunks per row */
    constexpr int KS = D / 16;           /* k-steps of the QK MFMA */
    constexpr int DB = D / 32;           /* 32-row d-blocks of O^T */
    constexpr int KB = BN / 32;          /* 32-key blocks of S^T per tile */
    constexpr int UNITS = BN * CPR;      /* 16-byte units per K (or V) tile */
    constexpr int UPT = (UNITS + T - 1) / T;
    constexpr int VS = D + TL_PF_VPAD;   /* V row stride (halves) */
    constexpr float NEG_INF = -__builtin_huge_valf();

    __shared__ uint4 s_k[2][UNITS];                      /* K rows, chunk-swizzled */
    __shared__ __attribute__((aligned(16))) _Float16 s_v[2][BN * VS];   /* V rows, row-major */

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5;             /* half-wave */
    const int lr = lane & 31;

    /* ---- fused append ----
     * The batch rows go into the cache at the launch's start, before any
     * workgroup reads the cache: workgroup b writes units b, b + grid, ...
     * (a unit = TL_PF_ROWS rows of one kv-head, the same conversion and
     * rotation as kv_append_kernel), waits for its stores, and sets the
     * units' flags to this launch's epoch (below: await_batch).  Stores and
     * flags cross XCDs with the device-coherent policy. */
    const bool fa = !Q8 && p.kin != nullptr;
    const u32 n_units = (p.n + TL_PF_ROWS - 1) / TL_PF_ROWS;
    u32 epoch = 0;
    __shared__ u32 s_direct;
    /* unit (kvh_u, rows r0..r0+TL_PF_ROWS) of the batch into the cache */
    auto write_unit = [&](u32 kvh_u, u32 r0) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rkw = buf_rsrc(p.k), rvw = buf_rsrc(p.v);
        constexpr int IPU = TL_PF_ROWS * CPR;             /* 16-byte items per unit */
        for (int i = tid; i < IPU; i += T) {
            const u32 row = r0 + (u32)(i / CPR), c = (u32)(i % CPR);
            if (row >= p.n) continue;
            const u32 key = p.pos + row;
            const u32 ph = p.ring ? key % p.ring : (p.slots ? p.slots[key] : key);
            if (ph >= p.cap) continue;
            const float *kr = p.kin + (u64)row * p.kv_stride + (u64)kvh_u * D;
            const float *vr = p.vin + (u64)row * p.kv_stride + (u64)kvh_u * D;
            const uint4 kk = ROPE ? cvt8_rope(kr, c * 8, key, p.rope.rdim, p.rope.theta,
                                              p.rope.neox)
                                  : cvt8_f16(kr + c * 8);
            const uint4 vv = cvt8_f16(vr + c * 8);
            const u32 off = (u32)((((u64)kvh_u * p.cap + ph) * D + c * 8) * 2);
            __builtin_amdgcn_raw_buffer_store_b128(u32x4v_t{kk.x, kk.y, kk.z, kk.w}, rkw, off, 0,
                                                   TL_SC1);
            __builtin_amdgcn_raw_buffer_store_b128(u32x4v_t{vv.x, vv.y, vv.z, vv.w}, rvw, off, 0,
                                                   TL_SC1);
        }
    };
    if (fa) {
        epoch = __builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(p.ctr), 0u, 0, TL_SC1) + 1u;
        for (u32 u = blockIdx.x; u < p.n_kv * n_units; u += gridDim.x)
            write_unit(u / n_units, (u % n_units) * TL_PF_ROWS);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (tid == 0) s_direct = 0u;
        __syncthreads();
        for (u32 u = blockIdx.x + (u32)tid * gridDim.x; u < p.n_kv * n_units;
             u += (u32)T * gridDim.x)
            __hip_atomic_store(&p.flags[u], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    /* block -> (K/V range x = kvh * n_split + split, query block); blocks that
     * read the same K/V range sit on the same XCD (block b runs on XCD b % 8) */
    const u32 nx = p.n_kv * p.n_split;
    const u32 x = blockIdx.x % nx, qblk = blockIdx.x / nx;
    const u32 kvh = x / p.n_split, split = x % p.n_split;

    const int g = wave % G, qsub = wave / G;
    const u32 hq = kvh * G + g;
    const u32 qb0 = qblk * ROWS;
    const u32 my_q = qb0 + qsub * 32 + lr;           /* lane's query row */
    const bool row_ok = my_q < p.n;
    const u32 qpos = p.pos + my_q;
    /* the wave's first and last valid query positions */
    const u32 wq0 = p.pos + qb0 + qsub * 32;
    const u32 wq1 = p.pos + min(qb0 + qsub * 32 + 31, p.n - 1);

    /* key range of the workgroup, then of this split */
    const u32 wg_last = min(p.pos + qb0 + ROWS, p.pos + p.n);
    const u32 first_pos = p.pos + qb0;
    const u32 wg_first = (p.window && first_pos + 1 > p.window) ? first_pos + 1 - p.window : 0;
    const u32 span = wg_last - wg_first;
    u32 chunk = (span + p.n_split - 1) / p.n_split;
    chunk = (chunk + BN - 1) / BN * BN;
    const u32 ks = wg_first + split * chunk;
    const u32 ke = min(ks + chunk, wg_last);
    /* keys this lane's row may see, inside the split's range: [klo, khi) */
    const u32 khi = row_ok ? min(ke, qpos + 1) : 0u;
    const u32 klo = (p.window && qpos + 1 > p.window) ? qpos + 1 - p.window : 0u;

    /* Q operand: lane holds Q[row lr][16s + 8h .. +8] (RoPE'd when p.rope is
     * set), f16, log2-scaled */
    half8_t qop[KS];
    {
        const float *qrow = p.q + (u64)(row_ok ? my_q : 0) * p.q_stride + (u64)hq * D;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            float t[8];
            load8_rope(qrow, 16 * s + 8 * h, qpos, ROPE ? p.rope.rdim : 0u, p.rope.theta,
                       p.rope.neox, t);
            const float sc = row_ok ? p.scale_log2 : 0.f;
            uint4 u = make_uint4(pack2(t[0] * sc, t[1] * sc), pack2(t[2] * sc, t[3] * sc),
                                 pack2(t[4] * sc, t[5] * sc), pack2(t[6] * sc, t[7] * sc));
            qop[s] = h8_from_u4(u);
        }
    }

    floatx16_t o[DB];
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[b][r] = 0.f;
    /* m: running max reference (NEG_INF until the row sees a key), mu: the
     * same or 0, held negated in every bias lane */
    float m = NEG_INF, mu = 0.f, lsum = 0.f;
    floatx16_t bias = {};
    const half2_t ones2 = {(_Float16)1.0f, (_Float16)1.0f};

    const u16 *Kb = p.k + (u64)kvh * p.cap * D;
    const u16 *Vb = p.v + (u64)kvh * p.cap * D;
    /* Q8_0 cache: int8 rows and one f16 scale per 32 elements */
    const uint8_t *K8 = (const uint8_t *)p.k + (u64)kvh * p.cap * D;
    const uint8_t *V8 = (const uint8_t *)p.v + (u64)kvh * p.cap * D;
    const u16 *Ksc = Q8 ? p.ks + (u64)kvh * p.cap * (D / 32) : nullptr;
    const u16 *Vsc = Q8 ? p.vs + (u64)kvh * p.cap * (D / 32) : nullptr;

    /* register staging, AHEAD tiles ahead of the compute (and the slot
     * table one tile further).  Unit u = tid + j*T -> row u / CPR, chunk
     * u % CPR; rows past ke load zeros.  A Q8_0
     * cache's units are held raw (8 int8 and their block's scale) and
     * dequantized on the LDS write, with two register sets at head_dim
     * <= 128: a tile's loads are issued one iteration before the iteration
     * that converts and writes it (measured: 482 -> 363 us for the last
     * config-4 chunk).  The f16 path keeps one set (a second one measured
     * no faster and costs occupancy at head_dim 64). */
    constexpr int AHEAD = (Q8 && D <= 128) ? 2 : 1;
    uint4 rk[AHEAD][UPT], rv[AHEAD][UPT];
    /* physical rows of this thread's units of the next tile to load: read
     * from the slot table one tile step before the tile's own loads, so the
     * slot round trip never stalls a step */
    u32 rows_next[UPT];
    /* branch-free slot reads (buffer loads: offsets past the table, and every
     * read when there is none, return 0), so nothing waits for them before
     * their use a step later */
    const __amdgpu_buffer_rsrc_t rslots = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.slots, (short)0, (p.slots && !p.ring) ? (int)(ke * 4u) : 0, 0x00020000);
    /* this kv head's K and V rows as buffer resources (f16 cache; the
     * launcher keeps cap * D * 2 within 32 bits, a multiple of 128, so at
     * most 0xffffff80: below the 0xfffffff0 offset that marks a unit to
     * zero-fill) */
    const int head_bytes = (int)(u32)((u64)p.cap * D * (Q8 ? 1 : 2));
    const __amdgpu_buffer_rsrc_t rsk = __builtin_amdgcn_make_buffer_rsrc(
        Q8 ? (void *)K8 : (void *)Kb, (short)0, head_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc(
        Q8 ? (void *)V8 : (void *)Vb, (short)0, head_bytes, 0x00020000);
    /* Q8_0 scale planes: cap * D / 16 bytes per head */
    const __amdgpu_buffer_rsrc_t rsks = __builtin_amdgcn_make_buffer_rsrc(
        (void *)Ksc, (short)0, Q8 ? (int)(p.cap * (D / 16)) : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsvs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)Vsc, (short)0, Q8 ? (int)(p.cap * (D / 16)) : 0, 0x00020000);
    auto fetch_rows = [&](u32 tb) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * T;
            const u32 key = tb + (u32)(u / CPR);
            rows_next[j] = __builtin_amdgcn_raw_buffer_load_b32(rslots, key * 4u, 0, 0);
        }
    };
    /* fused append: a workgroup whose keys reach the batch rows waits
     * (bounded) for the flags of every unit of its kv-head up to its last
     * key; units whose flag does not come (a writer not resident) it writes
     * itself (the same bytes).  Its tile loads stay plain: no CU or L2 of
     * this launch has read a batch row's cache lines before its flag (a row
     * is whole 128-byte lines, its slot holds no older position read here,
     * and the launch starts with the caches invalidated), and the writers'
     * stores were written through before their flags were set. */
    auto await_batch = [&]() __attribute__((always_inline)) {
        const u32 need = (wg_last - p.pos + TL_PF_ROWS - 1) / TL_PF_ROWS;
        if ((u32)tid < need) {
            const u32 *fl = p.flags + kvh * n_units + (u32)tid;
            bool ok = false;
            for (u32 it = 0; it < p.polls && !ok; it++) {
                if (it) __builtin_amdgcn_s_sleep(4);
                ok = __hip_atomic_load(fl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
            }
            if (!ok) s_direct = 1u;
        }
        __syncthreads();
        if (s_direct) {
            for (u32 b = 0; b < need; b++) write_unit(kvh, b * TL_PF_ROWS);
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
    };
    auto load_tile = [&](u32 tb, int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * T;
            const int row = u / CPR, c = u % CPR;
            const u32 key = tb + row;
            if constexpr (!Q8) {
                /* buffer loads: an offset past the head's rows (the unit
                 * beyond the tile, keys past ke, a slot past cap) reads 0 */
                u32 ph = p.ring ? key % p.ring : (p.slots ? rows_next[j] : key);
                const u32 off = (u < UNITS && key < ke && ph < p.cap) ? (ph * D + c * 8) * 2u
                                                                      : 0xfffffff0u;
                rk[s][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsk, off, 0, 0));
                rv[s][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsv, off, 0, 0));
            } else {
                /* the same for the int8 values and their block's scale: a
                 * unit out of range reads zero values and a zero scale */
                const u32 ph = p.ring ? key % p.ring : (p.slots ? rows_next[j] : key);
                const bool ok = u < UNITS && key < ke && ph < p.cap;
                const u32 off = ok ? ph * D + c * 8 : 0xfffffff0u;
                const u32 soff = ok ? (ph * (D / 32) + c / 4) * 2u : 0xfffffff0u;
                const pf_u2v kq = __builtin_amdgcn_raw_buffer_load_b64(rsk, off, 0, 0);
                const pf_u2v vq = __builtin_amdgcn_raw_buffer_load_b64(rsv, off, 0, 0);
                const u32 ks = __builtin_amdgcn_raw_buffer_load_b16(rsks, soff, 0, 0);
                const u32 vs = __builtin_amdgcn_raw_buffer_load_b16(rsvs, soff, 0, 0);
                rk[s][j] = make_uint4(kq[0], kq[1], ks, 0);
                rv[s][j] = make_uint4(vq[0], vq[1], vs, 0);
            }
        }
    };
    auto store_tile = [&](int buf, int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * T;
            if (u < UNITS) {
                const int row = u / CPR, c = u % CPR;
                uint4 kk = rk[s][j], vv = rv[s][j];
                if constexpr (Q8) {
                    kk = q8_dequant8(make_uint2(kk.x, kk.y), kk.z);
                    vv = q8_dequant8(make_uint2(vv.x, vv.y), vv.z);
                }
                s_k[buf][row * CPR + (c ^ (row % CPR))] = kk;
                *(uint4 *)&s_v[buf][row * VS + c * 8] = vv;
            }
        }
    };

    /* transpose-read coordinates of this lane (16-lane group gi, lane i) */
    const int gi = lane >> 4, li = lane & 15;
    const int tr_row = li >> 2;                       /* + 4h (+8) + 16 kb4 */
    const int tr_col = 16 * (gi & 1) + 4 * (li & 3);  /* + 32 b */

    /* the workgroup reads batch rows: all their units must be in the cache
     * before its first load (the writers published at their start) */
    if (fa && ke > p.pos) await_batch();
    if (ks < ke) {
        fetch_rows(ks);
        load_tile(ks, 0);
        store_tile(0, 0);
        if (ks + BN < ke) fetch_rows(ks + BN);
        if (AHEAD == 2 && ks + BN < ke) {
            load_tile(ks + BN, AHEAD - 1);
            if (ks + 2 * BN < ke) fetch_rows(ks + 2 * BN);
        }
    }
    __syncthreads();
    /* one tile: LDS buffer `buf` holds it, register set `sl` receives the
     * tile two ahead, set sl ^ 1 (loaded an iteration ago) holds the next
     * tile, written to the other buffer at the end */
    auto tile_step = [&](u32 tb, int buf, int sl) __attribute__((always_inline)) {
        if constexpr (AHEAD == 2) {
            if (tb + 2 * BN < ke) load_tile(tb + 2 * BN, sl);
            if (tb + 3 * BN < ke) fetch_rows(tb + 3 * BN);
        } else {
            if (tb + BN < ke) load_tile(tb + BN, 0);
            if (tb + 2 * BN < ke) fetch_rows(tb + 2 * BN);
        }
        const uint4 *sk = s_k[buf];
        const _Float16 *sv_t = s_v[buf];

        /* S^T - mu = K . Q^T + bias per 32-key block (the accumulators start
         * at -mu, this row's running reference): lane holds keys
         * 32 kb + 8(r/4) + 4h + r%4 of query lr */
        floatx16_t sacc[KB];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int krow = 32 * kb + lr;
            sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                h8_from_u4(sk[krow * CPR + (h ^ (krow % CPR))]), qop[0], bias, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < KS; s++) {
                const int c = 2 * s + h;
                const half8_t a = h8_from_u4(sk[krow * CPR + (c ^ (krow % CPR))]);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qop[s], sacc[kb], 0, 0, 0);
            }
        }

        /* mask (only tiles that cross a boundary; visible keys of this lane's
         * row are [klo, khi)) + online softmax.  The reference mu is raised
         * only when the tile's max exceeds it by more than TL_PF_RESCALE
         * (log2 units): then O and the sum are rescaled and the bias moved;
         * otherwise P = 2^(s - mu) <= 2^TL_PF_RESCALE needs no subtraction */
        const bool full = tb + BN <= ke && tb + BN - 1 <= wq0 &&
                          (!p.window || tb + p.window > wq1);
        float sv[KB][16];
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) sv[kb][r] = sacc[kb][r];
        if (!full) {
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const u32 key = tb + 32 * kb + 8 * (r / 4) + 4 * h + (r % 4);
                    sv[kb][r] = ((key >= klo) & (key < khi)) ? sv[kb][r] : NEG_INF;
                }
        }
        float mt = NEG_INF;
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) mt = fmaxf(mt, sv[kb][r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32));          /* relative to mu */
        const bool need = mt + mu > m + TL_PF_RESCALE;
        if (__builtin_amdgcn_ballot_w64(need)) {
            const float d = need ? mt : 0.f;         /* new mu - mu */
            const float alpha = (m == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(-d);
            if (need) {
                mu += d;
                m = mu;
            }
            lsum *= alpha;
#pragma unroll
            for (int b = 0; b < DB; b++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[b][r] *= alpha;
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) sv[kb][r] -= d;
#pragma unroll
            for (int r = 0; r < 16; r++) bias[r] = -mu;
        }
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) sv[kb][r] = __builtin_amdgcn_exp2f(sv[kb][r]);

        /* O^T += V^T . P^T per 16-key step; the MFMA's k = 8h + j maps to
         * keys 4h + j (j < 4) and 8 + 4h + (j - 4) of the step, the keys this
         * lane holds; V^T comes from row-major V by transpose reads */
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const int r0 = 8 * half;
                const uint4 pu = make_uint4(
                    pack2(sv[kb][r0 + 0], sv[kb][r0 + 1]), pack2(sv[kb][r0 + 2], sv[kb][r0 + 3]),
                    pack2(sv[kb][r0 + 4], sv[kb][r0 + 5]), pack2(sv[kb][r0 + 6], sv[kb][r0 + 7]));
                const half8_t pp = h8_from_u4(pu);
                /* the row sum of the f16 P the MFMA consumes */
                lsum = __builtin_amdgcn_fdot2(pf_h2(pu.x), ones2, lsum, false);
                lsum = __builtin_amdgcn_fdot2(pf_h2(pu.y), ones2, lsum, false);
                lsum = __builtin_amdgcn_fdot2(pf_h2(pu.z), ones2, lsum, false);
                lsum = __builtin_amdgcn_fdot2(pf_h2(pu.w), ones2, lsum, false);
                const int kbase = 32 * kb + 16 * half + 4 * h + tr_row;
#pragma unroll
                for (int b = 0; b < DB; b++) {
                    const _Float16 *vp = sv_t + kbase * VS + 32 * b + tr_col;
                    const uint2 x0 = ld_tr16(vp);
                    const uint2 x1 = ld_tr16(vp + 8 * VS);
                    const half8_t a = h8_from_u4(make_uint4(x0.x, x0.y, x1.x, x1.y));
                    o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pp, o[b], 0, 0, 0);
                }
            }
        }
        if (tb + BN < ke) store_tile(buf ^ 1, AHEAD == 2 ? sl ^ 1 : 0);
        __syncthreads();
    };
    if constexpr (AHEAD == 2) {
        for (u32 tb = ks; tb < ke; tb += 2 * BN) {
            tile_step(tb, 0, 0);
            if (tb + BN < ke) tile_step(tb + BN, 1, 1);
        }
    } else {
        int buf = 0;
        for (u32 tb = ks; tb < ke; tb += BN) {
            tile_step(tb, buf, 0);
            buf ^= 1;
        }
    }
    lsum += __shfl_xor(lsum, 32);

    /* the launch's last workgroup to finish advances the epoch: every
     * workgroup has read it by then */
    if (fa && tid == 0 &&
        __hip_atomic_fetch_add(p.ctr + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            gridDim.x - 1) {
        __hip_atomic_store(p.ctr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(p.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!row_ok) return;
    /* o[b][r] = O^T[d = 32b + 8(r/4) + 4h + r%4][row lr] */
    if (p.n_split == 1) {
        float *dst = p.dst + (u64)my_q * p.q_stride + (u64)hq * D;
        const float inv = 1.0f / lsum;
#pragma unroll
        for (int b = 0; b < DB; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) dst[32 * b + 8 * (r / 4) + 4 * h + (r % 4)] = o[b][r] * inv;
    } else {
        const u64 pi = ((u64)my_q * p.n_head + hq) * p.n_split + split;
        float *acc = p.ws_acc + pi * D;
#pragma unroll
        for (int b = 0; b < DB; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[32 * b + 8 * (r / 4) + 4 * h + (r % 4)] = o[b][r];
        if (h == 0) p.ws_ml[pi] = make_float2(m, lsum);
    }
}

/* One (ROPE, Q8) variant's instances over head_dim {64, 128, 256} x gqa 1..8;
 * returns the kernel entry point, or NULL for an unsupported shape. */
#define TL_PREFILL_PICKER(name, ROPE, Q8)                                              \
    template <int D>                                                                   \
    static const void *name##_d(int G) {                                               \
        switch (G) {                                                                   \
        case 1: return (const void *)attn_prefill_kernel<D, 1, ROPE, Q8>;              \
        case 2: return (const void *)attn_prefill_kernel<D, 2, ROPE, Q8>;              \
        case 3: return (const void *)attn_prefill_kernel<D, 3, ROPE, Q8>;              \
        case 4: return (const void *)attn_prefill_kernel<D, 4, ROPE, Q8>;              \
        case 5: return (const void *)attn_prefill_kernel<D, 5, ROPE, Q8>;              \
        case 6: return (const void *)attn_prefill_kernel<D, 6, ROPE, Q8>;              \
        case 7: return (const void *)attn_prefill_kernel<D, 7, ROPE, Q8>;              \
        case 8: return (const void *)attn_prefill_kernel<D, 8, ROPE, Q8>;              \
        default: return nullptr;                                                       \
        }                                                                              \
    }                                                                                  \
    const void *name(int D, int G) {                                                   \
        switch (D) {                                                                   \
        case 64: return name##_d<64>(G);                                               \
        case 128: return name##_d<128>(G);                                             \
        case 256: return name##_d<256>(G);                                             \
        default: return nullptr;                                                       \
        }                                                                              \
    }

const void *tl_prefill_fn(int D, int G);            /* tl_prefill.hip */
const void *tl_prefill_fn_rope(int D, int G);       /* tl_prefill_rope.hip */
const void *tl_prefill_fn_q8(int D, int G);         /* tl_prefill_q8.hip */
const void *tl_prefill_fn_q8_rope(int D, int G);    /* tl_prefill_q8_rope.hip */
