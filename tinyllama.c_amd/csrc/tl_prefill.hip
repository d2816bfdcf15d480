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
 *                                  range end; the O rescale is skipped when no
 *                                  row's max moved.  P^T is packed to f16
 *                                  straight from the accumulator registers.
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
    float m = NEG_INF, lsum = 0.f;

    const u16 *Kb = p.k + (u64)kvh * p.cap * D;
    const u16 *Vb = p.v + (u64)kvh * p.cap * D;
    /* Q8_0 cache: int8 rows and one f16 scale per 32 elements */
    const uint8_t *K8 = (const uint8_t *)p.k + (u64)kvh * p.cap * D;
    const uint8_t *V8 = (const uint8_t *)p.v + (u64)kvh * p.cap * D;
    const u16 *Ksc = Q8 ? p.ks + (u64)kvh * p.cap * (D / 32) : nullptr;
    const u16 *Vsc = Q8 ? p.vs + (u64)kvh * p.cap * (D / 32) : nullptr;

    /* register staging, AHEAD tiles ahead of the compute.  Unit u = tid + j*T
     * -> row u / CPR, chunk u % CPR; rows past ke load zeros.  A Q8_0
     * cache's units are held raw (8 int8 and their block's scale) and
     * dequantized on the LDS write, with two register sets at head_dim
     * <= 128: a tile's loads are issued one iteration before the iteration
     * that converts and writes it (measured: 482 -> 363 us for the last
     * config-4 chunk).  The f16 path keeps one set (a second one measured
     * no faster and costs occupancy at head_dim 64). */
    constexpr int AHEAD = (Q8 && D <= 128) ? 2 : 1;
    uint4 rk[AHEAD][UPT], rv[AHEAD][UPT];
    auto load_tile = [&](u32 tb, int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * T;
            const int row = u / CPR, c = u % CPR;
            const u32 key = tb + row;
            rk[s][j] = make_uint4(0, 0, 0, 0);
            rv[s][j] = make_uint4(0, 0, 0, 0);
            if (u < UNITS && key < ke) {
                u32 ph = p.ring ? key % p.ring : (p.slots ? p.slots[key] : key);
                ph = ph < p.cap ? ph : 0;
                if constexpr (Q8) {
                    const u64 e = (u64)ph * D + c * 8, sc = (u64)ph * (D / 32) + c / 4;
                    const uint2 kq = *(const uint2 *)(K8 + e), vq = *(const uint2 *)(V8 + e);
                    rk[s][j] = make_uint4(kq.x, kq.y, Ksc[sc], 0);
                    rv[s][j] = make_uint4(vq.x, vq.y, Vsc[sc], 0);
                } else {
                    rk[s][j] = *(const uint4 *)(Kb + (u64)ph * D + c * 8);
                    rv[s][j] = *(const uint4 *)(Vb + (u64)ph * D + c * 8);
                }
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

    if (ks < ke) {
        load_tile(ks, 0);
        store_tile(0, 0);
        if (AHEAD == 2 && ks + BN < ke) load_tile(ks + BN, AHEAD - 1);
    }
    __syncthreads();
    /* one tile: LDS buffer `buf` holds it, register set `sl` receives the
     * tile two ahead, set sl ^ 1 (loaded an iteration ago) holds the next
     * tile, written to the other buffer at the end */
    auto tile_step = [&](u32 tb, int buf, int sl) __attribute__((always_inline)) {
        if constexpr (AHEAD == 2) {
            if (tb + 2 * BN < ke) load_tile(tb + 2 * BN, sl);
        } else {
            if (tb + BN < ke) load_tile(tb + BN, 0);
        }
        const uint4 *sk = s_k[buf];
        const _Float16 *sv_t = s_v[buf];

        /* S^T = K . Q^T per 32-key block: lane holds keys
         * 32 kb + 8(r/4) + 4h + r%4 of query lr */
        floatx16_t sacc[KB];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int krow = 32 * kb + lr;
            const floatx16_t zero = {};
            sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                h8_from_u4(sk[krow * CPR + (h ^ (krow % CPR))]), qop[0], zero, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < KS; s++) {
                const int c = 2 * s + h;
                const half8_t a = h8_from_u4(sk[krow * CPR + (c ^ (krow % CPR))]);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qop[s], sacc[kb], 0, 0, 0);
            }
        }

        /* mask (only tiles that cross a boundary; visible keys of this lane's
         * row are [klo, khi)) + online softmax */
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
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float mu = (mn == NEG_INF) ? 0.f : mn;
        const float alpha = __builtin_amdgcn_exp2f(m - mu);
        m = mn;
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                sv[kb][r] = __builtin_amdgcn_exp2f(sv[kb][r] - mu);
                ps += sv[kb][r];
            }
        lsum = lsum * alpha + ps;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
            for (int b = 0; b < DB; b++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[b][r] *= alpha;
        }

        /* O^T += V^T . P^T per 16-key step; the MFMA's k = 8h + j maps to
         * keys 4h + j (j < 4) and 8 + 4h + (j - 4) of the step, the keys this
         * lane holds; V^T comes from row-major V by transpose reads */
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const int r0 = 8 * half;
                const half8_t pp = h8_from_u4(make_uint4(
                    pack2(sv[kb][r0 + 0], sv[kb][r0 + 1]), pack2(sv[kb][r0 + 2], sv[kb][r0 + 3]),
                    pack2(sv[kb][r0 + 4], sv[kb][r0 + 5]), pack2(sv[kb][r0 + 6], sv[kb][r0 + 7])));
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

/* ------------------------------------------------------------------------ */

bool tl_prefill_supported(const LayerView &L, const tl_attn_args *a) {
    if (getenv("TL_NO_PREFILL")) return false;
    const u32 G = a->n_head / L.n_kv_head;
    return (L.head_dim == 64 || L.head_dim == 128 || L.head_dim == 256) && G >= 1 && G <= 8;
}

template <int D, int G>
static void launch_pf(const PrefParams &p, u32 blocks, hipStream_t st) {
    const dim3 nt(64 * PCfg<D, G>::W);
    if (p.ks)   /* Q8_0 cache (no RoPE fusion on this path) */
        hipLaunchKernelGGL((attn_prefill_kernel<D, G, false, true>), dim3(blocks), nt, 0, st, p);
    else if (p.rope.rdim)
        hipLaunchKernelGGL((attn_prefill_kernel<D, G, true, false>), dim3(blocks), nt, 0, st, p);
    else
        hipLaunchKernelGGL((attn_prefill_kernel<D, G, false, false>), dim3(blocks), nt, 0, st, p);
}

template <int D>
static int launch_pf_d(const PrefParams &p, int G, u32 blocks, hipStream_t st) {
    switch (G) {
    case 1: launch_pf<D, 1>(p, blocks, st); break;
    case 2: launch_pf<D, 2>(p, blocks, st); break;
    case 3: launch_pf<D, 3>(p, blocks, st); break;
    case 4: launch_pf<D, 4>(p, blocks, st); break;
    case 5: launch_pf<D, 5>(p, blocks, st); break;
    case 6: launch_pf<D, 6>(p, blocks, st); break;
    case 7: launch_pf<D, 7>(p, blocks, st); break;
    case 8: launch_pf<D, 8>(p, blocks, st); break;
    default: return tl_fail(TL_EINVAL, "prefill: gqa %d", G);
    }
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

static u32 rows_per_wg(u32 D, u32 G) {
    const u32 wmax = D <= 128 ? 8 : 4;
    const u32 qb = wmax / G ? wmax / G : 1;
    return 32 * qb;
}

int tl_launch_prefill(const LayerView &L, const tl_attn_args *a, const RopeCfg &rope,
                      hipStream_t st) {
    const u32 D = L.head_dim, G = a->n_head / L.n_kv_head;
    if (L.q8 && (rope.rdim || !L.ks || !L.vs))
        return tl_fail(TL_EINVAL, "prefill: a Q8_0 cache takes scales and no fused RoPE");
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

    const u32 rows = rows_per_wg(D, G);
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
    if (const char *e = getenv("TL_PREFILL_SPLITS")) ns = (u32)atoi(e) ? (u32)atoi(e) : ns;
    p.n_split = ns;
    if (ns > 1) {
        TlWorkspace *w;
        size_t parts = (size_t)a->n * a->n_head * ns;
        int rc = tl_workspace_get(parts * D, parts, 0, &w);
        if (rc) return rc;
        p.ws_acc = w->acc;
        p.ws_ml = (float2 *)w->ml;
    }
    const u32 blocks = base * ns;
    int rc;
    switch (D) {
    case 64: rc = launch_pf_d<64>(p, (int)G, blocks, st); break;
    case 128: rc = launch_pf_d<128>(p, (int)G, blocks, st); break;
    case 256: rc = launch_pf_d<256>(p, (int)G, blocks, st); break;
    default: return tl_fail(TL_EINVAL, "prefill: head_dim %u", D);
    }
    if (rc || ns == 1) return rc;
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
