/*
 * tl_decode.hip — split-K decode attention over the slot-indexed f16 cache.
 *
 * Math of op_attn (reference src/backend/cpu/cpu_op.c:1011-1062): for each
 * q-head h and batch row r, n_keys = pos + r + 1, visible keys
 * [start, n_keys) with start = n_keys - window when window > 0 and
 * n_keys > window (cpu_op.c:1019-1022); s_t = (K[h/gqa][slot_t] . q) * scale;
 * out = softmax(s) @ V.
 *
 * Work decomposition (gfx950, wave64):
 *   grid = n_split x (rows x n_kv_head) workgroups of 4 waves, two resident
 *   per CU, mapped so that all splits of one (row, kv-head) group run on one
 *   XCD.  A workgroup streams one contiguous chunk of keys of one kv-head and
 *   serves every q-head of the GQA group from the same K/V bytes, so each
 *   cache byte is read from HBM once per step instead of gqa times.  The
 *   chunk's slot indices are staged in LDS first, so K/V loads never wait on
 *   a dependent slot-table load.
 *   Each wave owns every 4th tile of the chunk (4 KB of K+V by default):
 *   16-byte loads into registers, written to a per-wave LDS tile (K chunks
 *   XOR-swizzled by row against bank conflicts) while the next tile's loads
 *   are in flight.
 *   Scores: v_dot2_f32_f16 of the f16 K row with q (pre-scaled by
 *   scale*log2(e), rounded to f16), summed over the row's lanes with DPP
 *   moves; wave-uniform online softmax per q-head in f32 with exp2; p is
 *   rounded to f16 and PV runs as v_dot2 over key pairs of V.
 *   States merge across waves through LDS and across splits in the last
 *   workgroup of the group to finish (partials written with device-coherent
 *   stores, a per-group atomic counter that this workgroup resets), or in a
 *   separate merge launch when the partials exceed that workgroup's LDS.
 *   The fused append of decode rows: the split-0 workgroup writes the new
 *   K/V rows; workgroups that need a new key convert it from the f32 input.
 */
#include "tl_common.h"
#include "tl_internal.h"

#include <stdlib.h>
#include <string.h>
#include <type_traits>

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

TL_DEV half2_t as_h2(u32 w) { return __builtin_bit_cast(half2_t, w); }

/* 8 f32 -> 8 binary16 (RNE, NaN pinned), the append conversion */
TL_DEV uint4 cvt8_f16(const float *src) {
    const float4 a = *(const float4 *)src;
    const float4 b = *(const float4 *)(src + 4);
    return make_uint4(pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y),
                      pack_f16x2(b.z, b.w));
}

TL_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef u32 u32x4_t __attribute__((ext_vector_type(4)));

/* 16-byte streaming load (non-temporal: the cache is read once per step). */
TL_DEV uint4 ld_stream(const u16 *ptr) {
    u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)ptr);
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int D, int TB>
struct DCfg {
    static constexpr int CPR = D / 8;           /* 16-byte chunks per row */
    static constexpr int TK = TB / (2 * D);     /* keys per wave tile */
    static constexpr int LPK = D / 32;          /* lanes per key in QK (4 chunks each) */
    static constexpr int CPL = 4;               /* chunks per lane in QK */
    static constexpr int KPP = 64 / LPK;        /* keys per QK pass */
    static constexpr int PASSES = TK / KPP;     /* 1 or 2 */
    static constexpr int UNITS = TK * CPR;      /* 512 units per tile */
    static constexpr int LD = UNITS / 64;       /* 16-byte loads per lane per tile */
    static constexpr int DPL = (D <= 128) ? 2 : 4;  /* PV dims per lane */
    static constexpr int PVL = D / DPL;         /* lanes of one PV key group */
    static constexpr int KG = 64 / PVL;         /* PV key groups per wave */
    static constexpr int NPAIR = TK / 2;
};

TL_DEV u32 perm_lo(u32 a, u32 b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
TL_DEV u32 perm_hi(u32 a, u32 b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

/* the buffer builtins take and return GCC vectors; read their elements with
 * v[i] into scalars (this compiler mis-reads __builtin_bit_cast of a vector
 * element) */
typedef u32 u32x4v_t __attribute__((vector_size(16)));
typedef u32 u32x2v_t __attribute__((vector_size(8)));

/* Raw buffer resource over `base` (offsets are bytes from base). */
TL_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7ffffff0, 0x00020000);
}
/* Cache policy sc1: device-coherent access (written through to / read from
 * the level every XCD sees), the policy of agent-scope atomics. */
#define TL_SC1 16

template <int D, int G>
TL_DEV void split_merge(const DecParams &p, u32 grow, u32 kvh, u32 si, u32 r, float *lds,
                        float *s_hl);

template <int D, int G, int TB, bool ROPE>
__global__ __launch_bounds__(256) void attn_decode_kernel(const DecParams p) {
    using C = DCfg<D, TB>;
    constexpr int CPR = C::CPR, TK = C::TK, LPK = C::LPK, CPL = C::CPL, KPP = C::KPP;
    constexpr int PASSES = C::PASSES, UNITS = C::UNITS, LD = C::LD, DPL = C::DPL;
    constexpr int PVL = C::PVL, KG = C::KG, NPAIR = C::NPAIR;
    constexpr int GP = (G + 3) / 4 * 4;         /* p pairs padded to 16 bytes */
    constexpr float NEG_INF = -__builtin_huge_valf();

    __shared__ uint4 s_kv[4][2][UNITS];          /* per wave: K tile, V tile */
    __shared__ u32 s_p[4][NPAIR][GP];            /* per wave: (p_t, p_t+1) f16 pairs */
    __shared__ u32 s_slot[TL_DEC_MAX_CHUNK];
    __shared__ uint4 s_q[G * D / 8];             /* q, f16, scaled to log2 units */
    __shared__ float s_m[4][G];
    __shared__ float s_l[4][G];
    __shared__ uint4 s_newk[TL_DEC_MAX_NEW][D / 8];   /* new rows of a fused launch, f16 */
    __shared__ uint4 s_newv[TL_DEC_MAX_NEW][D / 8];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    /* XCD-aware block order: block b runs on XCD b % 8; all splits of one
     * (row, kv-head) group land on the same XCD when the group count is a
     * multiple of 8, so the split merge reads partials from that XCD's L2. */
    const u32 n_split = p.n_split;
    const u32 n_groups = gridDim.x / n_split;
    const u32 bid = blockIdx.x;
    u32 grp, split;
    if ((n_groups & 7) == 0) {
        const u32 xcd = bid & 7, local = bid >> 3;
        grp = xcd + 8 * (local / n_split);
        split = local % n_split;
    } else {
        grp = bid / n_split;
        split = bid % n_split;
    }
    const u32 kvh = grp % p.n_kv;
    const u32 grow = grp / p.n_kv;
    const u32 si = grow / p.rows_per_seq;
    const u32 r = grow % p.rows_per_seq;
    const DecSeq sq = p.seq[si];

    const u32 n_keys = sq.pos + r + 1;
    const u32 start = (p.window && n_keys > p.window) ? n_keys - p.window : 0;
    const u32 kbeg = start + split * p.chunk;
    const u32 kend = min(kbeg + p.chunk, n_keys);
    /* fused append: the launch's new rows (positions pos..pos+rows-1, K
     * RoPE'd when ROPE) are converted to f16 into LDS by every workgroup that
     * reads one of them and by the split-0 workgroup of row 0, which also
     * writes them to the cache.  No workgroup reads a cache row that is being
     * written in this launch, and the stream loop never runs the conversion
     * (or RoPE) code itself.
     * With ROPE, q and the new K rows are first copied to LDS as f32, rotated
     * one pair per thread while the first tile's loads are in flight, then
     * converted. */
    constexpr int VPR = D / 8;
    const bool fused = sq.kin != nullptr;
    const bool writer = fused && split == 0 && r == 0;
    const bool need_new = fused && (writer || kend > sq.pos);
    float *qf = (float *)&s_kv[0][0][0];             /* ROPE: [G][D] f32 */
    float *kf = qf + G * D;                          /* ROPE: [rows][D] f32 */
    const float *qb = sq.q + (u64)r * p.q_stride + (u64)kvh * G * D;
    if (need_new) {
        for (u32 i = tid; i < p.rows_per_seq * VPR; i += 256) {
            const u32 row = i / VPR, c8 = i % VPR;
            const u64 src = (u64)row * sq.kv_stride + (u64)kvh * D + c8 * 8;
            if constexpr (ROPE) {
                *(float4 *)(kf + row * D + c8 * 8) = *(const float4 *)(sq.kin + src);
                *(float4 *)(kf + row * D + c8 * 8 + 4) = *(const float4 *)(sq.kin + src + 4);
            } else {
                s_newk[row][c8] = cvt8_f16(sq.kin + src);
            }
            s_newv[row][c8] = cvt8_f16(sq.vin + src);
        }
    }

    /* physical rows of the chunk's keys, staged in LDS unless identity */
    const bool staged = (sq.ring != 0) || (sq.slots != nullptr);
    if (!staged) {
    } else if (sq.ring) {
        for (u32 i = kbeg + tid; i < kend; i += 256) s_slot[i - kbeg] = i % sq.ring;
    } else if (sq.slots) {
        for (u32 i = kbeg + tid; i < kend; i += 256) {
            u32 s = sq.slots[i];
            s_slot[i - kbeg] = s < sq.cap ? s : 0u;
        }
    }
    /* q of the GQA group, scaled to log2 units, staged once per workgroup */
    if constexpr (ROPE) {
        for (int i = tid; i < G * D / 4; i += 256)
            *(float4 *)(qf + i * 4) = *(const float4 *)(qb + i * 4);
    } else {
        for (int i = tid; i < G * D / 8; i += 256) {
            const float4 a = *(const float4 *)(qb + i * 8);
            const float4 b = *(const float4 *)(qb + i * 8 + 4);
            const float sc = p.scale_log2;
            s_q[i] = make_uint4(pack_f16x2_fast(a.x * sc, a.y * sc), pack_f16x2_fast(a.z * sc, a.w * sc),
                                pack_f16x2_fast(b.x * sc, b.y * sc), pack_f16x2_fast(b.z * sc, b.w * sc));
        }
    }
    __syncthreads();

    /* q chunks of this lane's QK position, scaled to log2 units, f16 pairs */
    const int qc0 = (lane % LPK) * CPL;

    float m[G], lsum[G], acc[G][DPL];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = NEG_INF;
        lsum[h] = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; e++) acc[h][e] = 0.f;
    }

    const u16 *Kbase = sq.k + (u64)kvh * sq.cap * D;
    const u16 *Vbase = sq.v + (u64)kvh * sq.cap * D;

    uint4 *tk = s_kv[wave][0];
    uint4 *tv = s_kv[wave][1];
    u32 *tp = &s_p[wave][0][0];

    /* register staging of one tile: K unit u = j*64 + lane holds chunk
     * (u % CPR) ^ (row % CPR) of tile row u / CPR; V is stored unswizzled
     * (unit u holds chunk u % CPR) because the PV phase reads whole rows.
     * Keys past the chunk load the chunk's last row (always valid memory)
     * and are zeroed when the tile is written to LDS. */
    uint4 rk[LD], rv[LD];
#define TL_PHYS(key) (staged ? s_slot[(key) - kbeg] : (key))
#define TL_LOAD_TILE(TBASE)                                                         \
    do {                                                                            \
        const u32 tb_ = (TBASE), klast_ = kend - 1;                                 \
        if (fused && tb_ + TK > sq.pos) {   /* tile holds new keys */               \
            _Pragma("unroll") for (int j = 0; j < LD; j++) {                        \
                const int u = j * 64 + lane;                                        \
                const int row = u / CPR;                                            \
                const u32 key = min(tb_ + (u32)row, klast_);                        \
                const int kc_ = (u % CPR) ^ (row % CPR), vc_ = u % CPR;             \
                if (key >= sq.pos) {                                                \
                    rk[j] = s_newk[key - sq.pos][kc_];                              \
                    rv[j] = s_newv[key - sq.pos][vc_];                              \
                } else {                                                            \
                    const u32 ph = TL_PHYS(key);                                    \
                    rk[j] = ld_stream(Kbase + (u64)ph * D + kc_ * 8);               \
                    rv[j] = ld_stream(Vbase + (u64)ph * D + vc_ * 8);               \
                }                                                                   \
            }                                                                       \
            break;                                                                  \
        }                                                                           \
        _Pragma("unroll") for (int j = 0; j < LD; j++) {                            \
            const int u = j * 64 + lane;                                            \
            const int row = u / CPR;                                                \
            const u32 key = min(tb_ + (u32)row, klast_);                            \
            const u32 ph = TL_PHYS(key);                                            \
            rk[j] = ld_stream(Kbase + (u64)ph * D + ((u % CPR) ^ (row % CPR)) * 8); \
            rv[j] = ld_stream(Vbase + (u64)ph * D + (u % CPR) * 8);                 \
        }                                                                           \
    } while (0)

    const u32 ntile = (kend > kbeg) ? (kend - kbeg + TK - 1) / TK : 0;
    u32 ti = wave;
    /* the first tile's loads go out now; with ROPE a tile that holds new
     * keys waits until they are converted */
    const bool defer_first = ROPE && fused && kbeg + ti * TK + TK > sq.pos;
    if (ti < ntile && !defer_first) TL_LOAD_TILE(kbeg + ti * TK);
    if constexpr (ROPE) {
        /* rotate q (G heads at pos + r) and the new K rows (at pos + row),
         * one pair per thread, in place in LDS */
        const u32 pairs = p.rope.rdim >> 1;
        const u32 nq = G * pairs, nk = need_new ? p.rows_per_seq * pairs : 0u;
        for (u32 t = tid; t < nq + nk; t += 256) {
            const bool isq = t < nq;
            const u32 tt = isq ? t : t - nq;
            const u32 hrow = tt / pairs, i = tt % pairs;
            float *row = (isq ? qf : kf) + hrow * D;
            const u32 ia = p.rope.neox ? i : 2 * i, ib = p.rope.neox ? i + pairs : 2 * i + 1;
            float c, sn, x, y;
            rope_cs(i, p.rope.rdim, p.rope.theta, isq ? sq.pos + r : sq.pos + hrow, c, sn);
            rope_rot(row[ia], row[ib], c, sn, x, y);
            row[ia] = x;
            row[ib] = y;
        }
        __syncthreads();
        const float sc = p.scale_log2;
        for (int i = tid; i < G * D / 8; i += 256) {
            const float *t = qf + i * 8;
            s_q[i] = make_uint4(pack_f16x2_fast(t[0] * sc, t[1] * sc), pack_f16x2_fast(t[2] * sc, t[3] * sc),
                                pack_f16x2_fast(t[4] * sc, t[5] * sc), pack_f16x2_fast(t[6] * sc, t[7] * sc));
        }
        if (need_new)
            for (u32 i = tid; i < p.rows_per_seq * VPR; i += 256) {
                const float *t = kf + (i / VPR) * D + (i % VPR) * 8;
                s_newk[i / VPR][i % VPR] = make_uint4(pack_f16x2(t[0], t[1]), pack_f16x2(t[2], t[3]),
                                                      pack_f16x2(t[4], t[5]), pack_f16x2(t[6], t[7]));
            }
        __syncthreads();   /* also: qf/kf (tile memory) are free again */
        if (ti < ntile && defer_first) TL_LOAD_TILE(kbeg + ti * TK);
    }
    if (writer) {
        for (u32 i = tid; i < p.rows_per_seq * VPR; i += 256) {
            const u32 row = i / VPR, c8 = i % VPR;
            const u32 key = sq.pos + row;
            const u32 ph = sq.ring ? key % sq.ring : (sq.slots ? sq.slots[key] : key);
            if (ph >= sq.cap) continue;
            const u64 dst = ((u64)kvh * sq.cap + ph) * D + c8 * 8;
            *(uint4 *)((u16 *)sq.k + dst) = s_newk[row][c8];
            *(uint4 *)((u16 *)sq.v + dst) = s_newv[row][c8];
        }
    }
    while (ti < ntile) {
        const u32 tbase = kbeg + ti * TK;
        if (tbase + TK <= kend) {
#pragma unroll
            for (int j = 0; j < LD; j++) {
                tk[j * 64 + lane] = rk[j];
                tv[j * 64 + lane] = rv[j];
            }
        } else {   /* tail tile: rows past kend contribute exactly 0 */
#pragma unroll
            for (int j = 0; j < LD; j++) {
                const bool ok = tbase + (u32)((j * 64 + lane) / CPR) < kend;
                uint4 a = rk[j], b = rv[j];
                a.x = ok ? a.x : 0u; a.y = ok ? a.y : 0u; a.z = ok ? a.z : 0u; a.w = ok ? a.w : 0u;
                b.x = ok ? b.x : 0u; b.y = ok ? b.y : 0u; b.z = ok ? b.z : 0u; b.w = ok ? b.w : 0u;
                tk[j * 64 + lane] = a;
                tv[j * 64 + lane] = b;
            }
        }
        __builtin_amdgcn_wave_barrier();
        const u32 tnext = ti + 4;
        if (tnext < ntile) TL_LOAD_TILE(kbeg + tnext * TK);

        /* ---- scores: LPK lanes per key, CPL chunks each ---- */
        float sc[PASSES][G];
#pragma unroll
        for (int ps = 0; ps < PASSES; ps++) {
            const int kt = ps * KPP + lane / LPK;
            float d[G];
#pragma unroll
            for (int h = 0; h < G; h++) d[h] = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; j++) {
                const int c = qc0 + j;
                const uint4 kv = tk[kt * CPR + (c ^ (kt % CPR))];
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const uint4 qv = s_q[h * CPR + c];
                    d[h] = __builtin_amdgcn_fdot2(as_h2(kv.x), as_h2(qv.x), d[h], false);
                    d[h] = __builtin_amdgcn_fdot2(as_h2(kv.y), as_h2(qv.y), d[h], false);
                    d[h] = __builtin_amdgcn_fdot2(as_h2(kv.z), as_h2(qv.z), d[h], false);
                    d[h] = __builtin_amdgcn_fdot2(as_h2(kv.w), as_h2(qv.w), d[h], false);
                }
            }
            const bool valid = tbase + kt < kend;
#pragma unroll
            for (int h = 0; h < G; h++) {
                float t = group_sum<LPK>(d[h]);
                sc[ps][h] = valid ? t : NEG_INF;
            }
        }

        /* ---- online softmax over the tile (wave-uniform max) ---- */
#pragma unroll
        for (int h = 0; h < G; h++) {
            float tm = sc[0][h];
#pragma unroll
            for (int ps = 1; ps < PASSES; ps++) tm = fmaxf(tm, sc[ps][h]);
            tm = group_max<64>(tm);
            const float mn = fmaxf(m[h], tm);
            const float mu = (mn == NEG_INF) ? 0.f : mn;
            const float alpha = fast_exp2(m[h] - mu);
            m[h] = mn;
            float ls = lsum[h] * alpha;
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[h][e] *= alpha;
#pragma unroll
            for (int ps = 0; ps < PASSES; ps++) {
                const float pr = fast_exp2(sc[ps][h] - mu);
                ls += pr;
                /* pair keys (2i, 2i+1): lane groups gi and gi+1 */
                const float pn = __shfl_xor(pr, LPK);
                const int gi = lane / LPK;
                if ((gi & 1) == 0 && (lane % LPK) == 0) {
                    const int kt = ps * KPP + gi;
                    tp[(kt >> 1) * GP + h] = pack_f16x2_fast(pr, pn);
                }
            }
            lsum[h] = ls;
        }
        __builtin_amdgcn_wave_barrier();

        /* ---- PV: lanes own DPL dims, v_dot2 over key pairs ---- */
        const int kg = lane / PVL;
        const int d0 = (lane % PVL) * DPL;
        const int vc = d0 / 8;
        const int vw = (d0 % 8) / 2;
#pragma unroll
        for (int ip = 0; ip < NPAIR / KG; ip++) {
            const int pi = ip * KG + kg;
            const int t0 = 2 * pi, t1 = 2 * pi + 1;
            const u32 *r0 = (const u32 *)&tv[t0 * CPR + vc] + vw;
            const u32 *r1 = (const u32 *)&tv[t1 * CPR + vc] + vw;
            u32 a[DPL / 2], b[DPL / 2];
#pragma unroll
            for (int w = 0; w < DPL / 2; w++) {
                a[w] = r0[w];
                b[w] = r1[w];
            }
            u32 pp[GP];
#pragma unroll
            for (int g4 = 0; g4 < GP; g4 += 4) {
                const uint4 t = *(const uint4 *)&tp[pi * GP + g4];
                pp[g4] = t.x; pp[g4 + 1] = t.y; pp[g4 + 2] = t.z; pp[g4 + 3] = t.w;
            }
#pragma unroll
            for (int w = 0; w < DPL / 2; w++) {
                const half2_t lo = as_h2(perm_lo(a[w], b[w]));
                const half2_t hi = as_h2(perm_hi(a[w], b[w]));
#pragma unroll
                for (int h = 0; h < G; h++) {
                    acc[h][2 * w] = __builtin_amdgcn_fdot2(lo, as_h2(pp[h]), acc[h][2 * w], false);
                    acc[h][2 * w + 1] = __builtin_amdgcn_fdot2(hi, as_h2(pp[h]), acc[h][2 * w + 1], false);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        ti = tnext;
    }

#undef TL_LOAD_TILE
#undef TL_PHYS

    /* ---- wave state -> LDS (tile memory is reused after the barrier) ---- */
#pragma unroll
    for (int h = 0; h < G; h++) {
        lsum[h] = group_sum<64>(lsum[h]) * (1.0f / LPK);
        if constexpr (KG > 1) {
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[h][e] += __shfl_xor(acc[h][e], PVL);
        }
    }
    __syncthreads();
    float *s_acc = (float *)&s_kv[0][0][0];       /* [4][G][D] */
    {
        const int d0 = (lane % PVL) * DPL;
        if (lane < PVL) {
#pragma unroll
            for (int h = 0; h < G; h++)
#pragma unroll
                for (int e = 0; e < DPL; e++) s_acc[(wave * G + h) * D + d0 + e] = acc[h][e];
        }
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < G; h++) {
                s_m[wave][h] = m[h];
                s_l[wave][h] = lsum[h];
            }
        }
    }
    __syncthreads();

    /* ---- merge the 4 waves; write the final row or this split's partial ---- */
    const bool single = (n_split == 1);
    const bool last_merges = p.counters != nullptr;
    for (int o = tid; o < G * D; o += 256) {
        const int h = o / D, d = o % D;
        float mm = fmaxf(fmaxf(s_m[0][h], s_m[1][h]), fmaxf(s_m[2][h], s_m[3][h]));
        float mu = (mm == NEG_INF) ? 0.f : mm;
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            float f = fast_exp2(s_m[w][h] - mu);
            L += s_l[w][h] * f;
            O += s_acc[(w * G + h) * D + d] * f;
        }
        const u32 hq = kvh * G + h;
        if (single) {
            sq.dst[(u64)r * p.q_stride + (u64)hq * D + d] = O / L;
        } else if (last_merges) {
            /* device-coherent stores: the merging workgroup may run on
             * another XCD and reads them with device-coherent loads */
            const u32 pb = ((grow * p.n_head + kvh * G) * n_split) ;
            const u32 pi = (u32)h * n_split + split;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(O),
                                                  buf_rsrc(p.ws_acc + (u64)pb * D),
                                                  (pi * D + d) * 4, 0, TL_SC1);
            if (d == 0)
                __builtin_amdgcn_raw_buffer_store_b64(
                    u32x2v_t{__float_as_uint(mm), __float_as_uint(L)},
                    buf_rsrc(p.ws_ml + pb), pi * 8, 0, TL_SC1);
        } else {
            u64 pi = ((u64)grow * p.n_head + hq) * n_split + split;
            p.ws_acc[pi * D + d] = O;
            if (d == 0) p.ws_ml[pi] = make_float2(mm, L);
        }
    }
    if (single || !last_merges) return;

    /* ---- the last split of this (row, kv-head) group to finish merges ----
     * Its partial stores are complete (vmcnt 0) before the counter add, so
     * the workgroup that sees n_split - 1 reads every partial. */
    __shared__ u32 s_last;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(&p.counters[grp], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_last != n_split - 1) return;
    if (tid == 0) __hip_atomic_store(&p.counters[grp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    split_merge<D, G>(p, grow, kvh, si, r, (float *)&s_kv[0][0][0], &s_l[0][0]);
}

/* Merge of the n_split partials of one (row, kv-head) group inside the
 * decode launch: weights w_s = exp2(m_s - M) per head, O = sum w_s acc_s,
 * out = O / sum w_s l_s.  Up to 32 partial float4 per thread and all (m, l)
 * pairs are requested together, so the common case costs one round trip
 * to memory; larger merges stream in batches.  lds: >= 2*G*n_split + 4*256
 * floats. */
template <int D, int G>
TL_DEV void split_merge(const DecParams &p, u32 grow, u32 kvh, u32 si, u32 r, float *lds,
                        float *s_hl) {
    constexpr float NEG_INF = -__builtin_huge_valf();
    constexpr int COLS = G * D / 4;                       /* float4 columns */
    constexpr int SUBS = COLS >= 256 ? 1 : 256 / COLS;    /* thread subsets over splits */
    constexpr int NIT = (COLS * SUBS + 255) / 256;        /* columns per thread */
    constexpr int BIG = 32 / NIT;    /* partials per column when all fit in one request wave */
    constexpr int B = 8 / NIT;       /* partials per column per batch otherwise */
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u32 ns = p.n_split;
    const u32 pb = (grow * p.n_head + kvh * G) * ns;
    const __amdgpu_buffer_rsrc_t rml = buf_rsrc(p.ws_ml + pb);
    const __amdgpu_buffer_rsrc_t racc = buf_rsrc(p.ws_acc + (u64)pb * D);
    float *s_w = lds;                 /* [G][ns] max, then weight */
    float *s_lv = lds + G * ns;       /* [G][ns] sums */
    float4 *s_part = (float4 *)(lds + 2 * G * ns + ((2 * G * ns) & 3 ? 4 - ((2 * G * ns) & 3) : 0));

    /* thread column k: it = tid + 256 k -> head h, dims (col % (D/4)) * 4,
     * splits sub, sub + SUBS, ... */
#define TL_COL(k)                                                                     \
    const int it = tid + (k) * 256;                                                   \
    const int col = it % COLS, sub = it / COLS;                                       \
    const bool live = it < COLS * SUBS;                                               \
    const u32 cb = (u32)(col / (D / 4)) * ns * D + (u32)(col % (D / 4)) * 4;          \
    const int h = col / (D / 4);                                                      \
    (void)h; (void)cb; (void)live
#define TL_LOAD(dst, s) \
    dst = (live && (s) < ns) ? __builtin_amdgcn_raw_buffer_load_b128(racc, (cb + (s) * D) * 4, 0, TL_SC1) \
                             : u32x4v_t{0u, 0u, 0u, 0u}
#define TL_FMA(a, v, s)                                                               \
    do {                                                                              \
        const float w_ = (live && (s) < ns) ? s_w[h * ns + (s)] : 0.f;                \
        a.x = fmaf(w_, __uint_as_float(v[0]), a.x);                                   \
        a.y = fmaf(w_, __uint_as_float(v[1]), a.y);                                   \
        a.z = fmaf(w_, __uint_as_float(v[2]), a.z);                                   \
        a.w = fmaf(w_, __uint_as_float(v[3]), a.w);                                   \
    } while (0)

    const bool one_wave = ns <= (u32)(SUBS * BIG);
    u32x4v_t v[NIT][BIG];
    if (one_wave) {
#pragma unroll
        for (int k = 0; k < NIT; k++) {
            TL_COL(k);
#pragma unroll
            for (int b = 0; b < BIG; b++) TL_LOAD(v[k][b], sub + b * SUBS);
        }
    }
    for (u32 i = tid; i < G * ns; i += 256) {
        const u32x2v_t ml = __builtin_amdgcn_raw_buffer_load_b64(rml, i * 8, 0, TL_SC1);
        s_w[i] = __uint_as_float(ml[0]);
        s_lv[i] = __uint_as_float(ml[1]);
    }
    __syncthreads();
    for (int hh = wave; hh < G; hh += 4) {
        float mx = NEG_INF;
        for (u32 s = lane; s < ns; s += 64) mx = fmaxf(mx, s_w[hh * ns + s]);
        mx = group_max<64>(mx);
        const float mu = (mx == NEG_INF) ? 0.f : mx;
        float L = 0.f;
        for (u32 s = lane; s < ns; s += 64) {
            const float w = fast_exp2(s_w[hh * ns + s] - mu);
            s_w[hh * ns + s] = w;
            L += w * s_lv[hh * ns + s];
        }
        L = group_sum<64>(L);
        if (lane == 0) s_hl[hh] = L;
    }
    __syncthreads();
    float4 acc[NIT];
#pragma unroll
    for (int k = 0; k < NIT; k++) {
        acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        TL_COL(k);
        if (one_wave) {
#pragma unroll
            for (int b = 0; b < BIG; b++) TL_FMA(acc[k], v[k][b], sub + b * SUBS);
        } else {
            for (u32 s0 = sub; s0 < ns; s0 += B * SUBS) {
                u32x4v_t t[B];
#pragma unroll
                for (int b = 0; b < B; b++) TL_LOAD(t[b], s0 + b * SUBS);
#pragma unroll
                for (int b = 0; b < B; b++) TL_FMA(acc[k], t[b], s0 + b * SUBS);
            }
        }
    }
#undef TL_COL
#undef TL_LOAD
#undef TL_FMA
#pragma unroll
    for (int k = 0; k < NIT; k++) {
        const int it = tid + k * 256;
        if (it < COLS * SUBS) s_part[(it / COLS) * COLS + it % COLS] = acc[k];
    }
    __syncthreads();
    const DecSeq &sq = p.seq[si];
    for (int col = tid; col < COLS; col += 256) {
        float4 o = s_part[col];
        for (int sb = 1; sb < SUBS; sb++) {
            const float4 t = s_part[sb * COLS + col];
            o.x += t.x; o.y += t.y; o.z += t.z; o.w += t.w;
        }
        const int h = col / (D / 4), d = (col % (D / 4)) * 4;
        const float inv = 1.0f / s_hl[h];
        float *dst = sq.dst + (u64)r * p.q_stride + (u64)(kvh * G + h) * D + d;
        dst[0] = o.x * inv;
        dst[1] = o.y * inv;
        dst[2] = o.z * inv;
        dst[3] = o.w * inv;
    }
}

/* Split merge as its own launch (no cross-workgroup synchronisation inside
 * the decode kernel).  grid = rows * n_head, 256 threads.  Weights
 * w_s = exp2(m_s - M) go to LDS; the n_split partial rows are then summed by
 * 256/D thread subsets with independent loads, and the subsets are added. */
#define TL_MERGE_MAX_SPLIT 1024
template <int D>
__global__ __launch_bounds__(256) void attn_merge_kernel(const DecParams p) {
    constexpr float NEG_INF = -__builtin_huge_valf();
    constexpr int SUB = 256 / D;      /* thread subsets over the splits */
    constexpr int B = 16;             /* partial rows in flight per thread */
    __shared__ float s_m[TL_MERGE_MAX_SPLIT];
    __shared__ float s_lw[TL_MERGE_MAX_SPLIT];
    __shared__ float s_red[8];
    __shared__ float s_part[SUB][D];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u32 hq = blockIdx.x % p.n_head;
    const u32 grow = blockIdx.x / p.n_head;
    const u32 si = grow / p.rows_per_seq, r = grow % p.rows_per_seq;
    const u32 ns = p.n_split;
    const u64 pb = ((u64)grow * p.n_head + hq) * ns;
    const int d = tid % D, sub = tid / D;
    const float *src = p.ws_acc + pb * D + d;

    /* one round trip: split maxima/sums and the first B partial elements */
    float a[B];
#pragma unroll
    for (int k = 0; k < B; k++) {
        const u32 s = sub + k * SUB;
        a[k] = s < ns ? src[(u64)s * D] : 0.f;
    }
    float mm = NEG_INF;
    for (u32 s = tid; s < ns; s += 256) {
        const float2 ml = p.ws_ml[pb + s];
        s_m[s] = ml.x;
        s_lw[s] = ml.y;
        mm = fmaxf(mm, ml.x);
    }
    mm = group_max<64>(mm);
    if (lane == 0) s_red[wave] = mm;
    __syncthreads();
    mm = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float mu = (mm == NEG_INF) ? 0.f : mm;
    float L = 0.f;
    for (u32 s = tid; s < ns; s += 256) {
        const float w = fast_exp2(s_m[s] - mu);
        s_m[s] = w;
        L += w * s_lw[s];
    }
    L = group_sum<64>(L);
    if (lane == 0) s_red[4 + wave] = L;
    __syncthreads();
    L = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);

    float O = 0.f;
#pragma unroll
    for (int k = 0; k < B; k++) {
        const u32 s = sub + k * SUB;
        if (s < ns) O = fmaf(s_m[s], a[k], O);
    }
    for (u32 s0 = B * SUB; s0 < ns; s0 += B * SUB) {   /* more than B*SUB splits */
#pragma unroll
        for (int k = 0; k < B; k++) {
            const u32 s = s0 + sub + k * SUB;
            a[k] = s < ns ? src[(u64)s * D] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < B; k++) {
            const u32 s = s0 + sub + k * SUB;
            if (s < ns) O = fmaf(s_m[s], a[k], O);
        }
    }
    s_part[sub][d] = O;
    __syncthreads();
    if (tid < D) {
        float o = 0.f;
#pragma unroll
        for (int k = 0; k < SUB; k++) o += s_part[k][tid];
        p.seq[si].dst[(u64)r * p.q_stride + (u64)hq * D + tid] = o / L;
    }
}

/* One decode kernel instance: entry point and K (or V) bytes per wave tile
 * (the RoPE-fusing instances are separate so the plain ones carry none of
 * its code):
 * 4 KB (16 keys at head_dim 128).  Small tiles give each wave more pipeline
 * iterations per chunk and keep GQA groups of up to 8 heads within two waves
 * per SIMD (8 KB tiles measured slower: 35.1 vs 31.8 us at config 4). */
struct DecKernel {
    const void *fn;
    int tile_bytes;
};

template <int D>
static DecKernel pick_kernel(int G, bool rope) {
    switch (G) {
#define TL_CASE(g)                                                                        \
    case g:                                                                               \
        if (rope) return {(const void *)attn_decode_kernel<D, g, 4096, true>, 4096};      \
        return {(const void *)attn_decode_kernel<D, g, 4096, false>, 4096};
        TL_CASE(1) TL_CASE(2) TL_CASE(3) TL_CASE(4)
        TL_CASE(5) TL_CASE(6) TL_CASE(7) TL_CASE(8)
#undef TL_CASE
    default:
        return {nullptr, 0};
    }
}

static u32 env_u32(const char *name, u32 dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    return (u32)strtoul(s, NULL, 10);
}

static int cu_count() {
    static int cus[16] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

/* resident workgroups per CU of a kernel (cached per entry point) */
static int resident_per_cu(const void *fn) {
    static const void *keys[64];
    static int vals[64];
    static int n = 0;
    for (int i = 0; i < n; i++)
        if (keys[i] == fn) return vals[i];
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, 256, 0) != hipSuccess || b < 1) b = 1;
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
int tl_launch_decode(DecParams &p, u32 n_rows_total, u32 head_dim, u32 G,
                     u32 max_vis, hipStream_t st) {
    DecKernel K;
    switch (head_dim) {
    case 64: K = pick_kernel<64>((int)G, p.rope.rdim != 0); break;
    case 128: K = pick_kernel<128>((int)G, p.rope.rdim != 0); break;
    case 256: K = pick_kernel<256>((int)G, p.rope.rdim != 0); break;
    default: return tl_fail(TL_EINVAL, "head_dim %u", head_dim);
    }
    if (!K.fn) return tl_fail(TL_EINVAL, "gqa ratio %u unsupported (1..8)", G);
    const u32 tk = (u32)K.tile_bytes / (2 * head_dim);   /* keys per wave tile */
    /* two workgroups per CU: measured best on MI355X for both tile sizes
     * (one resident wave of workgroups; more per CU only shortens chunks) */
    int per_cu = resident_per_cu(K.fn);
    if (per_cu > 2) per_cu = 2;
    const u32 target = env_u32("TL_DECODE_WGS", (u32)(per_cu * cu_count()));
    const u64 n_groups = (u64)n_rows_total * p.n_kv;
    u32 n_split = (u32)((target + n_groups - 1) / n_groups);
    const u32 max_split = (max_vis + 4 * tk - 1) / (4 * tk);    /* >= one tile per wave */
    const u32 min_split = (max_vis + TL_DEC_MAX_CHUNK - 1) / TL_DEC_MAX_CHUNK;
    if (n_split > max_split) n_split = max_split;
    if (n_split < min_split) n_split = min_split;
    if (n_split < 1) n_split = 1;
    const u32 chunk = (max_vis + n_split - 1) / n_split;
    n_split = (max_vis + chunk - 1) / chunk;
    if (n_split > TL_MERGE_MAX_SPLIT)
        return tl_fail(TL_EINVAL, "decode: %u keys need %u splits", max_vis, n_split);
    p.chunk = chunk;
    p.n_split = n_split;
    p.counters = nullptr;
    const bool in_kernel_merge = n_split > 1 && G * n_split <= 2048 &&
                                 !env_u32("TL_DECODE_MERGE_KERNEL", 0);
    if (n_split > 1) {
        TlWorkspace *w;
        size_t parts = (size_t)n_rows_total * p.n_head * n_split;
        int rc = tl_workspace_get(parts * head_dim, parts, in_kernel_merge ? n_groups : 0, &w);
        if (rc) return rc;
        p.ws_acc = w->acc;
        p.ws_ml = (float2 *)w->ml;
        if (in_kernel_merge) p.counters = w->cnt;
    }
    void *args[] = {(void *)&p};
    HIP_TRY(hipLaunchKernel(K.fn, dim3(n_split * (u32)n_groups), dim3(256), args, 0, st));
    if (n_split == 1 || in_kernel_merge) return TL_OK;
    return tl_launch_merge(p, n_rows_total, head_dim, st);
}

int tl_launch_merge(const DecParams &p, u32 n_rows_total, u32 head_dim, hipStream_t st) {
    if (p.n_split > TL_MERGE_MAX_SPLIT) return tl_fail(TL_EINVAL, "merge: %u splits", p.n_split);
    dim3 mg(n_rows_total * p.n_head);
    switch (head_dim) {
    case 64: hipLaunchKernelGGL(attn_merge_kernel<64>, mg, dim3(256), 0, st, p); break;
    case 128: hipLaunchKernelGGL(attn_merge_kernel<128>, mg, dim3(256), 0, st, p); break;
    case 256: hipLaunchKernelGGL(attn_merge_kernel<256>, mg, dim3(256), 0, st, p); break;
    default: return tl_fail(TL_EINVAL, "merge: head_dim %u", head_dim);
    }
    HIP_TRY(hipGetLastError());
    return TL_OK;
}
