/* tl_decode_kernels.h — the decode attention kernels (templates) and their
 * device helpers, shared by the translation units that instantiate them:
 * tl_decode.hip (f16 cache, launch code, split merge) and tl_decode_q8.hip
 * (Q8_0 cache instances).  The design is described in tl_decode.hip. */
#pragma once
#include "tl_common.h"
#include "tl_internal.h"

#include <stdlib.h>
#include <string.h>
#include <type_traits>
#include <utility>

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

TL_DEV half2_t as_h2(u32 w) { return __builtin_bit_cast(half2_t, w); }


TL_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef u32 u32x4_t __attribute__((ext_vector_type(4)));

/* 16-byte streaming load (non-temporal: the cache is read once per step). */
TL_DEV uint4 ld_stream(const u16 *ptr) {
    u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)ptr);
    return make_uint4(v.x, v.y, v.z, v.w);
}

TL_DEV u32 perm_lo(u32 a, u32 b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
TL_DEV u32 perm_hi(u32 a, u32 b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }


/* Split merge as its own launch (prefill key splits, and decode splits whose
 * partials exceed the in-launch merge).  D/4 threads per output row of one
 * head, each owning a float4: it folds the n_split partials of its float4
 * with an online max, in batches of 8 (all loads of a batch requested
 * together): out = sum_s exp2(m_s - M) acc_s / sum_s exp2(m_s - M) l_s.
 * grid = ceil(rows * n_head * D/4 / 256), no LDS, no barriers. */
#define TL_MERGE_MAX_SPLIT 1024
/* the merge's arguments: a small block (the kernel arguments are copied per
 * launch, and a chunked prefill runs one merge per layer and chunk) */
struct MergeParams {
    float *dst[TL_MAX_BATCH_SEQ];
    uint32_t rows_per_seq, n_head, q_stride, n_split;
    const float *ws_acc;
    const float2 *ws_ml;
};
template <int D>
__global__ __launch_bounds__(256) void attn_merge_kernel(const MergeParams p, u32 n_out) {
    constexpr float NEG_INF = -__builtin_huge_valf();
    constexpr int C4 = D / 4;
    constexpr int K = 8;
    const u32 gid = blockIdx.x * 256 + threadIdx.x;
    const u32 o = gid / C4;                       /* (row, head) */
    if (o >= n_out) return;
    const u32 d = (gid % C4) * 4;
    const u32 hq = o % p.n_head, grow = o / p.n_head;
    const u32 si = grow / p.rows_per_seq, r = grow % p.rows_per_seq;
    const u32 ns = p.n_split;
    const u64 pb = (u64)o * ns;
    float M = NEG_INF, L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (u32 s0 = 0; s0 < ns; s0 += K) {
        float2 ml[K];
        float4 a[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            /* splits past the last are not loaded (uniform branch) */
            ml[k] = make_float2(NEG_INF, 0.f);
            a[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (s0 + k < ns) {
                ml[k] = p.ws_ml[pb + s0 + k];
                a[k] = *(const float4 *)&p.ws_acc[(pb + s0 + k) * D + d];
            }
        }
        float bm = NEG_INF;
#pragma unroll
        for (int k = 0; k < K; k++) bm = fmaxf(bm, ml[k].x);
        const float nm = fmaxf(M, bm);
        const float mu = (nm == NEG_INF) ? 0.f : nm;
        const float sc = fast_exp2(M - mu);
        L *= sc;
        O.x *= sc; O.y *= sc; O.z *= sc; O.w *= sc;
        M = nm;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const float w = fast_exp2(ml[k].x - mu);
            L = fmaf(w, ml[k].y, L);
            O.x = fmaf(w, a[k].x, O.x);
            O.y = fmaf(w, a[k].y, O.y);
            O.z = fmaf(w, a[k].z, O.z);
            O.w = fmaf(w, a[k].w, O.w);
        }
    }
    const float inv = 1.0f / L;
    *(float4 *)&p.dst[si][(u64)r * p.q_stride + (u64)hq * D + d] =
        make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
}

/* ------------------------------------------------------------------------ */
/* Decode attention, LDS-direct ring                                        */
/* ------------------------------------------------------------------------ */

/* One 16-byte-per-lane load straight into LDS (global_load_lds_dwordx4,
 * non-temporal: the cache is streamed once per step): lane i's 16 bytes land
 * at LDS byte address m0 + 16*i.  Issued from inline
 * assembly so the compiler does not wait for it before every LDS read; the
 * caller waits with an explicit vmcnt.  `base` must be wave-uniform. */
TL_DEV void lds_dma16(u32 m0, const void *base, u32 voff) {
    const u64 g = (u64)base;
    const u32 lo = __builtin_amdgcn_readfirstlane((u32)g);
    const u32 hi = __builtin_amdgcn_readfirstlane((u32)(g >> 32));
    const void *sb = (const void *)(((u64)hi << 32) | lo);
    /* m0 is an input operand (the compiler writes it); s_nop covers the
     * one-wait-state hazard between an M0 write and an LDS-direct load */
    __asm__ volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                     :: "v"(voff), "s"(sb), "{m0}"(__builtin_amdgcn_readfirstlane(m0)) : "memory");
}

/* One 4-byte-per-lane load straight into LDS (global_load_lds_dword):
 * lane i's word lands at m0 + 4*i; otherwise as lds_dma16. */
TL_DEV void lds_dma4(u32 m0, const void *base, u32 voff) {
    const u64 g = (u64)base;
    const u32 lo = __builtin_amdgcn_readfirstlane((u32)g);
    const u32 hi = __builtin_amdgcn_readfirstlane((u32)(g >> 32));
    const void *sb = (const void *)(((u64)hi << 32) | lo);
    __asm__ volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1 nt"
                     :: "v"(voff), "s"(sb), "{m0}"(__builtin_amdgcn_readfirstlane(m0)) : "memory");
}

/* Q8_0 tiles: 6 loads each (K and V values 2 + 2, K and V scales 1 + 1) */
TL_DEV void wait_tiles_q8(u32 n) {
    switch (n) {
    case 0: __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: __asm__ volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 2: __asm__ volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    default: __asm__ volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    }
}

/* wait until at most n tiles (8 loads each) are still in flight */
TL_DEV void wait_tiles(u32 n) {
    switch (n) {
    case 0: __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 2: __asm__ volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    default: __asm__ volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    }
}

/* Ring-kernel tile geometry: a K (or V) tile is 4 KB; a lane owns 16
 * consecutive dims (two 16-byte chunks) of one key in each of the tile's
 * two passes, so LPK = D/16 lanes share a key and every lane holds one key
 * pair (t, t + KPP) for the v_dot2 PV products. */
template <int D>
struct RCfg {
    static constexpr int LPK = D / 16;       /* lanes per key */
    static constexpr int KPP = 64 / LPK;     /* keys per pass */
    static constexpr int TK = 2 * KPP;       /* keys per tile */
    static constexpr int CPR = D / 8;        /* 16-byte chunks per row */
    static constexpr int UNITS = TK * CPR;   /* 16-byte units per K (or V) tile */
    static constexpr int LD = UNITS / 64;    /* loads per lane per K (or V) tile */
};

/* Lazy rescale margin (log2 units): the wave's running max (common to all
 * its lanes) moves only when a score exceeds it by more than this, so
 * probabilities stay <= 2^8 and most tiles skip the rescale. */
#define TL_DEC_TAU 8.0f

/* Q8_0 ring tiles per softmax chain of the matrix-core tile: the chain's
 * tiles share one max, one rescale decision and one exponential pass, and
 * their LDS reads and MFMAs interleave (1: a chain per tile) */
#define TL_DEC_Q8_CHAIN 2

/* With G <= LPK every head of the group has its own lane in each key
 * group, and the softmax of a tile runs once per (key pair, head) instead
 * of once per lane: lane sub handles head sub and keeps that head's running
 * sum in l[0]. */
template <int G, int LPK>
constexpr bool own_head_softmax() { return G <= LPK && LPK <= 16; }

/* ds_swizzle in bit-mask mode (32-lane halves): every lane of an LPK-lane
 * group reads lane H of its group. */
template <int LPK, int H>
TL_DEV u32 group_bcast(u32 v) {
    return (u32)__builtin_amdgcn_ds_swizzle((int)v, (32 - LPK) | (H << 5));
}
template <int LPK, int G, int... H>
TL_DEV void group_bcast_all(u32 (&pp)[G], u32 v, std::integer_sequence<int, H...>) {
    ((pp[H] = group_bcast<LPK, H>(v)), ...);
}

/* Online-softmax step of one tile for the G heads of a lane's key pair:
 * scores s0/s1 (identical across the LPK lanes of a key group) -> packed
 * f16 probabilities pp[h].  The running max m[h] is common to the wave and
 * moves only when a score exceeds it by more than TL_DEC_TAU (then l and
 * acc are rescaled).  With own_head_softmax, lane sub computes the two
 * probabilities of head sub only and the group reads them with one swizzle
 * per head (2 exponentials per lane instead of 2G); l[0] then holds head
 * sub's sum.  Otherwise every lane computes every head and l[h] holds head
 * h's sum. */
template <int G, int LPK>
TL_DEV void tile_softmax(const float (&s0)[G], const float (&s1)[G], int sub, float (&m)[G],
                         float (&l)[G], float (&acc)[G][16], u32 (&pp)[G]) {
    constexpr float NEG_INF = -__builtin_huge_valf();
    if constexpr (own_head_softmax<G, LPK>()) {
        float a0 = s0[0], a1 = s1[0], mo = m[0];
#pragma unroll
        for (int h = 1; h < G; h++)
            if (sub == h) { a0 = s0[h]; a1 = s1[h]; mo = m[h]; }
        if (__builtin_amdgcn_ballot_w64(sub < G && fmaxf(a0, a1) > mo + TL_DEC_TAU)) {
            /* rare: move the wave's common max of each head that needs it */
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float mx = fmaxf(s0[h], s1[h]);
                if (__builtin_amdgcn_ballot_w64(mx > m[h] + TL_DEC_TAU)) {
                    const float mn = group_max<64>(mx);
                    const float alpha = fast_exp2(m[h] - mn);
                    if (sub == h) l[0] *= alpha;
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[h][e] *= alpha;
                    m[h] = mn;
                }
            }
            mo = m[0];
#pragma unroll
            for (int h = 1; h < G; h++)
                if (sub == h) mo = m[h];
        }
        const float mu = (mo == NEG_INF) ? 0.f : mo;
        const float p0 = fast_exp2(a0 - mu), p1 = fast_exp2(a1 - mu);
        l[0] += p0 + p1;
        group_bcast_all<LPK, G>(pp, pack_f16x2_fast(p0, p1), std::make_integer_sequence<int, G>{});
    } else {
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float mx = fmaxf(s0[h], s1[h]);
            if (__builtin_amdgcn_ballot_w64(mx > m[h] + TL_DEC_TAU)) {
                /* rare: move the wave's common max to this tile's max */
                const float mn = group_max<64>(mx);
                const float alpha = fast_exp2(m[h] - mn);
                l[h] *= alpha;
#pragma unroll
                for (int e = 0; e < 16; e++) acc[h][e] *= alpha;
                m[h] = mn;
            }
            const float mu = (m[h] == NEG_INF) ? 0.f : m[h];
            const float p0 = fast_exp2(s0[h] - mu), p1 = fast_exp2(s1[h] - mu);
            l[h] += p0 + p1;
            pp[h] = pack_f16x2_fast(p0, p1);
        }
    }
}

/* Scores, online softmax and PV of one staged tile (keys tbase..tbase+TK-1,
 * those >= kend masked) into the lane group's running state (l, acc); the
 * running max m is common to the wave.  Logical
 * chunk c of tile row t sits at LDS unit t*CPR + (c ^ (t & 1)). */
template <int D, int G>
TL_DEV void ring_tile(const uint4 *tk, const uint4 *tv, const u32 (&qr)[G][8], u32 tbase,
                      u32 kend, int lane, float (&m)[G], float (&l)[G], float (&acc)[G][16]) {
    using C = RCfg<D>;
    constexpr int LPK = C::LPK, KPP = C::KPP, CPR = C::CPR;
    constexpr float NEG_INF = -__builtin_huge_valf();
    const int g = lane / LPK, sub = lane % LPK;
    const int t0 = g, t1 = KPP + g;
    const int c0 = (2 * sub) ^ (g & 1), c1 = (2 * sub + 1) ^ (g & 1);
    const uint4 ka0 = tk[t0 * CPR + c0], ka1 = tk[t0 * CPR + c1];
    const uint4 kb0 = tk[t1 * CPR + c0], kb1 = tk[t1 * CPR + c1];
    const u32 ka[8] = {ka0.x, ka0.y, ka0.z, ka0.w, ka1.x, ka1.y, ka1.z, ka1.w};
    const u32 kb[8] = {kb0.x, kb0.y, kb0.z, kb0.w, kb1.x, kb1.y, kb1.z, kb1.w};
    float s0[G], s1[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            a = __builtin_amdgcn_fdot2(as_h2(ka[w]), as_h2(qr[h][w]), a, false);
            b = __builtin_amdgcn_fdot2(as_h2(kb[w]), as_h2(qr[h][w]), b, false);
        }
        s0[h] = a;
        s1[h] = b;
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
        s0[h] = group_sum<LPK>(s0[h]);
        s1[h] = group_sum<LPK>(s1[h]);
        /* keep the sums unconditional (the compiler would otherwise move
         * each dot-product chain into its own divergent branch) */
        __asm__ volatile("" : "+v"(s0[h]), "+v"(s1[h]));
    }
    if (tbase + (u32)(2 * KPP) > kend) {   /* wave-uniform: only a chunk's last tile */
        const bool v0 = tbase + (u32)t0 < kend, v1 = tbase + (u32)t1 < kend;
#pragma unroll
        for (int h = 0; h < G; h++) {
            s0[h] = v0 ? s0[h] : NEG_INF;
            s1[h] = v1 ? s1[h] : NEG_INF;
        }
    }
    const uint4 va0 = tv[t0 * CPR + c0], va1 = tv[t0 * CPR + c1];
    const uint4 vb0 = tv[t1 * CPR + c0], vb1 = tv[t1 * CPR + c1];
    u32 pp[G];
    tile_softmax<G, LPK>(s0, s1, sub, m, l, acc, pp);
    const u32 va[8] = {va0.x, va0.y, va0.z, va0.w, va1.x, va1.y, va1.z, va1.w};
    const u32 vb[8] = {vb0.x, vb0.y, vb0.z, vb0.w, vb1.x, vb1.y, vb1.z, vb1.w};
#pragma unroll
    for (int w = 0; w < 8; w++) {
        const half2_t lo = as_h2(perm_lo(va[w], vb[w]));   /* (V[t0][2w], V[t1][2w]) */
        const half2_t hi = as_h2(perm_hi(va[w], vb[w]));
#pragma unroll
        for (int h = 0; h < G; h++) {
            acc[h][2 * w] = __builtin_amdgcn_fdot2(lo, as_h2(pp[h]), acc[h][2 * w], false);
            acc[h][2 * w + 1] = __builtin_amdgcn_fdot2(hi, as_h2(pp[h]), acc[h][2 * w + 1], false);
        }
    }
}

/* ring_tile over a Q8_0 tile.  The tile's int8 rows are stored as loaded:
 * row t holds D bytes = LPK 16-byte units, and lane (g, sub) reads unit sub
 * of keys t0 = g and t1 = KPP + g (its 16 dims, as in ring_tile: one wave
 * read covers 1 KB of consecutive LDS).  sk / sv hold the tile's binary16
 * scales [TK][D/32]; the lane's 16 dims sit in block sub/2.
 * Scores: the exact int8 values (f16) dot q, times the key's scale (f32).
 * PV: V is dequantized to f16 (q * d rounded once) pairwise across the two
 * keys, then v_dot2 with the packed probabilities as in ring_tile. */
template <int D, int G>
TL_DEV void ring_tile_q8(const uint4 *tk, const uint4 *tv, const u16 *sk, const u16 *sv,
                         const u32 (&qr)[G][8], u32 tbase, u32 kend, int lane, float (&m)[G],
                         float (&l)[G], float (&acc)[G][16]) {
    using C = RCfg<D>;
    constexpr int LPK = C::LPK, KPP = C::KPP, NB = D / 32;
    constexpr float NEG_INF = -__builtin_huge_valf();
    const int g = lane / LPK, sub = lane % LPK;
    const int t0 = g, t1 = KPP + g;
    const uint4 ka = tk[t0 * LPK + sub], kb = tk[t1 * LPK + sub];
    const float dk0 = (float)__builtin_bit_cast(_Float16, sk[t0 * NB + sub / 2]);
    const float dk1 = (float)__builtin_bit_cast(_Float16, sk[t1 * NB + sub / 2]);
    const u32 kaw[4] = {ka.x, ka.y, ka.z, ka.w}, kbw[4] = {kb.x, kb.y, kb.z, kb.w};
    half2_t fa[8], fb[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        i8x4_to_f16(kaw[w], fa[2 * w], fa[2 * w + 1]);
        i8x4_to_f16(kbw[w], fb[2 * w], fb[2 * w + 1]);
    }
    float s0[G], s1[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            a = __builtin_amdgcn_fdot2(fa[w], as_h2(qr[h][w]), a, false);
            b = __builtin_amdgcn_fdot2(fb[w], as_h2(qr[h][w]), b, false);
        }
        s0[h] = a * dk0;
        s1[h] = b * dk1;
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
        s0[h] = group_sum<LPK>(s0[h]);
        s1[h] = group_sum<LPK>(s1[h]);
        __asm__ volatile("" : "+v"(s0[h]), "+v"(s1[h]));
    }
    if (tbase + (u32)(2 * KPP) > kend) {   /* wave-uniform: only a chunk's last tile */
        const bool v0 = tbase + (u32)t0 < kend, v1 = tbase + (u32)t1 < kend;
#pragma unroll
        for (int h = 0; h < G; h++) {
            s0[h] = v0 ? s0[h] : NEG_INF;
            s1[h] = v1 ? s1[h] : NEG_INF;
        }
    }
    const uint4 va = tv[t0 * LPK + sub], vb = tv[t1 * LPK + sub];
    const u32 dvb = (u32)sv[t0 * NB + sub / 2] | ((u32)sv[t1 * NB + sub / 2] << 16);
    u32 pp[G];
    tile_softmax<G, LPK>(s0, s1, sub, m, l, acc, pp);
    const half2_t dv2 = as_h2(dvb);                 /* (d of key t0, d of key t1) */
    const u32 vaw[4] = {va.x, va.y, va.z, va.w}, vbw[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        /* bytes (a0 b0 a1 b1) and (a2 b2 a3 b3): key pairs of dims 4w .. 4w+3 */
        const u32 x01 = __builtin_amdgcn_perm(vbw[w], vaw[w], 0x05010400u);
        const u32 x23 = __builtin_amdgcn_perm(vbw[w], vaw[w], 0x07030602u);
        half2_t e[4];
        i8x4_to_f16(x01, e[0], e[1]);
        i8x4_to_f16(x23, e[2], e[3]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const half2_t vv = e[k] * dv2;
#pragma unroll
            for (int h = 0; h < G; h++)
                acc[h][4 * w + k] = __builtin_amdgcn_fdot2(vv, as_h2(pp[h]), acc[h][4 * w + k], false);
        }
    }
}

/* ---- matrix-core tile (MF instances) ----
 * The same staged tile (row t, chunk c at LDS unit t*CPR + (c ^ (t & 1)))
 * computed on v_mfma 16x16 tiles with the G heads of the group as the
 * columns (16 - G columns carry q = 0 and are never written out):
 *   S^T[key][head] = K . Q^T   v_mfma_f32_16x16x32_f16 per 16-key block and
 *                              32 dims: A = 8 dims of key row (lane & 15)
 *                              (chunk 4j + lane/16), B = the same dims of q
 *                              (registers);
 *   O^T[dim][head] += V^T . P^T  v_mfma_f32_16x16x16f16 per 16-key block and
 *                              16 dims: A = V^T read with ds_read_b64_tr_b16,
 *                              B = the block's probabilities exactly as the
 *                              S accumulator leaves them (lane holds keys
 *                              4*(lane/16) + i of head lane & 15).
 * A lane owns one head column: its running max m (common to the column's
 * four lanes), its share l of the column's sum and D/4 output dims, so the
 * rescale and the final combine need no cross-lane moves besides the
 * column max of each tile (two shuffles).  Tiles of 8 keys (head_dim 256)
 * fill the block's other 8 rows with copies whose scores are masked. */
typedef _Float16 dh8_t __attribute__((ext_vector_type(8)));
typedef _Float16 dh4_t __attribute__((ext_vector_type(4)));
typedef float df4_t __attribute__((ext_vector_type(4)));
typedef short ds4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ds4_t lds_ds4_t;

TL_DEV dh8_t u4_as_h8(uint4 v) {
    const u32x4_t t = {v.x, v.y, v.z, v.w};
    return __builtin_bit_cast(dh8_t, t);
}

/* within each 16-lane group, lane i receives element (i & 3) of the 4-half
 * vector addressed by lane 4e + (i >> 2), e = 0..3 (a 4x16 -> 16x4
 * transpose when lane j addresses row j >> 2, columns 4 (j & 3) ..) */
TL_DEV dh4_t ld_tr16_h4(const _Float16 *lds_ptr) {
    const ds4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ds4_t *)(lds_ptr));
    return __builtin_bit_cast(dh4_t, v);
}

/* Mask, online softmax and PV of one tile's score blocks s (keys
 * tbase + 16b + 4*(lane/16) + i of head lane & 15) against the f16 V tile tv
 * (row t, chunk c at unit t*CPR + (c ^ (t & 1))). */
/* Column masks when a group holds several batch rows: column lane & 15 sees
 * the keys [klo, khi) of its own row; the rows' ranges differ only below
 * ulo (their window starts) and from uhi on (their ends), so tiles inside
 * [ulo, uhi) need no column mask. */
struct MfRows {
    u32 klo, khi;   /* this lane's column */
    u32 ulo, uhi;   /* keys every row of the group sees */
    bool multi;     /* more than one row */
};

/* NTL tiles' score blocks at once (tile t: s[t], V tile tv[t], first key
 * tbase[t]): one max, one rescale decision and one running sum for all of
 * them, so several tiles cost one softmax chain. */
template <int D, int G, int NTL>
TL_DEV void mf_softmax_pvn(df4_t (&s)[NTL][(RCfg<D>::TK + 15) / 16], const uint4 *const (&tv)[NTL],
                           const u32 (&tbase)[NTL], u32 kend, const MfRows &mr, int lane,
                           float &m, float &l, df4_t (&O)[D / 16]) {
    using C = RCfg<D>;
    constexpr int TK = C::TK, CPR = C::CPR, NB = (TK + 15) / 16, DB = D / 16;
    constexpr float NEG_INF = -__builtin_huge_valf();
    const int g = lane >> 4, c = lane & 15;
#pragma unroll
    for (int tl = 0; tl < NTL; tl++) {
        /* keys past the chunk (wave-uniform: only a chunk's last tiles),
         * the copied rows of 8-key tiles, and keys outside a column's own
         * row */
        const u32 tb = tbase[tl];
        const bool cols = mr.multi && (tb < mr.ulo || tb + (u32)TK > mr.uhi);
        if (TK < 16 || tb + (u32)TK > kend || cols) {
            /* the lane's visible keys [lo, hi) as one unsigned range test
             * (key - lo < n); a select per element, no branch */
            const u32 lo = cols ? mr.klo : 0u;
            const u32 hi = cols ? min(mr.khi, kend) : kend;
            const u32 n = hi > lo ? hi - lo : 0u;
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const u32 kk = (u32)(16 * b + 4 * g + i);
                    const bool live = kk < (u32)TK && tb + kk - lo < n;
                    s[tl][b][i] = live ? s[tl][b][i] : NEG_INF;
                }
        }
    }
    float mx = NEG_INF;
#pragma unroll
    for (int tl = 0; tl < NTL; tl++)
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[tl][b][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (__builtin_amdgcn_ballot_w64(mx > m + TL_DEC_TAU)) {
        /* rare: move the column's reference to this tile's max */
        const bool mv = mx > m + TL_DEC_TAU;
        const float a = mv ? fast_exp2(m - mx) : 1.f;
        m = mv ? mx : m;
        l *= a;
#pragma unroll
        for (int db = 0; db < DB; db++) O[db] *= a;
    }
    const float mu = (m == NEG_INF) ? 0.f : m;
    dh4_t pb[NTL][NB];
#pragma unroll
    for (int tl = 0; tl < NTL; tl++)
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[i] = fast_exp2(s[tl][b][i] - mu);
                l += p[i];
            }
            pb[tl][b] = dh4_t{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
        }
#pragma unroll
    for (int tl = 0; tl < NTL; tl++) {
        const _Float16 *vh = (const _Float16 *)tv[tl];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int t = (16 * b + 4 * g + (c >> 2)) % TK;
#pragma unroll
            for (int db = 0; db < DB; db++) {
                const int x = 16 * db + 4 * (c & 3);
                const dh4_t va = ld_tr16_h4(vh + (t * CPR + ((x >> 3) ^ (t & 1))) * 8 + (x & 7));
                O[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb[tl][b], O[db], 0, 0, 0);
            }
        }
    }
}

template <int D, int G>
TL_DEV void mf_softmax_pv(df4_t (&s)[(RCfg<D>::TK + 15) / 16], const uint4 *tv, u32 tbase,
                          u32 kend, const MfRows &mr, int lane, float &m, float &l,
                          df4_t (&O)[D / 16]) {
    constexpr int NB = (RCfg<D>::TK + 15) / 16;
    df4_t s1[1][NB];
#pragma unroll
    for (int b = 0; b < NB; b++) s1[0][b] = s[b];
    const uint4 *const tv1[1] = {tv};
    const u32 tb1[1] = {tbase};
    mf_softmax_pvn<D, G, 1>(s1, tv1, tb1, kend, mr, lane, m, l, O);
}

template <int D, int G>
TL_DEV void mfma_tile(const uint4 *tk, const uint4 *tv, const dh8_t (&qb)[D / 32], u32 tbase,
                      u32 kend, const MfRows &mr, int lane, float &m, float &l,
                      df4_t (&O)[D / 16]) {
    using C = RCfg<D>;
    constexpr int TK = C::TK, CPR = C::CPR, NB = (TK + 15) / 16, QS = D / 32;
    const int g = lane >> 4, c = lane & 15;
    df4_t s[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int t = (16 * b + c) % TK;
        df4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < QS; j++)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(u4_as_h8(tk[t * CPR + ((4 * j + g) ^ (t & 1))]),
                                                         qb[j], acc, 0, 0, 0);
        s[b] = acc;
    }
    mf_softmax_pv<D, G>(s, tv, tbase, kend, mr, lane, m, l, O);
}

/* mfma_tile over NTL Q8_0 tiles at once (tile t: int8 rows as loaded in
 * stage[t], row r at byte r*D; f16 scales [TK][D/32], K at scl[t], V at
 * scl[t] + 64).  Scores: every 32-dim step of the QK MFMA
 * is exactly one scale block, so the exact int8 values (f16) go into the
 * MFMA and each step's result is scaled by its key's block scale in f32, as
 * the vector tile does.  V: the wave reads its int8 K fragments and V rows
 * into registers, then writes V dequantized to f16 (RNE(q * d), as the
 * vector tile's PV operands) over the same stage, laid out like an f16 tile
 * (4 KB: the int8 K and V halves together), and the PV step reads it as
 * one.  The LDS operations of one wave run in order, so every lane's reads
 * precede the overwrite. */
template <int D, int G, int NTL>
TL_DEV void mfma_tile_q8n(uint4 *const (&stage)[NTL], const u16 *const (&scl)[NTL],
                          const dh8_t (&qb)[D / 32], const u32 (&tbase)[NTL], u32 kend,
                          const MfRows &mr, int lane, float &m, float &l, df4_t (&O)[D / 16]) {
    using C = RCfg<D>;
    constexpr int TK = C::TK, CPR = C::CPR, NB = (TK + 15) / 16, QS = D / 32, NSB = D / 32;
    constexpr int VU = TK * CPR / 64;              /* 8-byte V units per lane */
    const int g = lane >> 4, c = lane & 15;
    /* every LDS read of the tiles first (values, then the scales the lane
     * needs), so the wave waits once */
    uint2 kw[NTL][NB][QS], vw[NTL][VU];
    u16 ksc[NTL][NB][4][QS], vsc[NTL][VU];
#pragma unroll
    for (int tl = 0; tl < NTL; tl++) {
        const uint8_t *k8 = (const uint8_t *)stage[tl], *v8 = k8 + TK * D;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int t = (16 * b + c) % TK;
#pragma unroll
            for (int j = 0; j < QS; j++) kw[tl][b][j] = *(const uint2 *)(k8 + t * D + 8 * (4 * j + g));
        }
#pragma unroll
        for (int k = 0; k < VU; k++) {
            const int u = lane + 64 * k;
            vw[tl][k] = *(const uint2 *)(v8 + (u / CPR) * D + 8 * (u % CPR));
        }
    }
#pragma unroll
    for (int tl = 0; tl < NTL; tl++) {
        const u16 *sk = scl[tl], *sv = sk + 64;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const u16 *row = sk + ((16 * b + 4 * g + i) % TK) * NSB;   /* NSB scales, 4-byte aligned */
#pragma unroll
                for (int j = 0; j < QS; j += 2) {
                    const u32 w = *(const u32 *)(row + j);
                    ksc[tl][b][i][j] = (u16)(w & 0xffffu);
                    ksc[tl][b][i][j + 1] = (u16)(w >> 16);
                }
            }
#pragma unroll
        for (int k = 0; k < VU; k++) {
            const int u = lane + 64 * k;
            vsc[tl][k] = sv[(u / CPR) * NSB + (u % CPR) / 4];
        }
    }
    df4_t s[NTL][NB];
#pragma unroll
    for (int tl = 0; tl < NTL; tl++)
#pragma unroll
        for (int b = 0; b < NB; b++) {
            df4_t acc[QS];
#pragma unroll
            for (int j = 0; j < QS; j++) {
                tl_half2 h0, h1, h2, h3;
                i8x4_to_f16(kw[tl][b][j].x, h0, h1);
                i8x4_to_f16(kw[tl][b][j].y, h2, h3);
                const u32x4_t kx = {__builtin_bit_cast(u32, h0), __builtin_bit_cast(u32, h1),
                                    __builtin_bit_cast(u32, h2), __builtin_bit_cast(u32, h3)};
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dh8_t, kx), qb[j],
                                                                df4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
            s[tl][b] = df4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < QS; j++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    s[tl][b][i] = fmaf(acc[j][i], (float)__builtin_bit_cast(_Float16, ksc[tl][b][i][j]),
                                       s[tl][b][i]);
        }
#pragma unroll
    for (int tl = 0; tl < NTL; tl++)
#pragma unroll
        for (int k = 0; k < VU; k++) {
            const int u = lane + 64 * k, t = u / CPR, cc = u % CPR;
            stage[tl][t * CPR + (cc ^ (t & 1))] = q8_dequant8(vw[tl][k], (u32)vsc[tl][k]);
        }
    __builtin_amdgcn_wave_barrier();
    const uint4 *tv[NTL];
#pragma unroll
    for (int tl = 0; tl < NTL; tl++) tv[tl] = stage[tl];
    mf_softmax_pvn<D, G, NTL>(s, tv, tbase, kend, mr, lane, m, l, O);
}

/* mfma_tile over one Q8_0 tile (scales: K at scl, V at scl + 64) */
template <int D, int G>
TL_DEV void mfma_tile_q8(uint4 *stage, const u16 *scl, const dh8_t (&qb)[D / 32], u32 tbase,
                         u32 kend, const MfRows &mr, int lane, float &m, float &l,
                         df4_t (&O)[D / 16]) {
    uint4 *const st[1] = {stage};
    const u16 *const sc[1] = {scl};
    const u32 tb[1] = {tbase};
    mfma_tile_q8n<D, G, 1>(st, sc, qb, tb, kend, mr, lane, m, l, O);
}

constexpr int pow2_floor(int x) { return x >= 16 ? 16 : x >= 8 ? 8 : x >= 4 ? 4 : x >= 2 ? 2 : 1; }

/* Merge of a group's n_split partials by its last workgroup, in registers:
 * TPC threads per output float4 (h, d..d+3) each fold their share of the
 * splits with an online max, then combine across the TPC lanes with DPP:
 * out = sum_s exp2(m_s - M) acc_s / sum_s exp2(m_s - M) l_s.  The first
 * batch of partial rows and every (m, l) pair are requested together
 * (device-coherent loads); the pairs go through LDS (s_ml: G*n_split). */
template <int D, int G, int NT>
TL_DEV void split_merge_regs(const DecParams &p, u32 pb, u32 kvh, u32 r, u32 gh, u32 ncol,
                             const DecSeq &sq, float2 *s_ml) {
    constexpr float NEG_INF = -__builtin_huge_valf();
    constexpr int COLS_MAX = G * D / 4;
    const int COLS = (int)ncol * (D / 4);
    constexpr int TPC = pow2_floor(NT / COLS_MAX > 16 ? 16 : (NT / COLS_MAX < 1 ? 1 : NT / COLS_MAX));
    constexpr int K = 8;                       /* splits per load batch */
    const int tid = threadIdx.x;
    const u32 ns = p.n_split;
    const __amdgpu_buffer_rsrc_t rml = buf_rsrc(p.ws_ml + pb);
    const __amdgpu_buffer_rsrc_t racc = buf_rsrc(p.ws_acc + (u64)pb * D);
    const int part = tid % TPC;
    const int col0 = tid / TPC;
    u32x4v_t a[K];
    auto load_batch = [&](int col, u32 s0) {
        const int h = col / (D / 4), d = (col % (D / 4)) * 4;
#pragma unroll
        for (int k = 0; k < K; k++) {
            const u32 s = min(s0 + k * TPC, ns - 1);
            const u32 off = (((u32)h * ns + s) * D + d) * 4;
            a[k] = __builtin_amdgcn_raw_buffer_load_b128(racc, off, 0, TL_SC1);
        }
    };
    if (col0 < COLS) load_batch(col0, (u32)part);
    for (u32 i = tid; i < ncol * ns; i += NT) {
        const u32x2v_t ml = __builtin_amdgcn_raw_buffer_load_b64(rml, i * 8, 0, TL_SC1);
        s_ml[i] = make_float2(__uint_as_float(ml[0]), __uint_as_float(ml[1]));
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int col = col0; col < COLS; col += NT / TPC) {
        const int h = col / (D / 4), d = (col % (D / 4)) * 4;
        const float2 *mlh = s_ml + (u32)h * ns;
        float M = NEG_INF, L = 0.f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        for (u32 s0 = part; s0 < ns; s0 += K * TPC) {
            if (col != col0 || s0 != (u32)part) load_batch(col, s0);
            float2 ml[K];
            float bm = NEG_INF;
#pragma unroll
            for (int k = 0; k < K; k++) {
                const u32 s = s0 + k * TPC;
                ml[k] = mlh[min(s, ns - 1)];
                if (s >= ns) ml[k] = make_float2(NEG_INF, 0.f);   /* past the last split */
                bm = fmaxf(bm, ml[k].x);
            }
            const float nm = fmaxf(M, bm);
            const float mu = (nm == NEG_INF) ? 0.f : nm;
            const float sc = fast_exp2(M - mu);
            L *= sc;
            O.x *= sc; O.y *= sc; O.z *= sc; O.w *= sc;
            M = nm;
#pragma unroll
            for (int k = 0; k < K; k++) {
                const float w = fast_exp2(ml[k].x - mu);
                L = fmaf(w, ml[k].y, L);
                O.x = fmaf(w, __uint_as_float(a[k][0]), O.x);
                O.y = fmaf(w, __uint_as_float(a[k][1]), O.y);
                O.z = fmaf(w, __uint_as_float(a[k][2]), O.z);
                O.w = fmaf(w, __uint_as_float(a[k][3]), O.w);
            }
        }
        if constexpr (TPC > 1) {
            const float Mg = group_max<TPC>(M);
            const float mu = (Mg == NEG_INF) ? 0.f : Mg;
            const float e = fast_exp2(M - mu);
            L = group_sum<TPC>(L * e);
            O.x = group_sum<TPC>(O.x * e);
            O.y = group_sum<TPC>(O.y * e);
            O.z = group_sum<TPC>(O.z * e);
            O.w = group_sum<TPC>(O.w * e);
        }
        if (part == 0) {
            const float inv = 1.0f / L;
            *(float4 *)&sq.dst[(u64)(r + h / gh) * p.q_stride + (u64)(kvh * gh + h % gh) * D + d] =
                make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
        }
    }
}

/* Bounded waits of the in-launch split merge (polls of device-coherent
 * words, each a memory round trip): a split that waits longer gives up, and
 * the last split to arrive merges what nobody else claimed. */
#define TL_MERGE_SPIN 64
#define TL_MERGE_BACKOFF 4   /* s_sleep units (64 clocks) between polls */

/* Merge one slice of a group's output: columns [slice*cps, slice*cps + cps)
 * of the G*D/4 float4 columns (head, 4 dims).  One wave per column, lane s
 * holding split s (n_split <= 64): out = sum_s w_s acc_s / sum_s w_s l_s,
 * w_s = exp2(m_s - max m).  Partial rows and their (m, l, epoch) records
 * (float4 per partial) are read with device-coherent loads. */
template <int D, int W>
TL_DEV void merge_slice(const DecParams &p, u32 pb, u32 r, u32 kvh, u32 gh, u32 ncol,
                        const DecSeq &sq, u32 slice, u32 cps) {
    constexpr float NEG_INF = -__builtin_huge_valf();
    const u32 COLS = ncol * (D / 4);
    const u32 ns = p.n_split;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const u32 c0 = slice * cps, c1 = min(c0 + cps, COLS);
    const __amdgpu_buffer_rsrc_t rrec = buf_rsrc((const float4 *)p.ws_ml + pb);
    const __amdgpu_buffer_rsrc_t racc = buf_rsrc(p.ws_acc + (u64)pb * D);
    for (u32 col = c0 + (u32)wave; col < c1; col += W) {
        const u32 h = col / (D / 4), d = (col % (D / 4)) * 4;
        float m = NEG_INF, l = 0.f;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if ((u32)lane < ns) {
            const u32 pi = h * ns + (u32)lane;
            const u32x4v_t ml = __builtin_amdgcn_raw_buffer_load_b128(rrec, pi * 16, 0, TL_SC1);
            const u32x4v_t v = __builtin_amdgcn_raw_buffer_load_b128(racc, (pi * D + d) * 4, 0, TL_SC1);
            m = __uint_as_float(ml[0]);
            l = __uint_as_float(ml[1]);
            a = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                            __uint_as_float(v[3]));
        }
        const float M = group_max<64>(m);
        const float mu = (M == NEG_INF) ? 0.f : M;
        const float w = fast_exp2(m - mu);
        const float L = group_sum<64>(w * l);
        const float ox = group_sum<64>(w * a.x), oy = group_sum<64>(w * a.y);
        const float oz = group_sum<64>(w * a.z), ow = group_sum<64>(w * a.w);
        if (lane == 0) {
            const float inv = 1.0f / L;
            *(float4 *)&sq.dst[(u64)(r + h / gh) * p.q_stride + (u64)(kvh * gh + h % gh) * D + d] =
                make_float4(ox * inv, oy * inv, oz * inv, ow * inv);
        }
    }
}

/* Decode attention with one workgroup of 8 waves per CU.  Each wave streams
 * its tiles (every 8th tile of the chunk) through a ring of two LDS stages
 * filled by LDS-direct loads: while one tile is computed the next is in
 * flight, and two waves per SIMD hide each other's latency.  Every group of
 * LPK lanes keeps its own online-softmax state (no cross-lane exchange in
 * the stream loop); the groups and waves merge once at the end.  Split
 * decomposition, XCD-aware block order, GQA sharing, the fused append and
 * the split merge are described at the top of this file.  Tiles that hold rows
 * appended by this launch (the last tiles of the last split) stream through
 * the ring like the others; their new rows are then overwritten in LDS with
 * the rows staged from the f32 input. */
#define TL_RING_WAVES 8
#define TL_RING_STAGES 2
template <int D, int G, bool ROPE, bool Q8, bool MF, bool S16>
__device__ __attribute__((always_inline)) inline void decode_ring_body(const DecParams &p) {
    using C = RCfg<D>;
    constexpr int LPK = C::LPK, CPR = C::CPR, TK = C::TK, UNITS = C::UNITS, LD = C::LD;
    /* a Q8_0 tile is half the bytes of an f16 one: twice the stages in the
     * same ring memory, plus the scales (64 words per stage) */
    constexpr int W = TL_RING_WAVES, S = Q8 ? 2 * TL_RING_STAGES : TL_RING_STAGES, NT = 64 * W;
    constexpr int STAGE_U = Q8 ? UNITS : 2 * UNITS;   /* 16-byte units per stage (K + V) */
    constexpr int RING_U = 2 * TL_RING_STAGES * UNITS;
    constexpr int VPR = D / 8;
    constexpr float NEG_INF = -__builtin_huge_valf();
    static_assert(LD == 4, "wait_tiles assumes 8 loads per tile");
    static_assert(S * STAGE_U <= RING_U, "ring stages");

    __shared__ uint4 s_ring[W][RING_U];          /* per wave: S stages of (K, V) */
    __shared__ u32 s_scl[Q8 ? W : 1][Q8 ? S * 64 : 1];
    __shared__ u32 s_slot[TL_DEC_MAX_CHUNK];
    /* columns of the group's state: the G heads of one row, or with the
     * matrix-core tile up to 16 (8 at head_dim 256, for LDS) = (batch rows
     * of the group) x G */
    constexpr int CGT = MF ? (D == 256 ? 8 : 16) : G;
    static_assert(CGT >= G, "a row's heads fit the columns");
    __shared__ uint4 s_q[CGT * D / 8];
    __shared__ float s_m[W][CGT];
    __shared__ uint4 s_newk[Q8 ? 1 : TL_DEC_MAX_NEW][D / 8];
    __shared__ uint4 s_newv[Q8 ? 1 : TL_DEC_MAX_NEW][D / 8];
    /* Q8_0: the launch's new rows quantized as the append kernel does (int8
     * in 8-value units, binary16 block scales).  With RoPE the rotated K rows
     * pass through s_nv8 as f32 first (at most TL_DEC_Q8_ROPE_NEW rows) */
    constexpr bool Q8NEW = Q8;
    __shared__ uint2 s_nk8[Q8NEW ? TL_DEC_MAX_NEW : 1][Q8NEW ? D / 8 : 1];
    __shared__ uint2 s_nv8[Q8NEW ? TL_DEC_MAX_NEW : 1][Q8NEW ? D / 8 : 1];
    __shared__ u16 s_nks[Q8NEW ? TL_DEC_MAX_NEW : 1][Q8NEW ? D / 32 : 1];
    __shared__ u16 s_nvs[Q8NEW ? TL_DEC_MAX_NEW : 1][Q8NEW ? D / 32 : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    /* this launch's epoch (dist merge) is the launch counter + 1: the
     * counter is read now (device-coherent, as the closers' increments are)
     * and first used at the end, so nothing waits for it here */
    const u32 launches = __builtin_amdgcn_raw_buffer_load_b32(
        buf_rsrc(p.dist ? p.counters + TL_MERGE_LAUNCHES : nullptr), p.dist ? 0u : 0xfffffff0u, 0,
        TL_SC1);                                   /* without dist: out of range, reads 0 */

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
    /* group = (session, block of R batch rows, kv-head); R > 1 only with the
     * matrix-core tile.  The group's keys run from its first row's window
     * start to its last row's last key; each column masks its own row's. */
    const u32 R = MF && p.rows_per_wg > 1 ? p.rows_per_wg : 1u;
    const u32 RB = (p.rows_per_seq + R - 1) / R;
    const u32 kvh = grp % p.n_kv;
    const u32 gblk = grp / p.n_kv;
    const u32 si = gblk / RB;
    const u32 r = (gblk % RB) * R;                    /* the group's first row */
    const u32 nr = min(R, p.rows_per_seq - r);        /* its rows */
    const u32 cg = MF ? nr * G : (u32)G;              /* its columns */
    const DecSeq sq = p.seq[si];

    const u32 n_keys = sq.pos + r + nr;
    const u32 n_keys0 = sq.pos + r + 1;
    const u32 start = (p.window && n_keys0 > p.window) ? n_keys0 - p.window : 0;
    const u32 kbeg = start + split * p.chunk;
    const u32 kend = min(kbeg + p.chunk, n_keys);
    const bool fused = sq.kin != nullptr && (!(Q8 && ROPE) || p.rows_per_seq <= TL_DEC_Q8_ROPE_NEW);
    const bool writer = fused && split == 0 && r == 0;
    const bool need_new = fused && (writer || kend > sq.pos);
    const float *qb = sq.q + (u64)r * p.q_stride + (u64)kvh * G * D;

    /* physical rows of the chunk's keys */
    const bool staged = (sq.ring == 0) && (sq.slots != nullptr);
    /* S16: the slots staged as u16, twice as many in the same LDS */
    u16 *const s_slot16 = (u16 *)&s_slot[0];
    /* the chunk's slots are loaded here and stored to LDS after q and the new
     * rows have been requested too, so the prologue waits for one round
     * trip, not one per load */
    constexpr int SPT = (S16 ? TL_DEC_MAX_CHUNK16 : TL_DEC_MAX_CHUNK) / NT;   /* slots per thread */
    u32 slot_v[SPT];
    if (staged) {
#pragma unroll
        for (int j = 0; j < SPT; j++) {
            const u32 i = kbeg + tid + j * NT;
            slot_v[j] = i < kend ? sq.slots[i] : 0u;
        }
    }
    const u16 *Kbase = sq.k + (u64)kvh * sq.cap * D;
    const u16 *Vbase = sq.v + (u64)kvh * sq.cap * D;
    const u32 ring_lds = (u32)(uintptr_t)&s_ring[wave][0];
    /* Q8_0: int8 rows and their scale planes (f16 [n_kv][cap][D/32]) */
    const uint8_t *K8 = (const uint8_t *)sq.k + (u64)kvh * sq.cap * D;
    const uint8_t *V8 = (const uint8_t *)sq.v + (u64)kvh * sq.cap * D;
    const u16 *KS = Q8 ? sq.ks + (u64)kvh * sq.cap * (D / 32) : nullptr;
    const u16 *VS = Q8 ? sq.vs + (u64)kvh * sq.cap * (D / 32) : nullptr;
    const u32 scl_lds = (u32)(uintptr_t)&s_scl[Q8 ? wave : 0][0];

    /* tiles of the chunk, all streamed through the ring; rows appended by
     * this launch (key >= pos) are read from memory too (stale or new: the
     * writer may be storing them now) and replaced in LDS by the staged new
     * rows before the tile is used */
    const u32 ntile = (kend > kbeg) ? (kend - kbeg + TK - 1) / TK : 0;
    const u32 nj = ntile > (u32)wave ? (ntile - wave + W - 1) / W : 0;   /* this wave's ring tiles */
    const u32 klast = kend - 1;
    const bool patch = fused && klast >= sq.pos;

    auto phys = [&](u32 key) -> u32 {
        if (sq.ring) return key % sq.ring;
        if (!staged) return key;
        if constexpr (S16) return (u32)s_slot16[key - kbeg];
        return s_slot[key - kbeg];
    };
    /* unit u = jj*64 + lane of a K (or V) tile holds chunk (u % CPR) ^ (row & 1)
     * of tile row u / CPR.  Rows past the chunk load its last row (their
     * scores are masked to -inf, so they add exactly 0). */
    auto issue = [&](u32 j) {
        const u32 tb = kbeg + (wave + W * j) * TK;
        const u32 lk = ring_lds + (j % S) * (STAGE_U * 16);
        if constexpr (Q8) {
            /* values: unit u = jj*64 + lane is 16-byte unit u % LPK of tile
             * row u / LPK, stored as loaded; K then V (UNITS/2 units each) */
#pragma unroll
            for (int jj = 0; jj < LD / 2; jj++) {
                const int u = jj * 64 + lane;
                const u32 ph = phys(min(tb + (u32)(u / LPK), klast));
                const u32 off = ph * D + (u % LPK) * 16;
                lds_dma16(lk + jj * 1024, K8, off);
                lds_dma16(lk + UNITS * 8 + jj * 1024, V8, off);
            }
            /* scales: 32 words per plane (TK rows x D/32 f16), lanes 0..31 */
            const int srow = lane / (D / 64), sw = lane % (D / 64);
            const u32 sph = phys(min(tb + (u32)srow, klast));
            const u32 soff = (sph * (D / 32) + 2 * sw) * 2;
            const u32 ls = scl_lds + (j % S) * 256;
            if (lane < 32) {
                lds_dma4(ls, KS, soff);
                lds_dma4(ls + 128, VS, soff);
            }
            return;
        }
#pragma unroll
        for (int jj = 0; jj < LD; jj++) {
            const int u = jj * 64 + lane;
            const int row = u / CPR;
            const u32 ph = phys(min(tb + (u32)row, klast));
            const u32 off = (ph * D + (((u % CPR) ^ (row & 1)) * 8)) * 2;
            lds_dma16(lk + jj * 1024, Kbase, off);
            lds_dma16(lk + UNITS * 16 + jj * 1024, Vbase, off);
        }
    };

    /* Q8_0 fused append: a landed tile holding rows of this launch (key >=
     * pos) gets them, and their block scales, from the staged new rows */
    auto patch_q8 = [&](u32 j) __attribute__((always_inline)) {
        if constexpr (Q8NEW) {
            const u32 tb = kbeg + (wave + W * j) * TK;
            if (!patch || tb + TK <= sq.pos) return;
            uint2 *k8 = (uint2 *)&s_ring[wave][(j % S) * STAGE_U];   /* row t at t * D/8 */
            uint2 *v8 = k8 + TK * (D / 8);
#pragma unroll
            for (int jj = 0; jj < (TK * (D / 8) + 63) / 64; jj++) {
                const u32 u = (u32)(jj * 64 + lane);
                const u32 key = min(tb + u / (D / 8), klast);
                if (u < (u32)(TK * (D / 8)) && key >= sq.pos) {
                    k8[u] = s_nk8[key - sq.pos][u % (D / 8)];
                    v8[u] = s_nv8[key - sq.pos][u % (D / 8)];
                }
            }
            u16 *ss = (u16 *)&s_scl[wave][(j % S) * 64];              /* [TK][D/32], V at +64 */
            const u32 key = min(tb + (u32)lane / (D / 32), klast);
            if ((u32)lane < (u32)(TK * (D / 32)) && key >= sq.pos) {
                ss[lane] = s_nks[key - sq.pos][lane % (D / 32)];
                ss[64 + lane] = s_nvs[key - sq.pos][lane % (D / 32)];
            }
            __builtin_amdgcn_wave_barrier();
        }
    };
    const u32 npre = nj < (u32)S ? nj : (u32)S;
    /* the chunk's slots to LDS (one barrier), then the first tiles' loads */
    auto stage_and_issue = [&]() __attribute__((always_inline)) {
        if (staged) {
#pragma unroll
            for (int j = 0; j < SPT; j++) {
                const u32 i = tid + j * NT;
                if (kbeg + i < kend) {
                    const u32 ph = slot_v[j] < sq.cap ? slot_v[j] : 0u;
                    if constexpr (S16)
                        s_slot16[i] = (u16)ph;
                    else
                        s_slot[i] = ph;
                }
            }
        }
        __syncthreads();
        for (u32 j = 0; j < npre; j++) issue(j);
    };
    /* q of the GQA group (RoPE'd at pos + r when ROPE), scaled to log2 units,
     * f16; the launch's new K/V rows (K RoPE'd at pos + row), f16 */
    const float sc = p.scale_log2;
    if constexpr (ROPE) {
        /* pairs (ia, ib) of q and of the new K rows, rotated by position,
         * and the new V rows: every thread requests its (few) items first,
         * then rotates, converts and stores them */
        constexpr int QI = (CGT * (D / 2) + NT - 1) / NT;              /* q pairs */
        constexpr int KI = (TL_DEC_MAX_NEW * (D / 2) + NT - 1) / NT;   /* K pairs */
        constexpr int VI = (TL_DEC_MAX_NEW * (D / 8) + NT - 1) / NT;   /* V 8-element units */
        const u32 pairs = p.rope.rdim >> 1;
        const u32 nkp = need_new ? p.rows_per_seq * (D / 2) : 0u;
        const u32 nvu = need_new ? p.rows_per_seq * VPR : 0u;
        /* element indices of pair i: rotated pairs per the RoPE variant,
         * the rest (i >= pairs) stay adjacent */
        auto pair_of = [&](u32 i, u32 &ia, u32 &ib) {
            const bool rot = i < pairs;
            ia = (rot && p.rope.neox) ? i : 2 * i;
            ib = (rot && p.rope.neox) ? i + pairs : 2 * i + 1;
        };
        float qx[QI], qy[QI], kx[KI], ky[KI];
        float4 va[VI], vc[VI];
#pragma unroll
        for (int j = 0; j < QI; j++) {
            const u32 t = tid + j * NT;
            qx[j] = qy[j] = 0.f;
            if (t < cg * (D / 2)) {
                u32 ia, ib;
                pair_of(t % (D / 2), ia, ib);
                /* column t / (D/2) = batch row (of the group) x G + head */
                const u32 col = t / (D / 2);
                const float *row = qb + (u64)(col / G) * p.q_stride + (col % G) * D;
                qx[j] = row[ia];
                qy[j] = row[ib];
            }
        }
#pragma unroll
        for (int j = 0; j < KI; j++) {
            const u32 t = tid + j * NT;
            kx[j] = ky[j] = 0.f;
            if (t < nkp) {
                u32 ia, ib;
                pair_of(t % (D / 2), ia, ib);
                const float *src = sq.kin + (u64)(t / (D / 2)) * sq.kv_stride + (u64)kvh * D;
                kx[j] = src[ia];
                ky[j] = src[ib];
            }
        }
#pragma unroll
        for (int j = 0; j < VI; j++) {
            const u32 i = tid + j * NT;
            va[j] = vc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < nvu) {
                const float *src = sq.vin + (u64)(i / VPR) * sq.kv_stride + (u64)kvh * D + (i % VPR) * 8;
                va[j] = *(const float4 *)src;
                vc[j] = *(const float4 *)(src + 4);
            }
        }
        /* the rotation (powf + sincosf per pair, ~1 us per thread) runs
         * while the first tiles are in flight: the loaded values are pinned
         * here (the compiler waits for them now, not behind the tile
         * loads), then the slots are staged, the tiles issued, and q and
         * the new rows rotated, converted and stored */
#pragma unroll
        for (int j = 0; j < QI; j++) __asm__ volatile("" : "+v"(qx[j]), "+v"(qy[j]));
#pragma unroll
        for (int j = 0; j < KI; j++) __asm__ volatile("" : "+v"(kx[j]), "+v"(ky[j]));
#pragma unroll
        for (int j = 0; j < VI; j++)
            __asm__ volatile("" : "+v"(va[j].x), "+v"(va[j].y), "+v"(va[j].z), "+v"(va[j].w),
                             "+v"(vc[j].x), "+v"(vc[j].y), "+v"(vc[j].z), "+v"(vc[j].w));
        stage_and_issue();
        u16 *q16 = (u16 *)s_q;
#pragma unroll
        for (int j = 0; j < QI; j++) {
            const u32 t = tid + j * NT;
            if (t < cg * (D / 2)) {
                const u32 h = t / (D / 2), i = t % (D / 2);
                u32 ia, ib;
                pair_of(i, ia, ib);
                float x = qx[j], y = qy[j];
                if (i < pairs) {
                    float c, sn;
                    rope_cs(i, p.rope.rdim, p.rope.theta, sq.pos + r + h / G, c, sn);
                    rope_rot(qx[j], qy[j], c, sn, x, y);
                }
                const u32 pk = pack_f16x2_fast(x * sc, y * sc);
                q16[h * D + ia] = (u16)(pk & 0xffffu);
                q16[h * D + ib] = (u16)(pk >> 16);
            }
        }
#pragma unroll
        for (int j = 0; j < KI; j++) {
            const u32 t = tid + j * NT;
            if (t < nkp) {
                const u32 row = t / (D / 2), i = t % (D / 2);
                u32 ia, ib;
                pair_of(i, ia, ib);
                float x = kx[j], y = ky[j];
                if (i < pairs) {
                    float c, sn;
                    rope_cs(i, p.rope.rdim, p.rope.theta, sq.pos + row, c, sn);
                    rope_rot(kx[j], ky[j], c, sn, x, y);
                }
                if constexpr (Q8) {
                    float *kf = (float *)&s_nv8[0][0] + row * D;   /* f32 rows, quantized below */
                    kf[ia] = x;
                    kf[ib] = y;
                } else {
                    u16 *k16 = (u16 *)s_newk[row];
                    k16[ia] = (u16)f32_to_f16_bits(x);
                    k16[ib] = (u16)f32_to_f16_bits(y);
                }
            }
        }
        if constexpr (!Q8) {
#pragma unroll
            for (int j = 0; j < VI; j++) {
                const u32 i = tid + j * NT;
                if (i < nvu) s_newv[i / VPR][i % VPR] = cvt8_f16_regs(va[j], vc[j]);
            }
        }
        __syncthreads();   /* q and the new rows */
        if constexpr (Q8) {
            /* the rotated K rows (f32 over s_nv8) and the V rows (registers:
             * item tid, VI == 1) to Q8_0, one 8-value unit per thread; the
             * 4 lanes of a block are an aligned group */
            static_assert(VI == 1 && TL_DEC_Q8_ROPE_NEW * D * 4 <= (int)sizeof(s_nv8), "staging");
            const bool has_new = (u32)tid < nvu;
            const u32 nrow = (u32)tid / VPR, nc8 = (u32)tid % VPR;
            float kq[8];
            if (has_new) {
                const float *kf = (const float *)&s_nv8[0][0] + nrow * D + nc8 * 8;
#pragma unroll
                for (int e = 0; e < 8; e++) kq[e] = kf[e];
            }
            __syncthreads();   /* every f32 read before the int8 rows overwrite them */
            if (has_new) {
                const float vq[8] = {va[0].x, va[0].y, va[0].z, va[0].w,
                                     vc[0].x, vc[0].y, vc[0].z, vc[0].w};
                const float dk = group_max<4>(amax8(kq)) / 127.0f;
                const float dv = group_max<4>(amax8(vq)) / 127.0f;
                s_nk8[nrow][nc8] = q8_pack8(kq, dk > 0.0f ? 1.0f / dk : 0.0f);
                s_nv8[nrow][nc8] = q8_pack8(vq, dv > 0.0f ? 1.0f / dv : 0.0f);
                if ((nc8 & 3) == 0) {
                    s_nks[nrow][nc8 / 4] = (u16)f32_to_f16_bits(dk);
                    s_nvs[nrow][nc8 / 4] = (u16)f32_to_f16_bits(dv);
                }
            }
            __syncthreads();   /* the quantized rows */
        }
    } else {
        /* one q item and at most one new-row item per thread (G * D / 8 and
         * TL_DEC_MAX_NEW * D / 8 are at most NT): all loads first */
        static_assert(CGT * D / 8 <= NT && TL_DEC_MAX_NEW * (D / 8) <= NT, "one item per thread");
        float4 qa = make_float4(0.f, 0.f, 0.f, 0.f), qc = qa;
        float4 ka = qa, kc = qa, va = qa, vc = qa;
        const bool has_q = (u32)tid < cg * (D / 8);
        /* column tid / (D/8) = batch row (of the group) x G + head */
        const float *qrow = qb + (u64)((u32)tid / (G * D / 8)) * p.q_stride + ((u32)tid % (G * D / 8)) * 8;
        const bool has_new = need_new && (u32)tid < p.rows_per_seq * VPR;
        const u32 nrow = (u32)tid / VPR, nc8 = (u32)tid % VPR;
        if (has_q) {
            qa = *(const float4 *)qrow;
            qc = *(const float4 *)(qrow + 4);
        }
        if (has_new) {
            const u64 src = (u64)nrow * sq.kv_stride + (u64)kvh * D + nc8 * 8;
            ka = *(const float4 *)(sq.kin + src);
            kc = *(const float4 *)(sq.kin + src + 4);
            va = *(const float4 *)(sq.vin + src);
            vc = *(const float4 *)(sq.vin + src + 4);
        }
        if (has_q)
            s_q[tid] = make_uint4(pack_f16x2_fast(qa.x * sc, qa.y * sc), pack_f16x2_fast(qa.z * sc, qa.w * sc),
                                  pack_f16x2_fast(qc.x * sc, qc.y * sc), pack_f16x2_fast(qc.z * sc, qc.w * sc));
        if (has_new) {
            if constexpr (Q8) {
                /* the 4 lanes of a 32-value block are an aligned group (rows
                 * x D/8 items, D/8 a multiple of 4), all of them here */
                const float kx[8] = {ka.x, ka.y, ka.z, ka.w, kc.x, kc.y, kc.z, kc.w};
                const float vx[8] = {va.x, va.y, va.z, va.w, vc.x, vc.y, vc.z, vc.w};
                const float dk = group_max<4>(amax8(kx)) / 127.0f;
                const float dv = group_max<4>(amax8(vx)) / 127.0f;
                s_nk8[nrow][nc8] = q8_pack8(kx, dk > 0.0f ? 1.0f / dk : 0.0f);
                s_nv8[nrow][nc8] = q8_pack8(vx, dv > 0.0f ? 1.0f / dv : 0.0f);
                if ((nc8 & 3) == 0) {
                    s_nks[nrow][nc8 / 4] = (u16)f32_to_f16_bits(dk);
                    s_nvs[nrow][nc8 / 4] = (u16)f32_to_f16_bits(dv);
                }
            } else {
                s_newk[nrow][nc8] = cvt8_f16_regs(ka, kc);
                s_newv[nrow][nc8] = cvt8_f16_regs(va, vc);
            }
        }
    }
    if constexpr (!ROPE) stage_and_issue();


    /* q of this lane's 16 dims, every head of the group */
    u32 qr[G][8];
    {
        const int sub = lane % LPK;
#pragma unroll
        for (int h = 0; h < G; h++) {
            const uint4 a = s_q[h * CPR + 2 * sub], b = s_q[h * CPR + 2 * sub + 1];
            qr[h][0] = a.x; qr[h][1] = a.y; qr[h][2] = a.z; qr[h][3] = a.w;
            qr[h][4] = b.x; qr[h][5] = b.y; qr[h][6] = b.z; qr[h][7] = b.w;
        }
    }
    float m[G], l[G], acc[G][16];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = NEG_INF;
        l[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 16; e++) acc[h][e] = 0.f;
    }
    /* MF: q as the QK B operand (head lane & 15, chunk 4j + lane / 16; zero
     * past the group's heads) and one head column's state per lane */
    dh8_t qm[MF ? D / 32 : 1];
    df4_t O1[MF ? D / 16 : 1];
    float m1 = NEG_INF, l1 = 0.f;
    MfRows mr = {0u, 0xffffffffu, 0u, 0xffffffffu, false};
    if constexpr (MF) {
        const int c = lane & 15, g = lane >> 4;
        if (nr > 1) {
            /* per-column key ranges of the group's rows (columns past the
             * group's rows see everything: their q is zero) */
            auto row_start = [&](u32 n) { return (p.window && n > p.window) ? n - p.window : 0u; };
            mr.multi = true;
            mr.ulo = row_start(n_keys);      /* the last row's window start */
            mr.uhi = n_keys0;                /* the first row's end */
            if ((u32)c < cg) {
                mr.khi = sq.pos + r + (u32)c / G + 1;
                mr.klo = row_start(mr.khi);
            }
        }
#pragma unroll
        for (int j = 0; j < D / 32; j++) qm[j] = (u32)c < cg ? u4_as_h8(s_q[c * CPR + 4 * j + g]) : dh8_t{};
#pragma unroll
        for (int db = 0; db < D / 16; db++) O1[db] = df4_t{0.f, 0.f, 0.f, 0.f};
    }

    u32 j0 = 0;
    /* Q8_0 on the matrix cores: TL_DEC_Q8_CHAIN ring tiles per softmax
     * chain (the ring's other tiles stay in flight meanwhile); one at
     * head_dim 256, where two tiles' registers would spill */
    constexpr int NC = D == 256 ? 1 : TL_DEC_Q8_CHAIN;
    if constexpr (Q8 && MF && NC > 1) {
        static_assert(NC < S, "tiles in flight during a chain");
        for (; j0 + NC <= nj; j0 += NC) {
            const u32 after = nj - NC - j0;
            wait_tiles_q8(after < (u32)(S - NC) ? after : (u32)(S - NC));
#pragma unroll
            for (int t = 0; t < NC; t++) patch_q8(j0 + t);
            uint4 *st[NC];
            const u16 *sc[NC];
            u32 tb[NC];
#pragma unroll
            for (int t = 0; t < NC; t++) {
                st[t] = &s_ring[wave][((j0 + t) % S) * STAGE_U];
                sc[t] = (const u16 *)&s_scl[wave][((j0 + t) % S) * 64];
                tb[t] = kbeg + (wave + W * (j0 + t)) * TK;
            }
            mfma_tile_q8n<D, G, NC>(st, sc, qm, tb, kend, mr, lane, m1, l1, O1);
#pragma unroll
            for (int t = 0; t < NC; t++)
                if (j0 + t + S < nj) issue(j0 + t + S);
        }
    }
    for (u32 j = j0; j < nj; j++) {
        const u32 after = nj - 1 - j;
        if constexpr (Q8) {
            wait_tiles_q8(after < (u32)(S - 1) ? after : (u32)(S - 1));
            patch_q8(j);
        } else {
            wait_tiles(after < (u32)(S - 1) ? after : (u32)(S - 1));
        }
        const uint4 *st = &s_ring[wave][(j % S) * STAGE_U];
        if constexpr (!Q8) {
            const u32 tb = kbeg + (wave + W * j) * TK;
            if (patch && tb + TK > sq.pos) {
                /* unit u holds chunk (u % CPR) ^ (row & 1) of row u / CPR;
                 * rows past the chunk hold a copy of its last row */
                uint4 *sw = &s_ring[wave][(j % S) * STAGE_U];
#pragma unroll
                for (int jj = 0; jj < LD; jj++) {
                    const int u = jj * 64 + lane;
                    const int row = u / CPR;
                    const u32 key = min(tb + (u32)row, klast);
                    if (key >= sq.pos) {
                        const int c = (u % CPR) ^ (row & 1);
                        sw[u] = s_newk[key - sq.pos][c];
                        sw[UNITS + u] = s_newv[key - sq.pos][c];
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        if constexpr (Q8) {
            const u16 *ss = (const u16 *)&s_scl[wave][(j % S) * 64];
            if constexpr (MF)
                mfma_tile_q8<D, G>(&s_ring[wave][(j % S) * STAGE_U], ss, qm,
                                   kbeg + (wave + W * j) * TK, kend, mr, lane, m1, l1, O1);
            else
                ring_tile_q8<D, G>(st, st + UNITS / 2, ss, ss + 64, qr, kbeg + (wave + W * j) * TK,
                                   kend, lane, m, l, acc);
        } else if constexpr (MF) {
            mfma_tile<D, G>(st, st + UNITS, qm, kbeg + (wave + W * j) * TK, kend, mr, lane, m1,
                            l1, O1);
        } else {
            ring_tile<D, G>(st, st + UNITS, qr, kbeg + (wave + W * j) * TK, kend, lane, m, l, acc);
        }
        if (j + S < nj) issue(j + S);
    }
    if constexpr (Q8NEW) {
        if (writer) {
            /* the new rows and their scales into the cache (the append
             * kernel's layout: int8 [n_kv][cap][D], f16 [n_kv][cap][D/32]) */
            for (u32 i = tid; i < p.rows_per_seq * VPR; i += NT) {
                const u32 row = i / VPR, c8 = i % VPR;
                const u32 key = sq.pos + row;
                const u32 ph = sq.ring ? key % sq.ring : (sq.slots ? sq.slots[key] : key);
                if (ph >= sq.cap) continue;
                const u64 prow = (u64)kvh * sq.cap + ph;
                *(uint2 *)((uint8_t *)sq.k + prow * D + c8 * 8) = s_nk8[row][c8];
                *(uint2 *)((uint8_t *)sq.v + prow * D + c8 * 8) = s_nv8[row][c8];
                if ((c8 & 3) == 0) {
                    ((u16 *)sq.ks)[prow * (D / 32) + c8 / 4] = s_nks[row][c8 / 4];
                    ((u16 *)sq.vs)[prow * (D / 32) + c8 / 4] = s_nvs[row][c8 / 4];
                }
            }
        }
    }
    if (!Q8 && writer) {
        for (u32 i = tid; i < p.rows_per_seq * VPR; i += NT) {
            const u32 row = i / VPR, c8 = i % VPR;
            const u32 key = sq.pos + row;
            const u32 ph = sq.ring ? key % sq.ring : (sq.slots ? sq.slots[key] : key);
            if (ph >= sq.cap) continue;
            const u64 dst = ((u64)kvh * sq.cap + ph) * D + c8 * 8;
            *(uint4 *)((u16 *)sq.k + dst) = s_newk[row][c8];
            *(uint4 *)((u16 *)sq.v + dst) = s_newv[row][c8];
        }
    }

    /* ---- one state per workgroup and head, then its output or partial ---- */
    const bool single = (n_split == 1);
    const bool last_merges = p.counters != nullptr;
    /* the group's partials: [column][split][D] from pb (R = 1: the layout
     * attn_merge_kernel reads, [row][head][split][D]) */
    const u32 pb = grp * (R * G) * n_split;
    __shared__ float2 s_rec[CGT];
    /* output float4 (column h = batch row of the group x G + head, dims
     * d..d+3) of the workgroup's state: the result itself (one split) or
     * the split's partial */
    auto emit = [&](int h, int d, float mm, float L, float4 O) __attribute__((always_inline)) {
        const u32 hq = kvh * G + (u32)h % G, row = r + (u32)h / G;
        if (single) {
            const float inv = 1.0f / L;
            *(float4 *)&sq.dst[(u64)row * p.q_stride + (u64)hq * D + d] =
                make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
        } else if (last_merges) {
            /* device-coherent stores: the merging workgroup may run
             * on another XCD and reads them with device-coherent loads */
            const u32 pi = (u32)h * n_split + split;
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4v_t{__float_as_uint(O.x), __float_as_uint(O.y), __float_as_uint(O.z),
                         __float_as_uint(O.w)},
                buf_rsrc(p.ws_acc + (u64)pb * D), (pi * D + d) * 4, 0, TL_SC1);
            if (d == 0) {
                if (p.dist)
                    s_rec[h] = make_float2(mm, L);   /* record written below */
                else
                    __builtin_amdgcn_raw_buffer_store_b64(
                        u32x2v_t{__float_as_uint(mm), __float_as_uint(L)},
                        buf_rsrc(p.ws_ml + pb), pi * 8, 0, TL_SC1);
            }
        } else {
            const u64 pi = ((u64)gblk * p.n_head + hq) * n_split + split;
            *(float4 *)&p.ws_acc[pi * D + d] = O;
            if (d == 0) p.ws_ml[pi] = make_float2(mm, L);
        }
    };
    if constexpr (MF) {
        /* a column's sum over its four lanes; then every wave writes its
         * columns' (m, l) and O^T rows into its own ring region (no barrier:
         * that region is no longer read), and after one barrier thread
         * (h, d4) combines the waves with weights exp2(m_w - M_h) */
        __shared__ float s_lw[MF ? CGT : 1][W];
        static_assert(G <= 16, "one column per lane");
        const int c = lane & 15, g = lane >> 4;
        l1 += __shfl_xor(l1, 16);
        l1 += __shfl_xor(l1, 32);
        float *so = (float *)&s_ring[wave][0];
        static_assert(CGT * D * 4 <= RING_U * 16, "wave state exceeds its ring region");
        if ((u32)c < cg) {
#pragma unroll
            for (int db = 0; db < D / 16; db++)
                *(float4 *)&so[c * D + 16 * db + 4 * g] =
                    make_float4(O1[db][0], O1[db][1], O1[db][2], O1[db][3]);
            if (g == 0) {
                s_m[wave][c] = m1;
                s_lw[c][wave] = l1;
            }
        }
        __syncthreads();
        for (u32 t = (u32)tid; t < cg * (D / 4); t += NT) {
            const int h = (int)(t / (D / 4)), d = (int)(t % (D / 4)) * 4;
            float mm = s_m[0][h];
#pragma unroll
            for (int w = 1; w < W; w++) mm = fmaxf(mm, s_m[w][h]);
            const float mu = (mm == NEG_INF) ? 0.f : mm;
            float L = 0.f;
            float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < W; w++) {
                const float e = fast_exp2(s_m[w][h] - mu);
                const float4 t = *(const float4 *)((const float *)&s_ring[w][0] + h * D + d);
                L = fmaf(e, s_lw[h][w], L);
                O.x = fmaf(e, t.x, O.x);
                O.y = fmaf(e, t.y, O.y);
                O.z = fmaf(e, t.z, O.z);
                O.w = fmaf(e, t.w, O.w);
            }
            emit(h, d, mm, L, O);
        }
    } else {
        /* ---- one state per workgroup and head ----
         * The running max is wave-uniform, so the lanes of a wave add directly;
         * the waves combine with weights exp2(m_w - M_h).  The lane groups of a
         * DPP row are added in registers first; then a wave writes its state
         * into its own ring region (no barrier: that region is no longer read):
         * acc as float4 [head][k4][row-sum lane] (up to HB heads, 16 KB), l per
         * remaining lane group.  After one barrier, TPC threads per output
         * float4 each add a share of the W * GV lane groups (lanes sub +
         * LPK*part: every 8-lane phase of a read touches distinct banks), then
         * add across with shuffles.  More than HB heads take further rounds
         * through the same memory. */
        /* lane groups of one DPP row (16 lanes) are first added in registers
         * (row rotations by 8, then 4), so only one group per row goes through
         * LDS: PRE rotation steps, LV lanes per wave written, GV groups each */
        constexpr int PRE = LPK == 8 ? 1 : LPK == 4 ? 2 : 0;
        constexpr int LV = 64 >> PRE;
        constexpr int GV = LV / LPK;                      /* lane groups per wave in LDS */
        constexpr int NGRP = W * GV;                      /* lane groups per workgroup */
        constexpr int WREG = RING_U;                      /* float4 per wave region */
        constexpr int HB0 = WREG / (4 * LV);              /* heads that fit one round */
        constexpr int HB = G < HB0 ? G : HB0;             /* heads per round */
        constexpr int COLB = HB * D / 4;                  /* float4 columns per round */
        constexpr int TPC0 = NT / COLB > GV ? GV : NT / COLB;
        constexpr int TPC = pow2_floor(TPC0 < 1 ? 1 : TPC0);   /* threads per column */
        static_assert(HB * 4 * LV <= WREG, "wave state exceeds its ring region");
        static_assert(GV % TPC == 0, "lane groups per thread");
        if constexpr (PRE >= 1) {
    #pragma unroll
            for (int h = 0; h < G; h++) {
                l[h] += dpp_f<DPP_ROW_ROR8>(l[h]);
    #pragma unroll
                for (int e = 0; e < 16; e++) acc[h][e] += dpp_f<DPP_ROW_ROR8>(acc[h][e]);
            }
        }
        if constexpr (PRE >= 2) {
    #pragma unroll
            for (int h = 0; h < G; h++) {
                l[h] += dpp_f<DPP_ROW_ROR4>(l[h]);
    #pragma unroll
                for (int e = 0; e < 16; e++) acc[h][e] += dpp_f<DPP_ROW_ROR4>(acc[h][e]);
            }
        }
        /* lanes that hold their row's sums, and their place among them */
        const bool vlane = (lane & (PRE == 2 ? 12 : PRE == 1 ? 8 : 0)) == 0;
        const int ci = PRE == 0 ? lane : (lane % LPK) | ((lane >> 4) * LPK);
        __shared__ float s_lg[G][NGRP];
        float4 *s_w4 = (float4 *)&s_ring[0][0];
        const int sub = lane % LPK, gv = ci / LPK;
    #pragma unroll
        for (int h = 0; h < G; h++) {
            if (vlane) {
                if constexpr (own_head_softmax<G, LPK>()) {
                    if (sub == h) s_lg[h][wave * GV + gv] = l[0];
                } else {
                    if (sub == 0) s_lg[h][wave * GV + gv] = l[h];
                }
            }
            if (lane == 0) s_m[wave][h] = m[h];
        }
        /* reader mapping: t -> (sub, part, k4, hh) */
        const int rsub = tid % LPK, rpart = (tid / LPK) % TPC, rest = tid / (LPK * TPC);
        const int rk4 = rest % 4, rhh = rest / 4;
    #pragma unroll
        for (int h0 = 0; h0 < G; h0 += HB) {
            if (h0) __syncthreads();                      /* previous round read */
            float4 *mine = s_w4 + wave * WREG;
            if (vlane)
    #pragma unroll
                for (int hh = 0; hh < HB; hh++)
                    if (h0 + hh < G)
    #pragma unroll
                        for (int k4 = 0; k4 < 4; k4++)
                            mine[(hh * 4 + k4) * LV + ci] =
                                make_float4(acc[h0 + hh][4 * k4], acc[h0 + hh][4 * k4 + 1],
                                            acc[h0 + hh][4 * k4 + 2], acc[h0 + hh][4 * k4 + 3]);
            __syncthreads();
            const int h = h0 + rhh;
            if (rhh < HB && h < G) {
                const int d = rsub * 16 + rk4 * 4;
                float mm = s_m[0][h];
    #pragma unroll
                for (int w = 1; w < W; w++) mm = fmaxf(mm, s_m[w][h]);
                const float mu = (mm == NEG_INF) ? 0.f : mm;
                float L = 0.f;
                float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
                const float4 *src = s_w4 + (rhh * 4 + rk4) * LV + rsub;
    #pragma unroll
                for (int w = 0; w < W; w++) {
                    const float e = fast_exp2(s_m[w][h] - mu);
                    float lw = 0.f;
                    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    #pragma unroll
                    for (int g = 0; g < GV; g += TPC) {
                        const float4 t = src[w * WREG + (g + rpart) * LPK];
                        lw += s_lg[h][w * GV + g + rpart];
                        a.x += t.x; a.y += t.y; a.z += t.z; a.w += t.w;
                    }
                    L = fmaf(e, lw, L);
                    O.x = fmaf(e, a.x, O.x);
                    O.y = fmaf(e, a.y, O.y);
                    O.z = fmaf(e, a.z, O.z);
                    O.w = fmaf(e, a.w, O.w);
                }
    #pragma unroll
                for (int x = LPK; x < LPK * TPC; x *= 2) {
                    L += __shfl_xor(L, x);
                    O.x += __shfl_xor(O.x, x);
                    O.y += __shfl_xor(O.y, x);
                    O.z += __shfl_xor(O.z, x);
                    O.w += __shfl_xor(O.w, x);
                }
                if (rpart == 0) emit(h, d, mm, L, O);
            }
        }
    }
    if (single || !last_merges) return;

    /* ---- split merge ----
     * A workgroup's partial stores are complete (vmcnt 0) before anything
     * that announces them: its arrival in the group's counter (which the
     * last to arrive sets back to zero) and, in dist mode, the partials'
     * (m, l, epoch, ~epoch) records.
     * dist: the output columns of the group are cut into n_split slices and
     * split i merges slice i once every record of its heads carries this
     * launch's epoch (bounded wait), after tagging it as claimed; the last to
     * arrive merges its own slice, then waits (bounded) for the other slices'
     * claim tags and merges any slice still without one.  A slice merged
     * twice gets the same bits twice.  Otherwise the last to arrive merges
     * the whole group. */
    __shared__ u32 s_last, s_flag;
    __shared__ u64 s_todo;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    u32 *arrive = p.counters + grp * TL_MERGE_PAD;
    if (p.dist) {
        __shared__ u32 s_epoch;
        if (tid == 0) s_epoch = launches + 1u;
        __syncthreads();
        const u32 epoch = s_epoch;
        const u32 COLS = cg * (D / 4);
        const u32 cps = (COLS + n_split - 1) / n_split;   /* columns per slice */
        const u32 c0 = split * cps, c1 = min(c0 + cps, COLS);
        const __amdgpu_buffer_rsrc_t rrec = buf_rsrc((const float4 *)p.ws_ml + pb);
        if ((u32)tid < cg) {
            const u32 pi = (u32)tid * n_split + split;
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4v_t{__float_as_uint(s_rec[tid].x), __float_as_uint(s_rec[tid].y), epoch,
                         ~epoch},
                rrec, pi * 16, 0, TL_SC1);
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        if (tid == 64)   /* wave 1 counts the arrival while wave 0 polls */
            s_last = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (wave == 0) {
            u32 ok = c0 >= c1;   /* an empty slice needs nothing */
            for (u32 it = 0; it < p.polls && !ok; it++) {
                u64 missing = 0;
                for (u32 h = c0 / (D / 4); h <= (c1 - 1) / (D / 4); h++) {
                    bool have = true;
                    if ((u32)lane < n_split) {
                        const u32x4v_t rec = __builtin_amdgcn_raw_buffer_load_b128(
                            rrec, (h * n_split + (u32)lane) * 16, 0, TL_SC1);
                        have = rec[2] == epoch && rec[3] == ~epoch;
                    }
                    missing |= __builtin_amdgcn_ballot_w64(!have);
                }
                if (!missing) ok = 1;
                else __builtin_amdgcn_s_sleep(TL_MERGE_BACKOFF);
            }
            if (lane == 0) s_flag = ok;
        }
        __syncthreads();
        u32 *tags = p.counters + TL_MERGE_TAGS + grp * TL_MERGE_MAX_SPLIT_DIST;
        const bool closer = s_last == n_split - 1;
        if (!closer) {
            if (!s_flag || c0 >= c1) return;                 /* the last to arrive covers it */
            /* claim the slice: from here this workgroup merges it unconditionally */
            if (tid == 0)
                __hip_atomic_store(&tags[split], epoch, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            merge_slice<D, W>(p, pb, r, kvh, G, cg, sq, split, cps);
            return;
        }
        if (tid == 0) {
            __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            /* the last group of the launch to close advances the launch
             * counter: by then every workgroup of the launch has arrived, so
             * has read the counter, and all of them use the same epoch (a
             * workgroup dispatched after an early group's close would
             * otherwise see the next one and make its peers' polls time out) */
            const u32 closed = __hip_atomic_fetch_add(p.counters + TL_MERGE_CLOSED, 1u,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (closed == n_groups - 1) {
                __hip_atomic_store(p.counters + TL_MERGE_CLOSED, 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(p.counters + TL_MERGE_LAUNCHES, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        merge_slice<D, W>(p, pb, r, kvh, G, cg, sq, split, cps);
        /* slices whose owner has not claimed them (yet) */
        if (wave == 0) {
            u64 todo = 0;
            for (u32 it = 0; it <= p.polls; it++) {
                const u32 s = (u32)lane;
                bool need = s < n_split && s != split && s * cps < COLS;
                if (need)
                    need = __hip_atomic_load(&tags[s], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT) != epoch;
                todo = __builtin_amdgcn_ballot_w64(need);
                if (!todo || it == p.polls) break;
                __builtin_amdgcn_s_sleep(TL_MERGE_BACKOFF);
            }
            if (lane == 0) s_todo = todo;
        }
        __syncthreads();
        for (u64 todo = s_todo; todo; todo &= todo - 1)
            merge_slice<D, W>(p, pb, r, kvh, G, cg, sq, (u32)__builtin_ctzll(todo), cps);
        return;
    }
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const bool closer = s_last == n_split - 1;
    if (closer && tid == 0)
        __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!closer) return;
    /* (m, l) pairs of the partials: cg * n_split <= 2048 (ring memory) */
    split_merge_regs<D, CGT, NT>(p, pb, kvh, r, G, cg, sq, (float2 *)&s_ring[0][0]);
}

/* The kernel: slot indices staged as u32, at most TL_DEC_MAX_CHUNK keys per
 * workgroup when a slot table is staged. */
template <int D, int G, bool ROPE, bool Q8, bool MF>
__global__ __launch_bounds__(64 * TL_RING_WAVES) void attn_decode_ring_kernel(const DecParams p) {
    decode_ring_body<D, G, ROPE, Q8, MF, false>(p);
}

/* The same with slot indices staged as u16 (pools of at most 65536 rows), up
 * to TL_DEC_MAX_CHUNK16 keys per workgroup: launches whose chunks exceed
 * TL_DEC_MAX_CHUNK (f16 cache, matrix-core tile; tl_decode_s16.hip). */
template <int D, int G, bool ROPE, bool MF>
__global__ __launch_bounds__(64 * TL_RING_WAVES) void attn_decode_ring_kernel_s16(const DecParams p) {
    decode_ring_body<D, G, ROPE, false, MF, true>(p);
}

/* One decode kernel instance: entry point, K (or V) bytes per wave tile and
 * threads per workgroup.  The RoPE-fusing instances are separate so the
 * plain ones carry none of its code. */
struct DecKernel {
    const void *fn;
    int tile_bytes;
    int threads;
};

/* the Q8_0 instances (tl_decode_q8.hip) */
DecKernel tl_pick_decode_q8(int D, int G, bool rope, bool mf);
/* the u16-slot instances (f16 cache, matrix-core tile; tl_decode_s16.hip) */
DecKernel tl_pick_decode_s16(int D, int G, bool rope);

