/* tl_common.h — shared device helpers for the gfx950 KV-cache kernels. */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define TL_DEV __device__ __forceinline__
#define TL_HOSTDEV __host__ __device__ __forceinline__

typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;

/* f32 -> binary16 bits, round-to-nearest-even (v_cvt_f16_f32 in the default
 * RNE mode); NaN is pinned to quiet-NaN | top 9 payload bits so the result
 * does not depend on how the hardware canonicalises NaN. */
TL_DEV u32 f32_to_f16_bits(float x) {
    _Float16 h = (_Float16)x;
    u32 r = (u32)__builtin_bit_cast(u16, h);
    u32 b = __float_as_uint(x);
    if ((b & 0x7fffffffu) > 0x7f800000u)
        r = ((b >> 16) & 0x8000u) | 0x7e00u | ((b >> 13) & 0x3ffu);
    return r;
}

TL_DEV u32 pack_f16x2(float lo, float hi) {
    return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
}

/* RNE pack without the NaN pinning (operands of dot products): one
 * v_cvt_pk_f16_f32 on gfx950. */
typedef float tl_f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 tl_f16x2_t __attribute__((ext_vector_type(2)));
TL_DEV u32 pack_f16x2_fast(float lo, float hi) {
    const tl_f32x2_t v = {lo, hi};
    return __builtin_bit_cast(u32, __builtin_convertvector(v, tl_f16x2_t));
}

TL_DEV float f16lo(u32 w) {
    return (float)__builtin_bit_cast(_Float16, (u16)(w & 0xffffu));
}
TL_DEV float f16hi(u32 w) {
    return (float)__builtin_bit_cast(_Float16, (u16)(w >> 16));
}

/* DPP lane moves inside a row of 16 lanes. */
template <int CTRL>
TL_DEV float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
#define DPP_QUAD_XOR1  0xB1   /* quad_perm [1,0,3,2] */
#define DPP_QUAD_XOR2  0x4E   /* quad_perm [2,3,0,1] */
#define DPP_ROW_HMIRROR 0x141 /* lane i <- lane 7-i within 8 */
#define DPP_ROW_MIRROR  0x140 /* lane i <- lane 15-i within 16 */
#define DPP_ROW_ROR4    0x124 /* lane i <- lane (i+4) % 16 within 16 (rotate) */
#define DPP_ROW_ROR8    0x128 /* lane i <- lane (i+8) % 16 within 16 */

/* Sum over aligned groups of N consecutive lanes (N in 1..64, power of 2);
 * every lane of a group receives the group total.  Within 16 lanes the moves
 * are DPP (quad_perm xor1/xor2, row_half_mirror, row_mirror: after the quad
 * steps every lane of a quad holds the quad sum, so the mirrors add the other
 * quad / half); across rows they are shuffles. */
template <int N>
TL_DEV float group_sum(float x) {
    if constexpr (N >= 2) x += dpp_f<DPP_QUAD_XOR1>(x);
    if constexpr (N >= 4) x += dpp_f<DPP_QUAD_XOR2>(x);
    if constexpr (N >= 8) x += dpp_f<DPP_ROW_HMIRROR>(x);
    if constexpr (N >= 16) x += dpp_f<DPP_ROW_MIRROR>(x);
    if constexpr (N >= 32) x += __shfl_xor(x, 16);
    if constexpr (N >= 64) x += __shfl_xor(x, 32);
    return x;
}

template <int N>
TL_DEV float group_max(float x) {
    if constexpr (N >= 2) x = fmaxf(x, dpp_f<DPP_QUAD_XOR1>(x));
    if constexpr (N >= 4) x = fmaxf(x, dpp_f<DPP_QUAD_XOR2>(x));
    if constexpr (N >= 8) x = fmaxf(x, dpp_f<DPP_ROW_HMIRROR>(x));
    if constexpr (N >= 16) x = fmaxf(x, dpp_f<DPP_ROW_MIRROR>(x));
    if constexpr (N >= 32) x = fmaxf(x, __shfl_xor(x, 16));
    if constexpr (N >= 64) x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

/* 8 f32 -> 8 binary16 (RNE, NaN pinned), the append conversion */
TL_DEV uint4 cvt8_f16_regs(float4 a, float4 b) {
    return make_uint4(pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y),
                      pack_f16x2(b.z, b.w));
}
TL_DEV uint4 cvt8_f16(const float *src) {
    return cvt8_f16_regs(*(const float4 *)src, *(const float4 *)(src + 4));
}
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

/* ---- RoPE (reference: src/backend/cpu/cpu_op.c:637-700) -------------------
 * Pair i of a head row rotates by angle pos * theta_i, theta_i =
 * 1 / powf(base, 2i / rdim).  NORM pairs elements (2i, 2i+1), NEOX pairs
 * (i, i + rdim/2).  The rotation is written with explicit fmaf so every
 * kernel that applies it (the rope op and the fused append / attention
 * staging) produces the same bits. */
TL_DEV void rope_rot(float a, float b, float c, float s, float &x, float &y) {
    x = fmaf(a, c, -(b * s));
    y = fmaf(a, s, b * c);
}
TL_DEV void rope_cs(u32 i, u32 rdim, float base, u32 pos, float &c, float &s) {
    const float th = 1.0f / powf(base, (float)(2 * i) / (float)rdim);
    sincosf((float)pos * th, &s, &c);
}
/* elements e0..e0+7 of one head row (hrow = its element 0), rotated at
 * position pos when rdim > 0 */
TL_DEV void load8_rope(const float *hrow, u32 e0, u32 pos, u32 rdim, float base, int neox,
                       float out[8]) {
    const float4 a = *(const float4 *)(hrow + e0);
    const float4 b = *(const float4 *)(hrow + e0 + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    if (rdim == 0 || e0 >= rdim) return;
    if (!neox) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            if (e0 + j < rdim) {
                float c, s, x, y;
                rope_cs((e0 + j) >> 1, rdim, base, pos, c, s);
                rope_rot(out[j], out[j + 1], c, s, x, y);
                out[j] = x;
                out[j + 1] = y;
            }
        }
        return;
    }
    const u32 half = rdim >> 1;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const u32 e = e0 + j;
        if (e < rdim) {
            const bool lo = e < half;
            const u32 i = lo ? e : e - half;
            const float pa = lo ? out[j] : hrow[i];           /* element i */
            const float pb = lo ? hrow[e + half] : out[j];    /* element i + half */
            float c, s, x, y;
            rope_cs(i, rdim, base, pos, c, s);
            rope_rot(pa, pb, c, s, x, y);
            out[j] = lo ? x : y;
        }
    }
}

/* 8 f32 -> 8 binary16 (RNE, NaN pinned) of one K unit, RoPE'd at pos */
TL_DEV uint4 cvt8_rope(const float *hrow, u32 e0, u32 pos, u32 rdim, float base, int neox) {
    float t[8];
    load8_rope(hrow, e0, pos, rdim, base, neox, t);
    return make_uint4(pack_f16x2(t[0], t[1]), pack_f16x2(t[2], t[3]), pack_f16x2(t[4], t[5]),
                      pack_f16x2(t[6], t[7]));
}

/* ---- Q8_0 cache helpers ---------------------------------------------------- */

typedef _Float16 tl_half2 __attribute__((ext_vector_type(2)));

/* 4 int8 (element 0 in the low byte) -> f16 pairs (elements 0,1) and (2,3),
 * exact: byte ^ 0x80 = q + 128 placed under the binary16 exponent of 1024
 * (high byte 0x64) is the f16 value 1152 + q; one packed subtract leaves q. */
TL_DEV void i8x4_to_f16(u32 w, tl_half2 &lo, tl_half2 &hi) {
    const u32 x = w ^ 0x80808080u;
    const tl_half2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(tl_half2, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) - bias;
    hi = __builtin_bit_cast(tl_half2, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) - bias;
}

/* Q8_0 quantizer (gpu.cu:1077-1086): a lane holds 8 values of a 32-value
 * block, the block max comes from its 4-lane group (amax8, group_max<4>),
 * d = max / 127, q = rint(x / d) with 1/d formed once; shared by the append
 * kernel and the decode launch's fused append, so both write the same bits.
 * 8 values of a block whose scale is 1/id -> 8 int8 in two words: */
TL_DEV uint2 q8_pack8(const float (&x)[8], float id) {
    u32 w[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int a = (int)rintf(x[4 * h] * id), b = (int)rintf(x[4 * h + 1] * id);
        const int c = (int)rintf(x[4 * h + 2] * id), d = (int)rintf(x[4 * h + 3] * id);
        w[h] = (u32)(a & 0xff) | ((u32)(b & 0xff) << 8) | ((u32)(c & 0xff) << 16) |
               ((u32)(d & 0xff) << 24);
    }
    return make_uint2(w[0], w[1]);
}

TL_DEV float amax8(const float (&x)[8]) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(x[j]));
    return m;
}

/* 8 int8 of one 32-element block and its binary16 scale d -> 8 binary16
 * values RNE(q * d) (the product is formed exactly, then rounded once) */
TL_DEV uint4 q8_dequant8(uint2 w, u32 d_bits) {
    const tl_half2 d2 = __builtin_bit_cast(tl_half2, d_bits * 0x10001u);
    tl_half2 a, b, c, e;
    i8x4_to_f16(w.x, a, b);
    i8x4_to_f16(w.y, c, e);
    a *= d2; b *= d2; c *= d2; e *= d2;
    return make_uint4(__builtin_bit_cast(u32, a), __builtin_bit_cast(u32, b),
                      __builtin_bit_cast(u32, c), __builtin_bit_cast(u32, e));
}
