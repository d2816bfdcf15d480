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
