/*
 * tl_decode_s16.hip — the instances of the decode kernel that stage slot
 * indices as u16 (attn_decode_ring_kernel_s16, tl_decode_kernels.h; design
 * in tl_decode.hip): f16 cache, matrix-core tile, launches whose chunks
 * exceed TL_DEC_MAX_CHUNK keys.  Their own translation unit so the kernel
 * instances build in parallel.
 */
#include "tl_decode_kernels.h"

template <int D>
static DecKernel pick_s16(int G, bool rope) {
    constexpr int NT = 64 * TL_RING_WAVES;
    switch (G) {
#define TL_CASE(g)                                                                                 \
    case g:                                                                                        \
        if (rope) return {(const void *)attn_decode_ring_kernel_s16<D, g, true, true>, 4096, NT}; \
        return {(const void *)attn_decode_ring_kernel_s16<D, g, false, true>, 4096, NT};
        TL_CASE(1) TL_CASE(2) TL_CASE(3) TL_CASE(4)
        TL_CASE(5) TL_CASE(6) TL_CASE(7) TL_CASE(8)
#undef TL_CASE
    default:
        return {nullptr, 0, 0};
    }
}

DecKernel tl_pick_decode_s16(int D, int G, bool rope) {
    switch (D) {
    case 64: return pick_s16<64>(G, rope);
    case 128: return pick_s16<128>(G, rope);
    case 256: return pick_s16<256>(G, rope);
    default: return {nullptr, 0, 0};
    }
}
