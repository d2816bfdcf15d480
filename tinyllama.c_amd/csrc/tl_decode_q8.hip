/*
 * tl_decode_q8.hip — the Q8_0-cache instances of attn_decode_ring_kernel
 * (tl_decode_kernels.h; design in tl_decode.hip), in their own translation
 * unit so the kernel instances build in parallel.
 */
#include "tl_decode_kernels.h"

template <int D>
static DecKernel pick_q8(int G, bool rope, bool mf) {
    constexpr int NT = 64 * TL_RING_WAVES;
    switch (G) {
#define TL_CASE(g)                                                                                   \
    case g:                                                                                          \
        if (mf) {                                                                                    \
            if (rope) return {(const void *)attn_decode_ring_kernel<D, g, true, true, true>, 4096, NT}; \
            return {(const void *)attn_decode_ring_kernel<D, g, false, true, true>, 4096, NT};         \
        }                                                                                            \
        if (rope) return {(const void *)attn_decode_ring_kernel<D, g, true, true, false>, 4096, NT};  \
        return {(const void *)attn_decode_ring_kernel<D, g, false, true, false>, 4096, NT};
        TL_CASE(1) TL_CASE(2) TL_CASE(3) TL_CASE(4)
        TL_CASE(5) TL_CASE(6) TL_CASE(7) TL_CASE(8)
#undef TL_CASE
    default:
        return {nullptr, 0, 0};
    }
}

DecKernel tl_pick_decode_q8(int D, int G, bool rope, bool mf) {
    switch (D) {
    case 64: return pick_q8<64>(G, rope, mf);
    case 128: return pick_q8<128>(G, rope, mf);
    case 256: return pick_q8<256>(G, rope, mf);
    default: return {nullptr, 0, 0};
    }
}
