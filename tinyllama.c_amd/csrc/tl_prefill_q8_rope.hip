/*
 * tl_prefill_q8_rope.hip — the Q8_0 cache, fused RoPE instances of attn_prefill_kernel
 * (tl_prefill_kernels.h; design in tl_prefill.hip), in their own translation
 * unit so the kernel instances build in parallel.
 */
#include "tl_prefill_kernels.h"

TL_PREFILL_PICKER(tl_prefill_fn_q8_rope, true, true)
