/*
 * tl_prefill_rope.hip — the f16 cache, fused RoPE instances of attn_prefill_kernel
 * (tl_prefill_kernels.h; design in tl_prefill.hip), in their own translation
 * unit so the kernel instances build in parallel.
 */
#include "tl_prefill_kernels.h"

TL_PREFILL_PICKER(tl_prefill_fn_rope, true, false)
