/* tl_prefill.hip — MFMA chunked-prefill attention (gfx950). */
#include "tl_common.h"
#include "tl_internal.h"

bool tl_prefill_supported(const tl_kv_layer *, const tl_attn_args *) { return false; }

int tl_launch_prefill(const tl_kv_layer *, const tl_attn_args *, hipStream_t) {
    return tl_fail(TL_EINVAL, "prefill kernel not available");
}
