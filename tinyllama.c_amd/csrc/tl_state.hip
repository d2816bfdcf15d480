/*
 * tl_state.hip — recurrent-state snapshots as device-to-device copies.
 *
 * The reference saves and restores the recurrent state of stateful archs
 * (Gated DeltaNet / SSM conv rings and states) through host memory:
 * graph_state_save / graph_state_load (src/graph.c:368-408) issue one
 * cudaMemcpy per registered buffer to / from a host snapshot that
 * kv_cache_checkpoint / kv_cache_restore manage (src/kvcache.c:272-321).
 * Here the snapshot lives in device memory and one launch moves every
 * segment: a grid-stride loop over the concatenated byte range, 16 bytes per
 * lane where the segment and its snapshot offset are both 16-byte aligned,
 * bytes otherwise.  HBM bound (each byte read once and written once).
 */
#include "tl_common.h"
#include "tl_internal.h"
#include "../../include/tlkv.h"

#include <string.h>

#define TL_STATE_MAX_SEG 64

struct StateParams {
    uint8_t *seg[TL_STATE_MAX_SEG];
    u64 off[TL_STATE_MAX_SEG + 1];   /* prefix sums of the segment sizes */
    uint8_t *snap;
    u32 n_seg;
    int dir;
};

/* segment holding snapshot byte b (off[] is sorted; n_seg <= 64) */
TL_DEV u32 seg_of(const StateParams &p, u64 b) {
    u32 lo = 0, hi = p.n_seg - 1;
    while (lo < hi) {
        const u32 mid = (lo + hi + 1) >> 1;
        if (p.off[mid] <= b) lo = mid; else hi = mid - 1;
    }
    return lo;
}

/* grid-stride over 16-byte units of the concatenation; a unit that lies
 * inside one aligned segment moves as one uint4, any other unit byte by byte */
__global__ __launch_bounds__(256) void state_copy_kernel(const StateParams p) {
    const u64 total = p.off[p.n_seg];
    const u64 units = (total + 15) / 16;
    for (u64 u = (u64)blockIdx.x * blockDim.x + threadIdx.x; u < units;
         u += (u64)gridDim.x * blockDim.x) {
        const u64 b0 = u * 16;
        const u32 s = seg_of(p, b0);
        const u64 in = b0 - p.off[s];
        uint8_t *d = p.seg[s] + in;
        const uintptr_t so = p.dir == TL_STATE_ZERO ? 0 : (uintptr_t)(p.snap + b0);
        const bool whole = b0 + 16 <= p.off[s + 1] && ((((uintptr_t)d) | so) & 15) == 0;
        if (whole) {
            uint4 *sv = (uint4 *)(p.snap + b0);
            if (p.dir == TL_STATE_SAVE) *sv = *(const uint4 *)d;
            else if (p.dir == TL_STATE_LOAD) *(uint4 *)d = *sv;
            else *(uint4 *)d = make_uint4(0, 0, 0, 0);
            continue;
        }
        const u64 end = b0 + 16 < total ? b0 + 16 : total;
        u32 t = s;
        for (u64 b = b0; b < end; b++) {
            while (b >= p.off[t + 1]) t++;
            uint8_t *x = p.seg[t] + (b - p.off[t]);
            if (p.dir == TL_STATE_SAVE) p.snap[b] = *x;
            else if (p.dir == TL_STATE_LOAD) *x = p.snap[b];
            else *x = 0;
        }
    }
}

extern "C" int tl_state_copy(const tl_state_seg *segs, uint32_t n_seg, void *snap, int dir,
                             void *stream) {
    if (n_seg == 0) return TL_OK;
    if (!segs || (dir != TL_STATE_SAVE && dir != TL_STATE_LOAD && dir != TL_STATE_ZERO))
        return tl_fail(TL_EINVAL, "state copy: bad arguments");
    if (dir != TL_STATE_ZERO && !snap) return tl_fail(TL_EINVAL, "state copy: null snapshot");
    u64 base = 0;
    u32 i = 0;
    while (i < n_seg) {
        StateParams p;
        memset(&p, 0, sizeof(p));
        u32 k = 0;
        for (; i < n_seg && k < TL_STATE_MAX_SEG; i++) {
            if (!segs[i].bytes) continue;
            if (!segs[i].ptr) return tl_fail(TL_EINVAL, "state copy: segment %u is null", i);
            p.seg[k] = (uint8_t *)segs[i].ptr;
            p.off[k + 1] = p.off[k] + segs[i].bytes;
            k++;
        }
        if (k == 0) break;
        p.n_seg = k;
        p.dir = dir;
        p.snap = dir == TL_STATE_ZERO ? nullptr : (uint8_t *)snap + base;
        const u64 units = (p.off[k] + 15) / 16;
        u64 blocks = (units + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(state_copy_kernel, dim3((u32)blocks), dim3(256), 0,
                           (hipStream_t)stream, p);
        HIP_TRY(hipGetLastError());
        base += p.off[k];
    }
    return TL_OK;
}
