/*
 * tl_q8.hip — the Q8_0 KV cache: storage, quantizing append, gather and the
 * OP_ATTN entry points over it.
 *
 * The reference's cache is f32 (src/def.h:289-294) and its notes list a
 * quantized KV cache as missing (REMEMBER.md:18).  This cache keeps each
 * row of each kv-head as blocks of 32 values in the GGUF Q8_0 form the
 * reference dequantizes (src/quants.c:368-373: value = q * d, q int8, d
 * binary16), planar so rows stay 16-byte aligned for the DMA loads:
 *   k, v    int8 [n_kv][cap][head_dim]
 *   ks, vs  f16  [n_kv][cap][head_dim / 32]
 * Quantization is the reference's Q8_0 quantizer
 * (src/backend/gpu/gpu.cu:1077-1086): amax = max |x|, d = amax / 127,
 * id = d > 0 ? 1/d : 0, q = rint(x * id); d is stored RNE as binary16.
 *
 *   kv_append_q8_kernel  4 lanes per 32-element block: 8 values of K (RoPE'd
 *                        on the way when asked) and of V each, the block max
 *                        by DPP within the 4 lanes, one 8-byte store of q per
 *                        lane, lane 0 the scale.
 *   kv_gather_q8_kernel  rows by slot (values and scales).
 *   kv_copy_q8_kernel    row copies across layers (fork / compaction).
 * Attention: decode-sized batches run the split-K ring kernel's Q8_0
 * instance (tl_decode.hip), larger ones the MFMA prefill kernel, which
 * dequantizes its tiles to f16 as it stages them (tl_prefill.hip).
 */
#include "tl_common.h"
#include "tl_internal.h"
#include "../../include/tlkv.h"

#include <string.h>

static int check_layer_q8(const tl_kv_layer_q8 *L) {
    if (!L || !L->k || !L->v || !L->ks || !L->vs)
        return tl_fail(TL_EINVAL, "q8 layer: null storage");
    if (L->head_dim != 64 && L->head_dim != 128 && L->head_dim != 256)
        return tl_fail(TL_EINVAL, "head_dim %u unsupported (64/128/256)", L->head_dim);
    if (L->n_kv_head == 0 || L->cap == 0) return tl_fail(TL_EINVAL, "q8 layer: empty shape");
    if (L->ring > L->cap) return tl_fail(TL_EINVAL, "ring %u > cap %u", L->ring, L->cap);
    if ((u64)L->cap * L->head_dim > 0xFFFFFFFFull)
        return tl_fail(TL_ERANGE, "q8 layer: %u rows of head_dim %u exceed 4 GiB per kv-head",
                       L->cap, L->head_dim);
    if (((uintptr_t)L->k | (uintptr_t)L->v) & 15)
        return tl_fail(TL_EINVAL, "q8 cache values not 16-byte aligned");
    if (((uintptr_t)L->ks | (uintptr_t)L->vs) & 3)
        return tl_fail(TL_EINVAL, "q8 cache scales not 4-byte aligned");
    return TL_OK;
}

static LayerView view_q8(const tl_kv_layer_q8 *L) {
    LayerView v;
    v.k = L->k;
    v.v = L->v;
    v.ks = (const u16 *)L->ks;
    v.vs = (const u16 *)L->vs;
    v.cap = L->cap;
    v.n_kv_head = L->n_kv_head;
    v.head_dim = L->head_dim;
    v.ring = L->ring;
    v.q8 = true;
    return v;
}

extern "C" int tl_kv_layer_alloc_q8(tl_kv_layer_q8 *L, uint32_t cap, uint32_t n_kv_head,
                                    uint32_t head_dim, uint32_t ring) {
    if (!L) return tl_fail(TL_EINVAL, "null layer");
    memset(L, 0, sizeof(*L));
    const size_t vb = (size_t)cap * n_kv_head * head_dim;
    const size_t sb = vb / 32 * sizeof(u16);
    if (vb == 0) return tl_fail(TL_EINVAL, "empty layer");
    /* shape rules first, so a rejected layer holds no memory */
    {
        tl_kv_layer_q8 probe = {(void *)16, (void *)16, (void *)16, (void *)16,
                                cap, n_kv_head, head_dim, ring};
        int rc = check_layer_q8(&probe);
        if (rc) return rc;
    }
    void **p[4] = {&L->k, &L->v, &L->ks, &L->vs};
    const size_t bytes[4] = {vb, vb, sb, sb};
    for (int i = 0; i < 4; i++) {
        if (hipMalloc(p[i], bytes[i]) != hipSuccess) {
            *p[i] = NULL;
            tl_kv_layer_free_q8(L);
            return tl_fail(TL_ENOMEM, "q8 layer: %zu bytes", bytes[i]);
        }
        if (hipMemset(*p[i], 0, bytes[i]) != hipSuccess) {
            tl_kv_layer_free_q8(L);
            return tl_fail(TL_EHIP, "q8 layer: clearing %zu bytes failed", bytes[i]);
        }
    }
    L->cap = cap;
    L->n_kv_head = n_kv_head;
    L->head_dim = head_dim;
    L->ring = ring;
    return TL_OK;
}

extern "C" int tl_kv_layer_free_q8(tl_kv_layer_q8 *L) {
    if (!L) return TL_OK;
    void **p[4] = {&L->k, &L->v, &L->ks, &L->vs};
    for (int i = 0; i < 4; i++) {
        if (*p[i]) HIP_TRY(hipFree(*p[i]));
        *p[i] = NULL;
    }
    return TL_OK;
}

/* ------------------------------------------------------------------------ */
/* quantizing append                                                         */
/* ------------------------------------------------------------------------ */

/* one segment: n rows of one layer of one session */
struct Q8AppendSeg {
    int8_t *k8, *v8;
    u16 *ks, *vs;
    const float *k, *v;
    const u32 *slots;
    u32 cap, ring, n_kv, head_dim, kv_stride, pos, n;
};
template <int NS>
struct Q8AppendParamsN {
    Q8AppendSeg seg[NS];
    RopeCfg rope;            /* applied to K before quantizing (rdim 0: none) */
};
typedef Q8AppendParamsN<TL_MAX_BATCH_SEQ> Q8AppendParams;

/* grid: (blocks, segments).  One lane per 8 elements (K RoPE'd first when
 * ROPE, by the routine rope_kernel uses, so the bits equal tl_rope then the
 * plain append); the 4 lanes of a block are an aligned group of a wave
 * (grid stride and row length are multiples of 4), so the block max is a
 * DPP max within the group. */
template <bool ROPE, int NS>
__global__ __launch_bounds__(256) void kv_append_q8_kernel(const Q8AppendParamsN<NS> pp) {
    const Q8AppendSeg &p = pp.seg[blockIdx.y];
    const u32 opr = p.head_dim >> 3;
    const u64 total = (u64)p.n * p.n_kv * opr;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        const u32 e = (u32)(idx % opr);
        const u64 t = idx / opr;
        const u32 h = (u32)(t % p.n_kv);
        const u32 i = (u32)(t / p.n_kv);
        const u64 rowoff = (u64)i * p.kv_stride + (u64)h * p.head_dim;
        float kx[8], vx[8];
        if constexpr (ROPE) {
            load8_rope(p.k + rowoff, e * 8, p.pos + i, pp.rope.rdim, pp.rope.theta,
                       pp.rope.neox, kx);
        } else {
            const float4 a = *(const float4 *)(p.k + rowoff + e * 8);
            const float4 b = *(const float4 *)(p.k + rowoff + e * 8 + 4);
            kx[0] = a.x; kx[1] = a.y; kx[2] = a.z; kx[3] = a.w;
            kx[4] = b.x; kx[5] = b.y; kx[6] = b.z; kx[7] = b.w;
        }
        {
            const float4 a = *(const float4 *)(p.v + rowoff + e * 8);
            const float4 b = *(const float4 *)(p.v + rowoff + e * 8 + 4);
            vx[0] = a.x; vx[1] = a.y; vx[2] = a.z; vx[3] = a.w;
            vx[4] = b.x; vx[5] = b.y; vx[6] = b.z; vx[7] = b.w;
        }
        const float kmax = group_max<4>(amax8(kx));
        const float vmax = group_max<4>(amax8(vx));
        const u32 key = p.pos + i;
        const u32 slot = p.ring ? key % p.ring : (p.slots ? p.slots[key] : key);
        if (slot >= p.cap) continue;
        const float dk = kmax / 127.0f, dv = vmax / 127.0f;
        const float ik = dk > 0.0f ? 1.0f / dk : 0.0f;
        const float iv = dv > 0.0f ? 1.0f / dv : 0.0f;
        const u64 row = (u64)h * p.cap + slot;
        *(uint2 *)(p.k8 + row * p.head_dim + e * 8) = q8_pack8(kx, ik);
        *(uint2 *)(p.v8 + row * p.head_dim + e * 8) = q8_pack8(vx, iv);
        if ((e & 3) == 0) {
            p.ks[row * (p.head_dim / 32) + e / 4] = (u16)f32_to_f16_bits(dk);
            p.vs[row * (p.head_dim / 32) + e / 4] = (u16)f32_to_f16_bits(dv);
        }
    }
}

static int fill_seg_q8(Q8AppendSeg &p, const tl_kv_layer_q8 *L, const float *k, const float *v,
                       u32 kv_stride, const u32 *slots, u32 pos, u32 n) {
    if (!k || !v) return tl_fail(TL_EINVAL, "append: null rows");
    if (kv_stride < L->n_kv_head * L->head_dim || (kv_stride & 3) ||
        (((uintptr_t)k | (uintptr_t)v) & 15))
        return tl_fail(TL_EINVAL, "append: rows must be 16-byte aligned, stride %u", kv_stride);
    p.k8 = (int8_t *)L->k;
    p.v8 = (int8_t *)L->v;
    p.ks = (u16 *)L->ks;
    p.vs = (u16 *)L->vs;
    p.k = k;
    p.v = v;
    p.slots = slots;
    p.cap = L->cap;
    p.ring = L->ring;
    p.n_kv = L->n_kv_head;
    p.head_dim = L->head_dim;
    p.kv_stride = kv_stride;
    p.pos = pos;
    p.n = n;
    return TL_OK;
}

static int launch_append_q8(const Q8AppendParams &p, u32 n_seg, hipStream_t st) {
    u64 most = 0;
    for (u32 i = 0; i < n_seg; i++) {
        const u64 t = (u64)p.seg[i].n * p.seg[i].n_kv * (p.seg[i].head_dim / 8);
        if (t > most) most = t;
    }
    if (most == 0) return TL_OK;
    u64 blocks = (most + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (n_seg == 1) {   /* one segment's arguments: a smaller per-launch copy */
        Q8AppendParamsN<1> p1;
        p1.seg[0] = p.seg[0];
        p1.rope = p.rope;
        if (p.rope.rdim)
            hipLaunchKernelGGL((kv_append_q8_kernel<true, 1>), dim3((u32)blocks, 1), dim3(256), 0, st, p1);
        else
            hipLaunchKernelGGL((kv_append_q8_kernel<false, 1>), dim3((u32)blocks, 1), dim3(256), 0, st, p1);
    } else if (p.rope.rdim) {
        hipLaunchKernelGGL((kv_append_q8_kernel<true, TL_MAX_BATCH_SEQ>), dim3((u32)blocks, n_seg),
                           dim3(256), 0, st, p);
    } else {
        hipLaunchKernelGGL((kv_append_q8_kernel<false, TL_MAX_BATCH_SEQ>), dim3((u32)blocks, n_seg),
                           dim3(256), 0, st, p);
    }
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

static int append_q8(const tl_kv_layer_q8 *L, const float *k, const float *v, u32 kv_stride,
                     const u32 *slots, u32 pos, u32 n, const RopeCfg &rope, hipStream_t st) {
    if (n == 0) return TL_OK;
    Q8AppendParams p;
    memset(&p, 0, sizeof(p));
    int rc = fill_seg_q8(p.seg[0], L, k, v, kv_stride, slots, pos, n);
    if (rc) return rc;
    p.rope = rope;
    return launch_append_q8(p, 1, st);
}

extern "C" int tl_kv_append_q8(const tl_kv_layer_q8 *L, const float *k, const float *v,
                               uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                               uint32_t n, void *stream) {
    int rc = check_layer_q8(L);
    if (rc) return rc;
    RopeCfg none;
    tl_rope_cfg(L->head_dim, nullptr, none);
    return append_q8(L, k, v, kv_stride, slots, pos, n, none, (hipStream_t)stream);
}

extern "C" int tl_kv_append_rope_q8(const tl_kv_layer_q8 *L, const float *k, const float *v,
                                    uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                                    uint32_t n, const tl_rope_params *rope, void *stream) {
    int rc = check_layer_q8(L);
    if (rc) return rc;
    RopeCfg c;
    rc = tl_rope_cfg(L->head_dim, rope, c);
    if (rc) return rc;
    return append_q8(L, k, v, kv_stride, slots, pos, n, c, (hipStream_t)stream);
}

extern "C" int tl_kv_append_layers_q8(const tl_kv_layer_q8 *layers, uint32_t n_layer,
                                      const float *const *k, const float *const *v,
                                      uint32_t kv_stride, const uint32_t *slots, uint32_t pos,
                                      uint32_t n, void *stream) {
    if (n == 0 || n_layer == 0) return TL_OK;
    if (!layers || !k || !v) return tl_fail(TL_EINVAL, "append_layers: null pointer");
    for (u32 l0 = 0; l0 < n_layer; l0 += TL_MAX_BATCH_SEQ) {
        const u32 nl = n_layer - l0 < TL_MAX_BATCH_SEQ ? n_layer - l0 : TL_MAX_BATCH_SEQ;
        Q8AppendParams p;
        memset(&p, 0, sizeof(p));
        for (u32 j = 0; j < nl; j++) {
            const tl_kv_layer_q8 *L = &layers[l0 + j];
            int rc = check_layer_q8(L);
            if (!rc) rc = fill_seg_q8(p.seg[j], L, k[l0 + j], v[l0 + j], kv_stride, slots, pos, n);
            if (rc) return rc;
        }
        int rc = launch_append_q8(p, nl, (hipStream_t)stream);
        if (rc) return rc;
    }
    return TL_OK;
}

/* ------------------------------------------------------------------------ */
/* gather                                                                    */
/* ------------------------------------------------------------------------ */

/* one thread per 16 values (and, for the first of a block's two, its scale) */
__global__ __launch_bounds__(256) void kv_gather_q8_kernel(
    const int8_t *k8, const int8_t *v8, const u16 *ks, const u16 *vs, u32 cap, u32 n_kv,
    u32 head_dim, const u32 *slots, u32 n, int8_t *ko, u16 *kso, int8_t *vo, u16 *vso) {
    const u32 upr = head_dim >> 4;
    const u64 total = (u64)n * n_kv * upr;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        const u32 c = (u32)(idx % upr);
        const u64 t = idx / upr;
        const u32 h = (u32)(t % n_kv);
        const u32 i = (u32)(t / n_kv);
        const u32 slot = slots[i];
        uint4 kk = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
        u16 a = 0, b = 0;
        const bool ok = slot < cap;
        if (ok) {
            const u64 src = ((u64)h * cap + slot) * head_dim + c * 16;
            kk = *(const uint4 *)(k8 + src);
            vv = *(const uint4 *)(v8 + src);
        }
        const u64 dst = ((u64)i * n_kv + h) * head_dim + c * 16;
        *(uint4 *)(ko + dst) = kk;
        *(uint4 *)(vo + dst) = vv;
        if ((c & 1) == 0) {
            if (ok) {
                a = ks[((u64)h * cap + slot) * (head_dim / 32) + c / 2];
                b = vs[((u64)h * cap + slot) * (head_dim / 32) + c / 2];
            }
            kso[dst / 32] = a;
            vso[dst / 32] = b;
        }
    }
}

extern "C" int tl_kv_gather_q8(const tl_kv_layer_q8 *L, const uint32_t *slots, uint32_t n,
                               int8_t *k_out, uint16_t *ks_out, int8_t *v_out,
                               uint16_t *vs_out, void *stream) {
    int rc = check_layer_q8(L);
    if (rc) return rc;
    if (n == 0) return TL_OK;
    if (!slots || !k_out || !v_out || !ks_out || !vs_out)
        return tl_fail(TL_EINVAL, "gather: null pointer");
    if (((uintptr_t)k_out | (uintptr_t)v_out) & 15)
        return tl_fail(TL_EINVAL, "gather: outputs not 16-byte aligned");
    const u64 total = (u64)n * L->n_kv_head * (L->head_dim / 16);
    u64 blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(kv_gather_q8_kernel, dim3((u32)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const int8_t *)L->k, (const int8_t *)L->v, (const u16 *)L->ks,
                       (const u16 *)L->vs, L->cap, L->n_kv_head, L->head_dim, slots, n, k_out,
                       ks_out, v_out, vs_out);
    HIP_TRY(hipGetLastError());
    return TL_OK;
}

/* ------------------------------------------------------------------------ */
/* row copies (fork / compaction)                                            */
/* ------------------------------------------------------------------------ */

#define TL_COPY_Q8_MAX_LAYERS 32
struct Q8CopyParams {
    int8_t *k[TL_COPY_Q8_MAX_LAYERS], *v[TL_COPY_Q8_MAX_LAYERS];          /* destination */
    u16 *ks[TL_COPY_Q8_MAX_LAYERS], *vs[TL_COPY_Q8_MAX_LAYERS];
    const int8_t *sk[TL_COPY_Q8_MAX_LAYERS], *sv[TL_COPY_Q8_MAX_LAYERS];  /* source */
    const u16 *sks[TL_COPY_Q8_MAX_LAYERS], *svs[TL_COPY_Q8_MAX_LAYERS];
    u32 cap, src_cap, n_kv, head_dim;
};

/* grid: (blocks, layers-in-batch).  One thread per 16 values of K and of V;
 * the first thread of each 32-value block also moves the two scales. */
__global__ __launch_bounds__(256) void kv_copy_q8_kernel(const Q8CopyParams p, const u32 *src,
                                                         const u32 *dst, u32 n) {
    const u32 l = blockIdx.y;
    const u32 upr = p.head_dim >> 4;
    const u64 total = (u64)n * p.n_kv * upr;
    for (u64 idx = (u64)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (u64)gridDim.x * blockDim.x) {
        const u32 c = (u32)(idx % upr);
        const u64 t = idx / upr;
        const u32 h = (u32)(t % p.n_kv);
        const u32 i = (u32)(t / p.n_kv);
        const u32 s = src[i], d = dst[i];
        if (s >= p.src_cap || d >= p.cap) continue;
        const u64 so = ((u64)h * p.src_cap + s) * p.head_dim + c * 16;
        const u64 dof = ((u64)h * p.cap + d) * p.head_dim + c * 16;
        *(uint4 *)(p.k[l] + dof) = *(const uint4 *)(p.sk[l] + so);
        *(uint4 *)(p.v[l] + dof) = *(const uint4 *)(p.sv[l] + so);
        if ((c & 1) == 0) {
            p.ks[l][dof / 32] = p.sks[l][so / 32];
            p.vs[l][dof / 32] = p.svs[l][so / 32];
        }
    }
}

static int copy_rows_q8(const tl_kv_layer_q8 *dl, const tl_kv_layer_q8 *sl, uint32_t n_layer,
                        const uint32_t *src, const uint32_t *dst, uint32_t n, void *stream) {
    if (n == 0 || n_layer == 0) return TL_OK;
    if (!dl || !sl || !src || !dst) return tl_fail(TL_EINVAL, "copy: null pointer");
    for (u32 l0 = 0; l0 < n_layer; l0 += TL_COPY_Q8_MAX_LAYERS) {
        const u32 nl = n_layer - l0 < TL_COPY_Q8_MAX_LAYERS ? n_layer - l0 : TL_COPY_Q8_MAX_LAYERS;
        Q8CopyParams p;
        memset(&p, 0, sizeof(p));
        for (u32 j = 0; j < nl; j++) {
            const tl_kv_layer_q8 *D = &dl[l0 + j], *S = &sl[l0 + j];
            int rc = check_layer_q8(D);
            if (!rc) rc = check_layer_q8(S);
            if (rc) return rc;
            if (D->ring || S->ring) return tl_fail(TL_EINVAL, "copy: ring layers hold no slot rows");
            if (j == 0) {
                p.cap = D->cap;
                p.src_cap = S->cap;
                p.n_kv = D->n_kv_head;
                p.head_dim = D->head_dim;
            }
            if (D->cap != p.cap || S->cap != p.src_cap || D->n_kv_head != p.n_kv ||
                S->n_kv_head != p.n_kv || D->head_dim != p.head_dim || S->head_dim != p.head_dim)
                return tl_fail(TL_EINVAL, "copy: layers differ in shape");
            p.k[j] = (int8_t *)D->k;
            p.v[j] = (int8_t *)D->v;
            p.ks[j] = (u16 *)D->ks;
            p.vs[j] = (u16 *)D->vs;
            p.sk[j] = (const int8_t *)S->k;
            p.sv[j] = (const int8_t *)S->v;
            p.sks[j] = (const u16 *)S->ks;
            p.svs[j] = (const u16 *)S->vs;
        }
        const u64 total = (u64)n * p.n_kv * (p.head_dim >> 4);
        u64 blocks = (total + 255) / 256;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL(kv_copy_q8_kernel, dim3((u32)blocks, nl), dim3(256), 0,
                           (hipStream_t)stream, p, src, dst, n);
        HIP_TRY(hipGetLastError());
    }
    return TL_OK;
}

extern "C" int tl_kv_copy_q8(const tl_kv_layer_q8 *layers, uint32_t n_layer, const uint32_t *src,
                             const uint32_t *dst, uint32_t n, void *stream) {
    return copy_rows_q8(layers, layers, n_layer, src, dst, n, stream);
}

extern "C" int tl_kv_copy_between_q8(const tl_kv_layer_q8 *dst_layers,
                                     const tl_kv_layer_q8 *src_layers, uint32_t n_layer,
                                     const uint32_t *src, const uint32_t *dst, uint32_t n,
                                     void *stream) {
    return copy_rows_q8(dst_layers, src_layers, n_layer, src, dst, n, stream);
}

/* ------------------------------------------------------------------------ */
/* OP_ATTN over a Q8_0 cache                                                 */
/* ------------------------------------------------------------------------ */

static int attn_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a, bool append,
                   const tl_rope_params *rp, hipStream_t st) {
    int rc = check_layer_q8(L);
    if (rc) return rc;
    const LayerView lv = view_q8(L);
    rc = tl_check_attn_args(lv, a);
    if (rc) return rc;
    RopeCfg rope;
    rc = tl_rope_cfg(L->head_dim, rp, rope);
    if (rc) return rc;
    if (a->n == 0) return TL_OK;
    const bool prefill = tl_use_prefill(lv, a);
    /* decode-sized batches (with RoPE: up to TL_DEC_Q8_ROPE_NEW rows): the
     * decode launch quantizes and writes the new rows itself */
    const bool fuse = append && !prefill && a->n <= TL_DEC_MAX_NEW &&
                      (rope.rdim == 0 || a->n <= TL_DEC_Q8_ROPE_NEW);
    if (append && !fuse) {
        rc = append_q8(L, a->k, a->v, a->kv_stride, a->slots, a->pos, a->n, rope, st);
        if (rc) return rc;
    }
    if (prefill)
        return tl_launch_prefill(lv, a, rope, st);
    DecParams p;
    memset(&p, 0, sizeof(p));
    if (fuse) {
        Q8AppendSeg chk;
        rc = fill_seg_q8(chk, L, a->k, a->v, a->kv_stride, a->slots, a->pos, a->n);
        if (rc) return rc;
        p.seq[0].kin = a->k;
        p.seq[0].vin = a->v;
        p.seq[0].kv_stride = a->kv_stride;
    }
    p.seq[0].k = (const u16 *)L->k;
    p.seq[0].v = (const u16 *)L->v;
    p.seq[0].ks = (const u16 *)L->ks;
    p.seq[0].vs = (const u16 *)L->vs;
    p.seq[0].slots = a->slots;
    p.seq[0].q = a->q;
    p.seq[0].dst = a->dst;
    p.seq[0].cap = L->cap;
    p.seq[0].ring = L->ring;
    p.seq[0].pos = a->pos;
    p.rows_per_seq = a->n;
    p.n_kv = L->n_kv_head;
    p.n_head = a->n_head;
    p.q_stride = a->q_stride;
    p.window = a->window;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.rope = rope;
    const u32 max_keys = a->pos + a->n;
    const u32 max_vis = (a->window && max_keys > a->window) ? a->window : max_keys;
    return tl_launch_decode(p, a->n, L->head_dim, a->n_head / L->n_kv_head, max_vis, st, true);
}

extern "C" int tl_attn_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a, void *stream) {
    return attn_q8(L, a, true, nullptr, (hipStream_t)stream);
}

extern "C" int tl_attn_rope_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a,
                               const tl_rope_params *rope, void *stream) {
    return attn_q8(L, a, true, rope, (hipStream_t)stream);
}

extern "C" int tl_attn_noappend_q8(const tl_kv_layer_q8 *L, const tl_attn_args *a,
                                   void *stream) {
    return attn_q8(L, a, false, nullptr, (hipStream_t)stream);
}

extern "C" int tl_attn_decode_batch_q8(const tl_decode_seq_q8 *seqs, uint32_t n_seq,
                                       uint32_t n_head, uint32_t window, float scale,
                                       void *stream) {
    if (n_seq == 0) return TL_OK;
    if (!seqs || n_seq > TL_MAX_BATCH_SEQ)
        return tl_fail(TL_EINVAL, "decode_batch: 1..%d sessions", TL_MAX_BATCH_SEQ);
    const tl_kv_layer_q8 *L0 = &seqs[0].layer;
    Q8AppendParams ap;
    memset(&ap, 0, sizeof(ap));
    DecParams p;
    memset(&p, 0, sizeof(p));
    u32 max_vis = 1;
    for (u32 i = 0; i < n_seq; i++) {
        const tl_decode_seq_q8 *s = &seqs[i];
        int rc = check_layer_q8(&s->layer);
        if (rc) return rc;
        if (s->layer.n_kv_head != L0->n_kv_head || s->layer.head_dim != L0->head_dim)
            return tl_fail(TL_EINVAL, "decode_batch: sessions differ in shape");
        tl_attn_args a;
        memset(&a, 0, sizeof(a));
        a.q = s->q; a.k = s->k; a.v = s->v; a.dst = s->dst; a.slots = s->slots;
        a.pos = s->pos; a.n = 1; a.n_head = n_head;
        a.q_stride = n_head * s->layer.head_dim;
        a.kv_stride = s->layer.n_kv_head * s->layer.head_dim;
        a.window = window; a.scale = scale;
        rc = tl_check_attn_args(view_q8(&s->layer), &a);
        if (!rc) rc = fill_seg_q8(ap.seg[i], &s->layer, s->k, s->v, a.kv_stride, s->slots, s->pos, 1);
        if (rc) return rc;
        p.seq[i].k = (const u16 *)s->layer.k;
        p.seq[i].v = (const u16 *)s->layer.v;
        p.seq[i].ks = (const u16 *)s->layer.ks;
        p.seq[i].vs = (const u16 *)s->layer.vs;
        p.seq[i].slots = s->slots;
        p.seq[i].q = s->q;
        p.seq[i].dst = s->dst;
        p.seq[i].cap = s->layer.cap;
        p.seq[i].ring = s->layer.ring;
        p.seq[i].pos = s->pos;
        p.seq[i].kin = s->k;                /* appended by the decode launch */
        p.seq[i].vin = s->v;
        p.seq[i].kv_stride = a.kv_stride;
        const u32 nk = s->pos + 1;
        const u32 vis = (window && nk > window) ? window : nk;
        if (vis > max_vis) max_vis = vis;
    }
    p.rows_per_seq = 1;
    p.n_kv = L0->n_kv_head;
    p.n_head = n_head;
    p.q_stride = n_head * L0->head_dim;
    p.window = window;
    p.scale_log2 = scale * 1.4426950408889634f;
    tl_rope_cfg(L0->head_dim, nullptr, p.rope);
    return tl_launch_decode(p, n_seq, L0->head_dim, n_head / L0->n_kv_head, max_vis,
                            (hipStream_t)stream, true);
}
