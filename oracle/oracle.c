/*
 * oracle.c — CPU restatement of the reference's KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU port.
 *
 * What it restates (reference paths relative to the tinyllama.c tree):
 *   or_f32_to_f16      IEEE-754 binary32 -> binary16, round-to-nearest-even.
 *                      The reference cache is f32 (src/def.h:289-294); the
 *                      f16-cache contract is "device byte = RNE(f32 row)".
 *                      Pinned by tests against numpy.astype(float16) and
 *                      hand-picked special values (zeros, subnormals, ties,
 *                      overflow, NaN).
 *   or_kv_append       op_attn's K/V write-through, src/backend/cpu/cpu_op.c:995-1008
 *                      (slot = slots ? slots[pos+i] : pos+i; head-major
 *                      [head][cap][dim] layout, hs = cap*khd, cpu_op.c:986).
 *   or_kv_gather       inverse view of the above (read rows by slot).
 *   or_attn            op_attn, src/backend/cpu/cpu_op.c:964-1064, incl. the
 *                      sliding-window rule :1019-1022 and softmax :338-349.
 *                      Pinned against the compiled reference (cpu_graph_op)
 *                      through committed golden vectors, plus closed forms.
 *   or_q8_quantize     one 32-element Q8_0 block, the reference's quantizer
 *                      src/backend/gpu/gpu.cu:1077-1086 (amax, d = amax/127,
 *                      id = d > 0 ? 1/d : 0, q = rint(x*id)), with d kept as
 *                      binary16 as the GGUF Q8_0 block stores it.  Pinned by
 *                      tests on constructed blocks (ties to even, the amax
 *                      element -> +-127, zero blocks, error <= d/2).
 *   or_q8_dequant      quants.c:368-373 (value = q * f16_to_f32(d)).  Pinned
 *                      against the compiled reference's gguf_dequant.
 *   or_kv_append_q8 /  the write-through and op_attn over a Q8_0 cache: the
 *   or_attn_q8         rows are quantized on write; attention reads the
 *                      dequantized values (same loop as or_attn).
 *   or_rope_norm/neox  op_rope_norm cpu_op.c:674-700, rope_partial/op_rope_neox
 *                      cpu_op.c:632-670 (f32 libm powf/cosf/sinf).  Pinned by
 *                      golden vectors from the compiled reference, within
 *                      tolerance (the reference builds with -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;

/* ---- binary16 conversion ------------------------------------------------ */

u16 or_f32_to_f16(float f) {
    u32 x;
    memcpy(&x, &f, 4);
    u32 sign = (x >> 16) & 0x8000u;
    u32 exp  = (x >> 23) & 0xffu;
    u32 mant = x & 0x7fffffu;
    if (exp == 0xffu) {
        /* Inf stays Inf; NaN becomes a quiet NaN keeping the top 9 payload bits. */
        if (mant) return (u16)(sign | 0x7e00u | (mant >> 13));
        return (u16)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (u16)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (u16)sign;
        u32 m     = mant | 0x800000u;
        u32 shift = (u32)(14 - e);
        u32 hm    = m >> shift;
        u32 rem   = m & ((1u << shift) - 1u);
        u32 half  = 1u << (shift - 1u);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (u16)(sign | hm);
    }
    u32 hm  = mant >> 13;
    u32 rem = mant & 0x1fffu;
    u32 h   = sign | ((u32)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;
    return (u16)h;
}

float or_f16_to_f32(u16 h) {
    u32 sign = ((u32)h & 0x8000u) << 16;
    u32 exp  = ((u32)h >> 10) & 0x1fu;
    u32 mant = (u32)h & 0x3ffu;
    u32 x;
    if (exp == 0) {
        if (mant == 0) {
            x = sign;
        } else {
            /* subnormal: normalise */
            int e = -1;
            do { mant <<= 1; e++; } while (!(mant & 0x400u));
            mant &= 0x3ffu;
            x = sign | ((u32)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void or_f32_to_f16_array(const float *src, u16 *dst, u64 n) {
    for (u64 i = 0; i < n; i++) dst[i] = or_f32_to_f16(src[i]);
}

void or_f16_to_f32_array(const u16 *src, float *dst, u64 n) {
    for (u64 i = 0; i < n; i++) dst[i] = or_f16_to_f32(src[i]);
}

/* ---- K/V write-through (cpu_op.c:995-1008) ------------------------------ */

/* Cache layout per layer: [n_kv][cap][khd], element type f16 (cache_f16=1)
 * or f32 (cache_f16=0).  Rows come from k/v [n][kv_dim] f32.
 * Returns 0, or -1 when a slot is outside the cache (op_attn returns false). */
int or_kv_append(void *kc, void *vc, int cache_f16, u32 cap, u32 n_kv, u32 khd,
                 const float *k, const float *v, u32 kv_dim,
                 const u32 *slots, u32 pos, u32 n) {
    u64 hs = (u64)cap * khd;
    for (u32 i = 0; i < n; i++) {
        u32 slot = slots ? slots[pos + i] : pos + i;
        if (slot >= cap) return -1;
        const float *kr = k + (u64)i * kv_dim;
        const float *vr = v + (u64)i * kv_dim;
        for (u32 h = 0; h < n_kv; h++) {
            u64 off = (u64)h * hs + (u64)slot * khd;
            if (cache_f16) {
                for (u32 d = 0; d < khd; d++) {
                    ((u16 *)kc)[off + d] = or_f32_to_f16(kr[(u64)h * khd + d]);
                    ((u16 *)vc)[off + d] = or_f32_to_f16(vr[(u64)h * khd + d]);
                }
            } else {
                memcpy((float *)kc + off, kr + (u64)h * khd, (size_t)khd * 4);
                memcpy((float *)vc + off, vr + (u64)h * khd, (size_t)khd * 4);
            }
        }
    }
    return 0;
}

/* Read f16 rows slot[i] -> out [n][n_kv][khd]. */
int or_kv_gather(const u16 *kc, const u16 *vc, u32 cap, u32 n_kv, u32 khd,
                 const u32 *slots, u32 n, u16 *k_out, u16 *v_out) {
    u64 hs = (u64)cap * khd;
    for (u32 i = 0; i < n; i++) {
        if (slots[i] >= cap) return -1;
        for (u32 h = 0; h < n_kv; h++) {
            u64 src = (u64)h * hs + (u64)slots[i] * khd;
            u64 dst = ((u64)i * n_kv + h) * khd;
            memcpy(k_out + dst, kc + src, (size_t)khd * 2);
            memcpy(v_out + dst, vc + src, (size_t)khd * 2);
        }
    }
    return 0;
}

/* ---- attention (cpu_op.c:964-1064) -------------------------------------- */

static void or_softmax(float *x, u32 n) {          /* cpu_op.c:338-349 */
    float mx = x[0];
    for (u32 i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (u32 i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (u32 i = 0; i < n; i++) x[i] /= sum;
}

/* binary16 -> f32 table (filled from or_f16_to_f32 on first use) */
static float g_h2f[65536];
static int g_h2f_ready;

static void h2f_init(void) {
    if (g_h2f_ready) return;
    for (u32 i = 0; i < 65536; i++) g_h2f[i] = or_f16_to_f32((u16)i);
    g_h2f_ready = 1;
}

/* A layer cache as the attention loop reads it: f32, f16, or Q8_0 (int8
 * values plus one binary16 scale per 32 elements, planar). */
typedef struct {
    int type;                      /* 0 f32, 1 f16, 2 q8_0 */
    const void *k, *v;
    const u16 *ks, *vs;
    u32 cap, khd;
} CacheView;

/* one cached row (kv-head h, physical row slot) of K (which 0) or V as f32 */
static const float *view_row(const CacheView *c, int which, u32 h, u32 slot, float *tmp) {
    u64 off = ((u64)h * c->cap + slot) * c->khd;
    const void *base = which ? c->v : c->k;
    if (c->type == 0) return (const float *)base + off;
    if (c->type == 1) {
        const u16 *x = (const u16 *)base + off;
        for (u32 d = 0; d < c->khd; d++) tmp[d] = g_h2f[x[d]];
        return tmp;
    }
    const int8_t *x = (const int8_t *)base + off;
    const u16 *sc = (which ? c->vs : c->ks) + off / 32;
    for (u32 d = 0; d < c->khd; d++) tmp[d] = (float)x[d] * g_h2f[sc[d / 32]];
    return tmp;
}

/* attention of the batch over a cache that already holds its rows
 * (cpu_op.c:1011-1062) */
static int attn_rows(const float *q, float *dst, const CacheView *c, u32 ring,
                     const u32 *slots, u32 pos, u32 n, u32 n_head, u32 n_kv, u32 hd,
                     u32 win, float scale) {
    u32 khd = c->khd, q_dim = n_head * hd, gqa = n_head / n_kv;
    h2f_init();
    float *scr = (float *)malloc(((size_t)pos + n) * sizeof(float));
    float *row = (float *)malloc((size_t)khd * sizeof(float));
    if (!scr || !row) {
        free(scr);
        free(row);
        return -2;
    }
    memset(dst, 0, (size_t)n * q_dim * sizeof(float));
    for (u32 h = 0; h < n_head; h++) {
        u32 kv_h = h / gqa;
        for (u32 qi = 0; qi < n; qi++) {
            const float *qh = q + (u64)qi * q_dim + (u64)h * hd;
            u32 n_keys = pos + qi + 1;
            u32 start = (win && n_keys > win) ? n_keys - win : 0;
            u32 n_vis = n_keys - start;
            for (u32 t = 0; t < n_vis; t++) {
                u32 lp = start + t;
                u32 slot = ring ? lp % ring : (slots ? slots[lp] : lp);
                if (slot >= c->cap) {
                    free(scr);
                    free(row);
                    return -1;
                }
                const float *kr = view_row(c, 0, kv_h, slot, row);
                float sum = 0.0f;
                for (u32 d = 0; d < khd; d++) sum += kr[d] * qh[d];
                scr[t] = sum * scale;
            }
            or_softmax(scr, n_vis);
            float *oh = dst + (u64)qi * q_dim + (u64)h * hd;
            for (u32 t = 0; t < n_vis; t++) {
                u32 lp = start + t;
                u32 slot = ring ? lp % ring : (slots ? slots[lp] : lp);
                const float *vr = view_row(c, 1, kv_h, slot, row);
                float st = scr[t];
                for (u32 d = 0; d < khd; d++) oh[d] += st * vr[d];
            }
        }
    }
    free(scr);
    free(row);
    return 0;
}

/* op_attn restated: write the batch's K/V rows (converted to the cache
 * type), then for every q-head h and batch row qi attend over the visible
 * keys start..pos+qi through the slot table.  dst [n][n_head*hd] f32.
 * ring != 0 selects the ring layout for windowed layers: the physical row
 * of logical position p is p % ring (slots ignored); it is only valid when
 * ring >= win + n - 1 so no row still visible to this batch is overwritten. */
int or_attn(const float *q, const float *k, const float *v, float *dst,
            void *kc, void *vc, int cache_f16, u32 cap, u32 ring,
            const u32 *slots, u32 pos, u32 n,
            u32 n_head, u32 n_kv, u32 hd, u32 khd, u32 win, float scale) {
    u32 kv_dim = n_kv * khd;
    if (ring) {
        if (ring > cap || (win && ring < win + n - 1) || !win) return -1;
        for (u32 i = 0; i < n; i++) {
            u32 slot = (pos + i) % ring;
            int rc = or_kv_append(kc, vc, cache_f16, cap, n_kv, khd,
                                  k + (u64)i * kv_dim, v + (u64)i * kv_dim, kv_dim,
                                  NULL, slot, 1);
            if (rc) return rc;
        }
    } else if (or_kv_append(kc, vc, cache_f16, cap, n_kv, khd, k, v, kv_dim,
                            slots, pos, n)) {
        return -1;
    }
    CacheView c = {cache_f16 ? 1 : 0, kc, vc, NULL, NULL, cap, khd};
    return attn_rows(q, dst, &c, ring, slots, pos, n, n_head, n_kv, hd, win, scale);
}

/* ---- Q8_0 cache ----------------------------------------------------------- */

/* Quantize one block of 32 (gpu.cu:1077-1086): amax = max |x|,
 * d = amax / 127 (f32), id = d > 0 ? 1/d : 0, q = rint(x * id) in the
 * default round-to-nearest-even mode (__float2int_rn); the stored scale is
 * binary16(d), RNE, as the GGUF Q8_0 block holds it (quants.c:370-372). */
void or_q8_quantize(const float *x, int8_t *q, u16 *d_out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    float d = amax / 127.0f;
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    for (int j = 0; j < 32; j++) q[j] = (int8_t)(int)rintf(x[j] * id);
    *d_out = or_f32_to_f16(d);
}

void or_q8_quantize_n(const float *x, u64 nblk, int8_t *q, u16 *d) {
    for (u64 b = 0; b < nblk; b++) or_q8_quantize(x + 32 * b, q + 32 * b, d + b);
}

/* n elements of Q8_0 data (planar: q[n], d[n/32]) -> f32 (quants.c:368-373) */
void or_q8_dequant(const int8_t *q, const u16 *d, u64 n, float *out) {
    for (u64 i = 0; i < n; i++) out[i] = (float)q[i] * or_f16_to_f32(d[i >> 5]);
}

/* write-through into a Q8_0 cache: k8/v8 int8 [n_kv][cap][khd], ks/vs f16
 * [n_kv][cap][khd/32]; slot rule of or_kv_append (ring: p % ring). */
int or_kv_append_q8(int8_t *k8, u16 *ks, int8_t *v8, u16 *vs, u32 cap, u32 ring,
                    u32 n_kv, u32 khd, const float *k, const float *v, u32 kv_dim,
                    const u32 *slots, u32 pos, u32 n) {
    if (khd % 32) return -1;
    for (u32 i = 0; i < n; i++) {
        u32 lp = pos + i;
        u32 slot = ring ? lp % ring : (slots ? slots[lp] : lp);
        if (slot >= cap) return -1;
        for (u32 h = 0; h < n_kv; h++) {
            u64 off = ((u64)h * cap + slot) * khd;
            const float *kr = k + (u64)i * kv_dim + (u64)h * khd;
            const float *vr = v + (u64)i * kv_dim + (u64)h * khd;
            for (u32 b = 0; b < khd / 32; b++) {
                or_q8_quantize(kr + 32 * b, k8 + off + 32 * b, ks + off / 32 + b);
                or_q8_quantize(vr + 32 * b, v8 + off + 32 * b, vs + off / 32 + b);
            }
        }
    }
    return 0;
}

/* op_attn over a Q8_0 cache: quantize-append the batch rows (when k != NULL),
 * then attend over the dequantized cache. */
int or_attn_q8(const float *q, const float *k, const float *v, float *dst,
               int8_t *k8, u16 *ks, int8_t *v8, u16 *vs, u32 cap, u32 ring,
               const u32 *slots, u32 pos, u32 n, u32 n_head, u32 n_kv, u32 khd,
               u32 win, float scale) {
    if (ring && (ring > cap || !win || ring < win + n - 1)) return -1;
    if (k && or_kv_append_q8(k8, ks, v8, vs, cap, ring, n_kv, khd, k, v, n_kv * khd,
                             slots, pos, n))
        return -1;
    CacheView c = {2, k8, v8, ks, vs, cap, khd};
    return attn_rows(q, dst, &c, ring, slots, pos, n, n_head, n_kv, khd, win, scale);
}

/* ---- RoPE (cpu_op.c:632-700) -------------------------------------------- */

/* Consecutive-pair rotation (OP_ROPE_NORM, cpu_op.c:674-700).  buf holds
 * `rows` rows of `row_stride` floats; row p sits at absolute position pos+p. */
void or_rope_norm(float *buf, u32 rows, u32 row_stride, u32 heads, u32 hdim,
                  u32 rdim, u32 pos, float theta_base) {
    for (u32 p = 0; p < rows; p++) {
        u32 abspos = pos + p;
        float *dp = buf + (u64)p * row_stride;
        for (u32 h = 0; h < heads; h++) {
            float *bh = dp + (u64)h * hdim;
            for (u32 i = 0; i < rdim; i += 2) {
                float t  = 1.0f / powf(theta_base, (float)i / (float)rdim);
                float cs = cosf((float)abspos * t);
                float sn = sinf((float)abspos * t);
                float a = bh[i], b = bh[i + 1];
                bh[i]     = a * cs - b * sn;
                bh[i + 1] = a * sn + b * cs;
            }
        }
    }
}

/* Split-half rotation (OP_ROPE_NEOX via rope_partial, cpu_op.c:637-670). */
void or_rope_neox(float *buf, u32 rows, u32 row_stride, u32 heads, u32 hdim,
                  u32 rdim, u32 pos, float theta_base) {
    u32 half = rdim / 2;
    for (u32 p = 0; p < rows; p++) {
        u32 abspos = pos + p;
        float *dp = buf + (u64)p * row_stride;
        for (u32 h = 0; h < heads; h++) {
            float *bh = dp + (u64)h * hdim;
            for (u32 i = 0; i < half; i++) {
                float theta = 1.0f / powf(theta_base, (float)(2 * i) / (float)rdim);
                float c = cosf((float)abspos * theta);
                float s = sinf((float)abspos * theta);
                float a = bh[i], b = bh[i + half];
                bh[i]        = a * c - b * s;
                bh[i + half] = a * s + b * c;
            }
        }
    }
}
