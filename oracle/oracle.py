"""numpy front end of the CPU oracle (oracle.c) and of the compiled reference
harness (oracle/_ref/libtlref.so, present only where the reference tree was
available at build time).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product library.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtlref.so")
SHIM_SO = os.path.join(HERE, "_ref", "libtlshim.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
_u32 = ctypes.c_uint32
_vp = ctypes.c_void_p

_or = None
_ref = None


def build():
    """Compile liboracle.so (and _ref/ when the reference tree is present)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE, "-j8"], check=True)


def lib():
    global _or
    if _or is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f32_to_f16_array.argtypes = [_f32p, _u16p, ctypes.c_uint64]
        L.or_f16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_uint64]
        L.or_kv_append.argtypes = [_vp, _vp, ctypes.c_int, _u32, _u32, _u32,
                                   _f32p, _f32p, _u32, _vp, _u32, _u32]
        L.or_kv_append.restype = ctypes.c_int
        L.or_kv_gather.argtypes = [_u16p, _u16p, _u32, _u32, _u32, _u32p, _u32,
                                   _u16p, _u16p]
        L.or_kv_gather.restype = ctypes.c_int
        L.or_attn.argtypes = [_f32p, _f32p, _f32p, _f32p, _vp, _vp, ctypes.c_int,
                              _u32, _u32, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                              _u32, ctypes.c_float]
        L.or_attn.restype = ctypes.c_int
        _i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
        L.or_q8_quantize.argtypes = [_f32p, _i8p, _u16p]
        L.or_q8_quantize_n.argtypes = [_f32p, ctypes.c_uint64, _i8p, _u16p]
        L.or_q8_dequant.argtypes = [_i8p, _u16p, ctypes.c_uint64, _f32p]
        L.or_kv_append_q8.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                      _f32p, _f32p, _u32, _vp, _u32, _u32]
        L.or_kv_append_q8.restype = ctypes.c_int
        L.or_attn_q8.argtypes = [_f32p, _vp, _vp, _f32p, _vp, _vp, _vp, _vp, _u32, _u32,
                                 _vp, _u32, _u32, _u32, _u32, _u32, _u32, ctypes.c_float]
        L.or_attn_q8.restype = ctypes.c_int
        for nm in ("or_rope_norm", "or_rope_neox"):
            getattr(L, nm).argtypes = [_f32p, _u32, _u32, _u32, _u32, _u32, _u32,
                                       ctypes.c_float]
        _or = L
    return _or


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    """The compiled reference harness, or None when it was not built."""
    global _ref
    if _ref is None and ref_available():
        R = ctypes.CDLL(REF_SO)
        R.rh_attn.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _u32, _vp,
                              _u32, _u32, _u32, _u32, _u32, _u32, _u32]
        R.rh_attn.restype = ctypes.c_int
        R.rh_attn_radix.argtypes = [_vp, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _u32,
                                    _u32, _u32, _u32, _u32, _u32, _u32]
        R.rh_attn_radix.restype = ctypes.c_int
        R.rh_radix_layout.argtypes = [_u64p]
        R.rh_rope.argtypes = [ctypes.c_int, _f32p, _f32p, _u32, _u32, _u32, _u32,
                              _u32, _u32, ctypes.c_float]
        R.rh_rope.restype = ctypes.c_int
        R.rh_kv_create.argtypes = [_u32]
        R.rh_kv_create.restype = _vp
        R.rh_kv_destroy.argtypes = [_vp]
        R.rh_kv_match.argtypes = [_vp, _u32p, _u32]
        R.rh_kv_match.restype = _u32
        R.rh_kv_lookup.argtypes = [_vp, _u32p, _u32]
        R.rh_kv_lookup.restype = _u32
        R.rh_kv_append.argtypes = [_vp, _u32p, _u32, _u32]
        R.rh_kv_append.restype = ctypes.c_int
        R.rh_kv_req.argtypes = [_vp, _u32p]
        R.rh_kv_slots.argtypes = [_vp, _u32p, _u32]
        R.rh_kv_stats.argtypes = [_vp, _u64p]
        R.rh_kv_meta.argtypes = [_vp, _u32, _u32p]
        R.rh_dequant_q8_0.argtypes = [_vp, ctypes.c_uint64, _f32p]
        R.rh_kvs_create.argtypes = [_u32, ctypes.c_uint64]
        R.rh_kvs_create.restype = _vp
        R.rh_kvs_destroy.argtypes = [_vp]
        R.rh_kvs_set_state.argtypes = [_vp, _vp]
        R.rh_kvs_get_state.argtypes = [_vp, _vp]
        R.rh_kvs_cap_snaps.argtypes = [_vp]
        R.rh_kvs_cap_snaps.restype = _u32
        R.rh_kvs_checkpoint.argtypes = [_vp, _u32]
        R.rh_kvs_checkpoint.restype = ctypes.c_int
        R.rh_kvs_restore.argtypes = [_vp, _u32, _u32, _u32p]
        R.rh_kvs_restore.restype = _u32
        _ref = R
    return _ref


_shim = None


def shim_available():
    return os.path.exists(SHIM_SO)


def shim():
    """The executor shim (tinyllama.c_amd/integration/hip_graph_op.c) with its
    harness, built against the reference's headers, or None."""
    global _shim
    if _shim is None and os.path.exists(SHIM_SO):
        S = ctypes.CDLL(SHIM_SO)
        S.rh_attn_shim.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32,
                                   _u32, _u32, _u32, _u32, _vp]
        S.rh_attn_shim.restype = ctypes.c_int
        S.rh_layer_shim.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32,
                                    _u32, _u32, _u32, _u32, _u32, ctypes.c_int,
                                    ctypes.c_float, _u32, ctypes.c_int, _vp]
        S.rh_layer_shim.restype = ctypes.c_int
        S.rh_fallthrough.argtypes = [ctypes.c_int]
        S.rh_fallthrough.restype = ctypes.c_int
        S.rh_op_id.argtypes = [ctypes.c_char_p]
        S.rh_op_id.restype = ctypes.c_int
        S.rh_shim_release.argtypes = [_vp]
        _shim = S
    return _shim


def scale_of(head_dim):
    """1.0f / sqrtf((float)kv_head_dim), as graph.c:1275 forms it."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


# ---- binary16 ---------------------------------------------------------------

def f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_f16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(h.reshape(-1), out.reshape(-1), h.size)
    return out


# ---- cache -----------------------------------------------------------------

class Cache:
    """One layer's K/V cache in the reference layout [n_kv][cap][khd]."""

    def __init__(self, cap, n_kv, khd, f16=True):
        dt = np.uint16 if f16 else np.float32
        self.k = np.zeros((n_kv, cap, khd), dtype=dt)
        self.v = np.zeros((n_kv, cap, khd), dtype=dt)
        self.f16, self.cap, self.n_kv, self.khd = f16, cap, n_kv, khd

    def append(self, k, v, slots, pos, n):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.uint32)
        rc = lib().or_kv_append(self.k.ctypes.data, self.v.ctypes.data, int(self.f16),
                                self.cap, self.n_kv, self.khd, k.reshape(-1),
                                v.reshape(-1), self.n_kv * self.khd,
                                None if sl is None else sl.ctypes.data, pos, n)
        return rc

    def gather(self, slots):
        sl = np.ascontiguousarray(slots, dtype=np.uint32)
        n = sl.size
        ko = np.zeros((n, self.n_kv, self.khd), dtype=np.uint16)
        vo = np.zeros_like(ko)
        rc = lib().or_kv_gather(self.k.reshape(-1), self.v.reshape(-1), self.cap,
                                self.n_kv, self.khd, sl, n, ko.reshape(-1),
                                vo.reshape(-1))
        if rc:
            raise ValueError("gather: slot outside cache")
        return ko, vo


def attn(cache, q, k, v, slots, pos, n, n_head, window=0, ring=0, scale=None):
    """op_attn restated (oracle.c or_attn).  Returns dst [n][n_head*khd] f32."""
    khd = cache.khd
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    dst = np.zeros(n * n_head * khd, dtype=np.float32)
    sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.uint32)
    rc = lib().or_attn(q, k, v, dst, cache.k.ctypes.data, cache.v.ctypes.data,
                       int(cache.f16), cache.cap, ring,
                       None if sl is None else sl.ctypes.data, pos, n, n_head,
                       cache.n_kv, khd, khd, window,
                       scale_of(khd) if scale is None else scale)
    if rc:
        raise ValueError(f"or_attn failed ({rc})")
    return dst.reshape(n, n_head * khd)


# ---- Q8_0 ---------------------------------------------------------------------

def q8_quantize(x):
    """f32 [..., 32k] -> (int8 values, f16 scale bits [..., k]) (oracle.c or_q8_quantize)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    blocks = x.reshape(-1, 32)
    q = np.empty(blocks.shape, dtype=np.int8)
    d = np.empty(blocks.shape[0], dtype=np.uint16)
    lib().or_q8_quantize_n(blocks.reshape(-1), blocks.shape[0], q.reshape(-1), d)
    return q.reshape(x.shape), d.reshape(x.shape[:-1] + (x.shape[-1] // 32,))


def q8_dequant(q, d):
    """planar Q8_0 (int8 values, f16 scale bits) -> f32 (quants.c:368-373)."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    d = np.ascontiguousarray(d, dtype=np.uint16)
    out = np.empty(q.shape, dtype=np.float32)
    lib().or_q8_dequant(q.reshape(-1), d.reshape(-1), q.size, out.reshape(-1))
    return out


class CacheQ8:
    """One layer's Q8_0 cache: int8 [n_kv][cap][khd] + f16 scales [n_kv][cap][khd/32]."""

    def __init__(self, cap, n_kv, khd, ring=0):
        self.k = np.zeros((n_kv, cap, khd), dtype=np.int8)
        self.v = np.zeros_like(self.k)
        self.ks = np.zeros((n_kv, cap, khd // 32), dtype=np.uint16)
        self.vs = np.zeros_like(self.ks)
        self.cap, self.n_kv, self.khd, self.ring = cap, n_kv, khd, ring

    def _ptrs(self):
        return (self.k.ctypes.data, self.ks.ctypes.data, self.v.ctypes.data,
                self.vs.ctypes.data)

    def append(self, k, v, slots, pos, n):
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.uint32)
        return lib().or_kv_append_q8(*self._ptrs(), self.cap, self.ring, self.n_kv, self.khd,
                                     k, v, self.n_kv * self.khd,
                                     None if sl is None else sl.ctypes.data, pos, n)

    def attn(self, q, k, v, slots, pos, n, n_head, window=0, scale=None):
        """op_attn over this cache (k None: rows already appended)."""
        khd = self.khd
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        if k is not None:
            k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
            v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        dst = np.zeros(n * n_head * khd, dtype=np.float32)
        sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.uint32)
        rc = lib().or_attn_q8(q, None if k is None else k.ctypes.data,
                              None if v is None else v.ctypes.data, dst, *self._ptrs(),
                              self.cap, self.ring, None if sl is None else sl.ctypes.data,
                              pos, n, n_head, self.n_kv, khd, window,
                              scale_of(khd) if scale is None else scale)
        if rc:
            raise ValueError(f"or_attn_q8 failed ({rc})")
        return dst.reshape(n, n_head * khd)


def rope(x, heads, hdim, rdim, pos, theta, neox):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    rows, stride = x.shape
    fn = lib().or_rope_neox if neox else lib().or_rope_norm
    fn(x.reshape(-1), rows, stride, heads, hdim, rdim, pos, theta)
    return x


# ---- compiled reference ------------------------------------------------------

def ref_attn(kc, vc, q, k, v, slots, pos, n, n_head, window=0):
    """cpu_graph_op(OP_ATTN) of the compiled reference over an f32 cache
    (kc/vc float32 [n_kv][cap][khd], updated in place)."""
    R = ref()
    n_kv, cap, khd = kc.shape
    dst = np.zeros(n * n_head * khd, dtype=np.float32)
    sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.uint32)
    rc = R.rh_attn(np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                   np.ascontiguousarray(k, dtype=np.float32).reshape(-1),
                   np.ascontiguousarray(v, dtype=np.float32).reshape(-1), dst,
                   kc.reshape(-1), vc.reshape(-1), cap,
                   None if sl is None else sl.ctypes.data, pos, n, n_head, n_kv,
                   khd, khd, window)
    if rc:
        raise ValueError("reference op_attn returned false")
    return dst.reshape(n, n_head * khd)


def ref_attn_radix(radix, kc, vc, q, k, v, pos, n, n_head, window=0):
    """cpu_graph_op(OP_ATTN) with plan->radix = `radix` (a KvRadixCache*
    made by another library); op_attn reads its req.slots / req.len through
    the reference's struct layout (cpu_op.c:988-993)."""
    n_kv, cap, khd = kc.shape
    dst = np.zeros(n * n_head * khd, dtype=np.float32)
    rc = ref().rh_attn_radix(radix, np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                             np.ascontiguousarray(k, dtype=np.float32).reshape(-1),
                             np.ascontiguousarray(v, dtype=np.float32).reshape(-1), dst,
                             kc.reshape(-1), vc.reshape(-1), cap, pos, n, n_head, n_kv,
                             khd, window)
    if rc:
        raise ValueError("reference op_attn returned false")
    return dst.reshape(n, n_head * khd)


def ref_radix_layout():
    """offsetof / sizeof of the reference's KvRadixCache and KvSlotMeta fields."""
    o = np.zeros(16, dtype=np.uint64)
    ref().rh_radix_layout(o)
    return [int(x) for x in o]


def ref_rope(x, heads, hdim, rdim, pos, theta, neox):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, od = x.shape
    out = np.zeros_like(x)
    rc = ref().rh_rope(int(neox), x.reshape(-1), out.reshape(-1), rows, od, heads,
                       hdim, rdim, pos, theta)
    if rc:
        raise ValueError("reference rope returned false")
    return out


def ref_dequant_q8_0(blocks):
    """GGUF Q8_0 blocks uint8 [nblk][34] -> f32 [nblk*32] via the reference."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.shape[0] * 32
    out = np.empty(n, dtype=np.float32)
    ref().rh_dequant_q8_0(blocks.ctypes.data, n, out)
    return out


class RefKv:
    """The reference's kv_cache_* (src/kvcache.c) through the harness."""

    def __init__(self, ctx):
        self.R = ref()
        self.h = self.R.rh_kv_create(ctx)
        self.ctx = ctx

    def __del__(self):
        if getattr(self, "h", None):
            self.R.rh_kv_destroy(self.h)
            self.h = None

    def match(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        return self.R.rh_kv_match(self.h, t, t.size)

    def append(self, tokens, pos, n):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        return bool(self.R.rh_kv_append(self.h, t, pos, n))

    def lookup_len(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        return int(self.R.rh_kv_lookup(self.h, t, t.size))

    def req(self):
        o = np.zeros(4, dtype=np.uint32)
        self.R.rh_kv_req(self.h, o)
        return dict(len=int(o[0]), shared_len=int(o[1]), active=bool(o[2]),
                    n_free=int(o[3]))

    def slots(self, n=None):
        n = self.ctx if n is None else n
        o = np.zeros(n, dtype=np.uint32)
        self.R.rh_kv_slots(self.h, o, n)
        return o

    def stats(self):
        o = np.zeros(5, dtype=np.uint64)
        self.R.rh_kv_stats(self.h, o)
        return dict(hit_tokens=int(o[0]), computed_tokens=int(o[1]),
                    evictions=int(o[2]), allocations=int(o[3]), clock=int(o[4]))

    def meta(self, slot):
        o = np.zeros(7, dtype=np.uint32)
        self.R.rh_kv_meta(self.h, slot, o)
        return dict(token=int(o[0]), parent=int(o[1]), child_count=int(o[2]),
                    ref_count=int(o[3]), in_tree=bool(o[4]),
                    last_used=int(o[5]) | (int(o[6]) << 32))
