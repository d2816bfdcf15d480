"""ctypes binding of libtlkv.so (the C ABI declared in include/tlkv.h and
include/tl_kvcache.h).

Device buffers are torch tensors on a HIP device; only their addresses cross
the ABI.  The library must be built (``make -C tinyllama.c_amd``); loading
fails loudly when it is missing — there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# TLKV_LIB selects another build of the same library (e.g. the host-sanitizer
# build, `make -C tinyllama.c_amd asan`)
LIB_PATH = os.environ.get("TLKV_LIB") or os.path.join(HERE, "libtlkv.so")

u32 = ctypes.c_uint32
vp = ctypes.c_void_p


class KvLayer(ctypes.Structure):
    _fields_ = [("k", vp), ("v", vp), ("cap", u32), ("n_kv_head", u32),
                ("head_dim", u32), ("ring", u32)]


class KvLayerQ8(ctypes.Structure):
    _fields_ = [("k", vp), ("v", vp), ("ks", vp), ("vs", vp), ("cap", u32),
                ("n_kv_head", u32), ("head_dim", u32), ("ring", u32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", vp), ("k", vp), ("v", vp), ("dst", vp), ("slots", vp),
                ("pos", u32), ("n", u32), ("n_head", u32), ("q_stride", u32),
                ("kv_stride", u32), ("window", u32), ("scale", ctypes.c_float)]


class DecodeSeq(ctypes.Structure):
    _fields_ = [("layer", KvLayer), ("slots", vp), ("pos", u32), ("pad_", u32),
                ("q", vp), ("k", vp), ("v", vp), ("dst", vp)]


class DecodeSeqQ8(ctypes.Structure):
    _fields_ = [("layer", KvLayerQ8), ("slots", vp), ("pos", u32), ("pad_", u32),
                ("q", vp), ("k", vp), ("v", vp), ("dst", vp)]


MAX_BATCH_SEQ = 16


class RopeParams(ctypes.Structure):
    _fields_ = [("rope_dim", u32), ("theta", ctypes.c_float), ("neox", ctypes.c_int32)]

_lib = None


class TlError(RuntimeError):
    pass


# return codes (include/tlkv.h)
TL_OK, TL_EINVAL, TL_ERANGE, TL_EHIP, TL_ENOMEM, TL_EBUSY = 0, -1, -2, -3, -4, -5


# launch-shape overrides (include/tlkv.h TL_TUNE_*)
TUNE_DECODE_WGS, TUNE_DECODE_MIN_KEYS, TUNE_DECODE_MERGE_KERNEL = 0, 1, 2
TUNE_PREFILL_SPLITS, TUNE_NO_PREFILL, TUNE_DECODE_SINGLE_MERGE = 3, 4, 5
TUNE_DECODE_MERGE_POLLS = 6
TUNE_PREFILL_APPEND_POLLS, TUNE_PREFILL_SEPARATE_APPEND = 7, 8
TUNE_DECODE_MFMA, TUNE_DECODE_ROWS = 9, 10


class tuning:
    """Context manager: set a TL_TUNE_* override, restore the old value on exit."""

    def __init__(self, key, value):
        self.key, self.value = key, int(value)

    def __enter__(self):
        L = lib()
        self.old = int(L.tl_get_tuning(self.key))
        check(L.tl_set_tuning(self.key, self.value))
        return self

    def __exit__(self, *exc):
        check(lib().tl_set_tuning(self.key, self.old))
        return False


def lib():
    """Load libtlkv.so once (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise TlError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` "
                      "(or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    L.tl_last_error.restype = ctypes.c_char_p
    sigs = {
        "tl_init": [ctypes.c_int],
        "tl_kv_layer_alloc": [ctypes.POINTER(KvLayer), u32, u32, u32, u32],
        "tl_kv_layer_free": [ctypes.POINTER(KvLayer)],
        "tl_kv_append": [ctypes.POINTER(KvLayer), vp, vp, u32, vp, u32, u32, vp],
        "tl_kv_gather": [ctypes.POINTER(KvLayer), vp, u32, vp, vp, vp],
        "tl_kv_copy": [ctypes.POINTER(KvLayer), u32, vp, vp, u32, vp],
        "tl_kv_copy_between": [ctypes.POINTER(KvLayer), ctypes.POINTER(KvLayer), u32, vp, vp,
                               u32, vp],
        "tl_attn": [ctypes.POINTER(KvLayer), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_noalloc": [ctypes.POINTER(KvLayer), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_noappend": [ctypes.POINTER(KvLayer), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_decode_batch": [ctypes.POINTER(DecodeSeq), u32, u32, u32,
                                 ctypes.c_float, vp],
        "tl_attn_rope": [ctypes.POINTER(KvLayer), ctypes.POINTER(AttnArgs),
                         ctypes.POINTER(RopeParams), vp],
        "tl_kv_append_rope": [ctypes.POINTER(KvLayer), vp, vp, u32, vp, u32, u32,
                              ctypes.POINTER(RopeParams), vp],
        "tl_attn_decode_batch_rope": [ctypes.POINTER(DecodeSeq), u32, u32, u32,
                                      ctypes.c_float, ctypes.POINTER(RopeParams), vp],
        "tl_rope": [vp, u32, u32, u32, u32, u32, u32, ctypes.c_float,
                    ctypes.c_int, vp],
        "tl_probe_read": [vp, ctypes.c_uint64, vp, u32, u32, vp],
        "tl_probe_mfma": [ctypes.c_uint64, u32, vp, vp],
        "tl_set_tuning": [ctypes.c_int, u32],
        "tl_get_tuning": [ctypes.c_int],
        "tl_kv_append_layers": [ctypes.POINTER(KvLayer), u32, ctypes.POINTER(vp),
                                ctypes.POINTER(vp), u32, vp, u32, u32, vp],
        "tl_kv_append_layers_q8": [ctypes.POINTER(KvLayerQ8), u32, ctypes.POINTER(vp),
                                   ctypes.POINTER(vp), u32, vp, u32, u32, vp],
        "tl_state_copy": [ctypes.POINTER(StateSeg), u32, vp, ctypes.c_int, vp],
        "tl_kv_layer_alloc_q8": [ctypes.POINTER(KvLayerQ8), u32, u32, u32, u32],
        "tl_kv_layer_free_q8": [ctypes.POINTER(KvLayerQ8)],
        "tl_kv_append_q8": [ctypes.POINTER(KvLayerQ8), vp, vp, u32, vp, u32, u32, vp],
        "tl_kv_gather_q8": [ctypes.POINTER(KvLayerQ8), vp, u32, vp, vp, vp, vp, vp],
        "tl_attn_decode_batch_q8": [ctypes.POINTER(DecodeSeqQ8), u32, u32, u32, ctypes.c_float,
                                    vp],
        "tl_kv_copy_q8": [ctypes.POINTER(KvLayerQ8), u32, vp, vp, u32, vp],
        "tl_kv_copy_between_q8": [ctypes.POINTER(KvLayerQ8), ctypes.POINTER(KvLayerQ8), u32, vp,
                                  vp, u32, vp],
        "tl_attn_q8": [ctypes.POINTER(KvLayerQ8), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_noappend_q8": [ctypes.POINTER(KvLayerQ8), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_rope_q8": [ctypes.POINTER(KvLayerQ8), ctypes.POINTER(AttnArgs),
                            ctypes.POINTER(RopeParams), vp],
        "tl_kv_append_rope_q8": [ctypes.POINTER(KvLayerQ8), vp, vp, u32, vp, u32, u32,
                                 ctypes.POINTER(RopeParams), vp],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = ctypes.c_int
    L.tl_get_tuning.restype = u32
    _lib = L
    return L


def check(rc):
    if rc != 0:
        raise TlError(f"tlkv error {rc}: {lib().tl_last_error().decode()}")
    return rc


def ptr(t):
    """Device address of a torch tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class Layer:
    """One layer of f16 K/V storage, allocated by torch (16-byte aligned)."""

    def __init__(self, cap, n_kv_head, head_dim, ring=0, device="cuda"):
        import torch
        self.k = torch.zeros((n_kv_head, cap, head_dim), dtype=torch.float16,
                             device=device)
        self.v = torch.zeros_like(self.k)
        self.desc = KvLayer(self.k.data_ptr(), self.v.data_ptr(), cap,
                            n_kv_head, head_dim, ring)

    @property
    def cap(self):
        return self.desc.cap


class LayerQ8:
    """One layer of Q8_0 K/V storage (int8 values + f16 scales), allocated by
    torch: values [n_kv][cap][head_dim] int8, scales [n_kv][cap][head_dim/32]."""

    def __init__(self, cap, n_kv_head, head_dim, ring=0, device="cuda"):
        import torch
        self.k = torch.zeros((n_kv_head, cap, head_dim), dtype=torch.int8, device=device)
        self.v = torch.zeros_like(self.k)
        self.ks = torch.zeros((n_kv_head, cap, head_dim // 32), dtype=torch.int16,
                              device=device)
        self.vs = torch.zeros_like(self.ks)
        self.desc = KvLayerQ8(self.k.data_ptr(), self.v.data_ptr(), self.ks.data_ptr(),
                              self.vs.data_ptr(), cap, n_kv_head, head_dim, ring)

    @property
    def cap(self):
        return self.desc.cap


def attn_args(q, k, v, dst, slots, pos, n, n_head, head_dim, n_kv, window,
              scale=None):
    if scale is None:
        scale = 1.0 / (head_dim ** 0.5)
    return AttnArgs(q.data_ptr(), None if k is None else k.data_ptr(),
                    None if v is None else v.data_ptr(), dst.data_ptr(),
                    None if slots is None else slots.data_ptr(), pos, n, n_head,
                    n_head * head_dim, n_kv * head_dim, window, scale)


# ---- host KV bookkeeping (include/tl_kvcache.h) ------------------------------

class KvSlotMeta(ctypes.Structure):
    _fields_ = [("token", u32), ("parent", u32), ("child_count", u32),
                ("ref_count", u32), ("last_used", ctypes.c_uint64), ("snap", u32),
                ("in_tree", ctypes.c_bool)]


class KvRequestState(ctypes.Structure):
    _fields_ = [("slots", ctypes.POINTER(u32)), ("len", u32), ("shared_len", u32),
                ("active", ctypes.c_bool)]


class KvRequstStats(ctypes.Structure):
    _fields_ = [("hit_tokens", ctypes.c_uint64), ("computed_tokens", ctypes.c_uint64),
                ("evictions", ctypes.c_uint64), ("allocations", ctypes.c_uint64)]


STATE_BYTES_FN = ctypes.CFUNCTYPE(ctypes.c_size_t, vp)
STATE_SAVE_FN = ctypes.CFUNCTYPE(ctypes.c_bool, vp, vp, ctypes.c_size_t)
STATE_LOAD_FN = ctypes.CFUNCTYPE(ctypes.c_bool, vp, vp, ctypes.c_size_t)
STATE_ALLOC_FN = ctypes.CFUNCTYPE(vp, vp, ctypes.c_size_t)
STATE_RELEASE_FN = ctypes.CFUNCTYPE(None, vp, vp)


class TlKvStateOps(ctypes.Structure):
    _fields_ = [("bytes", STATE_BYTES_FN), ("save", STATE_SAVE_FN), ("load", STATE_LOAD_FN),
                ("alloc", STATE_ALLOC_FN), ("release", STATE_RELEASE_FN)]


class StateSeg(ctypes.Structure):
    _fields_ = [("ptr", vp), ("bytes", ctypes.c_uint64)]


TL_STATE_SAVE, TL_STATE_LOAD, TL_STATE_ZERO = 0, 1, 2

_kv_sigs_done = False


def _kv_sigs():
    global _kv_sigs_done
    L = lib()
    if _kv_sigs_done:
        return L
    u32p = ctypes.POINTER(u32)
    L.kv_cache_create.argtypes = [vp, vp, u32]
    L.kv_cache_create.restype = vp
    L.kv_cache_destroy.argtypes = [vp]
    L.kv_cache_destroy.restype = None
    L.kv_cache_match.argtypes = [vp, u32p, u32]
    L.kv_cache_match.restype = u32
    L.kv_cache_append.argtypes = [vp, u32p, u32, u32]
    L.kv_cache_append.restype = ctypes.c_bool
    L.tl_kv_cache_req.argtypes = [vp]
    L.tl_kv_cache_req.restype = ctypes.POINTER(KvRequestState)
    L.tl_kv_cache_stats.argtypes = [vp]
    L.tl_kv_cache_stats.restype = ctypes.POINTER(KvRequstStats)
    L.tl_kv_cache_meta.argtypes = [vp, u32]
    L.tl_kv_cache_meta.restype = ctypes.POINTER(KvSlotMeta)
    L.tl_kv_cache_n_free.argtypes = [vp]
    L.tl_kv_cache_n_free.restype = u32
    L.tl_kv_cache_clock.argtypes = [vp]
    L.tl_kv_cache_clock.restype = ctypes.c_uint64
    L.tl_kv_cache_take_dirty.argtypes = [vp]
    L.tl_kv_cache_take_dirty.restype = u32
    L.tl_kv_cache_compact.argtypes = [vp, u32p, u32p, u32]
    L.tl_kv_cache_compact.restype = u32
    L.tl_kv_cache_lookup.argtypes = [vp, u32p, u32, u32p]
    L.tl_kv_cache_lookup.restype = u32
    L.tl_kv_cache_trim.argtypes = [vp, u32]
    L.tl_kv_cache_trim.restype = u32
    L.tl_kv_cache_set_state_ops.argtypes = [vp, ctypes.POINTER(TlKvStateOps)]
    L.tl_kv_cache_set_state_ops.restype = None
    L.kv_cache_checkpoint.argtypes = [vp, u32]
    L.kv_cache_checkpoint.restype = ctypes.c_bool
    L.kv_cache_restore.argtypes = [vp, u32, u32, ctypes.POINTER(ctypes.c_bool)]
    L.kv_cache_restore.restype = u32
    _kv_sigs_done = True
    return L


def _u32_array(tokens):
    import numpy as np
    a = np.ascontiguousarray(tokens, dtype=np.uint32)
    return a, a.ctypes.data_as(ctypes.POINTER(u32))


class KvCache:
    """kv_cache_* of libtlkv (the product's host prefix cache)."""

    def __init__(self, ctx):
        self.L = _kv_sigs()
        self._dummy = ctypes.c_uint32(1)          # stands for the opaque KvCache*
        self.h = self.L.kv_cache_create(None, ctypes.addressof(self._dummy), ctx)
        if not self.h:
            raise TlError("kv_cache_create failed")
        self.ctx = ctx

    def close(self):
        if getattr(self, "h", None):
            self.L.kv_cache_destroy(self.h)
            self.h = None

    __del__ = close

    def match(self, tokens):
        a, p = _u32_array(tokens)
        return int(self.L.kv_cache_match(self.h, p, a.size))

    def append(self, tokens, pos, n):
        a, p = _u32_array(tokens)
        return bool(self.L.kv_cache_append(self.h, p, pos, n))

    def req(self):
        r = self.L.tl_kv_cache_req(self.h).contents
        return dict(len=int(r.len), shared_len=int(r.shared_len), active=bool(r.active),
                    n_free=int(self.L.tl_kv_cache_n_free(self.h)))

    def slots(self, n=None):
        import numpy as np
        n = self.ctx if n is None else n
        r = self.L.tl_kv_cache_req(self.h).contents
        return np.ctypeslib.as_array(r.slots, shape=(self.ctx,))[:n].copy()

    def stats(self):
        s = self.L.tl_kv_cache_stats(self.h).contents
        return dict(hit_tokens=int(s.hit_tokens), computed_tokens=int(s.computed_tokens),
                    evictions=int(s.evictions), allocations=int(s.allocations),
                    clock=int(self.L.tl_kv_cache_clock(self.h)))

    def meta(self, slot):
        m = self.L.tl_kv_cache_meta(self.h, slot).contents
        return dict(token=int(m.token), parent=int(m.parent), child_count=int(m.child_count),
                    ref_count=int(m.ref_count), in_tree=bool(m.in_tree),
                    last_used=int(m.last_used))

    def take_dirty(self):
        return int(self.L.tl_kv_cache_take_dirty(self.h))

    def compact(self, max_moves=None):
        """Renumber live slots into [0, n_live); returns (src, dst) move arrays."""
        import numpy as np
        m = self.ctx if max_moves is None else max_moves
        src = np.zeros(max(m, 1), dtype=np.uint32)
        dst = np.zeros(max(m, 1), dtype=np.uint32)
        n = self.L.tl_kv_cache_compact(self.h, src.ctypes.data_as(ctypes.POINTER(u32)),
                                       dst.ctypes.data_as(ctypes.POINTER(u32)), m)
        if n == 0xFFFFFFFF:
            raise TlError("compaction needs more moves than allowed")
        return src[:n].copy(), dst[:n].copy()

    def trim(self, keep):
        """Evict LRU leaves until at most `keep` slots are live; returns evictions."""
        return int(self.L.tl_kv_cache_trim(self.h, keep))

    def set_host_state(self, nbytes):
        """Install state callbacks over a host buffer of nbytes (self.state, a
        ctypes array standing for the session's recurrent state); snapshots
        are host memory.  nbytes = 0 removes them."""
        if not nbytes:
            self.L.tl_kv_cache_set_state_ops(self.h, None)
            self._ops = None
            return
        self.state = (ctypes.c_uint8 * nbytes)()
        st = self.state

        def _bytes(_s):
            return nbytes

        def _save(_s, dst, cap):
            if cap < nbytes:
                return False
            ctypes.memmove(dst, st, nbytes)
            return True

        def _load(_s, src, ln):
            if ln < nbytes:
                return False
            ctypes.memmove(st, src, nbytes)
            return True

        self._ops = TlKvStateOps(STATE_BYTES_FN(_bytes), STATE_SAVE_FN(_save),
                                 STATE_LOAD_FN(_load), STATE_ALLOC_FN(), STATE_RELEASE_FN())
        self.L.tl_kv_cache_set_state_ops(self.h, ctypes.byref(self._ops))

    def checkpoint(self, pos):
        return bool(self.L.kv_cache_checkpoint(self.h, pos))

    def restore(self, matched, n):
        flag = ctypes.c_bool(False)
        pos = int(self.L.kv_cache_restore(self.h, matched, n, ctypes.byref(flag)))
        return pos, bool(flag.value)

    def lookup(self, tokens):
        """Read-only longest cached prefix: (length, slots)."""
        import numpy as np
        a, p = _u32_array(tokens)
        out = np.zeros(max(a.size, 1), dtype=np.uint32)
        n = self.L.tl_kv_cache_lookup(self.h, p, a.size, out.ctypes.data_as(ctypes.POINTER(u32)))
        return int(n), out[:n].copy()


# ---- session (include/tl_session.h) -------------------------------------------

def _ptr_array(tensors, n):
    """ctypes array of the n tensors' device addresses (each distinct tensor
    asked once: callers often pass one buffer for every layer)."""
    seen = {}
    out = (vp * n)()
    for i, t in enumerate(tensors):
        a = seen.get(id(t))
        if a is None:
            a = seen[id(t)] = t.data_ptr()
        out[i] = a
    return out


class SessionCfg(ctypes.Structure):
    _fields_ = [("n_layer", u32), ("n_head", u32), ("n_kv_head", u32), ("head_dim", u32),
                ("ctx_size", u32), ("n_ubatch", u32), ("window", ctypes.POINTER(u32)),
                ("ring", ctypes.POINTER(u32)), ("use_radix", ctypes.c_int),
                ("stream", vp), ("kv_q8", ctypes.c_int)]


class Session:
    """tl_session: device KV storage + host prefix cache + micro-batch loop."""

    def __init__(self, n_layer, n_head, n_kv_head, head_dim, ctx_size, n_ubatch,
                 window=None, ring=None, use_radix=True, stream=None, kv_q8=False):
        L = lib()
        if not getattr(L, "_sess_sigs", False):
            L.tl_session_create.argtypes = [ctypes.POINTER(SessionCfg), ctypes.POINTER(vp)]
            L.tl_session_create.restype = ctypes.c_int
            L.tl_session_destroy.argtypes = [vp]
            L.tl_session_destroy.restype = None
            L.tl_session_kv_prepare.argtypes = [vp, ctypes.POINTER(u32), u32,
                                                ctypes.POINTER(u32), ctypes.POINTER(u32)]
            L.tl_session_kv_prepare.restype = ctypes.c_int
            L.tl_session_execute.argtypes = [vp, ctypes.POINTER(u32), u32,
                                             ctypes.POINTER(vp), ctypes.POINTER(vp),
                                             ctypes.POINTER(vp), ctypes.POINTER(vp), u32, u32]
            L.tl_session_execute.restype = ctypes.c_int
            L.tl_session_pos.argtypes = [vp]
            L.tl_session_pos.restype = u32
            L.tl_session_radix.argtypes = [vp]
            L.tl_session_radix.restype = vp
            L.tl_session_layer.argtypes = [vp, u32]
            L.tl_session_layer.restype = ctypes.POINTER(KvLayer)
            L.tl_session_layer_q8.argtypes = [vp, u32]
            L.tl_session_layer_q8.restype = ctypes.POINTER(KvLayerQ8)
            L.tl_session_kv_prepare_from.argtypes = [vp, vp, ctypes.POINTER(u32), u32,
                                                     ctypes.POINTER(u32), ctypes.POINTER(u32),
                                                     ctypes.POINTER(u32)]
            L.tl_session_kv_prepare_from.restype = ctypes.c_int
            L.tl_session_compact.argtypes = [vp, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]
            L.tl_session_compact.restype = ctypes.c_int
            L.tl_session_append.argtypes = [vp, ctypes.POINTER(u32), u32, ctypes.POINTER(vp),
                                            ctypes.POINTER(vp), u32]
            L.tl_session_append.restype = ctypes.c_int
            L.tl_session_set_state.argtypes = [vp, ctypes.POINTER(StateSeg), u32]
            L.tl_session_set_state.restype = ctypes.c_int
            L.tl_session_checkpoint.argtypes = [vp]
            L.tl_session_checkpoint.restype = ctypes.c_int
            L._sess_sigs = True
        self.L = L
        self.n_layer = n_layer
        self._win = (u32 * n_layer)(*(window or [0] * n_layer))
        self._ring = (u32 * n_layer)(*(ring or [0] * n_layer))
        cfg = SessionCfg(n_layer, n_head, n_kv_head, head_dim, ctx_size, n_ubatch,
                         self._win, self._ring, int(use_radix),
                         None if stream is None else stream, int(kv_q8))
        h = vp()
        check(L.tl_session_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            self.L.tl_session_destroy(self.h)
            self.h = None

    __del__ = close

    def kv_prepare(self, tokens):
        a, p = _u32_array(tokens)
        m, r = u32(), u32()
        check(self.L.tl_session_kv_prepare(self.h, p, a.size, ctypes.byref(m), ctypes.byref(r)))
        return int(m.value), int(r.value)

    def kv_prepare_from(self, donor, tokens):
        """Match, forking a longer prefix from `donor`: (matched, resume, forked)."""
        a, p = _u32_array(tokens)
        m, r, f = u32(), u32(), u32()
        check(self.L.tl_session_kv_prepare_from(self.h, donor.h, p, a.size, ctypes.byref(m),
                                                ctypes.byref(r), ctypes.byref(f)))
        return int(m.value), int(r.value), int(f.value)

    def compact(self, keep=0xFFFFFFFF):
        """Trim to `keep` live rows (LRU), then compact: (evicted, moved)."""
        e, n = u32(), u32()
        check(self.L.tl_session_compact(self.h, keep, ctypes.byref(e), ctypes.byref(n)))
        return int(e.value), int(n.value)

    @property
    def radix(self):
        return self.L.tl_session_radix(self.h)

    def set_state(self, tensors):
        """Register device tensors as the session's recurrent state (they must
        stay alive while registered); [] = stateless."""
        segs = (StateSeg * max(len(tensors), 1))(
            *[StateSeg(t.data_ptr(), t.numel() * t.element_size()) for t in tensors])
        check(self.L.tl_session_set_state(self.h, segs, len(tensors)))
        self._state = list(tensors)

    def checkpoint(self):
        check(self.L.tl_session_checkpoint(self.h))

    def append(self, tokens, k, v, kv_stride):
        """K/V write-through only (per-layer device tensors [n_tokens][kv_stride])."""
        a, p = _u32_array(tokens)
        check(self.L.tl_session_append(self.h, p, a.size, _ptr_array(k, self.n_layer),
                                       _ptr_array(v, self.n_layer), kv_stride))

    def execute(self, tokens, q, k, v, out, q_stride, kv_stride):
        """q/k/v/out: per-layer device tensors [n_tokens][stride]."""
        a, p = _u32_array(tokens)
        n = self.n_layer
        check(self.L.tl_session_execute(self.h, p, a.size, _ptr_array(q, n), _ptr_array(k, n),
                                        _ptr_array(v, n), _ptr_array(out, n), q_stride, kv_stride))

    @property
    def pos(self):
        return int(self.L.tl_session_pos(self.h))

    def radix_slots(self, n):
        import numpy as np
        r = self.L.tl_session_radix(self.h)
        req = _kv_sigs().tl_kv_cache_req(r).contents
        return np.ctypeslib.as_array(req.slots, shape=(n,)).copy()

    def layer(self, l):
        return self.L.tl_session_layer(self.h, l).contents

    def layer_q8(self, l):
        return self.L.tl_session_layer_q8(self.h, l).contents
