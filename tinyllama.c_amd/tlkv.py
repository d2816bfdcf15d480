"""ctypes binding of libtlkv.so (the C ABI declared in include/tlkv.h and
include/tl_kvcache.h).

Device buffers are torch tensors on a HIP device; only their addresses cross
the ABI.  The library must be built (``make -C tinyllama.c_amd``); loading
fails loudly when it is missing — there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtlkv.so")

u32 = ctypes.c_uint32
vp = ctypes.c_void_p


class KvLayer(ctypes.Structure):
    _fields_ = [("k", vp), ("v", vp), ("cap", u32), ("n_kv_head", u32),
                ("head_dim", u32), ("ring", u32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", vp), ("k", vp), ("v", vp), ("dst", vp), ("slots", vp),
                ("pos", u32), ("n", u32), ("n_head", u32), ("q_stride", u32),
                ("kv_stride", u32), ("window", u32), ("scale", ctypes.c_float)]


class DecodeSeq(ctypes.Structure):
    _fields_ = [("layer", KvLayer), ("slots", vp), ("pos", u32), ("pad_", u32),
                ("q", vp), ("k", vp), ("v", vp), ("dst", vp)]


MAX_BATCH_SEQ = 16

_lib = None


class TlError(RuntimeError):
    pass


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
        "tl_attn": [ctypes.POINTER(KvLayer), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_noappend": [ctypes.POINTER(KvLayer), ctypes.POINTER(AttnArgs), vp],
        "tl_attn_decode_batch": [ctypes.POINTER(DecodeSeq), u32, u32, u32,
                                 ctypes.c_float, vp],
        "tl_rope": [vp, u32, u32, u32, u32, u32, u32, ctypes.c_float,
                    ctypes.c_int, vp],
        "tl_probe_read": [vp, ctypes.c_uint64, vp, u32, u32, vp],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = ctypes.c_int
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


def attn_args(q, k, v, dst, slots, pos, n, n_head, head_dim, n_kv, window,
              scale=None):
    if scale is None:
        scale = 1.0 / (head_dim ** 0.5)
    return AttnArgs(q.data_ptr(), None if k is None else k.data_ptr(),
                    None if v is None else v.data_ptr(), dst.data_ptr(),
                    None if slots is None else slots.data_ptr(), pos, n, n_head,
                    n_head * head_dim, n_kv * head_dim, window, scale)
