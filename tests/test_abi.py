"""The C-ABI library loads (no GPU needed to load it) and exports every
function that include/*.h declares; the oracle and, when built, the compiled
reference harness load too."""
import ctypes
import glob
import os
import re

import pytest

import oracle as O
import tlkv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
        src = re.sub(r"//[^\n]*", " ", src)
        src = re.sub(r"#[^\n]*", " ", src).replace("extern \"C\" {", " ")
        # drop struct bodies (function-pointer members live there)
        while True:
            new = re.sub(r"\{[^{}]*\}", ";", src)
            if new == src:
                break
            src = new
        for stmt in src.split(";"):
            stmt = " ".join(stmt.split())
            if not stmt or stmt.startswith("typedef") or "extern \"C\"" in stmt:
                continue
            m = re.match(r"^[\w\s\*]*?\b(\w+)\s*\(", stmt)
            if m:
                names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_entry_points():
    names = declared_functions()
    for must in ("tl_attn", "tl_kv_append", "tl_kv_gather", "tl_kv_copy", "kv_cache_create",
                 "kv_cache_append", "kv_cache_match", "tl_session_execute"):
        assert must in names


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports(name):
    lib = ctypes.CDLL(tlkv.LIB_PATH)
    assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_oracle_loads():
    assert O.lib().or_f32_to_f16(1.0) == 0x3C00


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
def test_reference_harness_loads():
    assert O.ref() is not None


def test_argument_errors_need_no_device():
    """Shape and argument checks run before any HIP call: a rejected layer
    holds no memory and the calls below return TL_EINVAL without a GPU."""
    import ctypes
    lib = tlkv.lib()
    L8 = tlkv.KvLayerQ8()
    assert lib.tl_kv_layer_alloc_q8(ctypes.byref(L8), 16, 2, 48, 0) == -1
    assert not (L8.k or L8.v or L8.ks or L8.vs)
    assert b"head_dim" in lib.tl_last_error()
    L = tlkv.KvLayer()
    assert lib.tl_kv_layer_alloc(ctypes.byref(L), 16, 2, 96, 0) == -1
    assert not (L.k or L.v)
    assert lib.tl_kv_layer_alloc(ctypes.byref(L), 16, 2, 64, 17) == -1      # ring > cap
    a = tlkv.AttnArgs()
    assert lib.tl_attn_q8(None, ctypes.byref(a), None) == -1
    assert lib.tl_attn_noappend_q8(ctypes.byref(L8), ctypes.byref(a), None) == -1
    seg = (tlkv.StateSeg * 1)(tlkv.StateSeg(None, 64))
    assert lib.tl_state_copy(seg, 1, None, tlkv.TL_STATE_ZERO, None) == -1
    assert lib.tl_state_copy(seg, 1, None, 7, None) == -1
    assert lib.tl_state_copy(seg, 0, None, tlkv.TL_STATE_SAVE, None) == 0   # nothing to do


def test_size_limits_and_empty_batches_need_no_device():
    """A kv-head's rows are addressed with 32-bit byte offsets: layers past
    4 GiB per kv-head are refused before allocating; empty batches are
    no-ops (no launch)."""
    import ctypes
    lib = tlkv.lib()
    TL_ERANGE = -2
    L = tlkv.KvLayer()
    assert lib.tl_kv_layer_alloc(ctypes.byref(L), 1 << 24, 1, 256, 0) == TL_ERANGE
    assert not (L.k or L.v)
    L8 = tlkv.KvLayerQ8()
    assert lib.tl_kv_layer_alloc_q8(ctypes.byref(L8), 1 << 26, 1, 128, 0) == TL_ERANGE
    assert not (L8.k or L8.ks)
    # empty batches return before touching the device (storage pointers are fake)
    fake = tlkv.KvLayerQ8(16, 16, 16, 16, 64, 2, 64, 0)
    assert lib.tl_kv_append_q8(ctypes.byref(fake), None, None, 128, None, 0, 0, None) == 0
    a = tlkv.AttnArgs(16, 0, 0, 16, 0, 0, 0, 4, 256, 128, 0, 0.125)
    assert lib.tl_attn_noappend_q8(ctypes.byref(fake), ctypes.byref(a), None) == 0
    assert lib.tl_attn_decode_batch_q8(None, 0, 4, 0, 0.125, None) == 0


@pytest.mark.skipif(not O.shim_available(), reason="executor shim not built (no reference tree)")
def test_executor_shim_loads():
    S = O.shim()
    for name in ("hip_graph_op", "hip_graph_op_set_stream", "hip_graph_op_release",
                 "hip_graph_op_fused_count"):
        assert hasattr(S, name)


def test_tuning_overrides_need_no_device():
    """Launch-shape overrides: set/get round trip, restore through the context
    manager, unknown keys rejected."""
    lib = tlkv.lib()
    old = lib.tl_get_tuning(tlkv.TUNE_PREFILL_SPLITS)
    with tlkv.tuning(tlkv.TUNE_PREFILL_SPLITS, 5):
        assert lib.tl_get_tuning(tlkv.TUNE_PREFILL_SPLITS) == 5
    assert lib.tl_get_tuning(tlkv.TUNE_PREFILL_SPLITS) == old
    assert lib.tl_set_tuning(99, 1) == -1
    assert lib.tl_set_tuning(-1, 1) == -1
    assert lib.tl_get_tuning(99) == 0
