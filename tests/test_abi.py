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
