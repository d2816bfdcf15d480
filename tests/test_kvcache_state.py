"""Recurrent-state snapshots of the host prefix cache (kv_cache_checkpoint /
kv_cache_restore, src/kvcache.c:272-321) against the compiled reference.

The reference drives them with graph_state_save/load over a Session's
registered state buffers (src/graph.c:360-408); here the same op stream runs
through the product's kv_cache_* with host state callbacks
(tl_kv_cache_set_state_ops) and must give the same restore positions, flags
and restored state bytes — including the LRU replacement of snapshots once
the 16-snapshot cap (KV_SNAP_MAX, src/kvcache.c:9) is reached.  Fixture:
tests/golden/kvcache_state.npz (make_golden.gen_kvstate); live when
oracle/_ref is built.
"""
import importlib.util
import os

import numpy as np
import pytest

import oracle as O
import tlkv

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
MG = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(MG)


class OurStateApi:
    def __init__(self, ctx):
        self.kv = tlkv.KvCache(ctx)
        self.kv.set_host_state(MG.STATE_BYTES)

    def match(self, toks):
        return self.kv.match(toks)

    def restore(self, m, n):
        return self.kv.restore(m, n)

    def append(self, toks, pos, n):
        return self.kv.append(toks, pos, n)

    def checkpoint(self, pos):
        return self.kv.checkpoint(pos)

    def set_state(self, b):
        b = np.ascontiguousarray(b, dtype=np.uint8)
        self.kv.state[:] = b.tolist()

    def get_state(self):
        return np.array(self.kv.state[:], dtype=np.uint8)


def _run_ours():
    ctx, _, _ = MG.kvstate_ops()
    return MG.run_kvstate(OurStateApi(ctx))


def test_state_snapshots_vs_reference_golden():
    g = np.load(os.path.join(HERE, "golden", "kvcache_state.npz"))
    log, states = _run_ours()
    assert g["log"][:, 2].sum() > 10                       # restores happen
    assert np.array_equal(log, g["log"])
    assert np.array_equal(states, g["states"])


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
def test_state_snapshots_vs_reference_live():
    ctx, _, _ = MG.kvstate_ops()
    ref = MG.RefStateApi(ctx)
    try:
        rlog, rstates = MG.run_kvstate(ref)
    finally:
        ref.R.rh_kvs_destroy(ref.h)
    log, states = _run_ours()
    assert np.array_equal(log, rlog)
    assert np.array_equal(states, rstates)


def test_restored_state_is_the_checkpointed_one():
    """closed form: restoring at a checkpointed position returns exactly the
    bytes saved there, and nothing past the match is restored"""
    kv = OurStateApi(64)
    toks = np.arange(40, dtype=np.uint32)
    assert kv.match(toks) == 0
    assert kv.append(toks, 0, 20)
    kv.set_state(MG.state_pattern(1, 20))
    assert kv.checkpoint(20)
    assert kv.append(toks, 20, 20)
    kv.set_state(MG.state_pattern(1, 40))
    assert kv.checkpoint(40)
    # same prompt again: match 40, a restore must stay below n = 40
    m = kv.match(toks)
    assert m == 40
    kv.set_state(np.zeros(MG.STATE_BYTES, np.uint8))
    pos, restored = kv.restore(m, 40)
    assert (pos, restored) == (20, True)
    assert np.array_equal(kv.get_state(), MG.state_pattern(1, 20))
    # a longer prompt may restore the deepest snapshot
    longer = np.arange(50, dtype=np.uint32)
    m = kv.match(longer)
    pos, restored = kv.restore(m, 50)
    assert (pos, restored) == (40, True)
    assert np.array_equal(kv.get_state(), MG.state_pattern(1, 40))
