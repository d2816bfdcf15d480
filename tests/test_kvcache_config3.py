"""Config 3's exact request stream through the product's host prefix cache
(libtlkv kv_cache_*, fork lookup, compaction) against the compiled reference's
kvcache.c (src/kvcache.c:192-270) driven by the same calls.

Every request's match, fork length, resume position, hit / computed /
eviction / allocation counts, LRU clock, free-pool size and request map
(CRC) equal the reference's: the committed fixture (written by the compiled
reference, tests/golden/make_config3_trace.py) and, where oracle/_ref is
built, a live replay.  Compactions interleaved on the product side (every 16
requests, as the bench does) rename slots only, so every count stays equal
(the request maps then hold other slot numbers and are not compared).
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
import tlkv

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_config3_trace as C3  # noqa: E402

GOLD = os.path.join(HERE, "golden", "config3_trace.npz")
COUNTS = slice(0, 10)   # every column but the request-map CRC


def _product(between=None):
    return C3.replay(tlkv.KvCache, lambda c, t: c.lookup(t)[0], C3.requests(), between)


def test_config3_stream_equals_reference_fixture():
    rows, caches = _product()
    gold = np.load(GOLD)["rows"]
    assert rows.shape == gold.shape == (64, 11)
    for r in range(64):
        assert rows[r].tolist() == gold[r].tolist(), f"request {r}"
    # the stream does what config 3 is for: hits, forks and evictions
    assert gold[:, 0].sum() > 0 and gold[:, 2].sum() > 0 and gold[-1, 6] > 0
    for c in caches:
        c.close()


def test_config3_stream_with_compaction():
    """Compaction every 16 requests (the bench's cadence) leaves every count
    of the stream unchanged."""
    moved = []

    def between(r, caches):
        if r % 16 == 15:
            for c in caches:
                src, _ = c.compact()
                moved.append(len(src))

    rows, caches = _product(between)
    gold = np.load(GOLD)["rows"]
    for r in range(64):
        assert rows[r, COUNTS].tolist() == gold[r, COUNTS].tolist(), f"request {r}"
    for c in caches:
        c.close()


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
def test_config3_stream_live_reference():
    ref_rows, refs = C3.replay(O.RefKv, lambda c, t: c.lookup_len(t), C3.requests())
    rows, caches = _product()
    assert np.array_equal(rows, ref_rows)
    for a, b in zip(caches, refs):
        assert np.array_equal(a.slots(), b.slots())
        a.close()
