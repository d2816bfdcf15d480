"""Host prefix cache (libtlkv kv_cache_*) against the reference's kvcache.c.

- golden traces written by the compiled reference (tests/golden/kvcache_trace.npz):
  every match/append return value, request map, pool and statistics;
- live comparison with the compiled reference on longer random streams
  (skipped when oracle/_ref was not built);
- the unit cases of the reference's own design spec
  (docs/superpowers/specs/2026-10-28-prefix-kv-cache-design.md:916-985, §14.2).
"""
import os

import numpy as np
import pytest

import oracle as O
import tlkv

GOLD = os.path.join(os.path.dirname(__file__), "golden", "kvcache_trace.npz")
NONE = 0xFFFFFFFF


def test_golden_trace():
    g = np.load(GOLD)
    ctxs, ops, tokens, state, slots = g["ctx"], g["ops"], g["tokens"], g["state"], g["slots"]
    caches = {}
    for i, (si, kind, toff, tlen, pos, n) in enumerate(ops):
        kv = caches.setdefault(int(si), tlkv.KvCache(int(ctxs[si])))
        toks = tokens[toff:toff + tlen]
        ret = kv.match(toks) if kind == 0 else int(kv.append(toks, int(pos), int(n)))
        r, st = kv.req(), kv.stats()
        got = [ret, r["len"], r["shared_len"], int(r["active"]), r["n_free"],
               st["hit_tokens"], st["computed_tokens"], st["evictions"],
               st["allocations"], st["clock"]]
        exp = [int(x) for x in state[i][:10]]
        assert got == exp, f"op {i}: {got} != {exp}"
        so, sn = int(state[i][10]), int(state[i][11])
        assert np.array_equal(kv.slots(sn), slots[so:so + sn]), f"op {i}: slots differ"
    # the traces do evict (LRU) and do hit shared prefixes
    assert state[:, 7].max() > 100 and state[:, 5].max() > 100


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
@pytest.mark.parametrize("seed,ctx,vocab", [(11, 64, 50), (12, 300, 151936), (13, 40, 6)])
def test_live_vs_reference(seed, ctx, vocab):
    rng = np.random.default_rng(seed)
    a, b = tlkv.KvCache(ctx), O.RefKv(ctx)
    prefixes = [rng.integers(0, vocab, size=rng.integers(2, ctx // 2)) for _ in range(6)]
    for it in range(200):
        toks = np.concatenate([prefixes[rng.integers(len(prefixes))],
                               rng.integers(0, vocab, size=rng.integers(1, ctx // 2))])
        toks = toks[:ctx].astype(np.uint32)
        ma, mb = a.match(toks), b.match(toks)
        assert ma == mb
        pos = 0 if ma == 0 else (ma if ma < len(toks) else ma - 1)
        while pos < len(toks):
            n = int(min(rng.integers(1, 12), len(toks) - pos))
            ra, rb = a.append(toks, pos, n), b.append(toks, pos, n)
            assert ra == rb
            if not ra:
                break
            pos += n
        assert a.req() == b.req()
        assert np.array_equal(a.slots(a.req()["len"]), b.slots(b.req()["len"]))
        assert a.stats() == b.stats()
        if it % 20 == 0:
            for s in range(ctx):
                assert a.meta(s) == b.meta(s)


@pytest.fixture(params=["product", "reference"])
def make_kv(request):
    """The scenario tests run on the product and, when built, on the compiled
    reference itself, so their expectations are the reference's behaviour."""
    if request.param == "reference":
        if not O.ref_available():
            pytest.skip("compiled reference not built")
        return O.RefKv
    return tlkv.KvCache


def _fill(kv, toks):
    m = kv.match(toks)
    pos = 0 if m == 0 else (m if m < len(toks) else m - 1)
    assert kv.append(toks, pos, len(toks) - pos)
    return m


def test_fresh_pool_slot_order(make_kv):
    kv = make_kv(16)
    _fill(kv, [5, 6, 7, 8])
    assert list(kv.slots(4)) == [0, 1, 2, 3]       # slot 0 pops first
    assert kv.req() == dict(len=4, shared_len=0, active=False, n_free=12)


def test_branch_sharing(make_kv):
    kv = make_kv(16)
    _fill(kv, [1, 2, 3])
    abc = list(kv.slots(3))
    assert _fill(kv, [1, 2, 4]) == 2                 # A, B shared
    abd = list(kv.slots(3))
    assert abd[:2] == abc[:2] and abd[2] != abc[2]
    assert _fill(kv, [1, 2, 3]) == 3                 # ABC still cached
    assert list(kv.slots(3)) == abc


def test_full_hit_keeps_last_slot(make_kv):
    kv = make_kv(16)
    _fill(kv, [9, 8, 7, 6])
    before = list(kv.slots(4))
    m = kv.match([9, 8, 7, 6])
    assert m == 4
    # resume at m - 1: the last token is recomputed into its existing slot
    assert kv.append([9, 8, 7, 6], 3, 1)
    assert list(kv.slots(4)) == before
    assert kv.stats()["allocations"] == 4


def test_lru_evicts_oldest_unpinned_leaf(make_kv):
    kv = make_kv(6)
    _fill(kv, [1, 2, 3])             # slots 0,1,2
    _fill(kv, [4, 5, 6])             # slots 3,4,5 (releases 1,2,3)
    # pool full; the next request needs 1 slot: the oldest unpinned leaf is
    # slot 2 (token 3, last touched before anything of [4,5,6])
    _fill(kv, [4, 5, 6, 7][:3] + [8])   # [4,5,8]: shares 4,5; needs one slot
    assert kv.stats()["evictions"] == 1
    assert not kv.meta(2)["in_tree"] or kv.meta(2)["token"] == 8
    assert kv.meta(1)["in_tree"] and kv.meta(0)["in_tree"]


def test_pinned_prefix_never_evicted(make_kv):
    kv = make_kv(4)
    _fill(kv, [1, 2, 3, 4])          # whole pool pinned by the active request
    assert not kv.append([1, 2, 3, 4, 5], 4, 1) or kv.req()["len"] <= 4
    # match releases; now a fresh request can evict
    assert _fill(kv, [7, 8]) == 0
    assert kv.stats()["evictions"] == 2


def test_pool_exhaustion_all_pinned(make_kv):
    kv = make_kv(3)
    assert kv.match([1, 2, 3]) == 0
    assert kv.append([1, 2, 3], 0, 3)
    # ctx overflow and a position gap are refused (kvcache.c:222, :238)
    assert not kv.append([1, 2, 3, 4], 3, 1)
    kv2 = make_kv(8)
    assert not kv2.append([1, 2, 3], 1, 1)


def test_dirty_range_tracks_slot_writes():
    kv = tlkv.KvCache(32)
    assert kv.take_dirty() == 0
    kv.match([1, 2, 3])
    kv.append([1, 2, 3], 0, 3)
    assert kv.take_dirty() == 0
    assert kv.take_dirty() == NONE
    kv.append([1, 2, 3, 4], 3, 1)
    assert kv.take_dirty() == 3
    kv.match([1, 2, 9])              # releases, re-locks [1, 2]
    assert kv.take_dirty() == 0
