"""Eviction compaction and read-only lookup of the host prefix cache.

The reference never moves a cached row (src/kvcache.c:59-120), so compaction
is pinned by an invariant: it only renames slots.  A stream of requests run
with compactions interleaved must give the reference's own results for every
match/append return value, request length, pool occupancy and statistic
(the golden trace written by the compiled reference, and the compiled
reference live when it is built), and the request's logical view — the token
held by the slot of each position and the parent links between them — must
be unchanged.  After a compaction the live slots are exactly [0, n_live).
"""
import os

import numpy as np
import pytest

import oracle as O
import tlkv

GOLD = os.path.join(os.path.dirname(__file__), "golden", "kvcache_trace.npz")
NONE = 0xFFFFFFFF


def _live(kv, ctx):
    return [s for s in range(ctx) if kv.meta(s)["in_tree"]]


def _paths(kv, ctx):
    """token path (tuple) -> (ref_count, child_count, last_used) of every in-tree slot"""
    out = {}
    for s in range(ctx):
        m = kv.meta(s)
        if not m["in_tree"]:
            continue
        path, cur = [], s
        while cur != NONE:
            mc = kv.meta(cur)
            path.append(mc["token"])
            cur = mc["parent"]
        out[tuple(reversed(path))] = (m["ref_count"], m["child_count"], m["last_used"])
    return out


def _check_compaction(kv, ctx):
    before_live = _live(kv, ctx)
    before_paths = _paths(kv, ctx)
    req_len = kv.req()["len"]
    before_tokens = [kv.meta(s)["token"] for s in kv.slots(req_len)]
    src, dst = kv.compact()
    n_live = len(before_live)
    assert _live(kv, ctx) == list(range(n_live))
    assert len(src) == len(dst) == sum(1 for s in before_live if s >= n_live)
    assert np.all(src >= n_live) and np.all(dst < n_live)
    assert len(set(dst.tolist())) == len(dst)
    assert not set(dst.tolist()) & set(before_live)          # destinations were free
    assert _paths(kv, ctx) == before_paths                    # same tree, same LRU state
    sl = kv.slots(req_len)
    assert [kv.meta(s)["token"] for s in sl] == before_tokens
    for i in range(1, req_len):
        assert kv.meta(sl[i])["parent"] == sl[i - 1]
    assert kv.req()["n_free"] == ctx - n_live
    return len(src)


def test_golden_trace_with_compaction():
    """Replay the reference's golden trace, compacting after every third op."""
    g = np.load(GOLD)
    ctxs, ops, tokens, state = g["ctx"], g["ops"], g["tokens"], g["state"]
    caches = {}
    moved = 0
    for i, (si, kind, toff, tlen, pos, n) in enumerate(ops):
        ctx = int(ctxs[si])
        kv = caches.setdefault(int(si), tlkv.KvCache(ctx))
        toks = tokens[toff:toff + tlen]
        ret = kv.match(toks) if kind == 0 else int(kv.append(toks, int(pos), int(n)))
        r, st = kv.req(), kv.stats()
        got = [ret, r["len"], r["shared_len"], int(r["active"]), r["n_free"],
               st["hit_tokens"], st["computed_tokens"], st["evictions"],
               st["allocations"], st["clock"]]
        assert got == [int(x) for x in state[i][:10]], f"op {i}"
        # logical view of the request: position j holds token toks[j]
        sl = kv.slots(r["len"])
        assert [kv.meta(s)["token"] for s in sl] == [int(t) for t in toks[:r["len"]]]
        if i % 3 == 2:
            moved += _check_compaction(kv, ctx)
    # the reference pool only frees slots by evicting into an allocation, so
    # it stays dense and compaction has (almost) nothing to move here; the
    # trim test below is the one that moves rows
    assert moved >= 0


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
@pytest.mark.parametrize("seed,ctx,vocab", [(21, 96, 40), (22, 300, 151936)])
def test_live_vs_reference_with_trim_and_compaction(seed, ctx, vocab):
    """Every fourth request starts with `k` fresh tokens.  The reference
    evicts on demand while appending them to a full pool; the product first
    trims to ctx - k live slots (tl_kv_cache_trim), compacts, then appends
    without evicting.  Both must end with the same cached tree and counters."""
    rng = np.random.default_rng(seed)
    a, b = tlkv.KvCache(ctx), O.RefKv(ctx)
    prefixes = [rng.integers(0, vocab, size=rng.integers(2, ctx // 2)) for _ in range(6)]
    moved = trimmed = 0
    fresh_tok = vocab + 1000
    for it in range(120):
        if it % 4 == 3:
            k = int(rng.integers(1, ctx // 3))
            toks = np.arange(fresh_tok, fresh_tok + k, dtype=np.uint32)
            fresh_tok += k
            assert a.match(toks) == b.match(toks) == 0
            trimmed += a.trim(ctx - k)
            moved += _check_compaction(a, ctx)
            assert a.req()["n_free"] >= k
            ev0 = a.stats()["evictions"]
            assert a.append(toks, 0, k) and b.append(toks, 0, k)
            assert a.stats()["evictions"] == ev0          # room was made beforehand
        else:
            toks = np.concatenate([prefixes[rng.integers(len(prefixes))],
                                   rng.integers(0, vocab, size=rng.integers(1, ctx // 2))])
            toks = toks[:ctx].astype(np.uint32)
            assert a.match(toks) == b.match(toks)
            ma = a.req()["len"]
            pos = 0 if ma == 0 else (ma if ma < len(toks) else ma - 1)
            while pos < len(toks):
                n = int(min(rng.integers(1, 12), len(toks) - pos))
                ra, rb = a.append(toks, pos, n), b.append(toks, pos, n)
                assert ra == rb
                if not ra:
                    break
                pos += n
        assert a.req() == b.req()
        assert a.stats() == b.stats()
        assert _paths(a, ctx) == _paths(b, ctx)      # same cached tree under any numbering
    assert moved > 0 and trimmed > 0


def test_compact_fresh_and_full():
    kv = tlkv.KvCache(16)
    assert len(kv.compact()[0]) == 0
    toks = np.arange(100, 116, dtype=np.uint32)
    assert kv.match(toks) == 0 and kv.append(toks, 0, 16)
    src, dst = kv.compact()                 # a full pool is already dense
    assert len(src) == 0 and kv.req()["n_free"] == 0


def test_trim_then_compact_moves_rows():
    kv = tlkv.KvCache(8)
    a = np.array([1, 2, 3, 4], dtype=np.uint32)
    b = np.array([9, 8, 7], dtype=np.uint32)
    assert kv.match(a) == 0 and kv.append(a, 0, 4)   # slots 0..3
    assert kv.match(b) == 0 and kv.append(b, 0, 3)   # slots 4..6; releases `a`
    assert kv.trim(3) == 4                           # `a` leaf-first: 3, 2, 1, 0
    assert _live(kv, 8) == [4, 5, 6]
    with pytest.raises(tlkv.TlError):
        kv.compact(max_moves=2)
    assert _live(kv, 8) == [4, 5, 6]                 # nothing changed
    src, dst = kv.compact()
    assert src.tolist() == [4, 5, 6] and dst.tolist() == [0, 1, 2]
    assert kv.slots(3).tolist() == [0, 1, 2]
    assert [kv.meta(s)["token"] for s in range(3)] == [9, 8, 7]
    assert kv.match(b) == 3                          # still cached, renamed
    assert kv.stats()["evictions"] == 4


def test_lookup_is_read_only():
    kv = tlkv.KvCache(32)
    t = np.arange(1, 21, dtype=np.uint32)
    assert kv.match(t) == 0 and kv.append(t, 0, 20)
    st, req = kv.stats(), kv.req()
    q = np.concatenate([t[:12], np.array([999, 998], dtype=np.uint32)])
    n, sl = kv.lookup(q)
    assert n == 12
    assert np.array_equal(sl, kv.slots(12))
    assert kv.stats() == st and kv.req() == req     # no touches, no counts
    assert kv.lookup(np.array([5], dtype=np.uint32))[0] == 0
    assert kv.match(q) == 12                        # agrees with match
