"""Config 3 at its workload on the GPU: the bench's 64-request prefix-reuse
stream (tests/golden/make_config3_trace.py:requests(), the same draws as
bench.py run_config3) through two device sessions of 9216 rows at the
Qwen2.5-7B KV shape (Hkv 4, head_dim 128; 2 layers to keep the host-side
row generation short — every per-layer launch is the same kernel).

Per request: tl_session_kv_prepare_from (match, fork of a longer prefix held
by the other session through tl_kv_copy_between, the graph_kv_prepare resume
rule of src/graph.c:1440-1452), then tl_session_append of the rest in
512-row chunks (src/graph.c:1395-1413).  Every 16 requests both sessions are
compacted (tl_session_compact: optional LRU trim, then one tl_kv_copy launch
that renames live rows into [0, n_live)).

Checked:
- match, fork length and resume of every request, and the counts of the
  session's prefix cache, equal the compiled reference's kvcache.c
  (tests/golden/config3_trace.npz) when no trim is done, and the product's
  host-only replay of the same calls (itself pinned against that fixture by
  tests/test_kvcache_config3.py) with the bench's trim to 3/4 of the pool;
- after every request (fork and append) the rows behind the request's slot
  map are bit for bit the f16 of that request's rows, in every layer;
- after every compaction, every prefix that either session still caches
  (looked up read-only for the 8 shared prefixes and every request served
  so far) holds exactly its rows at its new slots.

K/V rows are a function of the token prefix, as a model's would be: a
rolling hash of tokens[0..p] picks each row's values from a fixed table of
N(0,1) draws, so a forked or relocated row has a known expected value.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_config3_trace as C3  # noqa: E402

pytestmark = pytest.mark.gpu

N_LAYER, HQ, HKV, HD = 2, 28, 4, 128
KD = HKV * HD
POOL, UB = C3.POOL, C3.UBATCH
GOLD = os.path.join(HERE, "golden", "config3_trace.npz")
TAB_BITS = 20
_TAB = np.random.default_rng(0xC3).standard_normal(1 << TAB_BITS).astype(np.float32)
_TAB16 = O.f16_bits(_TAB)
M64 = (1 << 64) - 1


def _prefix_hashes(tokens):
    """h[p] = 64-bit rolling hash of tokens[0..p] (splitmix64 steps)."""
    h = np.empty(len(tokens), np.uint64)
    x = 0x243F6A8885A308D3
    for p, t in enumerate(tokens.tolist()):
        x = (x ^ (t * 0x9E3779B97F4A7C15)) & M64
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
        x ^= x >> 31
        h[p] = x
    return h


def _rows_index(h, salt):
    """Table index of every element of the rows with prefix hashes h."""
    hs = h ^ np.uint64(salt)
    a = (hs & np.uint64((1 << TAB_BITS) - 1)).astype(np.int64)
    b = ((hs >> np.uint64(32)) | np.uint64(1)).astype(np.int64) & ((1 << TAB_BITS) - 1)
    j = np.arange(KD, dtype=np.int64)
    return (a[:, None] + j[None, :] * b[:, None]) & ((1 << TAB_BITS) - 1)


def _salt(layer, which):
    return (0x51ED270B27A4D5C1 * (2 * layer + which + 1)) & M64


class _Radix:
    """kv_cache_* views of a session's prefix cache (same calls as tlkv.KvCache)."""

    def __init__(self, h):
        import tlkv
        self.L, self.h, self.ctx = tlkv._kv_sigs(), h, POOL

    req = __import__("tlkv").KvCache.req
    stats = __import__("tlkv").KvCache.stats
    lookup = __import__("tlkv").KvCache.lookup


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def _gather(T, S, slots):
    import tlkv
    n = len(slots)
    sl = T.from_numpy(np.ascontiguousarray(slots, np.int32)).cuda()
    out = []
    for l in range(N_LAYER):
        ko = T.zeros((n, KD), dtype=T.float16, device="cuda")
        vo = T.zeros_like(ko)
        tlkv.check(tlkv.lib().tl_kv_gather(S.layer(l), tlkv.ptr(sl), n, tlkv.ptr(ko),
                                           tlkv.ptr(vo), None))
        out.append((ko, vo))
    T.cuda.synchronize()
    return [(k.cpu().numpy().view(np.uint16), v.cpu().numpy().view(np.uint16)) for k, v in out]


def _check_rows(T, S, slots, h, what):
    got = _gather(T, S, slots)
    for l, (k, v) in enumerate(got):
        for which, arr in ((0, k), (1, v)):
            exp = _TAB16[_rows_index(h[:len(slots)], _salt(l, which))]
            if not np.array_equal(arr, exp):
                bad = np.nonzero((arr != exp).any(axis=1))[0]
                raise AssertionError(f"{what}: layer {l} {'KV'[which]} rows differ at "
                                     f"positions {bad[:8].tolist()} (of {len(bad)})")


def _expected(trim):
    """Per-request columns [local match, donor match, forked, resume,
    hit_tokens, computed_tokens, evictions, allocations, clock, n_free]."""
    if not trim:
        return np.load(GOLD)["rows"][:, :10]
    import tlkv
    keep = POOL * 3 // 4

    def between(r, caches):
        if r % 16 == 15:
            for c in caches:
                c.trim(keep)
                c.compact()

    rows, caches = C3.replay(tlkv.KvCache, lambda c, t: c.lookup(t)[0], C3.requests(), between)
    for c in caches:
        c.close()
    return rows[:, :10]


@pytest.mark.parametrize("trim", [False, True], ids=["compact", "trim_compact"])
def test_config3_stream_on_device(T, trim):
    import tlkv
    reqs = C3.requests()
    hashes = [_prefix_hashes(t) for t in reqs]
    exp = _expected(trim)
    sess = [tlkv.Session(N_LAYER, HQ, HKV, HD, POOL, UB) for _ in range(2)]
    views = [_Radix(S.radix) for S in sess]
    keep = POOL * 3 // 4 if trim else 0xFFFFFFFF
    forked_total = moved_total = 0
    print(f"config3 on device, trim={trim}", flush=True)
    for r, toks in enumerate(reqs):
        S, other = sess[r % 2], sess[1 - r % 2]
        md = views[1 - r % 2].lookup(toks)[0]
        m, resume, f = S.kv_prepare_from(other, toks)
        n = len(toks)
        h = hashes[r]
        if f:
            # forked rows are the donor's, bit for bit, before anything is appended
            _check_rows(T, S, S.radix_slots(m), h, f"request {r} after fork of {f}")
        forked_total += f
        k = [T.from_numpy(_TAB[_rows_index(h[resume:], _salt(l, 0))]).cuda()
             for l in range(N_LAYER)]
        v = [T.from_numpy(_TAB[_rows_index(h[resume:], _salt(l, 1))]).cuda()
             for l in range(N_LAYER)]
        S.append(toks[resume:], k, v, KD)
        T.cuda.synchronize()
        st, rq = views[r % 2].stats(), views[r % 2].req()
        got = [m - f, md, f, resume, st["hit_tokens"], st["computed_tokens"], st["evictions"],
               st["allocations"], st["clock"], rq["n_free"]]
        assert got == exp[r].tolist(), f"request {r}: {got} != {exp[r].tolist()}"
        _check_rows(T, S, S.radix_slots(n), h, f"request {r} after append")
        if r % 16 == 15:
            for X in sess:
                ev, mv = X.compact(keep=keep)
                moved_total += mv
            for si, X in enumerate(sess):
                rq = views[si].req()
                live = POOL - rq["n_free"]
                checked = set()
                cands = [(reqs[j], hashes[j]) for j in range(r + 1)]
                for toks_j, h_j in cands:
                    ln, slots = views[si].lookup(toks_j)
                    if ln == 0:
                        continue
                    key = (ln, int(h_j[ln - 1]))
                    if key in checked:
                        continue
                    checked.add(key)
                    assert slots.max() < live, "compaction left a live row above n_live"
                    _check_rows(T, X, slots, h_j, f"session {si} after compaction at {r}")
                assert checked, "nothing cached after compaction"
    assert forked_total > 0
    # without the trim the pools stay full (eviction on demand), so there is
    # nothing to move; the trim frees a quarter of each pool first
    assert moved_total > 0 if trim else moved_total >= 0
    for S in sess:
        S.close()
