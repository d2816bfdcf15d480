"""The session layer on the GPU: prefix cache (kv_cache_*) + device slot-table
mirror + micro-batch loop + fused OP_ATTN, checked against the oracle.

K/V rows are a deterministic function of the token prefix (as a model's
would be), so a reused prefix holds exactly the rows a recomputation would
write.  Each request's outputs must match the oracle's op_attn over a
contiguous f16 cache holding that request's own rows, within 2e-3; the cache
contents behind the request's slot map must be bit-exact f16 of its rows.
"""
import hashlib

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def prefix_rows(tokens, p, width, salt):
    """K or V row of position p: a function of tokens[0..p] only."""
    h = hashlib.blake2b(np.asarray(tokens[:p + 1], np.uint32).tobytes() + salt, digest_size=8)
    rng = np.random.default_rng(int.from_bytes(h.digest(), "little"))
    return rng.standard_normal(width).astype(np.float32)


def run_session(T, n_layer, nh, nkv, hd, ctx, ub, prompts, decode_steps, window=None,
                ring=None, seed=0, S=None, prepare=None, between=None):
    """Serve `prompts` in order (prefill, then `decode_steps` one-token steps),
    checking every output against the oracle and the slot-mapped rows bit for
    bit.  prepare(S, tokens) replaces kv_prepare; between(S, i) runs after
    request i."""
    import tlkv
    if S is None:
        S = tlkv.Session(n_layer, nh, nkv, hd, ctx, ub, window=window, ring=ring)
    rng = np.random.default_rng(seed)
    qd, kd = nh * hd, nkv * hd
    results = []
    for pi, prompt in enumerate(prompts):
        full = list(prompt) + [int(x) for x in rng.integers(0, 1000, size=decode_steps)]
        if prepare is None:
            matched, resume = S.kv_prepare(np.array(prompt, np.uint32))
        else:
            matched, resume = prepare(S, np.array(prompt, np.uint32))
        calls = [(resume, len(prompt))] + [(p, p + 1) for p in range(len(prompt), len(full))]
        outs = []
        for (a, b) in calls:
            toks = np.array(full[a:b], np.uint32)
            n = b - a
            q = [rng.standard_normal((n, qd)).astype(np.float32) for _ in range(n_layer)]
            k = [np.stack([prefix_rows(full, p, kd, b"k%d" % l) for p in range(a, b)])
                 for l in range(n_layer)]
            v = [np.stack([prefix_rows(full, p, kd, b"v%d" % l) for p in range(a, b)])
                 for l in range(n_layer)]
            dq = [T.from_numpy(x).cuda() for x in q]
            dk = [T.from_numpy(x).cuda() for x in k]
            dv = [T.from_numpy(x).cuda() for x in v]
            do = [T.zeros((n, qd), dtype=T.float32, device="cuda") for _ in range(n_layer)]
            S.execute(toks, dq, dk, dv, do, qd, kd)
            T.cuda.synchronize()
            outs.append((a, b, q, [x.cpu().numpy() for x in do]))
        # oracle: the request's own rows in a contiguous f16 cache
        for l in range(n_layer):
            C = O.Cache(len(full), nkv, hd)
            allk = np.stack([prefix_rows(full, p, kd, b"k%d" % l) for p in range(len(full))])
            allv = np.stack([prefix_rows(full, p, kd, b"v%d" % l) for p in range(len(full))])
            C.append(allk[:outs[0][0]], allv[:outs[0][0]], None, 0, outs[0][0])
            win = window[l] if window else 0
            for (a, b, q, o) in outs:
                ref = O.attn(C, q[l], allk[a:b], allv[a:b], None, a, b - a, nh, window=win)
                err = np.abs(o[l] - ref).max()
                assert err < TOL, f"prompt {pi} layer {l} rows {a}:{b} err {err}"
            # slot-mapped cache rows are the request's rows, bit for bit
            if not (ring and ring[l]):
                slots = T.from_numpy(S.radix_slots(len(full))).cuda()
                ko = T.zeros((len(full), nkv, hd), dtype=T.float16, device="cuda")
                vo = T.zeros_like(ko)
                L = S.layer(l)
                tlkv.check(tlkv.lib().tl_kv_gather(L, tlkv.ptr(slots), len(full),
                                                   tlkv.ptr(ko), tlkv.ptr(vo), None))
                T.cuda.synchronize()
                assert np.array_equal(ko.cpu().numpy().view(np.uint16).reshape(len(full), -1),
                                      O.f16_bits(allk))
                assert np.array_equal(vo.cpu().numpy().view(np.uint16).reshape(len(full), -1),
                                      O.f16_bits(allv))
        results.append((matched, resume))
        if between is not None:
            between(S, pi)
    return S, results


def test_session_prefix_reuse_and_eviction(T):
    rng = np.random.default_rng(1)
    shared = [list(rng.integers(0, 1000, size=n)) for n in (20, 33)]
    prompts = []
    for i in range(6):
        prompts.append(shared[i % 2] + list(rng.integers(0, 1000, size=5 + i)))
    prompts.append(list(prompts[-1]))         # full hit: last token recomputed
    S, res = run_session(T, 2, 8, 2, 128, 96, 16, prompts, decode_steps=3)
    matched = [m for m, _ in res]
    assert matched[0] == 0 and matched[2] >= 20 and matched[3] >= 33
    assert res[-1][0] == len(prompts[-1]) and res[-1][1] == len(prompts[-1]) - 1


def test_session_gqa7_multi_chunk(T):
    rng = np.random.default_rng(2)
    prompts = [list(rng.integers(0, 151936, size=70)), list(rng.integers(0, 151936, size=40))]
    run_session(T, 2, 28, 4, 128, 256, 32, prompts, decode_steps=2, seed=3)


def test_session_window_ring_layer(T):
    rng = np.random.default_rng(3)
    prompts = [list(rng.integers(0, 1000, size=50))]
    # layer 0 windowed on a ring of win + ub - 1 rows, layer 1 global
    run_session(T, 2, 8, 4, 256, 128, 8, prompts, decode_steps=4, window=[16, 0],
                ring=[16 + 8 - 1, 0], seed=4)


# ---- eviction compaction and prefix fork -------------------------------------

def _cached_rows(T, S, n_layer, ctx):
    """token path -> (K rows, V rows) of every layer, for every in-tree slot."""
    import tlkv
    L = tlkv._kv_sigs()
    r = S.radix
    metas = [L.tl_kv_cache_meta(r, s).contents for s in range(ctx)]
    live = [s for s in range(ctx) if metas[s].in_tree]
    paths = {}
    for s in live:
        path, cur = [], s
        while cur != 0xFFFFFFFF:
            path.append(metas[cur].token)
            cur = metas[cur].parent
        paths[s] = tuple(reversed(path))
    sl = T.tensor(live, dtype=T.int32, device="cuda")
    out = {}
    per_layer = []
    for l in range(n_layer):
        lay = S.layer(l)
        ko = T.zeros((len(live), lay.n_kv_head, lay.head_dim), dtype=T.float16, device="cuda")
        vo = T.zeros_like(ko)
        tlkv.check(tlkv.lib().tl_kv_gather(lay, tlkv.ptr(sl), len(live), tlkv.ptr(ko),
                                           tlkv.ptr(vo), None))
        T.cuda.synchronize()
        per_layer.append((ko.cpu().numpy().view(np.uint16), vo.cpu().numpy().view(np.uint16)))
    for i, s in enumerate(live):
        out[paths[s]] = [(k[i].tobytes(), v[i].tobytes()) for (k, v) in per_layer]
    return out, live


def test_session_compaction_moves_rows_exactly(T):
    """Trim + compact between requests: every surviving cached prefix keeps its
    rows bit for bit at its new slot, the live rows end up in [0, n_live), and
    later requests that hit relocated prefixes still match the oracle."""
    rng = np.random.default_rng(5)
    n_layer, ctx = 2, 96
    shared = [list(rng.integers(0, 1000, size=n)) for n in (18, 27)]
    prompts = [shared[i % 2] + list(rng.integers(0, 1000, size=4 + i)) for i in range(6)]
    stats = {"moved": 0, "evicted": 0}

    def between(S, i):
        before, live0 = _cached_rows(T, S, n_layer, ctx)
        ev, mv = S.compact(keep=len(live0) - 8 if i % 2 else 0xFFFFFFFF)
        stats["moved"] += mv
        stats["evicted"] += ev
        after, live1 = _cached_rows(T, S, n_layer, ctx)
        assert live1 == list(range(len(live1)))
        assert len(live1) == len(live0) - ev
        assert set(after) <= set(before)
        for path, rows in after.items():
            assert rows == before[path], f"request {i}: rows of a cached prefix changed"

    run_session(T, n_layer, 8, 2, 128, ctx, 16, prompts, decode_steps=2, between=between)
    assert stats["moved"] > 0 and stats["evicted"] > 0


def test_session_fork_from_donor(T):
    """A prefix cached by one session is copied into another (tl_kv_copy_between)
    instead of recomputed: the copied rows are the donor's, bit for bit, and
    the receiving session's outputs over them match the oracle."""
    import tlkv
    rng = np.random.default_rng(6)
    n_layer, nh, nkv, hd, ctx, ub = 2, 8, 2, 128, 128, 16
    base = list(rng.integers(0, 1000, size=37))
    donor, _ = run_session(T, n_layer, nh, nkv, hd, ctx, ub, [base], decode_steps=0, seed=7)
    S = tlkv.Session(n_layer, nh, nkv, hd, 160, ub)      # different pool size
    forked = []

    def prep(S_, toks):
        m, r, f = S_.kv_prepare_from(donor, toks)
        forked.append(f)
        return m, r

    prompts = [base + list(rng.integers(0, 1000, size=9)), base[:20] + [5, 6, 7]]
    _, res = run_session(T, n_layer, nh, nkv, hd, 160, ub, prompts, decode_steps=2, seed=8,
                         S=S, prepare=prep)
    assert res[0] == (37, 37) and forked[0] == 37
    assert res[1][0] == 20 and forked[1] == 0          # already held locally
    a, _ = _cached_rows(T, donor, n_layer, ctx)
    b, _ = _cached_rows(T, S, n_layer, 160)
    for path, rows in a.items():
        assert b[path] == rows


@pytest.mark.parametrize("kv_q8", [False, True])
def test_session_append_only_multi_chunk(T, kv_q8):
    """tl_session_append: the prefix cache takes every n_ubatch chunk of a
    batch, then one slot upload and one write-through cover the batch.  With
    prefix reuse and LRU eviction (a pool of 96 rows, batches of up to 70
    tokens in 16-token chunks), the rows behind every request's slot map are
    the f16 (or Q8_0) conversion of that request's own rows, bit for bit, and
    the host trace equals a chunk-by-chunk replay through kv_cache_append."""
    import tlkv
    n_layer, nkv, hd, ctx, ub = 2, 2, 64, 96, 16
    kd = nkv * hd
    S = tlkv.Session(n_layer, 8, nkv, hd, ctx, ub, kv_q8=kv_q8)
    ref = tlkv.KvCache(ctx)                      # the same calls, host only
    rng = np.random.default_rng(31)
    shared = [list(rng.integers(0, 1000, size=n)) for n in (23, 40)]
    for i in range(8):
        toks = shared[i % 2] + list(rng.integers(0, 1000, size=int(rng.integers(5, 31))))
        arr = np.array(toks, np.uint32)
        m, resume = S.kv_prepare(arr)
        assert ref.match(arr) == m
        n = len(toks) - resume
        k = [T.from_numpy(np.stack([prefix_rows(toks, p, kd, b"k%d" % l)
                                    for p in range(resume, len(toks))])).cuda()
             for l in range(n_layer)]
        v = [T.from_numpy(np.stack([prefix_rows(toks, p, kd, b"v%d" % l)
                                    for p in range(resume, len(toks))])).cuda()
             for l in range(n_layer)]
        S.append(arr[resume:], k, v, kd)
        for p0 in range(resume, len(toks), ub):
            assert ref.append(arr, p0, min(ub, len(toks) - p0))
        T.cuda.synchronize()
        slots = S.radix_slots(len(toks))
        assert np.array_equal(slots, ref.slots(len(toks)))
        for l in range(n_layer):
            allk = np.stack([prefix_rows(toks, p, kd, b"k%d" % l) for p in range(len(toks))])
            allv = np.stack([prefix_rows(toks, p, kd, b"v%d" % l) for p in range(len(toks))])
            sl = T.tensor(slots.astype(np.int32), device="cuda")
            if kv_q8:
                lay = S.layer_q8(l)
                ko = T.zeros((len(toks), nkv, hd), dtype=T.int8, device="cuda")
                vo = T.zeros_like(ko)
                kso = T.zeros((len(toks), nkv, hd // 32), dtype=T.int16, device="cuda")
                vso = T.zeros_like(kso)
                tlkv.check(tlkv.lib().tl_kv_gather_q8(lay, tlkv.ptr(sl), len(toks), tlkv.ptr(ko),
                                                      tlkv.ptr(kso), tlkv.ptr(vo), tlkv.ptr(vso),
                                                      None))
                T.cuda.synchronize()
                qk, dk = O.q8_quantize(allk.reshape(len(toks), nkv, hd))
                qv, dv = O.q8_quantize(allv.reshape(len(toks), nkv, hd))
                assert np.array_equal(ko.cpu().numpy(), qk)
                assert np.array_equal(kso.cpu().numpy().view(np.uint16), dk)
                assert np.array_equal(vo.cpu().numpy(), qv)
                assert np.array_equal(vso.cpu().numpy().view(np.uint16), dv)
            else:
                lay = S.layer(l)
                ko = T.zeros((len(toks), nkv, hd), dtype=T.float16, device="cuda")
                vo = T.zeros_like(ko)
                tlkv.check(tlkv.lib().tl_kv_gather(lay, tlkv.ptr(sl), len(toks), tlkv.ptr(ko),
                                                   tlkv.ptr(vo), None))
                T.cuda.synchronize()
                assert np.array_equal(ko.cpu().numpy().view(np.uint16).reshape(len(toks), -1),
                                      O.f16_bits(allk))
                assert np.array_equal(vo.cpu().numpy().view(np.uint16).reshape(len(toks), -1),
                                      O.f16_bits(allv))
    st = tlkv._kv_sigs().tl_kv_cache_stats(S.radix).contents
    assert (st.hit_tokens, st.evictions, st.allocations) == (
        ref.stats()["hit_tokens"], ref.stats()["evictions"], ref.stats()["allocations"])
    assert st.evictions > 0


@pytest.mark.parametrize("kv_q8", [False, True])
def test_session_append_only_ring_layer(T, kv_q8):
    """tl_session_append with a batch longer than a ring layer's ring: the ring
    keeps the last `ring` positions, each at row p % ring, bit for bit (no
    launch may carry positions p and p + ring together), and the global layer
    holds every row behind the slot map."""
    import tlkv
    n_layer, nkv, hd, ctx, ub, win = 2, 2, 64, 160, 8, 16
    ring = win + ub - 1
    kd = nkv * hd
    S = tlkv.Session(n_layer, 8, nkv, hd, ctx, ub, window=[win, 0], ring=[ring, 0],
                     kv_q8=kv_q8)
    rng = np.random.default_rng(41)
    toks = [int(x) for x in rng.integers(0, 1000, size=150)]
    arr = np.array(toks, np.uint32)
    S.kv_prepare(arr)
    allk = [np.stack([prefix_rows(toks, p, kd, b"k%d" % l) for p in range(len(toks))])
            for l in range(n_layer)]
    allv = [np.stack([prefix_rows(toks, p, kd, b"v%d" % l) for p in range(len(toks))])
            for l in range(n_layer)]
    # two batches: 97 rows (over four rings' worth), then 53
    for a, b in ((0, 97), (97, 150)):
        S.append(arr[a:b], [T.from_numpy(x[a:b].copy()).cuda() for x in allk],
                 [T.from_numpy(x[a:b].copy()).cuda() for x in allv], kd)
        T.cuda.synchronize()
        n = b
        last = np.arange(n - ring, n)
        for l, sl in ((0, (last % ring).astype(np.int32)),
                      (1, S.radix_slots(n).astype(np.int32))):
            pos = last if l == 0 else np.arange(n)
            dsl = T.from_numpy(sl).cuda()
            m = len(sl)
            if kv_q8:
                src = S.layer_q8(l)
                phys = tlkv.KvLayerQ8(src.k, src.v, src.ks, src.vs,
                                      ring if l == 0 else src.cap, nkv, hd, 0)
                ko = T.zeros((m, nkv, hd), dtype=T.int8, device="cuda")
                kso = T.zeros((m, nkv, hd // 32), dtype=T.int16, device="cuda")
                vo, vso = T.zeros_like(ko), T.zeros_like(kso)
                tlkv.check(tlkv.lib().tl_kv_gather_q8(phys, tlkv.ptr(dsl), m,
                                                      tlkv.ptr(ko), tlkv.ptr(kso), tlkv.ptr(vo),
                                                      tlkv.ptr(vso), None))
                T.cuda.synchronize()
                qk, dk = O.q8_quantize(allk[l][pos].reshape(m, nkv, hd))
                qv, dv = O.q8_quantize(allv[l][pos].reshape(m, nkv, hd))
                assert np.array_equal(ko.cpu().numpy(), qk), f"layer {l} rows {n}"
                assert np.array_equal(kso.cpu().numpy().view(np.uint16), dk)
                assert np.array_equal(vo.cpu().numpy(), qv)
                assert np.array_equal(vso.cpu().numpy().view(np.uint16), dv)
            else:
                src = S.layer(l)
                phys = tlkv.KvLayer(src.k, src.v, ring if l == 0 else src.cap, nkv, hd, 0)
                ko = T.zeros((m, nkv, hd), dtype=T.float16, device="cuda")
                vo = T.zeros_like(ko)
                tlkv.check(tlkv.lib().tl_kv_gather(phys, tlkv.ptr(dsl), m,
                                                   tlkv.ptr(ko), tlkv.ptr(vo), None))
                T.cuda.synchronize()
                assert np.array_equal(ko.cpu().numpy().view(np.uint16).reshape(m, -1),
                                      O.f16_bits(allk[l][pos])), f"layer {l} rows {n}"
                assert np.array_equal(vo.cpu().numpy().view(np.uint16).reshape(m, -1),
                                      O.f16_bits(allv[l][pos]))

