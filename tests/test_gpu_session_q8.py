"""The session layer over a Q8_0 cache (tl_session_cfg.kv_q8): prefix cache +
device slot table + micro-batch loop with the quantizing append and
tl_attn_q8, prefix fork (tl_kv_copy_between_q8) and compaction
(tl_kv_copy_q8).

K/V rows are a deterministic function of the token prefix (as a model's
would be), so a reused or forked prefix holds exactly the rows a
recomputation would write.  Each request's outputs must match the oracle's
op_attn over a Q8_0 cache holding that request's own rows, within 2e-3; the
values and scales behind the request's slot map must be the oracle's
quantization of its rows, bit for bit.
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
    h = hashlib.blake2b(np.asarray(tokens[:p + 1], np.uint32).tobytes() + salt, digest_size=8)
    rng = np.random.default_rng(int.from_bytes(h.digest(), "little"))
    return rng.standard_normal(width).astype(np.float32)


def gather_q8(T, lay, slots):
    import tlkv
    n = len(slots)
    sl = T.tensor(np.asarray(slots, np.int64).astype(np.int32), device="cuda")
    ko = T.zeros((n, lay.n_kv_head, lay.head_dim), dtype=T.int8, device="cuda")
    vo = T.zeros_like(ko)
    kso = T.zeros((n, lay.n_kv_head, lay.head_dim // 32), dtype=T.int16, device="cuda")
    vso = T.zeros_like(kso)
    tlkv.check(tlkv.lib().tl_kv_gather_q8(lay, tlkv.ptr(sl), n, tlkv.ptr(ko), tlkv.ptr(kso),
                                          tlkv.ptr(vo), tlkv.ptr(vso), None))
    T.cuda.synchronize()
    return (ko.cpu().numpy(), kso.cpu().numpy().view(np.uint16), vo.cpu().numpy(),
            vso.cpu().numpy().view(np.uint16))


def run_session(T, n_layer, nh, nkv, hd, ctx, ub, prompts, decode_steps, seed=0, S=None,
                prepare=None, between=None):
    import tlkv
    if S is None:
        S = tlkv.Session(n_layer, nh, nkv, hd, ctx, ub, kv_q8=True)
    rng = np.random.default_rng(seed)
    qd, kd = nh * hd, nkv * hd
    results = []
    for pi, prompt in enumerate(prompts):
        full = list(prompt) + [int(x) for x in rng.integers(0, 1000, size=decode_steps)]
        toks0 = np.array(prompt, np.uint32)
        matched, resume = S.kv_prepare(toks0) if prepare is None else prepare(S, toks0)
        calls = [(resume, len(prompt))] + [(p, p + 1) for p in range(len(prompt), len(full))]
        outs = []
        for (a, b) in calls:
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
            S.execute(np.array(full[a:b], np.uint32), dq, dk, dv, do, qd, kd)
            T.cuda.synchronize()
            outs.append((a, b, q, [x.cpu().numpy() for x in do]))
        slots = S.radix_slots(len(full))
        for l in range(n_layer):
            allk = np.stack([prefix_rows(full, p, kd, b"k%d" % l) for p in range(len(full))])
            allv = np.stack([prefix_rows(full, p, kd, b"v%d" % l) for p in range(len(full))])
            C = O.CacheQ8(len(full), nkv, hd)
            a0 = outs[0][0]
            if a0:
                assert C.append(allk[:a0], allv[:a0], None, 0, a0) == 0
            for (a, b, q, o) in outs:
                ref = C.attn(q[l], allk[a:b], allv[a:b], None, a, b - a, nh)
                err = np.abs(o[l] - ref).max()
                assert err < TOL, f"prompt {pi} layer {l} rows {a}:{b} err {err}"
            gk, gks, gv, gvs = gather_q8(T, S.layer_q8(l), slots)
            qk, dk_ = O.q8_quantize(allk.reshape(len(full), nkv, hd))
            qv, dv_ = O.q8_quantize(allv.reshape(len(full), nkv, hd))
            assert np.array_equal(gk, qk) and np.array_equal(gks, dk_)
            assert np.array_equal(gv, qv) and np.array_equal(gvs, dv_)
        results.append((matched, resume))
        if between is not None:
            between(S, pi)
    return S, results


def test_session_q8_prefix_reuse_and_eviction(T):
    rng = np.random.default_rng(11)
    shared = [list(rng.integers(0, 1000, size=n)) for n in (20, 33)]
    prompts = [shared[i % 2] + list(rng.integers(0, 1000, size=5 + i)) for i in range(6)]
    prompts.append(list(prompts[-1]))
    S, res = run_session(T, 2, 8, 2, 128, 96, 16, prompts, decode_steps=3)
    matched = [m for m, _ in res]
    assert matched[0] == 0 and matched[2] >= 20 and matched[3] >= 33
    assert res[-1] == (len(prompts[-1]), len(prompts[-1]) - 1)


def test_session_q8_compaction_and_fork(T):
    """Compaction keeps every cached prefix's values and scales bit for bit;
    a prefix forked from a donor session holds the donor's rows."""
    import tlkv
    rng = np.random.default_rng(12)
    n_layer, nh, nkv, hd, ctx, ub = 2, 8, 2, 64, 96, 16
    shared = [list(rng.integers(0, 1000, size=n)) for n in (18, 27)]
    prompts = [shared[i % 2] + list(rng.integers(0, 1000, size=4 + i)) for i in range(5)]
    moved = []

    def live_rows(S):
        L = tlkv._kv_sigs()
        metas = [L.tl_kv_cache_meta(S.radix, s).contents for s in range(ctx)]
        live = [s for s in range(ctx) if metas[s].in_tree]
        paths = {}
        for s in live:
            path, cur = [], s
            while cur != 0xFFFFFFFF:
                path.append(metas[cur].token)
                cur = metas[cur].parent
            paths[s] = tuple(reversed(path))
        rows = {}
        g = [gather_q8(T, S.layer_q8(l), live) for l in range(n_layer)]
        for i, s in enumerate(live):
            rows[paths[s]] = [tuple(x[i].tobytes() for x in gl) for gl in g]
        return rows, live

    def between(S, i):
        before, live0 = live_rows(S)
        ev, mv = S.compact(keep=len(live0) - 6 if i % 2 else 0xFFFFFFFF)
        moved.append(mv)
        after, live1 = live_rows(S)
        assert live1 == list(range(len(live1)))
        for path, rows in after.items():
            assert rows == before[path]

    donor, _ = run_session(T, n_layer, nh, nkv, hd, ctx, ub, prompts, decode_steps=2,
                           between=between)
    assert sum(moved) > 0
    S = tlkv.Session(n_layer, nh, nkv, hd, 128, ub, kv_q8=True)
    forked = []

    def prep(S_, toks):
        m, r, f = S_.kv_prepare_from(donor, toks)
        forked.append(f)
        return m, r

    base = prompts[-1]
    run_session(T, n_layer, nh, nkv, hd, 128, ub, [base + [7, 8, 9]], decode_steps=1, seed=5,
                S=S, prepare=prep)
    assert forked[0] > 0


def test_session_q8_fork_rejects_mixed_cache_types(T):
    import tlkv
    a = tlkv.Session(1, 4, 1, 64, 64, 16, kv_q8=True)
    b = tlkv.Session(1, 4, 1, 64, 64, 16, kv_q8=False)
    toks = np.arange(10, dtype=np.uint32)
    kd = 64
    k = [T.randn((10, kd), device="cuda")]
    b.append(toks, k, k, kd)
    with pytest.raises(tlkv.TlError):
        a.kv_prepare_from(b, toks)
