"""The executor shim (tinyllama.c_amd/integration/hip_graph_op.c) in the
binding a tinyllama.c build uses: the reference's own OpCtx / Graph /
GraphPlan / KvCache structs, built as graph_compute builds them, and a prefix
cache made by libtlkv's kv_cache_create / match / append.

- OP_ATTN through the shim matches op_attn (src/backend/cpu/cpu_op.c:964-1064,
  restated in oracle/oracle.c and pinned there against the compiled
  reference) over the request's slot map read from the same libtlkv cache
  (within 2e-3), over multi-chunk request streams with prefix hits and LRU
  evictions; the shim uploads the slot table itself;
- the batch rows land at the request's slots, f16 RNE, bit for bit, and
  AttnKvCache.n = pos + n (src/backend/cpu/cpu_op.c:995-1009);
- RoPE nodes feeding only OP_ATTN are fused (same bits as running them on
  their own) and the result matches OP_ROPE_* (cpu_op.c:637-700) + OP_ATTN;
- other ops go on to the device backend's gpu_graph_op (a CPU test).
Needs oracle/_ref/libtlshim.so: the product shim and its harness, compiled
against the reference's headers (def.h, kvcache.h) where the reference tree
exists; it holds no reference code and travels with the repository."""
import numpy as np
import pytest

import oracle as O

_built = pytest.mark.skipif(not O.shim_available(), reason="executor shim not built")


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def _host_cache(L, n_kv, cap, hd):
    """the oracle's f16 cache holding a copy of the device cache's bits"""
    C = O.Cache(cap, n_kv, hd)
    C.k[...] = L.k.cpu().numpy().view(np.uint16).reshape(n_kv, cap, hd)
    C.v[...] = L.v.cpu().numpy().view(np.uint16).reshape(n_kv, cap, hd)
    return C


@_built
@pytest.mark.gpu
@pytest.mark.parametrize("nh,nkv,hd,cap,pos,n,win", [
    (32, 8, 128, 2048, 1500, 1, 0),     # decode, contiguous (no radix)
    (8, 4, 256, 1600, 1200, 3, 512),    # windowed multi-row decode
    (28, 4, 128, 1024, 300, 64, 0),     # prefill chunk (MFMA kernel), gqa 7
])
def test_shim_contiguous_matches_reference(T, nh, nkv, hd, cap, pos, n, win):
    import tlkv
    rng = np.random.default_rng(pos + n)
    kd, qd = nkv * hd, nh * hd
    hk = rng.standard_normal((pos, kd)).astype(np.float32)
    hv = rng.standard_normal((pos, kd)).astype(np.float32)
    q = rng.standard_normal((n, qd)).astype(np.float32)
    k = rng.standard_normal((n, kd)).astype(np.float32)
    v = rng.standard_normal((n, kd)).astype(np.float32)
    L = tlkv.Layer(cap, nkv, hd)
    dhk, dhv = T.from_numpy(hk).cuda(), T.from_numpy(hv).cuda()
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dhk), tlkv.ptr(dhv), kd, None, 0, pos,
                                       None))
    dq, dk, dv = T.from_numpy(q).cuda(), T.from_numpy(k).cuda(), T.from_numpy(v).cuda()
    out = T.zeros((n, qd), dtype=T.float32, device="cuda")
    n_after = np.zeros(1, dtype=np.uint32)
    rc = O.shim().rh_attn_shim(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(),
                               L.k.data_ptr(), L.v.data_ptr(), cap, None, pos, n, nh, nkv, hd,
                               win, n_after.ctypes.data)
    T.cuda.synchronize()
    assert rc == 0 and int(n_after[0]) == pos + n
    C = O.Cache(cap, nkv, hd)
    C.append(hk, hv, None, 0, pos)
    ref = O.attn(C, q, k, v, None, pos, n, nh, window=win)
    assert np.abs(out.cpu().numpy() - ref).max() < 2e-3
    got = L.k.cpu().numpy().view(np.uint16)[:, pos:pos + n].transpose(1, 0, 2).reshape(n, -1)
    assert np.array_equal(got, O.f16_bits(k))


@_built
@pytest.mark.gpu
@pytest.mark.parametrize("seed,nh,nkv,hd,ctx,ub,win", [
    (5, 8, 2, 128, 384, 64, 0),     # prefill chunks (MFMA) + decode, evictions
    (6, 12, 4, 64, 256, 37, 96),    # ragged chunks, windowed
])
def test_shim_over_libtlkv_radix_stream(T, seed, nh, nkv, hd, ctx, ub, win):
    import tlkv
    rng = np.random.default_rng(seed)
    kv = tlkv.KvCache(ctx)
    L = tlkv.Layer(ctx, nkv, hd)
    kd, qd = nkv * hd, nh * hd
    prefixes = [rng.integers(0, 50, size=rng.integers(40, ctx // 2)) for _ in range(3)]
    checked = 0
    try:
        for req in range(8):
            toks = np.concatenate([prefixes[rng.integers(3)],
                                   rng.integers(0, 50, size=rng.integers(20, ctx // 3))])
            toks = toks[:ctx - 4].astype(np.uint32)
            m = kv.match(toks)
            pos = 0 if m == 0 else (m if m < len(toks) else m - 1)
            steps = []
            while pos < len(toks):
                steps.append((pos, int(min(ub, len(toks) - pos))))
                pos += steps[-1][1]
            # then three decode steps past the prompt
            full = np.concatenate([toks, rng.integers(0, 50, size=3).astype(np.uint32)])
            steps += [(len(toks) + i, 1) for i in range(3)]
            for p, n in steps:
                assert kv.append(full, p, n)
                q = rng.standard_normal((n, qd)).astype(np.float32)
                k = rng.standard_normal((n, kd)).astype(np.float32)
                v = rng.standard_normal((n, kd)).astype(np.float32)
                C = _host_cache(L, nkv, ctx, hd)     # the cache before this op
                dq, dk, dv = (T.from_numpy(x).cuda() for x in (q, k, v))
                out = T.zeros((n, qd), dtype=T.float32, device="cuda")
                n_after = np.zeros(1, dtype=np.uint32)
                rc = O.shim().rh_attn_shim(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                           out.data_ptr(), L.k.data_ptr(), L.v.data_ptr(),
                                           ctx, kv.h, p, n, nh, nkv, hd, win,
                                           n_after.ctypes.data)
                T.cuda.synchronize()
                assert rc == 0 and int(n_after[0]) == p + n, f"req {req} pos {p}"
                ref = O.attn(C, q, k, v, kv.slots(p + n), p, n, nh, window=win)
                err = np.abs(out.cpu().numpy() - ref).max()
                assert err < 2e-3, f"req {req} pos {p} n {n}: {err}"
                sl = kv.slots(p + n)[p:]
                got = L.k.cpu().numpy().view(np.uint16)[:, sl].transpose(1, 0, 2).reshape(n, -1)
                assert np.array_equal(got, O.f16_bits(k))
                checked += 1
        assert kv.stats()["evictions"] > 0 and kv.stats()["hit_tokens"] > 0
        assert checked > 20
    finally:
        O.shim().rh_shim_release(kv.h)


@_built
@pytest.mark.gpu
@pytest.mark.parametrize("neox,theta,nh,nkv,hd,rdim,pos,n", [
    (0, 5e5, 32, 8, 128, 128, 900, 1),      # Llama NORM decode
    (1, 1e6, 28, 4, 128, 128, 700, 48),     # Qwen NEOX prefill chunk
    (1, 1e4, 8, 4, 256, 256, 1100, 2),      # Gemma local NEOX
    (1, 1e6, 16, 4, 128, 64, 300, 1),       # partial rope_dim
])
def test_shim_rope_fusion(T, neox, theta, nh, nkv, hd, rdim, pos, n):
    import tlkv
    rng = np.random.default_rng(pos + n + neox)
    cap = pos + n + 16
    kd, qd = nkv * hd, nh * hd
    toks = rng.integers(0, 1000, size=pos + n).astype(np.uint32)
    hk = rng.standard_normal((pos, kd)).astype(np.float32)
    hv = rng.standard_normal((pos, kd)).astype(np.float32)
    q = rng.standard_normal((n, qd)).astype(np.float32)
    k = rng.standard_normal((n, kd)).astype(np.float32)
    v = rng.standard_normal((n, kd)).astype(np.float32)
    results = []
    # separate slots; a second reader of the rotated K; the OP_ATTN output on
    # the Q projection's slot; the K rotation on the Q projection's slot (the
    # last two as arena_plan can place them, src/graph.c:671-724)
    for mode in ("separate", "extra", "dst_on_q", "krot_on_q"):
        extra = int(mode == "extra")
        kv = tlkv.KvCache(cap)
        try:
            assert kv.match(toks) == 0
            assert kv.append(toks, 0, pos) and kv.append(toks, pos, n)
            sl = kv.slots(pos + n)
            L = tlkv.Layer(cap, nkv, hd)
            d_sl = T.from_numpy(sl.astype(np.int64)).to(T.int32).cuda()
            dhk, dhv = T.from_numpy(hk).cuda(), T.from_numpy(hv).cuda()
            tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dhk), tlkv.ptr(dhv), kd,
                                               tlkv.ptr(d_sl), 0, pos, None))
            C = _host_cache(L, nkv, cap, hd)
            dq, dk, dv = (T.from_numpy(x).cuda() for x in (q, k, v))
            qr = T.zeros_like(dq)
            kr = dq if mode == "krot_on_q" else T.zeros_like(dk)
            out = dq if mode == "dst_on_q" else T.zeros((n, qd), dtype=T.float32, device="cuda")
            fused = np.zeros(1, dtype=np.uint32)
            rc = O.shim().rh_layer_shim(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                        qr.data_ptr(), kr.data_ptr(), out.data_ptr(),
                                        L.k.data_ptr(), L.v.data_ptr(), cap, kv.h, pos, n, nh,
                                        nkv, hd, 0, neox, theta, rdim, extra,
                                        fused.ctypes.data)
            T.cuda.synchronize()
            assert rc == 0
            # fused only when both RoPE sources outlive the walk up to OP_ATTN
            assert int(fused[0]) == (1 if mode == "separate" else 0), mode
            # OP_ROPE_* on q and k, then OP_ATTN over the same cache
            rq = O.rope(q, nh, hd, rdim, pos, theta, neox)
            rk = O.rope(k, nkv, hd, rdim, pos, theta, neox)
            ref = O.attn(C, rq, rk, v, sl, pos, n, nh)
            o = out.cpu().numpy()
            assert np.abs(o - ref).max() < 2e-3, mode
            rows = L.k.cpu().numpy().view(np.uint16)[:, sl[pos:]]
            results.append((o, rows))
            if extra:   # the rotated K was materialised for its other reader
                assert np.abs(kr.cpu().numpy() - rk).max() < 1e-3
        finally:
            O.shim().rh_shim_release(kv.h)
    # fused and unfused, on any slots: the same bits
    for o, rows in results[1:]:
        assert np.array_equal(results[0][0].view(np.uint32), o.view(np.uint32))
        assert np.array_equal(results[0][1], rows)


@_built
def test_shim_other_ops_fall_through():
    S = O.shim()
    for name in (b"OP_ADD", b"OP_SOFTMAX", b"OP_MATMUL"):
        op = S.rh_op_id(name)
        assert op >= 0
        assert S.rh_fallthrough(op) == op
