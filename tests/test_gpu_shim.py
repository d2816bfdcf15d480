"""The executor shim (tinyllama.c_amd/integration/hip_graph_op.c) in the
binding a tinyllama.c build uses: the reference's own OpCtx / Graph /
GraphPlan / KvCache structs, built as graph_compute builds them, and a prefix
cache made by libtlkv's kv_cache_create / match / append.

- OP_ATTN through the shim matches the compiled reference's
  cpu_graph_op(OP_ATTN) reading the same libtlkv cache through the
  reference's header (within 2e-3), over multi-chunk request streams with
  prefix hits and LRU evictions; the shim uploads the slot table itself;
- the batch rows land at the request's slots, f16 RNE, bit for bit, and
  AttnKvCache.n = pos + n (src/backend/cpu/cpu_op.c:995-1009);
- RoPE nodes feeding only OP_ATTN are fused (same bits as running them on
  their own) and the result matches the reference's OP_ROPE_* + OP_ATTN;
- other ops go on to the device backend's gpu_graph_op (a CPU test).
Needs oracle/_ref (built where the reference tree exists; it travels with the
repository)."""
import numpy as np
import pytest

import oracle as O

_built = pytest.mark.skipif(not (O.shim_available() and O.ref_available()),
                            reason="executor shim / compiled reference not built")


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def _f32_cache(L, n_kv, cap, hd):
    """the device f16 cache as f32 rows (the reference's f32 cache holding them)"""
    kc = O.f16_to_f32(L.k.cpu().numpy().view(np.uint16)).reshape(n_kv, cap, hd)
    vc = O.f16_to_f32(L.v.cpu().numpy().view(np.uint16)).reshape(n_kv, cap, hd)
    return np.ascontiguousarray(kc), np.ascontiguousarray(vc)


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
    kc = np.zeros((nkv, cap, hd), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :pos] = hk.reshape(pos, nkv, hd).transpose(1, 0, 2)
    vc[:, :pos] = hv.reshape(pos, nkv, hd).transpose(1, 0, 2)
    ref = O.ref_attn(kc, vc, q, k, v, None, pos, n, nh, window=win)
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
                kc, vc = _f32_cache(L, nkv, ctx, hd)     # the cache before this op
                dq, dk, dv = (T.from_numpy(x).cuda() for x in (q, k, v))
                out = T.zeros((n, qd), dtype=T.float32, device="cuda")
                n_after = np.zeros(1, dtype=np.uint32)
                rc = O.shim().rh_attn_shim(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                           out.data_ptr(), L.k.data_ptr(), L.v.data_ptr(),
                                           ctx, kv.h, p, n, nh, nkv, hd, win,
                                           n_after.ctypes.data)
                T.cuda.synchronize()
                assert rc == 0 and int(n_after[0]) == p + n, f"req {req} pos {p}"
                ref = O.ref_attn_radix(kv.h, kc, vc, q, k, v, p, n, nh, window=win)
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
    for extra in (0, 1):
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
            kc, vc = _f32_cache(L, nkv, cap, hd)
            dq, dk, dv = (T.from_numpy(x).cuda() for x in (q, k, v))
            qr = T.zeros_like(dq)
            kr = T.zeros_like(dk)
            out = T.zeros((n, qd), dtype=T.float32, device="cuda")
            fused = np.zeros(1, dtype=np.uint32)
            rc = O.shim().rh_layer_shim(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                        qr.data_ptr(), kr.data_ptr(), out.data_ptr(),
                                        L.k.data_ptr(), L.v.data_ptr(), cap, kv.h, pos, n, nh,
                                        nkv, hd, 0, neox, theta, rdim, extra,
                                        fused.ctypes.data)
            T.cuda.synchronize()
            assert rc == 0
            assert int(fused[0]) == (0 if extra else 1)
            # the reference: OP_ROPE_* on q and k, then OP_ATTN over the same cache
            rq = O.ref_rope(q, nh, hd, rdim, pos, theta, neox)
            rk = O.ref_rope(k, nkv, hd, rdim, pos, theta, neox)
            ref = O.ref_attn_radix(kv.h, kc, vc, rq, rk, v, pos, n, nh)
            o = out.cpu().numpy()
            assert np.abs(o - ref).max() < 2e-3
            rows = L.k.cpu().numpy().view(np.uint16)[:, sl[pos:]]
            results.append((o, rows))
            if extra:   # the rotated K was materialised for its other reader
                assert np.abs(kr.cpu().numpy() - rk).max() < 1e-3
        finally:
            O.shim().rh_shim_release(kv.h)
    # fused and unfused: the same bits
    assert np.array_equal(results[0][0].view(np.uint32), results[1][0].view(np.uint32))
    assert np.array_equal(results[0][1], results[1][1])


@_built
def test_shim_other_ops_fall_through():
    S = O.shim()
    for name in (b"OP_ADD", b"OP_SOFTMAX", b"OP_MATMUL"):
        op = S.rh_op_id(name)
        assert op >= 0
        assert S.rh_fallthrough(op) == op
