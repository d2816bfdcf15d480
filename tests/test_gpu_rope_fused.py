"""Fused RoPE entry points (tl_attn_rope, tl_kv_append_rope,
tl_attn_decode_batch_rope) against the unfused sequence they replace: the
reference runs OP_ROPE_NORM / OP_ROPE_NEOX on Q and K
(src/backend/cpu/cpu_op.c:637-700) and then OP_ATTN (cpu_op.c:964-1064); here
that sequence is tl_rope on q, tl_rope on k, then tl_attn / tl_kv_append.

The fused kernels apply the same rotation (shared device code, explicit fma),
so cache contents must match bit for bit and attention outputs exactly; the
unfused tl_rope itself is pinned against the oracle in test_gpu_kv.py.  The
fused path must also leave the caller's q and k unmodified.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def _gather(T, tlkv, L, slots, n):
    ko = T.zeros((n, L.desc.n_kv_head, L.desc.head_dim), dtype=T.float16, device="cuda")
    vo = T.zeros_like(ko)
    tlkv.check(tlkv.lib().tl_kv_gather(L.desc, tlkv.ptr(slots), n, tlkv.ptr(ko),
                                       tlkv.ptr(vo), None))
    T.cuda.synchronize()
    return ko.cpu().numpy().view(np.uint16), vo.cpu().numpy().view(np.uint16)


CASES = [
    # n_head, n_kv, hd, pos, n, rope_dim, neox, theta
    (32, 8, 128, 700, 1, 128, 0, 5e5),       # decode, NORM (configs 1, 4)
    (28, 4, 128, 900, 1, 128, 1, 1e6),       # decode, NEOX, gqa 7 (configs 2, 3)
    (8, 4, 256, 1500, 1, 256, 1, 1e4),       # decode, head_dim 256 (config 5)
    (16, 2, 128, 300, 5, 64, 1, 1e4),        # multi-row decode, partial rope_dim
    (32, 8, 128, 2000, 6, 128, 0, 5e5),      # multi-row decode, 4 rows per group, ragged
    (32, 8, 128, 1000, 100, 128, 0, 5e5),    # prefill batch (append + MFMA kernel)
    (8, 4, 64, 200, 40, 32, 0, 1e4),         # prefill, head_dim 64, partial NORM
    (32, 8, 64, 700, 1, 64, 0, 5e5),         # decode, head_dim 64 (config 1 shape)
    (8, 4, 256, 600, 64, 256, 1, 1e6),       # prefill, head_dim 256, NEOX (config 5 global)
]


@pytest.mark.parametrize("case", CASES)
def test_attn_rope_equals_rope_then_attn(T, case):
    _rope_case(T, case)


@pytest.mark.parametrize("case", [c for c in CASES if c[4] >= 16])
def test_attn_rope_prefill_kernel_forced(T, case):
    """The batches of 16+ rows on the prefill kernel, also where the plan
    takes the decode kernel (small rows x keys)."""
    import tlkv
    with tlkv.tuning(tlkv.TUNE_NO_PREFILL, 2):
        _rope_case(T, case)


def _rope_case(T, case):
    import tlkv
    n_head, n_kv, hd, pos, n, rdim, neox, theta = case
    lib = tlkv.lib()
    rng = np.random.default_rng(pos + n)
    cap = pos + n + 8
    kd, qd = n_kv * hd, n_head * hd
    slots = T.from_numpy(rng.permutation(cap).astype(np.uint32)).cuda()
    hist_k = T.from_numpy(rng.standard_normal((pos, kd)).astype(np.float32)).cuda()
    hist_v = T.from_numpy(rng.standard_normal((pos, kd)).astype(np.float32)).cuda()
    q0 = T.from_numpy(rng.standard_normal((n, qd)).astype(np.float32)).cuda()
    k0 = T.from_numpy(rng.standard_normal((n, kd)).astype(np.float32)).cuda()
    v0 = T.from_numpy(rng.standard_normal((n, kd)).astype(np.float32)).cuda()
    layers = [tlkv.Layer(cap, n_kv, hd) for _ in range(2)]
    for L in layers:
        tlkv.check(lib.tl_kv_append(L.desc, tlkv.ptr(hist_k), tlkv.ptr(hist_v), kd,
                                    tlkv.ptr(slots), 0, pos, None))
    scale = O.scale_of(hd)
    # unfused: rope q, rope k (in place on copies), then OP_ATTN
    q1, k1 = q0.clone(), k0.clone()
    tlkv.check(lib.tl_rope(tlkv.ptr(q1), n, qd, n_head, hd, rdim, pos, theta, neox, None))
    tlkv.check(lib.tl_rope(tlkv.ptr(k1), n, kd, n_kv, hd, rdim, pos, theta, neox, None))
    out1 = T.zeros((n, qd), dtype=T.float32, device="cuda")
    a1 = tlkv.attn_args(q1, k1, v0, out1, slots, pos, n, n_head, hd, n_kv, 0, scale)
    tlkv.check(lib.tl_attn(layers[0].desc, a1, None))
    # fused
    qs, ks = q0.clone(), k0.clone()
    out2 = T.zeros((n, qd), dtype=T.float32, device="cuda")
    a2 = tlkv.attn_args(q0, k0, v0, out2, slots, pos, n, n_head, hd, n_kv, 0, scale)
    rp = tlkv.RopeParams(rdim, theta, neox)
    tlkv.check(lib.tl_attn_rope(layers[1].desc, a2, rp, None))
    T.cuda.synchronize()
    assert T.equal(q0, qs) and T.equal(k0, ks), "fused path modified its inputs"
    assert np.array_equal(out1.cpu().numpy(), out2.cpu().numpy())
    g1 = _gather(T, tlkv, layers[0], slots, pos + n)
    g2 = _gather(T, tlkv, layers[1], slots, pos + n)
    assert np.array_equal(g1[0], g2[0]) and np.array_equal(g1[1], g2[1])
    # and the rotated rows are the oracle's RoPE of the inputs, within the
    # tolerance that pins tl_rope
    kr = O.rope(k0.cpu().numpy(), n_kv, hd, rdim, pos, theta, neox)
    got = O.f16_to_f32(g2[0][pos:pos + n].reshape(n, kd))
    assert np.abs(got - kr).max() < 2e-3 + np.abs(kr).max() * 1e-3


@pytest.mark.parametrize("neox", [0, 1])
def test_kv_append_rope_equals_rope_then_append(T, neox):
    import tlkv
    lib = tlkv.lib()
    rng = np.random.default_rng(40 + neox)
    n_kv, hd, cap, pos, n = 4, 128, 2048, 777, 600
    kd = n_kv * hd
    slots = T.from_numpy(rng.permutation(cap).astype(np.uint32)).cuda()
    k0 = T.from_numpy(rng.standard_normal((n, kd)).astype(np.float32)).cuda()
    v0 = T.from_numpy(rng.standard_normal((n, kd)).astype(np.float32)).cuda()
    L1, L2 = tlkv.Layer(cap, n_kv, hd), tlkv.Layer(cap, n_kv, hd)
    k1 = k0.clone()
    tlkv.check(lib.tl_rope(tlkv.ptr(k1), n, kd, n_kv, hd, hd, pos, 1e6, neox, None))
    tlkv.check(lib.tl_kv_append(L1.desc, tlkv.ptr(k1), tlkv.ptr(v0), kd, tlkv.ptr(slots),
                                pos, n, None))
    rp = tlkv.RopeParams(hd, 1e6, neox)
    tlkv.check(lib.tl_kv_append_rope(L2.desc, tlkv.ptr(k0), tlkv.ptr(v0), kd, tlkv.ptr(slots),
                                     pos, n, rp, None))
    T.cuda.synchronize()
    assert T.equal(L1.k, L2.k) and T.equal(L1.v, L2.v)


def test_decode_batch_rope_equals_unfused(T):
    import tlkv
    lib = tlkv.lib()
    n_head, n_kv, hd, n_seq = 28, 4, 128, 6
    rng = np.random.default_rng(41)
    keep, fused, plain, outs = [], [], [], []
    for s in range(n_seq):
        cap, pos = 600 + 32 * s, 250 + 31 * s
        kd, qd = n_kv * hd, n_head * hd
        slots = T.from_numpy(rng.permutation(cap).astype(np.uint32)).cuda()
        hk = T.from_numpy(rng.standard_normal((pos, kd)).astype(np.float32)).cuda()
        hv = T.from_numpy(rng.standard_normal((pos, kd)).astype(np.float32)).cuda()
        q = T.from_numpy(rng.standard_normal((1, qd)).astype(np.float32)).cuda()
        k = T.from_numpy(rng.standard_normal((1, kd)).astype(np.float32)).cuda()
        v = T.from_numpy(rng.standard_normal((1, kd)).astype(np.float32)).cuda()
        qr, kr = q.clone(), k.clone()
        tlkv.check(lib.tl_rope(tlkv.ptr(qr), 1, qd, n_head, hd, hd, pos, 1e6, 1, None))
        tlkv.check(lib.tl_rope(tlkv.ptr(kr), 1, kd, n_kv, hd, hd, pos, 1e6, 1, None))
        La, Lb = tlkv.Layer(cap, n_kv, hd), tlkv.Layer(cap, n_kv, hd)
        for L in (La, Lb):
            tlkv.check(lib.tl_kv_append(L.desc, tlkv.ptr(hk), tlkv.ptr(hv), kd, tlkv.ptr(slots),
                                        0, pos, None))
        oa = T.zeros((1, qd), dtype=T.float32, device="cuda")
        ob = T.zeros_like(oa)
        keep += [slots, hk, hv, q, k, v, qr, kr, La, Lb, oa, ob]
        plain.append(tlkv.DecodeSeq(La.desc, slots.data_ptr(), pos, 0, qr.data_ptr(),
                                    kr.data_ptr(), v.data_ptr(), oa.data_ptr()))
        fused.append(tlkv.DecodeSeq(Lb.desc, slots.data_ptr(), pos, 0, q.data_ptr(),
                                    k.data_ptr(), v.data_ptr(), ob.data_ptr()))
        outs.append((oa, ob, La, Lb))
    scale = O.scale_of(hd)
    tlkv.check(lib.tl_attn_decode_batch((tlkv.DecodeSeq * n_seq)(*plain), n_seq, n_head, 0,
                                        scale, None))
    tlkv.check(lib.tl_attn_decode_batch_rope((tlkv.DecodeSeq * n_seq)(*fused), n_seq, n_head, 0,
                                             scale, tlkv.RopeParams(hd, 1e6, 1), None))
    T.cuda.synchronize()
    for oa, ob, La, Lb in outs:
        assert T.equal(oa, ob)
        assert T.equal(La.k, Lb.k) and T.equal(La.v, Lb.v)


def test_rope_params_rejected(T):
    import tlkv
    lib = tlkv.lib()
    L = tlkv.Layer(64, 2, 128)
    q = T.zeros((1, 8 * 128), device="cuda")
    k = T.zeros((1, 2 * 128), device="cuda")
    out = T.zeros_like(q)
    a = tlkv.attn_args(q, k, k, out, None, 3, 1, 8, 128, 2, 0)
    for bad in (tlkv.RopeParams(130, 1e4, 0), tlkv.RopeParams(63, 1e4, 0),
                tlkv.RopeParams(128, 0.0, 0)):
        assert lib.tl_attn_rope(L.desc, a, bad, None) == -1
