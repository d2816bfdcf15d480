"""OP_ATTN on prefill batches with the append fused into the prefill launch:
the launch's workgroups write the batch rows (f32 -> f16 RNE, K rotated when
RoPE is fused) into the cache before any of them reads it, each publishing
its 16-row units with a flag; a workgroup whose keys reach the batch rows
waits (bounded) for the flags and reads those rows back device-coherently,
and writes a unit itself when its flag does not come.

Checked against the separate append launch (the previous path) on twin
layers: the cache contents and the outputs are the same bits, with the
bounded wait as usual and with no wait at all (every workgroup writes every
unit it reads itself: the fallback), and the outputs are within 2e-3 of the
oracle (src/backend/cpu/cpu_op.c:995-1062).  Shapes: config 4's chunk at
depth with a permuted slot table and several key splits, config 4's first
chunk (every key is a batch row), gqa 7, head_dim 64 and 256, a window on a
ring, a ragged batch, and the fused-RoPE entry point."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-3
_KEEP = []


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def dev(T, a):
    t = T.from_numpy(np.ascontiguousarray(a)).cuda()
    _KEEP.append(t)
    return t


CASES = [
    # n_head, n_kv, hd, cap, pos, n, window, ring, permuted slots, rope
    (32, 8, 128, 8800, 8192, 512, 0, 0, True, None),      # config 4 chunk at depth
    (32, 8, 128, 600, 0, 512, 0, 0, False, None),         # config 4 first chunk
    (28, 4, 128, 2048, 1000, 300, 0, 0, True, None),      # gqa 7, ragged batch
    (32, 8, 64, 1100, 512, 256, 0, 0, False, None),       # config 1 shape
    (8, 4, 256, 1600, 1200, 100, 256, 256 + 100 - 1, False, None),  # window on a ring
    (32, 8, 128, 4200, 3000, 200, 0, 0, True, (0, 5e5)),  # fused RoPE NORM
    (28, 4, 128, 1500, 700, 77, 0, 0, False, (1, 1e6)),   # fused RoPE NEOX, ragged
]


def _run(T, case, mode):
    """mode: 'separate' (own append launch), 'fused', 'fallback' (no wait)."""
    import tlkv
    nh, nkv, hd, cap, pos, n, win, ring, perm, rope = case
    rng = np.random.default_rng(pos + n + hd)
    kd, qd = nkv * hd, nh * hd
    hk = rng.standard_normal((pos, kd)).astype(np.float32)
    hv = rng.standard_normal((pos, kd)).astype(np.float32)
    q = rng.standard_normal((n, qd)).astype(np.float32)
    k = rng.standard_normal((n, kd)).astype(np.float32)
    v = rng.standard_normal((n, kd)).astype(np.float32)
    slots = rng.permutation(cap).astype(np.uint32) if perm else None
    L = tlkv.Layer(cap, nkv, hd, ring=ring)
    ds = None if slots is None else dev(T, slots)
    lib = tlkv.lib()
    if pos:
        lo = max(0, pos - ring) if ring else 0
        tlkv.check(lib.tl_kv_append(L.desc, tlkv.ptr(dev(T, hk[lo:])), tlkv.ptr(dev(T, hv[lo:])),
                                    kd, tlkv.ptr(ds), lo, pos - lo, None))
    out = T.zeros((n, qd), dtype=T.float32, device="cuda")
    a = tlkv.attn_args(dev(T, q), dev(T, k), dev(T, v), out, ds, pos, n, nh, hd, nkv, win,
                       O.scale_of(hd))
    sep = tlkv.tuning(tlkv.TUNE_PREFILL_SEPARATE_APPEND, 1 if mode == "separate" else 0)
    polls = tlkv.tuning(tlkv.TUNE_PREFILL_APPEND_POLLS, 1 if mode == "fallback" else 0)
    with sep, polls:
        if rope is None:
            tlkv.check(lib.tl_attn(L.desc, a, None))
        else:
            rp = tlkv.RopeParams(hd, rope[1], rope[0])
            tlkv.check(lib.tl_attn_rope(L.desc, a, rp, None))
    T.cuda.synchronize()
    _KEEP.clear()
    res = dict(out=out.cpu().numpy(), k=L.k.cpu().numpy().view(np.uint16),
               v=L.v.cpu().numpy().view(np.uint16))
    # the oracle: RoPE'd q/k (when fused), then op_attn over the f16 cache
    C = O.Cache(ring or cap, nkv, hd)
    if pos:
        lo = max(0, pos - ring) if ring else 0
        if ring:
            for p in range(lo, pos):
                C.append(hk[p:p + 1], hv[p:p + 1], None, p % ring, 1)
        else:
            C.append(hk, hv, slots, 0, pos)
    qq, kk = q, k
    if rope is not None:
        qq = O.rope(q, nh, hd, hd, pos, rope[1], rope[0])
        kk = O.rope(k, nkv, hd, hd, pos, rope[1], rope[0])
    res["ref"] = O.attn(C, qq, kk, v, slots, pos, n, nh, window=win, ring=ring)
    return res


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"h{c[0]}-kv{c[1]}-d{c[2]}-p{c[4]}-n{c[5]}")
def test_fused_append_equals_separate(T, case):
    base = _run(T, case, "separate")
    assert np.abs(base["out"] - base["ref"]).max() < TOL
    for mode in ("fused", "fallback"):
        got = _run(T, case, mode)
        assert np.array_equal(got["k"], base["k"]), f"{mode}: K cache differs"
        assert np.array_equal(got["v"], base["v"]), f"{mode}: V cache differs"
        assert np.array_equal(got["out"].view(np.uint32), base["out"].view(np.uint32)), mode
        assert np.abs(got["out"] - got["ref"]).max() < TOL, mode
