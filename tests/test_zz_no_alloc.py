"""tl_attn_noalloc (the entry point that allocates nothing: split partials and
merge counters in the library's fixed per-GPU region) against tl_attn on the
same inputs, through the C ABI: calls in a row, each followed by a smaller
one, so the second reads a region the first left behind.  Decode outputs are
bit-identical (same kernels, same split count); prefill batches may take
fewer key splits to fit the region, so they agree within 1e-4 and both stay
within 2e-3 of the oracle.  The appended cache rows are identical.  Also:
overlapping calls the library can see are refused with TL_EBUSY; the call
captured in a HIP graph replays bit-identically to the eager call; a first
call under capture before tl_init is refused with TL_EINVAL."""
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


def _pair(T, n_head, n_kv, hd, cap, pos, n, window, seed):
    """Two layers with the same history; OP_ATTN of the same batch through
    tl_attn and tl_attn_noalloc.  Returns (out_attn, out_noalloc, oracle,
    layers)."""
    import tlkv
    rng = np.random.default_rng(seed)
    kd = n_kv * hd
    hk = rng.standard_normal((pos, kd)).astype(np.float32)
    hv = rng.standard_normal((pos, kd)).astype(np.float32)
    q = rng.standard_normal((n, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((n, kd)).astype(np.float32)
    v = rng.standard_normal((n, kd)).astype(np.float32)
    slots = rng.permutation(cap).astype(np.uint32)
    ds = T.from_numpy(slots).cuda()
    dhk, dhv = T.from_numpy(hk).cuda(), T.from_numpy(hv).cuda()
    dq, dk, dv = (T.from_numpy(x).cuda() for x in (q, k, v))
    outs, layers = [], []
    for fn in ("tl_attn", "tl_attn_noalloc"):
        L = tlkv.Layer(cap, n_kv, hd)
        if pos:
            tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dhk), tlkv.ptr(dhv), kd,
                                               tlkv.ptr(ds), 0, pos, None))
        out = T.full((n, n_head * hd), float("nan"), dtype=T.float32, device="cuda")
        a = tlkv.attn_args(dq, dk, dv, out, ds, pos, n, n_head, hd, n_kv, window,
                           O.scale_of(hd))
        tlkv.check(getattr(tlkv.lib(), fn)(L.desc, a, None))
        T.cuda.synchronize()
        outs.append(out.cpu().numpy())
        layers.append(L)
    C = O.Cache(cap, n_kv, hd)
    C.append(hk, hv, slots, 0, pos)
    ref = O.attn(C, q, k, v, slots, pos, n, n_head, window=window)
    return outs[0], outs[1], ref, layers


@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_noalloc_equals_attn_twice(T, kind):
    if kind == "decode":
        # config 4's last step, then a smaller windowed multi-row decode
        calls = [(32, 8, 128, 33800, 33791, 1, 0), (16, 2, 128, 4096, 3000, 5, 700)]
    else:
        # a config-4 chunk at depth, then a smaller gqa-7 chunk
        calls = [(32, 8, 128, 8800, 8192, 512, 0), (28, 4, 128, 1200, 300, 100, 0)]
    for i, (nh, nkv, hd, cap, pos, n, win) in enumerate(calls):
        base, noalloc, ref, layers = _pair(T, nh, nkv, hd, cap, pos, n, win, seed=100 + i)
        assert np.isfinite(noalloc).all()
        if kind == "decode":
            assert np.array_equal(base.view(np.uint32), noalloc.view(np.uint32)), f"call {i}"
        else:
            assert np.abs(base - noalloc).max() < 1e-4, f"call {i}"
        assert np.abs(noalloc - ref).max() < TOL, f"call {i}"
        k0 = layers[0].k.cpu().numpy().view(np.uint16)
        k1 = layers[1].k.cpu().numpy().view(np.uint16)
        assert np.array_equal(k0, k1), f"call {i}: appended rows differ"


def test_noalloc_refuses_overlap_on_another_stream(T):
    """A call on another stream while the previous call's work is still
    queued fails with TL_EBUSY instead of racing on the shared region; once
    that work has finished the same call runs, and both calls match tl_attn
    bit for bit (each appends the same row, then attends over the cache)."""
    import tlkv
    n_head, n_kv, hd, cap, pos = 32, 8, 128, 4200, 4095
    rng = np.random.default_rng(77)
    kd = n_kv * hd
    L = tlkv.Layer(cap, n_kv, hd)
    hk = T.from_numpy(rng.standard_normal((pos, kd)).astype(np.float32)).cuda()
    hv = T.from_numpy(rng.standard_normal((pos, kd)).astype(np.float32)).cuda()
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(hk), tlkv.ptr(hv), kd, None, 0, pos,
                                       None))
    q, k, v = (T.from_numpy(rng.standard_normal((1, w)).astype(np.float32)).cuda()
               for w in (n_head * hd, kd, kd))
    outs = [T.zeros((1, n_head * hd), dtype=T.float32, device="cuda") for _ in range(3)]
    args = [tlkv.attn_args(q, k, v, o, None, pos, 1, n_head, hd, n_kv, 0, O.scale_of(hd))
            for o in outs]
    s1, s2 = T.cuda.Stream(), T.cuda.Stream()
    T.cuda.synchronize()
    lib = tlkv.lib()
    big = T.randn((8192, 8192), device="cuda")
    T.cuda.synchronize()
    with T.cuda.stream(s1):                 # ~0.2 s of queued work on s1
        for _ in range(20):
            big = T.mm(big, big).clamp_(-1, 1)
    assert lib.tl_attn_noalloc(L.desc, args[0], s1.cuda_stream) == tlkv.TL_OK
    assert lib.tl_attn_noalloc(L.desc, args[1], s2.cuda_stream) == tlkv.TL_EBUSY
    s1.synchronize()
    assert lib.tl_attn_noalloc(L.desc, args[1], s2.cuda_stream) == tlkv.TL_OK
    tlkv.check(lib.tl_attn(L.desc, args[2], s2.cuda_stream))
    s2.synchronize()
    a, b, c = (o.cpu().numpy().view(np.uint32) for o in outs)
    assert np.array_equal(a, c) and np.array_equal(b, c)


def test_noalloc_graph_replay(T):
    """The use case: tl_attn_noalloc captured in a HIP graph (after tl_init)
    and replayed, with new q written eagerly between replays; every replay
    equals the eager no-allocation call on the same inputs bit for bit and
    the oracle within tolerance."""
    import tlkv
    n_head, n_kv, hd, cap, pos = 32, 8, 128, 8400, 8191
    rng = np.random.default_rng(2025)
    kd, qd = n_kv * hd, n_head * hd
    hk = rng.standard_normal((pos + 1, kd)).astype(np.float32)
    hv = rng.standard_normal((pos + 1, kd)).astype(np.float32)
    L = tlkv.Layer(cap, n_kv, hd)
    dhk, dhv = T.from_numpy(hk[:pos]).cuda(), T.from_numpy(hv[:pos]).cuda()
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dhk), tlkv.ptr(dhv), kd, None, 0, pos,
                                       None))
    T.cuda.synchronize()
    C = O.Cache(cap, n_kv, hd)
    C.append(hk[:pos], hv[:pos], None, 0, pos)
    dq = T.zeros((1, qd), dtype=T.float32, device="cuda")
    dk = T.from_numpy(hk[pos:]).cuda()
    dv = T.from_numpy(hv[pos:]).cuda()
    out = T.zeros((1, qd), dtype=T.float32, device="cuda")
    a = tlkv.attn_args(dq, dk, dv, out, None, pos, 1, n_head, hd, n_kv, 0, O.scale_of(hd))
    lib = tlkv.lib()
    s = T.cuda.Stream()
    T.cuda.synchronize()
    g = T.cuda.CUDAGraph()
    with T.cuda.graph(g, stream=s):
        tlkv.check(lib.tl_attn_noalloc(L.desc, a, s.cuda_stream))
    for i in range(4):
        q = rng.standard_normal((1, qd)).astype(np.float32)
        dq.copy_(T.from_numpy(q))
        T.cuda.synchronize()
        g.replay()
        T.cuda.synchronize()
        got = out.cpu().numpy().copy()
        out.zero_()
        tlkv.check(lib.tl_attn_noalloc(L.desc, a, s.cuda_stream))
        s.synchronize()
        assert np.array_equal(got.view(np.uint32), out.cpu().numpy().view(np.uint32)), i
        ref = O.attn(C, q, hk[pos:], hv[pos:], None, pos, 1, n_head)
        assert np.abs(got - ref).max() < TOL, i


def test_noalloc_capture_before_init_is_refused():
    """In a process that has not called tl_init, a first tl_attn_noalloc under
    graph capture fails with TL_EINVAL (its one-time set-up would synchronise
    the device) instead of breaking the capture.  Run in a child process: this
    one has set the region up already."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    pkg = os.path.join(os.path.dirname(here), "tinyllama.c_amd")
    code = f"""
import sys
sys.path.insert(0, {pkg!r})
import torch, tlkv
L = tlkv.Layer(1024, 8, 128)
q = torch.zeros((1, 4096), device="cuda"); k = torch.zeros((1, 1024), device="cuda")
out = torch.zeros((1, 4096), device="cuda")
a = tlkv.attn_args(q, k, k, out, None, 100, 1, 32, 128, 8, 0, 0.088)
s = torch.cuda.Stream(); torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc = tlkv.lib().tl_attn_noalloc(L.desc, a, s.cuda_stream)
print("rc", rc, flush=True)
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "rc -1" in r.stdout, r.stdout + r.stderr[-2000:]
