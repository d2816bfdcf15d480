"""GPU parity of the Q8_0 cache against the CPU oracle (through the C ABI).

Append / gather: bit-exact against oracle.c's Q8_0 quantizer (the
reference's quantizer, gpu.cu:1077-1086, with the scale kept as binary16).
Attention: within 2e-3 max-abs of the oracle's op_attn over the dequantized
cache (quants.c:368-373), for the decode kernel (1..15 rows) and the MFMA
prefill kernel (16+ rows), with slot tables, windows and rings.
"""
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


_KEEP = []


def dev(T, a):
    """Device copy kept alive until the next sync (kernels run asynchronously)."""
    t = T.from_numpy(np.ascontiguousarray(a)).cuda()
    _KEEP.append(t)
    return t


def host(t):
    return t.cpu().numpy()


def sync(T):
    T.cuda.synchronize()
    _KEEP.clear()


def rows(rng, n, width, scale_spread=False):
    x = rng.standard_normal((n, width)).astype(np.float32)
    if scale_spread and n:
        # blocks of very different magnitudes, zero blocks, exact ties
        x *= rng.choice([1e-3, 0.1, 1.0, 30.0], size=(n, width // 32, 1)).repeat(32, 2).reshape(n, width)
        x[0, :32] = 0.0
        x[0, 32:64] = np.arange(32, dtype=np.float32) - 15.5
        x[0, 64] = 127.0
    return x


def _q8(L):
    return host(L.k), host(L.ks).view(np.uint16), host(L.v), host(L.vs).view(np.uint16)


@pytest.mark.parametrize("n_kv,hd,cap,n,pos,perm,ring", [
    (8, 128, 64, 17, 5, True, 0),
    (8, 64, 40, 33, 0, False, 0),
    (4, 256, 32, 9, 3, True, 0),
    (4, 128, 600, 512, 7, True, 0),
    (2, 128, 50, 40, 30, False, 50),     # wraps the ring once (no slot written twice)
])
def test_append_q8_bitexact(T, n_kv, hd, cap, n, pos, perm, ring):
    import tlkv
    rng = np.random.default_rng(n * 31 + hd)
    k = rows(rng, n, n_kv * hd, scale_spread=True)
    v = rows(rng, n, n_kv * hd, scale_spread=True)
    slots = (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    L = tlkv.LayerQ8(cap, n_kv, hd, ring=ring)
    ds = None if ring else dev(T, slots)
    tlkv.check(tlkv.lib().tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, k)), tlkv.ptr(dev(T, v)),
                                          n_kv * hd, tlkv.ptr(ds), pos, n, None))
    sync(T)
    C = O.CacheQ8(cap, n_kv, hd, ring)
    if ring:
        for i in range(n):   # rows in order: later rows overwrite earlier ones
            assert C.append(k[i:i + 1], v[i:i + 1], None, pos + i, 1) == 0
    else:
        assert C.append(k, v, slots, pos, n) == 0
    gk, gks, gv, gvs = _q8(L)
    assert np.array_equal(gk, C.k)
    assert np.array_equal(gks, C.ks)
    assert np.array_equal(gv, C.v)
    assert np.array_equal(gvs, C.vs)


def test_append_q8_out_of_range_slot_skipped(T):
    import tlkv
    rng = np.random.default_rng(5)
    n_kv, hd, cap = 2, 64, 16
    k = rows(rng, 4, n_kv * hd)
    slots = np.array([3, 99, 7, 15], dtype=np.uint32)
    L = tlkv.LayerQ8(cap, n_kv, hd)
    tlkv.check(tlkv.lib().tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, k)), tlkv.ptr(dev(T, k)),
                                          n_kv * hd, tlkv.ptr(dev(T, slots)), 0, 4, None))
    sync(T)
    gk = host(L.k)
    q, d = O.q8_quantize(k.reshape(4, n_kv, hd))
    for i, s in enumerate(slots):
        if s < cap:
            assert np.array_equal(gk[:, s], q[i])
    untouched = [s for s in range(cap) if s not in (3, 7, 15)]
    assert not gk[:, untouched].any()


def test_gather_q8_roundtrip(T):
    import tlkv
    rng = np.random.default_rng(11)
    n_kv, hd, cap = 4, 128, 100
    k = rows(rng, cap, n_kv * hd, scale_spread=True)
    v = rows(rng, cap, n_kv * hd, scale_spread=True)
    L = tlkv.LayerQ8(cap, n_kv, hd)
    tlkv.check(tlkv.lib().tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, k)), tlkv.ptr(dev(T, v)),
                                          n_kv * hd, None, 0, cap, None))
    sel = np.concatenate([rng.permutation(cap)[:37], [cap + 5]]).astype(np.uint32)
    n = sel.size
    ko = T.zeros((n, n_kv, hd), dtype=T.int8, device="cuda")
    vo = T.zeros_like(ko)
    kso = T.zeros((n, n_kv, hd // 32), dtype=T.int16, device="cuda")
    vso = T.zeros_like(kso)
    tlkv.check(tlkv.lib().tl_kv_gather_q8(L.desc, tlkv.ptr(dev(T, sel)), n, tlkv.ptr(ko),
                                          tlkv.ptr(kso), tlkv.ptr(vo), tlkv.ptr(vso), None))
    sync(T)
    qk, dk = O.q8_quantize(k.reshape(cap, n_kv, hd))
    qv, dv = O.q8_quantize(v.reshape(cap, n_kv, hd))
    assert np.array_equal(host(ko)[:-1], qk[sel[:-1]])
    assert np.array_equal(host(kso).view(np.uint16)[:-1], dk[sel[:-1]])
    assert np.array_equal(host(vo)[:-1], qv[sel[:-1]])
    assert np.array_equal(host(vso).view(np.uint16)[:-1], dv[sel[:-1]])
    assert not host(ko)[-1].any() and not host(kso)[-1].any()   # slot outside the cache


def _run_attn_q8(T, n_head, n_kv, hd, cap, pos, n, window, slots, seed, ring=0,
                 append=True):
    """Fill positions [0,pos) then run OP_ATTN over the Q8_0 cache on rows
    [pos,pos+n) on the device and in the oracle.  Returns (device, oracle)."""
    import tlkv
    rng = np.random.default_rng(seed)
    kd = n_kv * hd
    total = pos + n
    hk, hv = rows(rng, total, kd), rows(rng, total, kd)
    q = rows(rng, n, n_head * hd)
    L = tlkv.LayerQ8(cap, n_kv, hd, ring=ring)
    C = O.CacheQ8(cap, n_kv, hd, ring)
    ds = None if slots is None else dev(T, slots)
    fill = total if not append else pos
    lo = max(0, fill - ring) if ring else 0
    if fill > lo:
        tlkv.check(tlkv.lib().tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, hk[lo:fill])),
                                              tlkv.ptr(dev(T, hv[lo:fill])), kd, tlkv.ptr(ds),
                                              lo, fill - lo, None))
        assert C.append(hk[lo:fill], hv[lo:fill], slots, lo, fill - lo) == 0
    out = T.zeros((n, n_head * hd), dtype=T.float32, device="cuda")
    dk, dv = (dev(T, hk[pos:]), dev(T, hv[pos:])) if append else (None, None)
    a = tlkv.attn_args(dev(T, q), dk, dv, out, ds, pos, n, n_head, hd, n_kv, window,
                       O.scale_of(hd))
    fn = tlkv.lib().tl_attn_q8 if append else tlkv.lib().tl_attn_noappend_q8
    tlkv.check(fn(L.desc, a, None))
    sync(T)
    ref = C.attn(q, hk[pos:] if append else None, hv[pos:] if append else None, slots, pos, n,
                 n_head, window=window)
    return host(out), ref, L, C


Q8_CASES = [
    # n_head, n_kv, hd, cap, pos, n, window, permuted slots, ring
    (32, 8, 64, 1024, 700, 1, 0, True, 0),       # config 1 shape
    (28, 4, 128, 2048, 1500, 1, 0, True, 0),     # gqa 7
    (32, 8, 128, 4096, 4000, 1, 0, False, 0),    # config 4 shape
    (8, 4, 256, 2048, 1800, 1, 1024, True, 0),   # windowed, head_dim 256
    (8, 4, 256, 1535, 3000, 1, 1024, False, 1535),   # ring
    (32, 8, 128, 512, 0, 1, 0, False, 0),        # first token
    (32, 8, 128, 512, 3, 1, 0, True, 0),         # tiny history
    (16, 2, 128, 600, 200, 5, 0, True, 0),       # multi-row decode
    (16, 2, 128, 600, 200, 15, 64, True, 0),     # multi-row + window
    (8, 8, 64, 300, 100, 3, 0, False, 0),        # MHA
    (24, 8, 128, 700, 500, 1, 0, True, 0),       # gqa 3
    (40, 5, 128, 700, 500, 2, 0, True, 0),       # gqa 8
    (16, 2, 128, 1200, 300, 200, 0, True, 0),    # prefill (MFMA, dequant on load)
    (8, 4, 256, 1500, 700, 64, 256, False, 0),   # prefill, windowed, head_dim 256
    (8, 1, 64, 600, 0, 333, 0, True, 0),         # prefill from empty
    (28, 4, 128, 1200, 600, 100, 0, True, 0),    # prefill, gqa 7 (configs 2/3), ragged rows
    (24, 8, 128, 900, 300, 64, 0, True, 0),      # prefill, gqa 3
]


@pytest.mark.parametrize("case", Q8_CASES)
def test_attn_q8_vs_oracle(T, case):
    n_head, n_kv, hd, cap, pos, n, window, perm, ring = case
    rng = np.random.default_rng(hash(case) & 0xffff)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    out, ref, L, C = _run_attn_q8(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                  seed=pos + n, ring=ring)
    err = np.abs(out - ref).max()
    assert err < TOL, f"vs Q8_0 oracle {err}"
    # the batch rows were quantized into the cache bit-exactly
    gk, gks, gv, gvs = _q8(L)
    assert np.array_equal(gk, C.k) and np.array_equal(gks, C.ks)
    assert np.array_equal(gv, C.v) and np.array_equal(gvs, C.vs)


@pytest.mark.parametrize("case", [c for c in Q8_CASES if c[5] >= 16])
def test_attn_q8_prefill_kernel_forced(T, case):
    """Batches of 16+ rows over the Q8_0 cache on the prefill kernel, also
    where the plan takes the decode kernel (small rows x keys)."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm, ring = case
    rng = np.random.default_rng(hash(case) & 0xffff)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    with tlkv.tuning(tlkv.TUNE_NO_PREFILL, 2):
        out, ref, _, _ = _run_attn_q8(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                      seed=pos + n, ring=ring)
    assert np.abs(out - ref).max() < TOL


@pytest.mark.parametrize("tile", ["vector", "matrix"])
@pytest.mark.parametrize("case", [c for c in Q8_CASES if c[5] < 16] +
                         [(32, 8, 128, 33800, 33791, 1, 0, False, 0)])
def test_attn_q8_decode_tile_paths(T, case, tile):
    """Both decode tile computations over the Q8_0 cache (v_dot2 on the vector
    ALUs, v_mfma on the matrix cores), forced whatever the automatic choice
    for the shape, within tolerance of the Q8_0 oracle."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm, ring = case
    rng = np.random.default_rng(pos + 31 * n)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    with tlkv.tuning(tlkv.TUNE_DECODE_MFMA, 1 if tile == "vector" else 2):
        out, ref, _, _ = _run_attn_q8(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                      seed=pos + n, ring=ring)
    assert np.abs(out - ref).max() < TOL


@pytest.mark.parametrize("case", [
    # n_head, n_kv, hd, cap, pos, n, window, permuted slots, ring
    (40, 5, 128, 3000, 2900, 6, 0, True, 0),      # gqa 8: 2 rows per group
    (16, 4, 64, 2000, 1900, 7, 0, False, 0),      # gqa 4, head_dim 64: 4 rows, ragged
    (8, 8, 64, 1200, 1000, 15, 0, True, 0),       # MHA: 15 rows in one group
    (8, 4, 256, 2100, 1800, 9, 1024, True, 0),    # head_dim 256, windowed
    (32, 8, 128, 8300, 8000, 4, 0, False, 0),     # splits
])
def test_attn_q8_row_folding(T, case):
    """Batch rows folded into one matrix-core group over the Q8_0 cache:
    within tolerance of the Q8_0 oracle with and without folding."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm, ring = case
    rng = np.random.default_rng(pos + 7 * n)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    outs = []
    for rows in (0, 1):
        with tlkv.tuning(tlkv.TUNE_DECODE_MFMA, 2), tlkv.tuning(tlkv.TUNE_DECODE_ROWS, rows):
            out, ref, _, _ = _run_attn_q8(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                          seed=pos + n, ring=ring)
        assert np.abs(out - ref).max() < TOL, (case, rows)
        outs.append(out)
    # different split plans: P is rounded to f16 against different running
    # maxima (the same bound as the prefill split test)
    assert np.abs(outs[0] - outs[1]).max() < 3e-4


@pytest.mark.parametrize("case", [
    # n_head, n_kv, hd, cap, pos, n, window, ring
    (32, 8, 128, 4200, 4000, 1, 0, 0),        # config 4 shape
    (16, 2, 128, 600, 200, 5, 0, 0),          # folded batch rows
    (8, 8, 64, 1300, 1000, 15, 0, 0),         # MHA, 15 new rows
    (8, 4, 256, 0, 3000, 3, 1024, 1026),      # ring of a windowed layer
    (28, 4, 128, 9000, 8191, 2, 0, 0),        # gqa 7, rows across tiles
])
def test_attn_q8_fused_append_equals_separate(T, case):
    """tl_attn_q8 on decode-sized batches quantizes and writes the new rows
    inside the decode launch: the cache (values and scales) and the output
    equal tl_kv_append_q8 followed by tl_attn_noappend_q8, bit for bit."""
    import tlkv
    lib = tlkv.lib()
    n_head, n_kv, hd, cap, pos, n, window, ring = case
    cap = ring or cap
    rng = np.random.default_rng(pos + n)
    kd = n_kv * hd
    hist_k, hist_v = rows(rng, pos, kd, scale_spread=True), rows(rng, pos, kd, scale_spread=True)
    q, k, v = rows(rng, n, n_head * hd), rows(rng, n, kd, scale_spread=True), rows(rng, n, kd)
    slots = None if ring else rng.permutation(cap).astype(np.uint32)
    ds = None if slots is None else dev(T, slots)
    outs, layers = [], []
    for fused in (True, False):
        L = tlkv.LayerQ8(cap, n_kv, hd, ring=ring)
        lo = max(0, pos - ring) if ring else 0
        tlkv.check(lib.tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, hist_k[lo:])),
                                       tlkv.ptr(dev(T, hist_v[lo:])), kd, tlkv.ptr(ds), lo,
                                       pos - lo, None))
        out = T.zeros((n, n_head * hd), dtype=T.float32, device="cuda")
        dk, dv = dev(T, k), dev(T, v)
        a = tlkv.attn_args(dev(T, q), dk, dv, out, ds, pos, n, n_head, hd, n_kv, window,
                           O.scale_of(hd))
        if fused:
            tlkv.check(lib.tl_attn_q8(L.desc, a, None))
        else:
            tlkv.check(lib.tl_kv_append_q8(L.desc, tlkv.ptr(dk), tlkv.ptr(dv), kd, tlkv.ptr(ds),
                                           pos, n, None))
            tlkv.check(lib.tl_attn_noappend_q8(L.desc, a, None))
        sync(T)
        outs.append(host(out))
        layers.append(_q8(L))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), case
    for x, y in zip(layers[0], layers[1]):
        assert np.array_equal(x, y), case


@pytest.mark.parametrize("n", [1, 4, 40])
def test_attn_noappend_q8(T, n):
    rng = np.random.default_rng(n)
    cap = 900
    slots = rng.permutation(cap).astype(np.uint32)
    out, ref, _, _ = _run_attn_q8(T, 16, 4, 128, cap, 800, n, 0, slots, seed=n, append=False)
    assert np.abs(out - ref).max() < TOL


def test_attn_q8_full_size_config4(T):
    """Config 4's shape at its full key count (one layer, last decode step)."""
    out, ref, _, _ = _run_attn_q8(T, 32, 8, 128, 33800, 33791, 1, 0, None, seed=4)
    assert np.abs(out - ref).max() < TOL


def test_attn_q8_split_invariance(T):
    """Different split counts (decode workgroups) give results within rounding."""
    import tlkv
    rng = np.random.default_rng(9)
    cap = 6000
    slots = rng.permutation(cap).astype(np.uint32)
    outs = []
    for wgs in (8, 64, 0):
        with tlkv.tuning(tlkv.TUNE_DECODE_WGS, wgs):
            out, ref, _, _ = _run_attn_q8(T, 32, 8, 128, cap, 5900, 1, 0, slots, seed=3)
        assert np.abs(out - ref).max() < TOL, wgs
        outs.append(out)
    assert np.abs(outs[0] - outs[2]).max() < 1e-3


@pytest.mark.parametrize("window", [0, 300])
def test_decode_batch_q8_sessions(T, window):
    """tl_attn_decode_batch_q8: several sessions (own caches, slot tables or a
    ring, positions) in one append + one decode launch, each within 2e-3 of
    the oracle and its new row quantized bit-exactly into its cache."""
    import tlkv
    rng = np.random.default_rng(40 + window)
    n_head, n_kv, hd = 12, 4, 128
    # cap, pos, permuted slots, ring (a ring needs a window: ring >= window)
    last = (1100, 2500, False, 1100) if window else (1100, 1093, False, 0)
    specs = [(1200, 1100, True, 0), (700, 333, False, 0), (2000, 1999, True, 0),
             (900, 5, True, 0), last]
    seqs = (tlkv.DecodeSeqQ8 * len(specs))()
    refs, layers, oc = [], [], []
    for i, (cap, pos, perm, ring) in enumerate(specs):
        slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
        hk = rows(rng, pos + 1, n_kv * hd)
        hv = rows(rng, pos + 1, n_kv * hd)
        q = rows(rng, 1, n_head * hd)
        L = tlkv.LayerQ8(cap, n_kv, hd, ring=ring)
        C = O.CacheQ8(cap, n_kv, hd, ring)
        ds = None if slots is None else dev(T, slots)
        lo = max(0, pos - ring) if ring else 0
        if pos > lo:
            tlkv.check(tlkv.lib().tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, hk[lo:pos])),
                                                  tlkv.ptr(dev(T, hv[lo:pos])), n_kv * hd,
                                                  tlkv.ptr(ds), lo, pos - lo, None))
            assert C.append(hk[lo:pos], hv[lo:pos], slots, lo, pos - lo) == 0
        out = T.zeros((1, n_head * hd), dtype=T.float32, device="cuda")
        seqs[i] = tlkv.DecodeSeqQ8(L.desc, None if ds is None else ds.data_ptr(), pos, 0,
                                   dev(T, q).data_ptr(), dev(T, hk[pos:]).data_ptr(),
                                   dev(T, hv[pos:]).data_ptr(), out.data_ptr())
        refs.append(C.attn(q, hk[pos:], hv[pos:], slots, pos, 1, n_head, window=window))
        layers.append((L, out))
        oc.append(C)
    tlkv.check(tlkv.lib().tl_attn_decode_batch_q8(seqs, len(specs), n_head, window,
                                                  O.scale_of(hd), None))
    sync(T)
    for i, ((L, out), ref, C) in enumerate(zip(layers, refs, oc)):
        err = np.abs(host(out) - ref).max()
        assert err < TOL, f"session {i}: {err}"
        gk, gks, gv, gvs = _q8(L)
        assert np.array_equal(gk, C.k) and np.array_equal(gks, C.ks), i
        assert np.array_equal(gv, C.v) and np.array_equal(gvs, C.vs), i


@pytest.mark.parametrize("neox,rdim,n,window", [(0, 128, 1, 0), (1, 128, 3, 0), (1, 64, 40, 0),
                                                 (0, 128, 24, 100), (1, 128, 1, 200),
                                                 (1, 128, 4, 0), (0, 64, 9, 0)])
def test_attn_rope_q8_equals_rope_then_attn(T, neox, rdim, n, window):
    """tl_attn_rope_q8 (K rotated before quantizing, q while staged) gives the
    same bits as tl_rope on q and k followed by tl_attn_q8: outputs, values
    and scales."""
    import tlkv
    rng = np.random.default_rng(90 + n + neox)
    n_head, n_kv, hd, cap, pos = 16, 4, 128, 600, 300
    theta = 10000.0 if neox else 500000.0
    slots = rng.permutation(cap).astype(np.uint32)
    hk, hv = rows(rng, pos, n_kv * hd), rows(rng, pos, n_kv * hd)
    q, k, v = rows(rng, n, n_head * hd), rows(rng, n, n_kv * hd), rows(rng, n, n_kv * hd)
    rp = tlkv.RopeParams(rdim, theta, neox)
    outs, lays = [], []
    for fused in (False, True):
        L = tlkv.LayerQ8(cap, n_kv, hd)
        ds = dev(T, slots)
        tlkv.check(tlkv.lib().tl_kv_append_q8(L.desc, tlkv.ptr(dev(T, hk)), tlkv.ptr(dev(T, hv)),
                                              n_kv * hd, tlkv.ptr(ds), 0, pos, None))
        dq, dk, dv = dev(T, q), dev(T, k), dev(T, v)
        out = T.zeros((n, n_head * hd), dtype=T.float32, device="cuda")
        a = tlkv.attn_args(dq, dk, dv, out, ds, pos, n, n_head, hd, n_kv, window, O.scale_of(hd))
        if fused:
            tlkv.check(tlkv.lib().tl_attn_rope_q8(L.desc, a, rp, None))
        else:
            lib = tlkv.lib()
            tlkv.check(lib.tl_rope(tlkv.ptr(dq), n, n_head * hd, n_head, hd, rdim, pos, theta,
                                   neox, None))
            tlkv.check(lib.tl_rope(tlkv.ptr(dk), n, n_kv * hd, n_kv, hd, rdim, pos, theta,
                                   neox, None))
            tlkv.check(lib.tl_attn_q8(L.desc, a, None))
        sync(T)
        outs.append(host(out))
        lays.append(_q8(L))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for x, y in zip(lays[0], lays[1]):
        assert np.array_equal(x, y)
