"""GPU parity of the device path against the CPU oracle (through the C ABI).

Append / gather / copy: bit-exact against oracle.c (f16 RNE of the reference's
f32 rows, written at the reference's slot, cpu_op.c:995-1008).
Attention: within 2e-3 max-abs of the oracle's op_attn restatement, both over
the same f16 cache (kernel error alone) and over the reference's f32 cache
(the reference CPU semantics).
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
    """Device copy of a numpy array.  The tensor is kept alive until the
    module ends: kernels run asynchronously and only its address crosses the
    ABI, so a temporary could be freed and reused before the kernel reads it."""
    t = T.from_numpy(np.ascontiguousarray(a)).cuda()
    _KEEP.append(t)
    return t


def host(t):
    return t.cpu().numpy()


def sync(T):
    T.cuda.synchronize()
    _KEEP.clear()


def rows(rng, n, width, special=False):
    x = rng.standard_normal((n, width)).astype(np.float32)
    if special:
        sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 1e-8,
                       -6.0e-8, 2.9802322e-08, 5.9604645e-08, 1e5, -3e-5, 0.5 + 2**-12],
                      dtype=np.float32)
        flat = x.reshape(-1)
        flat[:sp.size] = sp
        # a signalling-pattern NaN with payload
        flat[sp.size] = np.frombuffer(np.uint32(0x7f800123).tobytes(), np.float32)[0]
        flat[sp.size + 1] = np.frombuffer(np.uint32(0xffc00001).tobytes(), np.float32)[0]
    return x


@pytest.mark.parametrize("n_kv,hd,cap,n,pos,perm", [
    (8, 128, 64, 17, 5, True),
    (8, 64, 40, 33, 0, False),
    (4, 256, 32, 9, 3, True),
    (4, 128, 600, 512, 7, True),
])
def test_append_bitexact(T, n_kv, hd, cap, n, pos, perm):
    import tlkv
    rng = np.random.default_rng(n * 31 + hd)
    k = rows(rng, n, n_kv * hd, special=True)
    v = rows(rng, n, n_kv * hd, special=True)
    slots = (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    L = tlkv.Layer(cap, n_kv, hd)
    ds = dev(T, slots)
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, k)), tlkv.ptr(dev(T, v)),
                                       n_kv * hd, tlkv.ptr(ds), pos, n, None))
    sync(T)
    C = O.Cache(cap, n_kv, hd)
    assert C.append(k, v, slots, pos, n) == 0
    assert np.array_equal(host(L.k).view(np.uint16), C.k)
    assert np.array_equal(host(L.v).view(np.uint16), C.v)


def test_append_identity_slots(T):
    import tlkv
    rng = np.random.default_rng(3)
    n_kv, hd, cap = 8, 128, 48
    k, v = rows(rng, 20, n_kv * hd), rows(rng, 20, n_kv * hd)
    L = tlkv.Layer(cap, n_kv, hd)
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, k)), tlkv.ptr(dev(T, v)),
                                       n_kv * hd, None, 11, 20, None))
    sync(T)
    C = O.Cache(cap, n_kv, hd)
    C.append(k, v, None, 11, 20)
    assert np.array_equal(host(L.k).view(np.uint16), C.k)
    assert np.array_equal(host(L.v).view(np.uint16), C.v)


def test_gather_roundtrip(T):
    """gather(append(x)) == f16(x) for any slot permutation."""
    import tlkv
    rng = np.random.default_rng(4)
    n_kv, hd, cap, n = 4, 128, 256, 200
    k, v = rows(rng, n, n_kv * hd, True), rows(rng, n, n_kv * hd, True)
    slots = rng.permutation(cap).astype(np.uint32)
    L = tlkv.Layer(cap, n_kv, hd)
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, k)), tlkv.ptr(dev(T, v)),
                                       n_kv * hd, tlkv.ptr(dev(T, slots)), 0, n, None))
    ko = T.zeros((n, n_kv, hd), dtype=T.float16, device="cuda")
    vo = T.zeros_like(ko)
    tlkv.check(tlkv.lib().tl_kv_gather(L.desc, tlkv.ptr(dev(T, slots[:n])), n,
                                       tlkv.ptr(ko), tlkv.ptr(vo), None))
    sync(T)
    assert np.array_equal(host(ko).view(np.uint16).reshape(n, -1), O.f16_bits(k))
    assert np.array_equal(host(vo).view(np.uint16).reshape(n, -1), O.f16_bits(v))


def test_copy_rows_all_layers(T):
    import tlkv
    rng = np.random.default_rng(5)
    n_kv, hd, cap, nl = 4, 128, 64, 3
    layers = [tlkv.Layer(cap, n_kv, hd) for _ in range(nl)]
    for L in layers:
        L.k.copy_(T.randn(L.k.shape, device="cuda").half())
        L.v.copy_(T.randn(L.v.shape, device="cuda").half())
    before = [(host(L.k).copy(), host(L.v).copy()) for L in layers]
    src = np.array([1, 5, 9, 30, 31], dtype=np.uint32)
    dst = np.array([40, 2, 63, 0, 10], dtype=np.uint32)
    arr = (tlkv.KvLayer * nl)(*[L.desc for L in layers])
    tlkv.check(tlkv.lib().tl_kv_copy(arr, nl, tlkv.ptr(dev(T, src)),
                                     tlkv.ptr(dev(T, dst)), src.size, None))
    sync(T)
    for L, (kb, vb) in zip(layers, before):
        ke, ve = kb.copy(), vb.copy()
        ke[:, dst] = kb[:, src]
        ve[:, dst] = vb[:, src]
        assert np.array_equal(host(L.k), ke)
        assert np.array_equal(host(L.v), ve)


def _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots, seed, ring=0):
    """Fill positions [0,pos) then run OP_ATTN on rows [pos,pos+n) on both the
    device and the oracle.  Returns (device, oracle f16 cache, oracle f32 cache)."""
    import tlkv
    rng = np.random.default_rng(seed)
    kd = n_kv * hd
    hist_k, hist_v = rows(rng, pos, kd), rows(rng, pos, kd)
    q = rows(rng, n, n_head * hd)
    k, v = rows(rng, n, kd), rows(rng, n, kd)

    L = tlkv.Layer(cap, n_kv, hd, ring=ring)
    ds = None if slots is None else dev(T, slots)
    Cf16 = O.Cache(cap, n_kv, hd, f16=True)
    Cf32 = O.Cache(cap, n_kv, hd, f16=False)
    if pos:
        if ring:
            for p in range(max(0, pos - ring), pos):   # older rows are overwritten
                tlkv.check(tlkv.lib().tl_kv_append(
                    L.desc, tlkv.ptr(dev(T, hist_k[p:p + 1])),
                    tlkv.ptr(dev(T, hist_v[p:p + 1])), kd, None, p, 1, None))
                Cf16.append(hist_k[p:p + 1], hist_v[p:p + 1], None, p % ring, 1)
                Cf32.append(hist_k[p:p + 1], hist_v[p:p + 1], None, p % ring, 1)
        else:
            tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hist_k)),
                                               tlkv.ptr(dev(T, hist_v)), kd, tlkv.ptr(ds),
                                               0, pos, None))
            Cf16.append(hist_k, hist_v, slots, 0, pos)
            Cf32.append(hist_k, hist_v, slots, 0, pos)
    dq, dk, dv = dev(T, q), dev(T, k), dev(T, v)
    out = T.zeros((n, n_head * hd), dtype=T.float32, device="cuda")
    a = tlkv.attn_args(dq, dk, dv, out, ds, pos, n, n_head, hd, n_kv, window,
                       O.scale_of(hd))
    tlkv.check(tlkv.lib().tl_attn(L.desc, a, None))
    sync(T)
    o16 = O.attn(Cf16, q, k, v, slots, pos, n, n_head, window=window, ring=ring)
    o32 = O.attn(Cf32, q, k, v, slots, pos, n, n_head, window=window, ring=ring)
    return host(out), o16, o32, L, Cf16


ATTN_CASES = [
    # n_head, n_kv, hd, cap, pos, n, window, permuted slots
    (32, 8, 64, 1024, 700, 1, 0, True),      # config 1 shape
    (28, 4, 128, 2048, 1500, 1, 0, True),    # config 2/3 shape, gqa 7
    (32, 8, 128, 4096, 4000, 1, 0, False),   # config 4 shape
    (8, 4, 256, 2048, 1800, 1, 1024, True),  # config 5 local layer
    (8, 4, 256, 2048, 1800, 1, 0, False),    # config 5 global layer
    (32, 8, 128, 512, 3, 1, 0, True),        # tiny history
    (32, 8, 128, 512, 0, 1, 0, False),       # first token
    (16, 2, 128, 600, 200, 5, 0, True),      # multi-row batch (decode kernel)
    (16, 2, 128, 600, 200, 6, 64, True),     # multi-row + window
    (8, 8, 64, 300, 100, 3, 0, False),       # MHA
]


@pytest.mark.parametrize("case", ATTN_CASES)
def test_attn_vs_oracle(T, case):
    n_head, n_kv, hd, cap, pos, n, window, perm = case
    rng = np.random.default_rng(hash(case) & 0xffff)
    slots = (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                    seed=pos + n)
    e16 = np.abs(out - o16).max()
    e32 = np.abs(out - o32).max()
    assert e16 < TOL, f"vs f16-cache oracle {e16}"
    assert e32 < TOL, f"vs f32-cache (reference) oracle {e32}"


FULL_SIZE_CASES = [
    # BASELINE shapes at their full key counts (one layer, one decode row)
    # n_head, n_kv, hd, cap, pos, window, permuted slots, ring
    (32, 8, 64, 800, 767, 0, True, 0),            # config 1, last decode step
    (28, 4, 128, 8800, 8703, 0, True, 0),         # config 2/3, last decode step
    (32, 8, 128, 33800, 33791, 0, False, 0),      # config 4, last decode step
    (8, 4, 256, 17000, 16895, 0, False, 0),       # config 5 global layer
    (8, 4, 256, 1535, 16895, 1024, False, 1535),  # config 5 local layer on its ring
]


@pytest.mark.parametrize("case", FULL_SIZE_CASES)
def test_attn_full_size_vs_oracle(T, case):
    n_head, n_kv, hd, cap, pos, window, perm, ring = case
    rng = np.random.default_rng(pos)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, 1, window, slots,
                                    seed=pos + 1, ring=ring)
    assert np.abs(out - o16).max() < TOL
    assert np.abs(out - o32).max() < TOL


@pytest.mark.parametrize("tile", ["vector", "matrix"])
@pytest.mark.parametrize("case", ATTN_CASES + [c[:5] + (1,) + c[5:] for c in FULL_SIZE_CASES])
def test_decode_tile_paths_vs_oracle(T, case, tile):
    """Both decode tile computations (v_dot2 on the vector ALUs, v_mfma
    16x16 on the matrix cores), forced whatever the automatic choice for the
    shape, within tolerance of the oracle and of each other."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm = case[:8]
    ring = case[8] if len(case) > 8 else 0
    rng = np.random.default_rng(pos + 17 * n)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    with tlkv.tuning(tlkv.TUNE_DECODE_MFMA, 1 if tile == "vector" else 2):
        out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                        seed=pos + n, ring=ring)
    assert np.abs(out - o16).max() < TOL
    assert np.abs(out - o32).max() < TOL


def _random_decode_cases(count=24, seed=2024):
    """Seeded decode shapes over the kernel's whole parameter range: head_dim
    64/128/256, gqa 1-8, 1-8 kv-heads, 1-15 batch rows, full / windowed /
    ring layers, identity or permuted slot tables."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        hd = int(rng.choice([64, 128, 256]))
        n_kv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.integers(1, 9))
        n = int(rng.choice([1, 1, 1, 2, 7, 15]))
        pos = int(rng.integers(0, 3000))
        window = int(rng.choice([0, 0, 64, 700]))
        ring = window + n - 1 + int(rng.integers(0, 16)) if window and rng.random() < 0.5 else 0
        cap = ring if ring else pos + n + int(rng.integers(0, 64))
        perm = bool(rng.random() < 0.5) and not ring
        cases.append((g * n_kv, n_kv, hd, cap, pos, n, window, perm, ring))
    return cases


@pytest.mark.parametrize("tile", ["vector", "matrix"])
@pytest.mark.parametrize("case", _random_decode_cases())
def test_decode_random_shapes_both_tiles(T, case, tile):
    """Both decode tile paths against the oracle over seeded random shapes."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm, ring = case
    rng = np.random.default_rng(cap + 7 * pos)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    with tlkv.tuning(tlkv.TUNE_DECODE_MFMA, 1 if tile == "vector" else 2):
        out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                        seed=pos + n, ring=ring)
    assert np.abs(out - o16).max() < TOL, case
    assert np.abs(out - o32).max() < TOL, case


def test_attn_noncontiguous_equals_contiguous(T):
    """Spec'd parity test of the reference design (slot table [7,3,9,12] vs
    [0,1,2,3]): identical outputs."""
    n_head, n_kv, hd = 8, 2, 64
    cap = 16
    perm = np.arange(cap, dtype=np.uint32)
    perm[:4] = [7, 3, 9, 12]
    perm[4:] = [s for s in range(cap) if s not in (7, 3, 9, 12)]
    ident = np.arange(cap, dtype=np.uint32)
    a, _, _, _, _ = _run_attn(T, n_head, n_kv, hd, cap, 3, 1, 0, perm, seed=9)
    b, _, _, _, _ = _run_attn(T, n_head, n_kv, hd, cap, 3, 1, 0, ident, seed=9)
    assert np.array_equal(a, b)


def test_attn_ring_window(T):
    """Ring layout for windowed layers equals the masked full cache."""
    n_head, n_kv, hd, win = 8, 4, 256, 64
    ring = win
    out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, 256, 200, 1, win, None,
                                    seed=11, ring=ring)
    assert np.abs(out - o32).max() < TOL
    assert np.abs(out - o16).max() < TOL


def test_attn_closed_form_identical_keys(T):
    """All keys equal -> uniform softmax -> output = mean of V rows (f16)."""
    import tlkv
    n_head, n_kv, hd, P = 8, 2, 128, 3000
    cap = P
    rng = np.random.default_rng(12)
    L = tlkv.Layer(cap, n_kv, hd)
    krow = rng.standard_normal(n_kv * hd).astype(np.float32)
    hk = np.tile(krow, (P - 1, 1))
    hv = rows(rng, P - 1, n_kv * hd)
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hk)), tlkv.ptr(dev(T, hv)),
                                       n_kv * hd, None, 0, P - 1, None))
    q = rows(rng, 1, n_head * hd)
    v_new = rows(rng, 1, n_kv * hd)
    out = T.zeros((1, n_head * hd), dtype=T.float32, device="cuda")
    a = tlkv.attn_args(dev(T, q), dev(T, krow[None]), dev(T, v_new), out, None,
                       P - 1, 1, n_head, hd, n_kv, 0, O.scale_of(hd))
    tlkv.check(tlkv.lib().tl_attn(L.desc, a, None))
    sync(T)
    allv = O.f16_to_f32(O.f16_bits(np.concatenate([hv, v_new]))).astype(np.float64)
    mean = allv.mean(axis=0).reshape(n_kv, hd)
    expect = np.repeat(mean, n_head // n_kv, axis=0).reshape(-1)
    assert np.abs(host(out)[0] - expect).max() < 1e-4


def test_split_count_invariance(T):
    """The split-K decomposition does not change the result beyond rounding
    (p is rounded to f16 against each tile's running max)."""
    outs = []
    import tlkv
    for wgs in (1, 64, 4096):
        with tlkv.tuning(tlkv.TUNE_DECODE_WGS, wgs):
            out, o16, _, _, _ = _run_attn(T, 32, 8, 128, 8192, 8000, 1, 0, None, seed=13)
        assert np.abs(out - o16).max() < TOL
        outs.append(out)
    assert np.abs(outs[0] - outs[1]).max() < 1e-4
    assert np.abs(outs[0] - outs[2]).max() < 1e-4


@pytest.mark.parametrize("shape", [(32, 8, 128, 8192, 8000), (28, 4, 128, 3000, 2900),
                                   (32, 8, 64, 1024, 700), (8, 4, 256, 4096, 4000),
                                   (28, 4, 128, 8300, 8192), (8, 4, 256, 17000, 16384)])
def test_decode_variants_agree(T, shape):
    """The three ways of merging decode splits: every split merging a slice
    of the output inside the launch (the default where it applies), the last
    workgroup of a group merging all of it, and the separate merge kernel:
    same result up to rounding, each within tolerance of the oracle."""
    n_head, n_kv, hd, cap, pos = shape
    import tlkv
    outs = []
    for merge_kernel, single in ((0, 0), (0, 1), (1, 0)):
        with tlkv.tuning(tlkv.TUNE_DECODE_MERGE_KERNEL, merge_kernel), \
                tlkv.tuning(tlkv.TUNE_DECODE_SINGLE_MERGE, single):
            out, o16, _, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, 1, 0, None, seed=pos)
        assert np.abs(out - o16).max() < TOL, (merge_kernel, single)
        outs.append(out)
    for o in outs[1:]:
        assert np.abs(outs[0] - o).max() < 1e-4


FOLD_CASES = [
    # n_head, n_kv, hd, cap, pos, n, window, permuted slots, ring
    (32, 8, 128, 8300, 8000, 4, 0, False, 0),   # config 4 shape: 4 rows per group, splits
    (28, 4, 128, 3000, 2900, 7, 0, True, 0),    # gqa 7: 2 rows per group, ragged last block
    (8, 8, 64, 1300, 1000, 15, 0, True, 0),     # MHA: 15 rows in one group
    (16, 2, 64, 2100, 2000, 15, 0, False, 0),   # gqa 8, head_dim 64
    (8, 4, 256, 2100, 1800, 9, 1024, True, 0),  # head_dim 256, windowed, ragged
    (16, 4, 128, 0, 600, 6, 200, False, 210),   # ring of a windowed layer
    (32, 8, 128, 600, 0, 15, 0, True, 0),       # from an empty cache
    (32, 8, 128, 33000, 32000, 4, 0, False, 0), # 32K keys
]


@pytest.mark.parametrize("case", [
    # n_head, n_kv, hd, cap, pos, n, slot table
    (32, 8, 128, 40100, 40000, 8, "perm"),    # 16 groups x 16 splits of 2501 keys: u16 slots
    (32, 8, 128, 70000, 66000, 1, "perm"),    # slots past 65535: u32, 33+ splits in even rounds
    (32, 8, 128, 40100, 40000, 8, None),      # no slot table: no chunk limit
])
def test_decode_long_chunks(T, case):
    """Chunks past 2048 keys per workgroup: the u16-slot instance for pools of
    at most 65536 rows, u32 slots (every value kept) and whole even rounds of
    workgroups above that, and no limit without a slot table."""
    n_head, n_kv, hd, cap, pos, n, table = case
    rng = np.random.default_rng(cap + n)
    slots = rng.permutation(cap).astype(np.uint32) if table else None
    out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, 0, slots, seed=pos + n)
    assert np.abs(out - o16).max() < TOL, case
    assert np.abs(out - o32).max() < TOL, case


@pytest.mark.parametrize("case", FOLD_CASES)
def test_decode_row_folding(T, case):
    """Several batch rows of a session in one matrix-core group (their heads
    side by side as MFMA columns, each column masked to its own row's keys):
    within tolerance of the oracle, and of the one-row-per-group launch up
    to rounding."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm, ring = case
    cap = ring or cap
    rng = np.random.default_rng(cap + pos + n)
    slots = None if ring else (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    outs = []
    for rows in (0, 1):
        with tlkv.tuning(tlkv.TUNE_DECODE_MFMA, 2), tlkv.tuning(tlkv.TUNE_DECODE_ROWS, rows):
            out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                            seed=pos + n, ring=ring)
        assert np.abs(out - o16).max() < TOL, (case, rows)
        assert np.abs(out - o32).max() < TOL, (case, rows)
        outs.append(out)
    # different split plans: P is rounded to f16 against different running
    # maxima (the same bound as the prefill split test)
    assert np.abs(outs[0] - outs[1]).max() < 3e-4


def test_decode_batch_sessions(T):
    """Multi-session one-token decode equals per-session OP_ATTN."""
    import tlkv
    n_head, n_kv, hd = 28, 4, 128
    n_seq = 8
    rng = np.random.default_rng(14)
    seqs, refs, keep = [], [], []
    for s in range(n_seq):
        cap = 512 + 64 * s
        pos = 300 + 17 * s
        slots = rng.permutation(cap).astype(np.uint32)
        L = tlkv.Layer(cap, n_kv, hd)
        hk, hv = rows(rng, pos, n_kv * hd), rows(rng, pos, n_kv * hd)
        ds = dev(T, slots)
        tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hk)),
                                           tlkv.ptr(dev(T, hv)), n_kv * hd,
                                           tlkv.ptr(ds), 0, pos, None))
        C = O.Cache(cap, n_kv, hd)
        C.append(hk, hv, slots, 0, pos)
        q, k, v = rows(rng, 1, n_head * hd), rows(rng, 1, n_kv * hd), rows(rng, 1, n_kv * hd)
        dq, dk, dv = dev(T, q), dev(T, k), dev(T, v)
        out = T.zeros((1, n_head * hd), dtype=T.float32, device="cuda")
        keep += [L, ds, dq, dk, dv]
        seqs.append(tlkv.DecodeSeq(L.desc, ds.data_ptr(), pos, 0, dq.data_ptr(),
                                   dk.data_ptr(), dv.data_ptr(), out.data_ptr()))
        refs.append((out, O.attn(C, q, k, v, slots, pos, 1, n_head)))
    arr = (tlkv.DecodeSeq * n_seq)(*seqs)
    tlkv.check(tlkv.lib().tl_attn_decode_batch(arr, n_seq, n_head, 0,
                                               O.scale_of(hd), None))
    sync(T)
    for out, ref in refs:
        assert np.abs(host(out) - ref).max() < TOL


@pytest.mark.parametrize("neox", [0, 1])
def test_rope_vs_oracle(T, neox):
    import tlkv
    rng = np.random.default_rng(15 + neox)
    heads, hd, rows_n, pos = 8, 128, 64, 3000
    x = rng.standard_normal((rows_n, heads * hd)).astype(np.float32)
    dx = dev(T, x)
    tlkv.check(tlkv.lib().tl_rope(tlkv.ptr(dx), rows_n, heads * hd, heads, hd, hd, pos,
                                  500000.0, neox, None))
    sync(T)
    ref = O.rope(x, heads, hd, hd, pos, 500000.0, neox)
    # angles up to ~3e3 rad: one f32 ulp of the angle is ~2.4e-4 rad; libm
    # (reference: -ffast-math glibc) and the device differ by a few ulp
    assert np.abs(host(dx) - ref).max() < 2e-3


PREFILL_CASES = [
    # n_head, n_kv, hd, cap, pos, n, window, permuted slots
    (32, 8, 128, 600, 0, 512, 0, False),     # config 4 first chunk
    (32, 8, 128, 1600, 1000, 512, 0, True),  # config 4 later chunk, slot table
    (32, 8, 64, 1100, 512, 512, 0, True),    # config 1 shape
    (28, 4, 128, 700, 300, 100, 0, True),    # gqa 7, ragged rows
    (8, 4, 256, 800, 600, 64, 128, True),    # config 5 local layer (window)
    (8, 4, 256, 800, 500, 200, 0, False),    # config 5 global layer
    (16, 2, 128, 300, 7, 16, 5, True),       # smallest prefill batch, tiny window
    (32, 8, 128, 2200, 2000, 64, 0, True),   # 64 rows x 2K keys (decode kernel when planned)
    (28, 4, 128, 700, 600, 40, 0, False),    # 40 rows, gqa 7
]


@pytest.mark.parametrize("kernel", ["auto", "prefill"])
@pytest.mark.parametrize("case", PREFILL_CASES)
def test_prefill_vs_oracle(T, case, kernel):
    """Batches of 16+ rows: as planned (small rows x keys run on the decode
    kernel) and forced onto the prefill kernel."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n, window, perm = case
    rng = np.random.default_rng(sum(case))
    slots = (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    with tlkv.tuning(tlkv.TUNE_NO_PREFILL, 2 if kernel == "prefill" else 0):
        out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                        seed=pos + 3 * n)
    e16 = np.abs(out - o16).max()
    e32 = np.abs(out - o32).max()
    assert e16 < TOL, f"vs f16-cache oracle {e16}"
    assert e32 < TOL, f"vs f32-cache (reference) oracle {e32}"


def test_prefill_split_invariance(T):
    outs = []
    import tlkv
    for ns in (1, 3, 7):
        with tlkv.tuning(tlkv.TUNE_PREFILL_SPLITS, ns):
            out, o16, _, _, _ = _run_attn(T, 32, 8, 128, 2100, 1500, 512, 0, None, seed=21)
        assert np.abs(out - o16).max() < TOL
        outs.append(out)
    # each split rounds its probabilities to f16 relative to its own running
    # max reference (raised lazily, up to 2^8 below the true max), so split
    # counts agree to f16 rounding of P, far inside the 2e-3 oracle bar
    assert np.abs(outs[0] - outs[1]).max() < 3e-4
    assert np.abs(outs[0] - outs[2]).max() < 3e-4


@pytest.mark.parametrize("case", [
    # n_head, n_kv, hd, cap, pos, n, window, permuted slots: GQA ratios the
    # BASELINE shapes do not use, and the largest fused decode batch
    (12, 4, 128, 2048, 1900, 1, 0, True),     # gqa 3
    (20, 4, 128, 2048, 1900, 1, 0, False),    # gqa 5
    (24, 4, 64, 2048, 1900, 1, 0, True),      # gqa 6, head_dim 64
    (16, 2, 256, 2048, 1500, 2, 0, True),     # gqa 8, head_dim 256, 2 rows
    (32, 8, 128, 4096, 3000, 15, 0, True),    # 15 new rows in one decode launch
    (32, 8, 128, 4096, 3000, 15, 700, False), # same, windowed
])
def test_attn_more_shapes_vs_oracle(T, case):
    n_head, n_kv, hd, cap, pos, n, window, perm = case
    rng = np.random.default_rng(pos + n)
    slots = (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
    out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, window, slots,
                                    seed=pos + 3 * n)
    assert np.abs(out - o16).max() < TOL
    assert np.abs(out - o32).max() < TOL


def test_decode_deterministic_across_launches(T):
    """The same decode call repeated on the same cache gives bit-identical
    outputs (fixed split boundaries and merge order)."""
    import tlkv
    n_head, n_kv, hd, cap, pos = 32, 8, 128, 20000, 19000
    rng = np.random.default_rng(21)
    L = tlkv.Layer(cap, n_kv, hd)
    kd = n_kv * hd
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, rows(rng, pos, kd))),
                                       tlkv.ptr(dev(T, rows(rng, pos, kd))), kd, None, 0, pos,
                                       None))
    q = dev(T, rows(rng, 1, n_head * hd))
    outs = []
    for _ in range(3):
        out = T.zeros((1, n_head * hd), dtype=T.float32, device="cuda")
        a = tlkv.attn_args(q, None, None, out, None, pos, 1, n_head, hd, n_kv, 0,
                           O.scale_of(hd))
        tlkv.check(tlkv.lib().tl_attn_noappend(L.desc, a, None))
        sync(T)
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("q8", [False, True])
def test_append_layers_equals_per_layer(T, q8):
    """tl_kv_append_layers(_q8): 20 layers (two launches of up to 16) write
    the same bytes as 20 per-layer appends."""
    import ctypes
    import tlkv
    rng = np.random.default_rng(77 + q8)
    n_layer, n_kv, hd, cap, pos, n = 20, 4, 128, 300, 17, 45
    slots = rng.permutation(cap).astype(np.uint32)
    ds = dev(T, slots)
    ks = [dev(T, rows(rng, n, n_kv * hd)) for _ in range(n_layer)]
    vs = [dev(T, rows(rng, n, n_kv * hd)) for _ in range(n_layer)]
    mk = (lambda: tlkv.LayerQ8(cap, n_kv, hd)) if q8 else (lambda: tlkv.Layer(cap, n_kv, hd))
    A = [mk() for _ in range(n_layer)]
    B = [mk() for _ in range(n_layer)]
    one = tlkv.lib().tl_kv_append_q8 if q8 else tlkv.lib().tl_kv_append
    for l in range(n_layer):
        tlkv.check(one(A[l].desc, tlkv.ptr(ks[l]), tlkv.ptr(vs[l]), n_kv * hd, tlkv.ptr(ds),
                       pos, n, None))
    Desc = tlkv.KvLayerQ8 if q8 else tlkv.KvLayer
    descs = (Desc * n_layer)(*[b.desc for b in B])
    karr = (ctypes.c_void_p * n_layer)(*[t.data_ptr() for t in ks])
    varr = (ctypes.c_void_p * n_layer)(*[t.data_ptr() for t in vs])
    many = tlkv.lib().tl_kv_append_layers_q8 if q8 else tlkv.lib().tl_kv_append_layers
    tlkv.check(many(descs, n_layer, karr, varr, n_kv * hd, tlkv.ptr(ds), pos, n, None))
    sync(T)
    for a, b in zip(A, B):
        assert T.equal(a.k, b.k) and T.equal(a.v, b.v)
        if q8:
            assert T.equal(a.ks, b.ks) and T.equal(a.vs, b.vs)


def test_attn_rejects_bad_arguments_without_side_effects(T):
    """Shapes the kernels do not support and positions past the cache are
    rejected before any launch (TL_EINVAL / TL_ERANGE); an empty batch (n = 0)
    is a no-op.  Neither touches the output or the cache."""
    import tlkv
    lib = tlkv.lib()
    n_kv, hd, cap = 2, 128, 64
    L = tlkv.Layer(cap, n_kv, hd)
    L.k.fill_(1.0)
    L.v.fill_(-2.0)
    k0, v0 = L.k.clone(), L.v.clone()
    rng = np.random.default_rng(3)
    q = dev(T, rows(rng, 2, 32 * hd))
    k = dev(T, rows(rng, 2, n_kv * hd))
    out = T.full((2, 32 * hd), 7.0, dtype=T.float32, device="cuda")

    def call(pos, n, n_head, window=0, qoff=0):
        a = tlkv.attn_args(q, k, k, out, None, pos, n, n_head, hd, n_kv, window)
        a.q = q.data_ptr() + qoff
        return lib.tl_attn(L.desc, a, None)

    TL_EINVAL, TL_ERANGE = -1, -2
    assert call(10, 1, 3) == TL_EINVAL            # n_head not a multiple of n_kv
    assert call(10, 1, 18) == TL_EINVAL           # gqa 9 > 8
    assert call(10, 1, 8, qoff=4) == TL_EINVAL    # q not 16-byte aligned
    assert call(cap - 1, 2, 8) == TL_ERANGE       # rows past the cache end
    assert call(10, 0, 8) == 0                    # empty batch
    sync(T)
    assert bool((out == 7.0).all())
    assert T.equal(L.k, k0) and T.equal(L.v, v0)
    # a ring layer needs a window that fits it
    R = tlkv.Layer(32, n_kv, hd, ring=32)
    a = tlkv.attn_args(q, k, k, out, None, 40, 1, 8, hd, n_kv, 0)
    assert lib.tl_attn(R.desc, a, None) == TL_EINVAL
    a = tlkv.attn_args(q, k, k, out, None, 40, 2, 8, hd, n_kv, 32)
    assert lib.tl_attn(R.desc, a, None) == TL_EINVAL   # window + n - 1 > ring
    sync(T)
    assert bool((out == 7.0).all())


# ---- depth, RoPE sweep, full-size batches, concurrent streams ---------------

@pytest.mark.parametrize("splits", [0, 1, 5])
def test_prefill_deep_chunk_vs_oracle(T, splits):
    """Config 4's last chunk depth: 64 query rows at pos 32256 over 32320 keys
    (505 key tiles) through a permuted slot table, heads reduced to 8 / 2 so
    the oracle stays fast; automatic key splits and forced 1 and 5 splits
    (the merge kernel)."""
    import tlkv
    n_head, n_kv, hd, pos, n = 8, 2, 128, 32256, 64
    cap = pos + n + 64
    rng = np.random.default_rng(32256 + splits)
    slots = rng.permutation(cap).astype(np.uint32)
    with tlkv.tuning(tlkv.TUNE_PREFILL_SPLITS, splits):
        out, o16, o32, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, n, 0, slots, seed=77)
    assert np.abs(out - o16).max() < TOL
    assert np.abs(out - o32).max() < TOL


ROPE_SWEEP = [
    # neox, theta, heads, head_dim, rope_dim: the configs' rotations
    (0, 5e5, 8, 128, 128),    # configs 1 / 4 (Llama NORM)
    (0, 5e5, 8, 64, 64),
    (1, 1e6, 4, 128, 128),    # configs 2 / 3 (Qwen NEOX), config 5 global
    (1, 1e4, 4, 256, 256),    # config 5 local
    (1, 1e6, 4, 256, 64),     # partial rotation
]


@pytest.mark.parametrize("pos", [0, 8192, 16384, 33791])
@pytest.mark.parametrize("rp", ROPE_SWEEP)
def test_rope_sweep_vs_oracle_and_reference(T, rp, pos):
    """tl_rope at the configs' theta / NORM-NEOX / rope_dim and positions up to
    config 4's last.  The angle pos * theta_i is formed in f32 on every side;
    theta_i = 1 / powf(base, e) may differ by an ulp between libms, which moves
    the angle by up to pos * theta_i * 2^-23: the tolerance scales with pos."""
    import tlkv
    neox, theta, heads, hd, rdim = rp
    rng = np.random.default_rng(pos + hd + rdim)
    rows_n = 16
    x = rng.standard_normal((rows_n, heads * hd)).astype(np.float32)
    dx = dev(T, x)
    tlkv.check(tlkv.lib().tl_rope(tlkv.ptr(dx), rows_n, heads * hd, heads, hd, rdim, pos,
                                  theta, neox, None))
    sync(T)
    got = host(dx)
    tol = 2e-6 + float(np.abs(x).max()) * (pos + rows_n) * 2.4e-7
    assert np.abs(got - O.rope(x, heads, hd, rdim, pos, theta, neox)).max() < tol
    # dims past rope_dim are copied unchanged
    if rdim < hd:
        xs, gs = x.reshape(rows_n, heads, hd), got.reshape(rows_n, heads, hd)
        assert np.array_equal(xs[..., rdim:], gs[..., rdim:])


def test_decode_batch_sessions_full_size(T):
    """Config 2 at full size: 8 sessions x 8193 visible keys (gqa 7, permuted
    slot tables), one batched launch with the fused append, against the
    oracle per session."""
    import tlkv
    n_head, n_kv, hd, n_seq, pos = 28, 4, 128, 8, 8192
    cap = 8704
    rng = np.random.default_rng(8192)
    seqs, refs, keep = [], [], []
    for s in range(n_seq):
        slots = rng.permutation(cap).astype(np.uint32)
        L = tlkv.Layer(cap, n_kv, hd)
        hk, hv = rows(rng, pos, n_kv * hd), rows(rng, pos, n_kv * hd)
        ds = dev(T, slots)
        tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hk)),
                                           tlkv.ptr(dev(T, hv)), n_kv * hd,
                                           tlkv.ptr(ds), 0, pos, None))
        C = O.Cache(cap, n_kv, hd)
        C.append(hk, hv, slots, 0, pos)
        q, k, v = rows(rng, 1, n_head * hd), rows(rng, 1, n_kv * hd), rows(rng, 1, n_kv * hd)
        dq, dk, dv = dev(T, q), dev(T, k), dev(T, v)
        out = T.zeros((1, n_head * hd), dtype=T.float32, device="cuda")
        keep += [L, ds, dq, dk, dv]
        seqs.append(tlkv.DecodeSeq(L.desc, ds.data_ptr(), pos, 0, dq.data_ptr(),
                                   dk.data_ptr(), dv.data_ptr(), out.data_ptr()))
        refs.append((out, O.attn(C, q, k, v, slots, pos, 1, n_head)))
    arr = (tlkv.DecodeSeq * n_seq)(*seqs)
    tlkv.check(tlkv.lib().tl_attn_decode_batch(arr, n_seq, n_head, 0, O.scale_of(hd), None))
    sync(T)
    for i, (out, ref) in enumerate(refs):
        assert np.abs(host(out) - ref).max() < TOL, f"session {i}"


def test_two_streams_interleaved_decode(T):
    """Two sessions on two streams (default priority) decode in turn without
    synchronising between launches: each stream has its own split partials and
    merge counters, so every output matches the oracle."""
    import tlkv
    n_head, n_kv, hd, pos0, steps = 32, 8, 128, 6000, 6
    cap = pos0 + steps
    streams = [T.cuda.Stream(), T.cuda.Stream()]
    sess = []
    for i in range(2):
        rng = np.random.default_rng(900 + i)
        slots = rng.permutation(cap).astype(np.uint32)
        L = tlkv.Layer(cap, n_kv, hd)
        hk, hv = rows(rng, pos0, n_kv * hd), rows(rng, pos0, n_kv * hd)
        ds = dev(T, slots)
        tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hk)),
                                           tlkv.ptr(dev(T, hv)), n_kv * hd, tlkv.ptr(ds),
                                           0, pos0, None))
        C = O.Cache(cap, n_kv, hd)
        C.append(hk, hv, slots, 0, pos0)
        qs = [rows(rng, 1, n_head * hd) for _ in range(steps)]
        ks = [rows(rng, 1, n_kv * hd) for _ in range(steps)]
        vs = [rows(rng, 1, n_kv * hd) for _ in range(steps)]
        outs = [T.zeros((1, n_head * hd), dtype=T.float32, device="cuda") for _ in range(steps)]
        sess.append(dict(L=L, ds=ds, C=C, slots=slots, q=qs, k=ks, v=vs, out=outs,
                         dq=[dev(T, x) for x in qs], dk=[dev(T, x) for x in ks],
                         dv=[dev(T, x) for x in vs]))
    T.cuda.synchronize()
    for t in range(steps):
        for i, S in enumerate(sess):
            a = tlkv.attn_args(S["dq"][t], S["dk"][t], S["dv"][t], S["out"][t], S["ds"],
                               pos0 + t, 1, n_head, hd, n_kv, 0, O.scale_of(hd))
            tlkv.check(tlkv.lib().tl_attn(S["L"].desc, a, streams[i].cuda_stream))
    sync(T)
    for i, S in enumerate(sess):
        for t in range(steps):
            ref = O.attn(S["C"], S["q"][t], S["k"][t], S["v"][t], S["slots"], pos0 + t, 1,
                         n_head)
            assert np.abs(host(S["out"][t]) - ref).max() < TOL, f"session {i} step {t}"


def test_two_host_threads_decode(T):
    """Two host threads, each driving its own session on its own stream
    (default priority) through decode steps at once: the launch path's
    process-wide caches (CU count, occupancy, per-stream workspaces) are
    shared by both, and every output matches the oracle."""
    import threading
    import tlkv
    n_head, n_kv, hd, pos0, steps = 28, 4, 128, 7000, 8
    cap = pos0 + steps
    sess = []
    for i in range(2):
        rng = np.random.default_rng(950 + i)
        slots = rng.permutation(cap).astype(np.uint32)
        L = tlkv.Layer(cap, n_kv, hd)
        hk, hv = rows(rng, pos0, n_kv * hd), rows(rng, pos0, n_kv * hd)
        ds = dev(T, slots)
        tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hk)),
                                           tlkv.ptr(dev(T, hv)), n_kv * hd, tlkv.ptr(ds),
                                           0, pos0, None))
        C = O.Cache(cap, n_kv, hd)
        C.append(hk, hv, slots, 0, pos0)
        qs = [rows(rng, 1, n_head * hd) for _ in range(steps)]
        ks = [rows(rng, 1, n_kv * hd) for _ in range(steps)]
        vs = [rows(rng, 1, n_kv * hd) for _ in range(steps)]
        sess.append(dict(L=L, ds=ds, C=C, slots=slots, q=qs, k=ks, v=vs,
                         out=[T.zeros((1, n_head * hd), dtype=T.float32, device="cuda")
                              for _ in range(steps)],
                         dq=[dev(T, x) for x in qs], dk=[dev(T, x) for x in ks],
                         dv=[dev(T, x) for x in vs], stream=T.cuda.Stream(), rc=[]))
    T.cuda.synchronize()
    start = threading.Barrier(2)

    def drive(S):
        start.wait()
        for t in range(steps):
            a = tlkv.attn_args(S["dq"][t], S["dk"][t], S["dv"][t], S["out"][t], S["ds"],
                               pos0 + t, 1, n_head, hd, n_kv, 0, O.scale_of(hd))
            S["rc"].append(tlkv.lib().tl_attn(S["L"].desc, a, S["stream"].cuda_stream))
        S["stream"].synchronize()

    th = [threading.Thread(target=drive, args=(S,)) for S in sess]
    for x in th:
        x.start()
    for x in th:
        x.join()
    sync(T)
    for i, S in enumerate(sess):
        assert S["rc"] == [0] * steps, f"session {i}: {S['rc']}"
        for t in range(steps):
            ref = O.attn(S["C"], S["q"][t], S["k"][t], S["v"][t], S["slots"], pos0 + t, 1,
                         n_head)
            assert np.abs(host(S["out"][t]) - ref).max() < TOL, f"session {i} step {t}"


@pytest.mark.parametrize("shape", [(32, 8, 128, 8192, 8000), (28, 4, 128, 8300, 8192)])
def test_decode_split_merge_fallback(T, shape):
    """The split merge's bounded waits, forced from the host: with no polls
    every split gives up its slice and the last split of each group to
    arrive merges all of them; with one poll some do and some do not.  The
    outputs equal the default run's bit for bit (every slice is merged by
    the same code from the same partials, whoever runs it)."""
    import tlkv
    n_head, n_kv, hd, cap, pos = shape
    outs = []
    for polls in (0, 1, 2):
        with tlkv.tuning(tlkv.TUNE_DECODE_MERGE_POLLS, polls):
            out, o16, _, _, _ = _run_attn(T, n_head, n_kv, hd, cap, pos, 1, 0, None, seed=pos)
        assert np.abs(out - o16).max() < TOL, polls
        outs.append(out)
    for o in outs[1:]:
        assert np.array_equal(outs[0].view(np.uint32), o.view(np.uint32))


@pytest.mark.parametrize("shape", [(32, 8, 128, 8200, 8000, 1), (32, 8, 128, 4200, 4000, 4)])
def test_decode_graph_replay(T, shape):
    """OP_ATTN captured in a HIP graph and replayed: each replay, with new q
    written eagerly between replays, equals the eager call on the same
    inputs bit for bit and the oracle within tolerance (the split merge's
    state carries nothing from one replay into the next)."""
    import tlkv
    n_head, n_kv, hd, cap, pos, n = shape
    rng = np.random.default_rng(pos + n)
    kd, qd = n_kv * hd, n_head * hd
    L = tlkv.Layer(cap, n_kv, hd)
    hk, hv = rows(rng, pos + n, kd), rows(rng, pos + n, kd)
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dev(T, hk)), tlkv.ptr(dev(T, hv)), kd,
                                       None, 0, pos + n, None))
    C = O.Cache(cap, n_kv, hd)
    C.append(hk, hv, None, 0, pos + n)
    dq = T.zeros((n, qd), dtype=T.float32, device="cuda")
    out = T.zeros((n, qd), dtype=T.float32, device="cuda")
    a = tlkv.attn_args(dq, None, None, out, None, pos, n, n_head, hd, n_kv, 0, O.scale_of(hd))
    s = T.cuda.Stream()
    sync(T)
    for _ in range(2):      # workspace of the capture stream allocated before capture
        tlkv.check(tlkv.lib().tl_attn_noappend(L.desc, a, s.cuda_stream))
    s.synchronize()
    g = T.cuda.CUDAGraph()
    with T.cuda.graph(g, stream=s):
        tlkv.check(tlkv.lib().tl_attn_noappend(L.desc, a, s.cuda_stream))
    for i in range(4):
        q = rows(rng, n, qd)
        dq.copy_(T.from_numpy(q))
        T.cuda.synchronize()
        g.replay()
        T.cuda.synchronize()
        got = host(out).copy()
        out.zero_()
        tlkv.check(tlkv.lib().tl_attn_noappend(L.desc, a, None))
        sync(T)
        assert np.array_equal(got.view(np.uint32), host(out).view(np.uint32)), f"replay {i}"
        ref = O.attn(C, q, hk[pos:], hv[pos:], None, pos, n, n_head)
        assert np.abs(got - ref).max() < TOL, f"replay {i}"
