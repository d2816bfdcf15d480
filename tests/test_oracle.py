"""Pins the CPU oracle (oracle/oracle.c) before it is used as the checker.

- binary16 conversion: numpy's IEEE round-to-nearest-even on 1M+ values and
  hand-picked special values (ties, subnormals, overflow, signed zeros, NaN);
- op_attn restatement: the compiled reference's cpu_graph_op(OP_ATTN) outputs
  (tests/golden/op_attn.npz, f32 cache) and live when oracle/_ref is built;
  closed forms (one key, identical keys, window >= keys) and a float64 brute
  force on tiny inputs;
- RoPE: the compiled reference's outputs within tolerance (the reference
  builds with -ffast-math; transcendental results are not bit-pinned).
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(1 << 20).astype(np.float32) * np.float32(100),
        rng.standard_normal(1 << 16).astype(np.float32) * np.float32(1e-5),
        rng.standard_normal(1 << 14).astype(np.float32) * np.float32(7e4),
        np.frombuffer(rng.integers(0, 2**32, size=1 << 16, dtype=np.uint64)
                      .astype(np.uint32).tobytes(), np.float32),
    ])
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_bits(x), ref)


@pytest.mark.parametrize("val,bits", [
    (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (65504.0, 0x7BFF),
    (65519.996, 0x7BFF), (65520.0, 0x7C00), (np.inf, 0x7C00), (-np.inf, 0xFC00),
    (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000), (1.5 * 2.0 ** -25, 0x0001),
    (2.0 ** -14, 0x0400), (1.0 + 2.0 ** -11, 0x3C00), (1.0 + 3 * 2.0 ** -11, 0x3C02),
    (6.097555e-05, 0x03FF),
])
def test_f16_special_values(val, bits):
    assert int(O.f16_bits(np.array([val], np.float32))[0]) == bits


def test_f16_nan_rule():
    """NaN -> quiet NaN keeping the sign and the top 9 payload bits."""
    for u, h in ((0x7FC00000, 0x7E00), (0x7F800001, 0x7E00), (0x7F812345, 0x7E09),
                 (0xFFC00001, 0xFE00), (0x7FFFFFFF, 0x7FFF)):
        x = np.frombuffer(np.uint32(u).tobytes(), np.float32)
        assert int(O.f16_bits(x)[0]) == h, hex(u)


def test_f16_roundtrip_exact_on_f16_values():
    h = np.arange(0, 1 << 16, dtype=np.uint16)
    f = O.f16_to_f32(h)
    finite = (h & 0x7C00) != 0x7C00
    assert np.array_equal(O.f16_bits(f)[finite], h[finite])
    assert np.array_equal(f[finite], h[finite].view(np.float16).astype(np.float32))


def _golden_attn():
    g = np.load(os.path.join(GOLD, "op_attn.npz"))
    for ci in range(int(g["n_cases"])):
        yield {k: g[f"c{ci}_{k}"] for k in ("meta", "kc", "vc", "q", "k", "v", "slots", "out")}


@pytest.mark.parametrize("case", list(range(8)))
def test_oracle_attn_vs_reference_golden(case):
    c = list(_golden_attn())[case]
    nh, nkv, hd, cap, pos, n, win, perm = (int(x) for x in c["meta"])
    C = O.Cache(cap, nkv, hd, f16=False)
    C.k[:] = c["kc"]
    C.v[:] = c["vc"]
    out = O.attn(C, c["q"], c["k"], c["v"], c["slots"] if perm else None, pos, n, nh,
                 window=win)
    # same f32 math; the reference's -ffast-math / SIMD summation order differs
    assert np.abs(out - c["out"]).max() < 2e-6


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
@pytest.mark.parametrize("nh,nkv,hd,pos,n,win", [(32, 8, 64, 300, 1, 0), (28, 4, 128, 200, 3, 0),
                                                 (8, 4, 256, 150, 2, 64), (16, 16, 64, 90, 5, 7)])
def test_oracle_attn_vs_reference_live(nh, nkv, hd, pos, n, win):
    rng = np.random.default_rng(pos + n)
    cap = pos + n + 5
    kc = rng.standard_normal((nkv, cap, hd), dtype=np.float32)
    vc = rng.standard_normal((nkv, cap, hd), dtype=np.float32)
    q = rng.standard_normal((n, nh * hd), dtype=np.float32)
    k = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    slots = rng.permutation(cap).astype(np.uint32)
    ref = O.ref_attn(kc.copy(), vc.copy(), q, k, v, slots, pos, n, nh, win)
    C = O.Cache(cap, nkv, hd, f16=False)
    C.k[:], C.v[:] = kc, vc
    out = O.attn(C, q, k, v, slots, pos, n, nh, window=win)
    assert np.abs(out - ref).max() < 2e-6


def _brute(kc, vc, q, slots, pos, n, nh, win):
    """float64 attention straight from the definition (cpu_op.c:1011-1062)."""
    nkv, cap, hd = kc.shape
    gqa = nh // nkv
    out = np.zeros((n, nh * hd))
    for qi in range(n):
        nk = pos + qi + 1
        start = nk - win if (win and nk > win) else 0
        rows = [slots[t] for t in range(start, nk)]
        for h in range(nh):
            K = kc[h // gqa][rows].astype(np.float64)
            V = vc[h // gqa][rows].astype(np.float64)
            s = K @ q[qi, h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[qi, h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


@pytest.mark.parametrize("f16", [False, True])
def test_oracle_attn_vs_float64_brute_force(f16):
    rng = np.random.default_rng(5)
    nh, nkv, hd, cap, pos, n = 6, 2, 64, 40, 20, 4
    q = rng.standard_normal((n, nh * hd), dtype=np.float32)
    k = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    hk = rng.standard_normal((pos, nkv * hd), dtype=np.float32)
    hv = rng.standard_normal((pos, nkv * hd), dtype=np.float32)
    slots = rng.permutation(cap).astype(np.uint32)
    for win in (0, 5):
        C = O.Cache(cap, nkv, hd, f16=f16)
        C.append(hk, hv, slots, 0, pos)
        out = O.attn(C, q, k, v, slots, pos, n, nh, window=win)
        kc = O.f16_to_f32(C.k) if f16 else C.k
        vc = O.f16_to_f32(C.v) if f16 else C.v
        ref = _brute(kc, vc, q, slots, pos, n, nh, win)
        assert np.abs(out - ref).max() < 1e-5


def test_oracle_attn_closed_forms():
    rng = np.random.default_rng(6)
    nh, nkv, hd, cap = 4, 2, 64, 16
    q = rng.standard_normal((1, nh * hd), dtype=np.float32)
    k = rng.standard_normal((1, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((1, nkv * hd), dtype=np.float32)
    # one visible key -> output is its V row, whatever q is
    C = O.Cache(cap, nkv, hd, f16=False)
    out = O.attn(C, q, k, v, None, 0, 1, nh)
    assert np.array_equal(out.reshape(nh, hd), np.repeat(v.reshape(nkv, hd), 2, axis=0))
    # window 1 -> only the current key, at any position
    C = O.Cache(cap, nkv, hd, f16=False)
    C.k[:] = rng.standard_normal(C.k.shape, dtype=np.float32)
    C.v[:] = rng.standard_normal(C.v.shape, dtype=np.float32)
    out = O.attn(C, q, k, v, None, 9, 1, nh, window=1)
    assert np.array_equal(out.reshape(nh, hd), np.repeat(v.reshape(nkv, hd), 2, axis=0))
    # window >= visible keys -> identical to full attention
    C1 = O.Cache(cap, nkv, hd, f16=False)
    C1.k[:], C1.v[:] = C.k, C.v
    a = O.attn(C, q, k, v, None, 9, 1, nh, window=10)
    b = O.attn(C1, q, k, v, None, 9, 1, nh, window=0)
    assert np.array_equal(a, b)
    # identical keys -> uniform weights -> mean of V
    C = O.Cache(cap, nkv, hd, f16=False)
    krow = rng.standard_normal((1, nkv * hd), dtype=np.float32)
    hv = rng.standard_normal((7, nkv * hd), dtype=np.float32)
    C.append(np.repeat(krow, 7, axis=0), hv, None, 0, 7)
    out = O.attn(C, q, krow, v, None, 7, 1, nh)
    mean = np.concatenate([hv, v]).astype(np.float64).mean(axis=0).reshape(nkv, hd)
    assert np.abs(out.reshape(nh, hd) - np.repeat(mean, 2, axis=0)).max() < 1e-6


def test_oracle_ring_equals_masked_full_cache():
    rng = np.random.default_rng(7)
    nh, nkv, hd, win, pos, n = 4, 2, 64, 6, 30, 3
    ring = win + n - 1
    q = rng.standard_normal((n, nh * hd), dtype=np.float32)
    k = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    hk = rng.standard_normal((pos, nkv * hd), dtype=np.float32)
    hv = rng.standard_normal((pos, nkv * hd), dtype=np.float32)
    full = O.Cache(pos + n, nkv, hd, f16=True)
    full.append(hk, hv, None, 0, pos)
    rc = O.Cache(ring, nkv, hd, f16=True)
    for p in range(pos):
        rc.append(hk[p:p + 1], hv[p:p + 1], None, p % ring, 1)
    a = O.attn(full, q, k, v, None, pos, n, nh, window=win)
    b = O.attn(rc, q, k, v, None, pos, n, nh, window=win, ring=ring)
    assert np.array_equal(a, b)


def test_oracle_append_layout():
    """Head-major rows at the slot, as cpu_op.c:995-1008 writes them."""
    rng = np.random.default_rng(8)
    nkv, hd, cap = 3, 64, 10
    k = rng.standard_normal((2, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((2, nkv * hd), dtype=np.float32)
    slots = np.array([0, 0, 0, 7, 2, 0, 0, 0, 0, 0], np.uint32)
    C = O.Cache(cap, nkv, hd, f16=True)
    assert C.append(k, v, slots, 3, 2) == 0
    for i, s in enumerate((7, 2)):
        for h in range(nkv):
            assert np.array_equal(C.k[h, s], O.f16_bits(k[i, h * hd:(h + 1) * hd]))
            assert np.array_equal(C.v[h, s], O.f16_bits(v[i, h * hd:(h + 1) * hd]))
    assert C.append(k, v, np.full(10, 99, np.uint32), 0, 1) == -1   # slot >= cap


def test_oracle_rope_vs_reference_golden():
    g = np.load(os.path.join(GOLD, "rope.npz"))
    for ci in range(int(g["n_cases"])):
        neox, heads, hd, rd, pos = (int(x) for x in g[f"c{ci}_meta"])
        theta = float(g[f"c{ci}_theta"])
        y = O.rope(g[f"c{ci}_x"], heads, hd, rd, pos, theta, neox)
        # the angle pos*theta_i carries ~pos * 2^-24 rad of f32 rounding; the
        # reference's -ffast-math sincos adds a few ulp
        tol = 5e-4 + pos * 1e-6
        assert np.abs(y - g[f"c{ci}_y"]).max() < tol, ci
