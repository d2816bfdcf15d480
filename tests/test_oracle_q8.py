"""Pins the Q8_0 part of the CPU oracle before it is used as the checker.

- dequantization: the compiled reference's gguf_dequant(GGUF_TYPE_Q8_0)
  (src/quants.c:368-373, 640-652) through tests/golden/q8_0_dequant.npz, and
  live when oracle/_ref is built;
- quantization (src/backend/gpu/gpu.cu:1077-1086): constructed blocks whose
  answers are fixed by hand -- ties to even (rint, not roundf), the amax
  element maps to +-127, zero blocks give d = 0 and q = 0 -- and the error
  bound |x - q d| <= d/2 + 127 |d - f16(d)| on random blocks;
- op_attn over the Q8_0 cache: bit-identical to or_attn (pinned against the
  reference) over an f32 cache holding the dequantized rows, and within
  tolerance of the compiled reference's OP_ATTN given those rows.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _blocks(q, d):
    nblk = q.shape[0]
    b = np.zeros((nblk, 34), dtype=np.uint8)
    b[:, 0:2] = np.ascontiguousarray(d, dtype=np.uint16).view(np.uint8).reshape(nblk, 2)
    b[:, 2:] = np.ascontiguousarray(q, dtype=np.int8).view(np.uint8)
    return b


def test_q8_dequant_vs_reference_golden():
    g = np.load(os.path.join(GOLD, "q8_0_dequant.npz"))
    out = O.q8_dequant(g["q"], g["d"])
    assert np.array_equal(out.reshape(-1).view(np.uint32), g["out"].view(np.uint32))


@pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")
def test_q8_dequant_vs_reference_live():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((64, 32)) * rng.uniform(1e-3, 50, size=(64, 1))).astype(np.float32)
    q, d = O.q8_quantize(x)
    ref = O.ref_dequant_q8_0(_blocks(q, d.reshape(-1)))
    assert np.array_equal(O.q8_dequant(q, d).reshape(-1), ref)


def test_q8_quantize_ties_to_even():
    # amax 127 -> d = 1, id = 1: q = rint(x); roundf would give 3, -3, 1, 5
    x = np.zeros(32, dtype=np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, 4.5, 1.5, -0.5, 3.49]
    q, d = O.q8_quantize(x)
    assert d[0] == 0x3C00
    assert list(q[:8]) == [127, 2, -2, 0, 4, 2, 0, 3]
    assert not q[8:].any()


def test_q8_quantize_amax_and_zero_block():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((200, 32)).astype(np.float32)
    x[5] = 0.0
    x[6] = -0.0
    q, d = O.q8_quantize(x)
    assert not q[5].any() and d[5] == 0 and not q[6].any() and d[6] == 0
    for i in (0, 1, 2, 50, 199):
        j = int(np.argmax(np.abs(x[i])))
        assert q[i, j] == (127 if x[i, j] > 0 else -127)
    assert q.min() >= -127 and q.max() <= 127
    # the stored scale is binary16(amax / 127) (numpy's RNE float16 cast)
    amax = np.abs(x).max(axis=1)
    want = (amax / np.float32(127.0)).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(d.reshape(-1), want)


def test_q8_quantize_error_bound():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((500, 32)) * rng.uniform(1e-4, 1e3, size=(500, 1))).astype(np.float32)
    q, d = O.q8_quantize(x)
    deq = O.q8_dequant(q, d).astype(np.float64)
    d32 = np.abs(x).max(axis=1).astype(np.float64) / 127.0
    d16 = O.f16_to_f32(d.reshape(-1)).astype(np.float64)
    bound = d32 / 2 * (1 + 1e-5) + 127 * np.abs(d16 - d32)
    assert (np.abs(deq - x) <= bound[:, None] + 1e-30).all()


@pytest.mark.parametrize("nh,nkv,hd,pos,n,win,ring,use_slots", [
    (4, 2, 64, 37, 1, 0, 0, True),
    (8, 2, 128, 70, 5, 0, 0, True),
    (4, 4, 128, 90, 3, 32, 40, False),
    (2, 1, 256, 20, 17, 0, 0, False),
])
def test_oracle_attn_q8_equals_attn_on_dequantized(nh, nkv, hd, pos, n, win, ring, use_slots):
    rng = np.random.default_rng(nh * 1000 + pos)
    cap = 128
    total = pos + n
    slots = rng.permutation(cap)[:total].astype(np.uint32) if use_slots else None
    hk = rng.standard_normal((total, nkv * hd)).astype(np.float32)
    hv = rng.standard_normal((total, nkv * hd)).astype(np.float32)
    q = rng.standard_normal((n, nh * hd)).astype(np.float32)
    C8 = O.CacheQ8(cap, nkv, hd, ring)
    assert C8.append(hk[:pos], hv[:pos], slots, 0, pos) == 0
    out8 = C8.attn(q, hk[pos:], hv[pos:], slots, pos, n, nh, window=win)
    # the same keys, dequantized, through the f32-cache oracle
    dk = O.q8_dequant(*O.q8_quantize(hk.reshape(total, nkv, hd))).reshape(total, -1)
    dv = O.q8_dequant(*O.q8_quantize(hv.reshape(total, nkv, hd))).reshape(total, -1)
    C = O.Cache(cap, nkv, hd, f16=False)
    if ring:
        for i in range(pos):
            assert C.append(dk[i:i + 1], dv[i:i + 1], None, i % ring, 1) == 0
    else:
        assert C.append(dk[:pos], dv[:pos], slots, 0, pos) == 0
    out = O.attn(C, q, dk[pos:], dv[pos:], slots, pos, n, nh, window=win, ring=ring)
    assert np.array_equal(out8, out)
    if O.ref_available() and not ring:
        kc = np.zeros((nkv, cap, hd), dtype=np.float32)
        vc = np.zeros_like(kc)
        for i in range(pos):
            s = slots[i] if slots is not None else i
            kc[:, s] = dk[i].reshape(nkv, hd)
            vc[:, s] = dv[i].reshape(nkv, hd)
        ref = O.ref_attn(kc, vc, q, dk[pos:], dv[pos:], slots, pos, n, nh, window=win)
        np.testing.assert_allclose(out8, ref, rtol=1e-5, atol=1e-5)
