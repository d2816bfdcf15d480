"""The executor shim (tinyllama.c_amd/integration/hip_graph_op.c): the
reference's own OpCtx / GraphPlan / KvCache / KvRadixCache structs, built as
graph_execute builds them for OP_ATTN, go through hip_graph_op to libtlkv;
the outputs must match the compiled reference's cpu_graph_op(OP_ATTN) over
an f32 cache holding the same rows (within 2e-3), the f16 rows must land at
the radix's slots bit for bit, and AttnKvCache.n must be pos + n, as op_attn
leaves it (src/backend/cpu/cpu_op.c:995-1009).  Needs oracle/_ref (built
where the reference tree exists; it travels with the repository)."""
import ctypes

import numpy as np
import pytest

import oracle as O

# checked by file, not loaded: loading libtlkv before torch initialises its
# HIP runtime would put two runtimes in the process
pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not (O.shim_available() and O.ref_available()),
                                 reason="executor shim / compiled reference not built")]


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


@pytest.mark.parametrize("nh,nkv,hd,cap,pos,n,win,radix", [
    (32, 8, 128, 2048, 1500, 1, 0, True),     # decode through the slot table
    (32, 8, 128, 2048, 1500, 1, 0, False),    # contiguous (no radix)
    (8, 4, 256, 1600, 1200, 3, 512, True),    # windowed multi-row decode
    (28, 4, 128, 1024, 300, 64, 0, True),     # prefill chunk (MFMA kernel), gqa 7
])
def test_shim_matches_reference_op_attn(T, nh, nkv, hd, cap, pos, n, win, radix):
    import tlkv
    rng = np.random.default_rng(pos + n)
    kd, qd = nkv * hd, nh * hd
    hk = rng.standard_normal((pos, kd)).astype(np.float32)
    hv = rng.standard_normal((pos, kd)).astype(np.float32)
    q = rng.standard_normal((n, qd)).astype(np.float32)
    k = rng.standard_normal((n, kd)).astype(np.float32)
    v = rng.standard_normal((n, kd)).astype(np.float32)
    slots = rng.permutation(cap).astype(np.uint32) if radix else None
    # the history already cached (earlier OP_ATTN calls)
    L = tlkv.Layer(cap, nkv, hd)
    d_slots = T.from_numpy(slots.astype(np.int64)).to(T.int32).cuda() if radix else None
    dhk, dhv = T.from_numpy(hk).cuda(), T.from_numpy(hv).cuda()
    tlkv.check(tlkv.lib().tl_kv_append(L.desc, tlkv.ptr(dhk), tlkv.ptr(dhv), kd,
                                       tlkv.ptr(d_slots), 0, pos, None))
    dq, dk, dv = T.from_numpy(q).cuda(), T.from_numpy(k).cuda(), T.from_numpy(v).cuda()
    out = T.zeros((n, qd), dtype=T.float32, device="cuda")
    n_after = np.zeros(1, dtype=np.uint32)
    hs = None if slots is None else np.ascontiguousarray(slots)
    rc = O.shim().rh_attn_shim(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(),
                               L.k.data_ptr(), L.v.data_ptr(), cap,
                               None if hs is None else hs.ctypes.data,
                               None if d_slots is None else d_slots.data_ptr(),
                               pos, n, nh, nkv, hd, win, n_after.ctypes.data)
    T.cuda.synchronize()
    assert rc == 0
    assert int(n_after[0]) == pos + n
    # the reference: cpu_graph_op(OP_ATTN) over an f32 cache with the same rows
    kc = np.zeros((nkv, cap, hd), np.float32)
    vc = np.zeros_like(kc)
    for i in range(pos):
        s = slots[i] if radix else i
        kc[:, s] = hk[i].reshape(nkv, hd)
        vc[:, s] = hv[i].reshape(nkv, hd)
    ref = O.ref_attn(kc, vc, q, k, v, slots, pos, n, nh, window=win)
    assert np.abs(out.cpu().numpy() - ref).max() < 2e-3
    # the batch rows were written through at their slots, f16 RNE
    rows = np.concatenate([hk, k])
    sl = slots[:pos + n] if radix else np.arange(pos + n, dtype=np.uint32)
    got = L.k.cpu().numpy().view(np.uint16)[:, sl[pos:]].transpose(1, 0, 2).reshape(n, -1)
    assert np.array_equal(got, O.f16_bits(rows[pos:]))
