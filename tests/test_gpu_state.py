"""Device-side recurrent-state snapshots (the reference's graph_state_save /
load + kv_cache_checkpoint / restore, src/graph.c:368-408, 1423-1460,
src/kvcache.c:272-321, with device-to-device copies).

- tl_state_copy: save / zero / load round trips are bit-exact for segments
  of any size and alignment, more segments than one launch takes, and
  empty segments;
- tl_session: with registered device state, kv_prepare follows
  graph_kv_prepare's stateful rule — a continuation keeps the state, a new
  request zeroes it and restores the deepest snapshot — with the resume
  positions of the host prefix cache (pinned against the compiled reference
  in tests/test_kvcache_state.py) and the snapshot bytes restored exactly.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import tlkv
    tlkv.check(tlkv.lib().tl_init(0))
    return torch


def _segs(tensors):
    import tlkv
    return (tlkv.StateSeg * len(tensors))(
        *[tlkv.StateSeg(t.data_ptr(), t.numel() * t.element_size()) for t in tensors])


def test_state_copy_roundtrip(T):
    import tlkv
    rng = np.random.default_rng(1)
    sizes = [0, 1, 15, 16, 17, 4096, 333, 64, 100000, 7] + list(rng.integers(1, 300, size=70))
    pool = T.from_numpy(rng.integers(0, 256, size=sum(sizes) + 4 * len(sizes) + 64,
                                     dtype=np.uint8)).cuda()
    tensors, off = [], 0
    for i, n in enumerate(sizes):
        off += (i % 3)                           # odd start offsets: unaligned segments
        tensors.append(pool[off:off + n])
        off += n
    orig = [t.clone() for t in tensors]
    total = sum(sizes)
    snap = T.zeros(total + 1, dtype=T.uint8, device="cuda")[1:]   # unaligned snapshot too
    lib = tlkv.lib()
    segs = _segs(tensors)
    tlkv.check(lib.tl_state_copy(segs, len(tensors), tlkv.ptr(snap), tlkv.TL_STATE_SAVE, None))
    T.cuda.synchronize()
    assert T.equal(snap, T.cat(orig))
    tlkv.check(lib.tl_state_copy(segs, len(tensors), None, tlkv.TL_STATE_ZERO, None))
    T.cuda.synchronize()
    assert all(int(t.sum()) == 0 for t in tensors if t.numel())
    tlkv.check(lib.tl_state_copy(segs, len(tensors), tlkv.ptr(snap), tlkv.TL_STATE_LOAD, None))
    T.cuda.synchronize()
    assert all(T.equal(a, b) for a, b in zip(tensors, orig))


def test_state_copy_aligned_fast_path(T):
    import tlkv
    x = [T.randn(n, device="cuda") for n in (1 << 16, 257, 4)]
    snap = T.empty(sum(t.numel() for t in x), device="cuda")
    tlkv.check(tlkv.lib().tl_state_copy(_segs(x), 3, tlkv.ptr(snap), tlkv.TL_STATE_SAVE, None))
    T.cuda.synchronize()
    assert T.equal(snap, T.cat(x))


def test_state_copy_rejects_bad_arguments(T):
    import tlkv
    segs = (tlkv.StateSeg * 1)(tlkv.StateSeg(None, 16))
    assert tlkv.lib().tl_state_copy(segs, 1, None, tlkv.TL_STATE_ZERO, None) != 0
    t = T.zeros(16, dtype=T.uint8, device="cuda")
    assert tlkv.lib().tl_state_copy(_segs([t]), 1, None, tlkv.TL_STATE_SAVE, None) != 0
    assert tlkv.lib().tl_state_copy(_segs([t]), 1, tlkv.ptr(t), 7, None) != 0


def _pattern(T, shape_bytes, key):
    g = np.random.default_rng(key).integers(0, 256, size=shape_bytes, dtype=np.uint8)
    return T.from_numpy(g).cuda()


def test_session_device_snapshots(T):
    import tlkv
    n_layer, n_head, n_kv, hd, ctx, ub = 2, 8, 2, 64, 256, 32
    sess = tlkv.Session(n_layer, n_head, n_kv, hd, ctx, ub)
    sizes = [1000, 37, 4096]
    state = [T.zeros(n, dtype=T.uint8, device="cuda") for n in sizes]
    sess.set_state(state)
    kd = n_kv * hd

    def set_state(key):
        for i, t in enumerate(state):
            t.copy_(_pattern(T, sizes[i], key * 10 + i))

    def state_is(key):
        T.cuda.synchronize()
        return all(T.equal(t, _pattern(T, sizes[i], key * 10 + i)) for i, t in enumerate(state))

    def run(tokens, start, req):
        """append tokens[start:] chunk by chunk; after each chunk the state a
        forward pass would leave, then a checkpoint (graph_kv_checkpoint)"""
        p = start
        while p < tokens.size:
            c = min(ub, tokens.size - p)
            k = [T.randn((c, kd), device="cuda") for _ in range(n_layer)]
            v = [T.randn((c, kd), device="cuda") for _ in range(n_layer)]
            sess.append(tokens[p:p + c], k, v, kd)
            p += c
            set_state(req * 1000 + p)
            sess.checkpoint()
        assert sess.pos == tokens.size

    a = np.arange(100, dtype=np.uint32)
    set_state(7)
    # a fresh session's history (0 tokens) is a prefix of any prompt: a
    # continuation, the state is kept (src/graph.c:1439-1443)
    assert sess.kv_prepare(a) == (0, 0)
    assert state_is(7)
    run(a, 0, 1)                                          # snapshots at 32, 64, 96, 100
    # a new request sharing 60 tokens: restore the snapshot at 32
    b = np.concatenate([a[:60], np.arange(500, 520, dtype=np.uint32)])
    m, r = sess.kv_prepare(b)
    assert (m, r) == (60, 32)
    assert state_is(1 * 1000 + 32)
    # a prompt with no cached prefix: reset (zeroed), resume 0
    m, r = sess.kv_prepare(np.arange(700, 720, dtype=np.uint32))
    assert (m, r) == (0, 0)
    T.cuda.synchronize()
    assert all(int(t.sum()) == 0 for t in state)
    m, r = sess.kv_prepare(b)
    assert (m, r) == (60, 32)
    assert state_is(1 * 1000 + 32)
    run(b, r, 2)                                          # snapshots at 64, 80 of b
    # continuation: the history is a prefix of the prompt -> keep the state
    set_state(99)
    c = np.concatenate([b, np.arange(900, 905, dtype=np.uint32)])
    m, r = sess.kv_prepare(c)
    assert (m, r) == (b.size, b.size)
    assert state_is(99)
    # the first request again (n = 100): deepest snapshot below n is 96
    m, r = sess.kv_prepare(a)
    assert (m, r) == (100, 96)
    assert state_is(1 * 1000 + 96)
    # stateless again: the stateless resume rule (matched - 1 at a full hit)
    sess.set_state([])
    assert sess.kv_prepare(a) == (100, 99)


def test_session_snapshot_positions_match_host_cache(T):
    """the session's restore positions equal the host prefix cache's over the
    same op stream (that cache is pinned against the compiled reference)"""
    import tlkv
    n_layer, n_kv, hd, ctx, ub = 1, 1, 64, 96, 16
    sess = tlkv.Session(n_layer, 4, n_kv, hd, ctx, ub)
    st = [T.zeros(64, dtype=T.uint8, device="cuda")]
    sess.set_state(st)
    host = tlkv.KvCache(ctx)
    host.set_host_state(64)
    rng = np.random.default_rng(3)
    prefixes = [rng.integers(0, 20, size=rng.integers(5, 40)).astype(np.uint32) for _ in range(3)]
    host_pos = 0
    for r in range(25):
        toks = np.concatenate([prefixes[r % 3], rng.integers(0, 20, size=rng.integers(1, 30))])
        toks = toks[:ctx].astype(np.uint32)
        n = toks.size
        m = host.match(toks)
        if m == host_pos and n > m:          # continuation (graph.c:1439-1443)
            pos = m
        else:
            pos, _ = host.restore(m, n)
        sm, sr = sess.kv_prepare(toks)
        assert sm == m
        assert sr == pos, (r, m, n)
        p = pos
        while p < n:
            c = min(ub, n - p)
            assert host.append(toks, p, c)
            kk = [T.randn((c, n_kv * hd), device="cuda")]
            sess.append(toks[p:p + c], kk, kk, n_kv * hd)
            p += c
            assert host.checkpoint(p)
            sess.checkpoint()
        host_pos = n
