"""Write the golden vectors under tests/golden/ from the COMPILED REFERENCE
(oracle/_ref/libtlref.so, built by `make -C oracle` from the reference's own
sources).  Run here, where the reference tree exists:

    python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  kvcache_trace.npz  kv_cache_match / kv_cache_append op streams over small
                     pools (heavy LRU eviction) and the reference's state after
                     every op: return value, req.len, req.shared_len,
                     req.active, pool.n_free, stats, clock, req.slots[0..len).
  op_attn.npz        cpu_graph_op(OP_ATTN) outputs over an f32 cache for tiny
                     GQA / window / slot-table cases (inputs included).
  rope.npz           cpu_graph_op(OP_ROPE_NORM / OP_ROPE_NEOX) outputs.
  kvcache_state.npz  kv_cache_checkpoint / kv_cache_restore over a Session
                     with one registered recurrent-state buffer: per request
                     the match, the restore result (position, flag) and the
                     state bytes after it, then chunked appends each followed
                     by a new state pattern and a checkpoint.
  q8_0_dequant.npz   gguf_dequant(GGUF_TYPE_Q8_0) over GGUF Q8_0 blocks with
                     random int8 values (all 256 codes) and binary16 scales
                     (normal, subnormal, zero, negative).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def kv_streams():
    """Op streams: (ctx, list of ops); op = ('m', tokens) or ('a', tokens, pos, n)."""
    out = []
    for seed, ctx, n_req, vocab in ((1, 48, 60, 40), (2, 96, 80, 500), (3, 32, 40, 8)):
        rng = np.random.default_rng(seed)
        prefixes = [rng.integers(0, vocab, size=rng.integers(3, ctx // 2)) for _ in range(4)]
        ops = []
        for _ in range(n_req):
            toks = np.concatenate([prefixes[rng.integers(len(prefixes))],
                                   rng.integers(0, vocab, size=rng.integers(1, ctx // 3))])
            toks = toks[:ctx].astype(np.uint32)
            ops.append(("m", toks))
            # resume rule of graph_kv_prepare, then chunked appends
            ops.append(("prep", toks))
        out.append((ctx, ops, seed))
    return out


def gen_kvcache():
    rec_ops, rec_tok, rec_state, rec_slots, rec_stream = [], [], [], [], []
    tok_off = 0
    slot_off = 0
    for si, (ctx, ops, seed) in enumerate(kv_streams()):
        rng = np.random.default_rng(seed + 100)
        kv = O.RefKv(ctx)
        for op in ops:
            toks = op[1]
            if op[0] == "m":
                calls = [("m", 0, 0)]
            else:
                m = last_match
                pos = 0 if m == 0 else (m if m < len(toks) else m - 1)
                calls = []
                while pos < len(toks):
                    n = int(min(rng.integers(1, 9), len(toks) - pos))
                    calls.append(("a", pos, n))
                    pos += n
            for kind, pos, n in calls:
                if kind == "m":
                    ret = kv.match(toks)
                    last_match = ret
                else:
                    ret = int(kv.append(toks, pos, n))
                r = kv.req()
                st = kv.stats()
                sl = kv.slots(r["len"])
                rec_ops.append([si, 0 if kind == "m" else 1, tok_off, len(toks), pos, n])
                rec_state.append([ret, r["len"], r["shared_len"], int(r["active"]), r["n_free"],
                                  st["hit_tokens"], st["computed_tokens"], st["evictions"],
                                  st["allocations"], st["clock"], slot_off, len(sl)])
                rec_slots.append(sl)
                slot_off += len(sl)
                if kind == "a" and not ret:
                    break
            rec_tok.append(toks)
            tok_off += len(toks)
        rec_stream.append(ctx)
    np.savez_compressed(os.path.join(HERE, "kvcache_trace.npz"),
                        ctx=np.array(rec_stream, dtype=np.uint32),
                        ops=np.array(rec_ops, dtype=np.int64),
                        tokens=np.concatenate(rec_tok).astype(np.uint32),
                        state=np.array(rec_state, dtype=np.uint64),
                        slots=np.concatenate(rec_slots).astype(np.uint32))


ATTN_CASES = [
    # n_head, n_kv, hd, cap, pos, n, window, permuted
    (4, 2, 64, 24, 0, 1, 0, False),
    (4, 2, 64, 24, 9, 1, 0, True),
    (8, 2, 64, 40, 5, 7, 0, True),
    (8, 2, 64, 40, 5, 7, 3, True),
    (8, 8, 128, 20, 11, 2, 0, False),
    (6, 2, 128, 33, 17, 4, 8, True),
    (4, 4, 256, 16, 6, 3, 0, True),
    (8, 4, 256, 16, 6, 3, 4, False),
]


def gen_attn():
    arrays = {}
    for ci, (nh, nkv, hd, cap, pos, n, win, perm) in enumerate(ATTN_CASES):
        rng = np.random.default_rng(1000 + ci)
        kc = rng.standard_normal((nkv, cap, hd), dtype=np.float32)
        vc = rng.standard_normal((nkv, cap, hd), dtype=np.float32)
        q = rng.standard_normal((n, nh * hd), dtype=np.float32)
        k = rng.standard_normal((n, nkv * hd), dtype=np.float32)
        v = rng.standard_normal((n, nkv * hd), dtype=np.float32)
        slots = (rng.permutation(cap) if perm else np.arange(cap)).astype(np.uint32)
        out = O.ref_attn(kc.copy(), vc.copy(), q, k, v, slots if perm else None, pos, n, nh, win)
        meta = np.array([nh, nkv, hd, cap, pos, n, win, int(perm)], dtype=np.int64)
        for name, a in (("meta", meta), ("kc", kc), ("vc", vc), ("q", q), ("k", k), ("v", v),
                        ("slots", slots), ("out", out)):
            arrays[f"c{ci}_{name}"] = a
    arrays["n_cases"] = np.array(len(ATTN_CASES))
    np.savez_compressed(os.path.join(HERE, "op_attn.npz"), **arrays)


def gen_rope():
    arrays = {}
    cases = [(0, 4, 64, 64, 0, 500000.0), (0, 8, 128, 128, 32000, 500000.0),
             (1, 4, 128, 128, 777, 1e6), (1, 2, 256, 256, 16000, 10000.0),
             (1, 2, 256, 64, 300, 1e6)]
    for ci, (neox, heads, hd, rd, pos, theta) in enumerate(cases):
        rng = np.random.default_rng(2000 + ci)
        x = rng.standard_normal((5, heads * hd), dtype=np.float32)
        y = O.ref_rope(x, heads, hd, rd, pos, theta, neox)
        arrays[f"c{ci}_meta"] = np.array([neox, heads, hd, rd, pos], dtype=np.int64)
        arrays[f"c{ci}_theta"] = np.array(theta, dtype=np.float32)
        arrays[f"c{ci}_x"] = x
        arrays[f"c{ci}_y"] = y
    arrays["n_cases"] = np.array(len(cases))
    np.savez_compressed(os.path.join(HERE, "rope.npz"), **arrays)


STATE_BYTES = 64


def state_pattern(req, pos):
    """the recurrent state a forward pass would leave at `pos` of request `req`"""
    return np.random.default_rng(req * 100003 + pos).integers(0, 256, STATE_BYTES).astype(np.uint8)


def kvstate_ops(seed=7, ctx=160, n_req=70, vocab=30, chunk=24):
    """requests sharing prefixes; ops per request: (req, tokens, n_chunks)"""
    rng = np.random.default_rng(seed)
    prefixes = [rng.integers(0, vocab, size=rng.integers(4, 60)) for _ in range(5)]
    reqs = []
    for r in range(n_req):
        toks = np.concatenate([prefixes[rng.integers(len(prefixes))],
                               rng.integers(0, vocab, size=rng.integers(1, 40))])
        reqs.append(toks[:ctx].astype(np.uint32))
    return ctx, chunk, reqs


def run_kvstate(api):
    """Drive one implementation (api: match, restore, append, checkpoint,
    set_state, get_state) through kvstate_ops; returns the per-request log
    [matched, restore_pos, restored, append_ok...] and the state bytes after
    each restore."""
    ctx, chunk, reqs = kvstate_ops()
    log, states = [], []
    for r, toks in enumerate(reqs):
        n = toks.size
        m = api.match(toks)
        api.set_state(np.zeros(STATE_BYTES, np.uint8))   # reset before restore
        pos, restored = api.restore(m, n)
        states.append(api.get_state())
        ok = []
        p = pos
        while p < n:
            c = min(chunk, n - p)
            ok.append(int(api.append(toks, p, c)))
            if not ok[-1]:
                break
            p += c
            api.set_state(state_pattern(r, p))
            ok.append(int(api.checkpoint(p)))
        log.append([m, pos, int(restored), len(ok), sum(ok)])
    return np.array(log, dtype=np.int64), np.array(states, dtype=np.uint8)


class RefStateApi:
    def __init__(self, ctx):
        self.R = O.ref()
        self.h = self.R.rh_kvs_create(ctx, STATE_BYTES)

    def match(self, toks):
        a = np.ascontiguousarray(toks, dtype=np.uint32)
        return int(self.R.rh_kv_match(self.h, a, a.size))

    def restore(self, m, n):
        flag = np.zeros(1, dtype=np.uint32)
        pos = int(self.R.rh_kvs_restore(self.h, m, n, flag))
        return pos, bool(flag[0])

    def append(self, toks, pos, n):
        a = np.ascontiguousarray(toks, dtype=np.uint32)
        return bool(self.R.rh_kv_append(self.h, a, pos, n))

    def checkpoint(self, pos):
        return bool(self.R.rh_kvs_checkpoint(self.h, pos))

    def set_state(self, b):
        b = np.ascontiguousarray(b, dtype=np.uint8)
        self.R.rh_kvs_set_state(self.h, b.ctypes.data)

    def get_state(self):
        out = np.zeros(STATE_BYTES, dtype=np.uint8)
        self.R.rh_kvs_get_state(self.h, out.ctypes.data)
        return out


def gen_kvstate():
    ctx, _, _ = kvstate_ops()
    api = RefStateApi(ctx)
    assert int(api.R.rh_kvs_cap_snaps(api.h)) == 16
    log, states = run_kvstate(api)
    api.R.rh_kvs_destroy(api.h)
    np.savez_compressed(os.path.join(HERE, "kvcache_state.npz"), log=log, states=states)


def gen_q8():
    rng = np.random.default_rng(3000)
    nblk = 96
    q = rng.integers(-128, 128, size=(nblk, 32)).astype(np.int8)
    q[0] = np.arange(-128, -96, dtype=np.int8)       # every code appears
    q[1:8] = np.arange(-96, 128, dtype=np.int16).reshape(7, 32).astype(np.int8)
    d = O.f16_bits(rng.uniform(1e-3, 2.0, size=nblk).astype(np.float32))
    d[8:12] = [0x0000, 0x8000, 0x0001, 0x03ff]       # zeros and subnormals
    d[12:16] = O.f16_bits(np.array([-0.5, 65504.0, 6.1035e-05, 1.0], dtype=np.float32))
    blocks = np.zeros((nblk, 34), dtype=np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    blocks[:, 2:] = q.view(np.uint8)
    out = O.ref_dequant_q8_0(blocks)
    np.savez_compressed(os.path.join(HERE, "q8_0_dequant.npz"), q=q, d=d, out=out)


if __name__ == "__main__":
    if not O.ref_available():
        O.build()
    if not O.ref_available():
        sys.exit("the compiled reference (oracle/_ref) is not available")
    gen_kvcache()
    gen_attn()
    gen_rope()
    gen_q8()
    gen_kvstate()
    print("golden vectors written to", HERE)
