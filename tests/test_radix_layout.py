"""libtlkv's KvRadixCache read by code compiled against the reference's header.

op_attn reads radix->req.slots / req.len straight from the struct
(src/backend/cpu/cpu_op.c:988-993), with the layout of src/kvcache.h:50-57.
These tests hand a prefix cache made by libtlkv's kv_cache_create/match/append
to the compiled reference's cpu_graph_op(OP_ATTN) and check:
- the field offsets of TlKvRadixHead (include/tl_kvcache.h) equal the
  reference's (the library asserts its own struct against TlKvRadixHead);
- over multi-chunk request streams with prefix hits and LRU evictions, the
  reference's op_attn over libtlkv's cache gives the same outputs, bit for bit,
  as over the reference's own kv_cache_* driven by the same stream, and agrees
  with the oracle restatement.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
import tlkv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="compiled reference not built")

_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "tl_kvcache.h"
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n",
        offsetof(TlKvRadixHead, tree), offsetof(TlKvRadixHead, pool),
        offsetof(TlKvRadixHead, pool.n_free), offsetof(TlKvRadixHead, pool.free_stack),
        offsetof(TlKvRadixHead, meta), offsetof(TlKvRadixHead, req),
        offsetof(TlKvRadixHead, req.len), offsetof(TlKvRadixHead, req.shared_len),
        offsetof(TlKvRadixHead, req.active), offsetof(TlKvRadixHead, kv),
        offsetof(TlKvRadixHead, n_layer), offsetof(TlKvRadixHead, ctx_size),
        offsetof(TlKvRadixHead, enabled), sizeof(KvSlotMeta),
        offsetof(KvSlotMeta, last_used), offsetof(KvSlotMeta, in_tree));
    return 0;
}
"""


def test_head_offsets_equal_reference(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    ours = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                           text=True).stdout.split()]
    assert ours == O.ref_radix_layout()


def _run_stream(seed, ctx, n_kv, hd, n_head, ub, n_req, vocab):
    rng = np.random.default_rng(seed)
    ours, theirs = tlkv.KvCache(ctx), O.RefKv(ctx)
    kc_a = np.zeros((n_kv, ctx, hd), np.float32)
    vc_a = np.zeros_like(kc_a)
    kc_b, vc_b = kc_a.copy(), vc_a.copy()
    oc = O.Cache(ctx, n_kv, hd, f16=False)
    prefixes = [rng.integers(0, vocab, size=rng.integers(8, ctx // 2)) for _ in range(3)]
    n_evict_seen = 0
    n_hits = 0
    for _ in range(n_req):
        toks = np.concatenate([prefixes[rng.integers(3)],
                               rng.integers(0, vocab, size=rng.integers(1, ctx // 3))])
        toks = toks[:ctx].astype(np.uint32)
        m = ours.match(toks)
        assert m == theirs.match(toks)
        n_hits += m
        pos = 0 if m == 0 else (m if m < len(toks) else m - 1)
        while pos < len(toks):
            n = int(min(ub, len(toks) - pos))
            ra, rb = ours.append(toks, pos, n), theirs.append(toks, pos, n)
            assert ra == rb
            if not ra:
                break
            q = rng.standard_normal((n, n_head * hd)).astype(np.float32)
            k = rng.standard_normal((n, n_kv * hd)).astype(np.float32)
            v = rng.standard_normal((n, n_kv * hd)).astype(np.float32)
            # the reference's op_attn reading libtlkv's struct ...
            out_a = O.ref_attn_radix(ours.h, kc_a, vc_a, q, k, v, pos, n, n_head)
            # ... and reading its own kv_cache_* state for the same stream
            sl = theirs.slots(pos + n)
            out_b = O.ref_attn(kc_b, vc_b, q, k, v, sl, pos, n, n_head)
            assert np.array_equal(out_a.view(np.uint32), out_b.view(np.uint32))
            assert np.array_equal(kc_a, kc_b) and np.array_equal(vc_a, vc_b)
            out_o = O.attn(oc, q, k, v, ours.slots(pos + n), pos, n, n_head)
            assert np.abs(out_a - out_o).max() < 1e-5
            pos += n
        n_evict_seen = ours.stats()["evictions"]
    assert n_evict_seen > 0 and n_hits > 0     # the stream did evict and hit


@pytest.mark.parametrize("seed,ctx,n_kv,hd,n_head,ub", [
    (1, 96, 2, 64, 8, 16),     # small pool: many evictions, multi-chunk requests
    (2, 160, 4, 32, 8, 7),     # ragged chunks
])
def test_reference_op_attn_over_libtlkv_radix(seed, ctx, n_kv, hd, n_head, ub):
    _run_stream(seed, ctx, n_kv, hd, n_head, ub, n_req=14, vocab=40)
