"""Config 3's request stream (prefix-reuse stress on the Qwen2.5-7B KV shape)
replayed through the host prefix cache, and the fixture the compiled
reference writes for it.

The stream is the bench's (bench.py run_config3, the same seed and draws):
64 requests, each one of 8 seeded prefixes (U[256,4096] tokens, vocab
151936) plus a unique suffix (U[32,512]); two sessions (-np 2) of 9216 slots
take them alternately.  Per request the host calls are those of
tl_session_kv_prepare_from + tl_session_append (without the device work):
  kv_cache_match on the session; the longest prefix the other session caches
  (a read-only lookup); when it is longer, one kv_cache_append over the
  difference (the fork: the reference would recompute those rows, through
  the same call); resume = the graph_kv_prepare rule (src/graph.c:1440-1452);
  kv_cache_append per 512-token chunk from there (src/graph.c:1395-1413).
The trim of the bench (LRU eviction ahead of demand) has no reference
counterpart and is not replayed; compaction only renames slots and is
replayed on the product side (tests/test_kvcache_config3.py).

    python tests/golden/make_config3_trace.py

writes tests/golden/config3_trace.npz from the compiled reference
(oracle/_ref/libtlref.so): per request [match, fork lookup, forked rows,
resume, hit_tokens, computed_tokens, evictions, allocations, clock, n_free]
of the session that served it, and a CRC of its request map.
"""
import os
import sys
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
POOL, UBATCH, VOCAB = 9216, 512, 151936


def requests():
    """bench.py run_config3's prompts (same generator, same order of draws)."""
    rng = np.random.default_rng(0x9E3779B97F4A7C15 ^ 3)
    prefixes = [rng.integers(0, VOCAB, size=int(rng.integers(256, 4097))).astype(np.uint32)
                for _ in range(8)]
    reqs = []
    for _ in range(64):
        suf = rng.integers(0, VOCAB, size=int(rng.integers(32, 513))).astype(np.uint32)
        reqs.append(np.concatenate([prefixes[int(rng.integers(8))], suf]))
    return reqs


def replay(make, lookup, reqs, between=None):
    """Run the stream over two caches made by make(POOL); lookup(cache,
    tokens) = longest cached prefix, read-only.  Returns one row per request
    (see the module docstring) and the caches."""
    caches = [make(POOL), make(POOL)]
    rows = []
    for r, toks in enumerate(reqs):
        s, other = caches[r % 2], caches[1 - r % 2]
        n = len(toks)
        m = s.match(toks)
        md = lookup(other, toks)
        forked = 0
        if md > m:
            assert s.append(toks, m, md - m)
            forked = md - m
            m = md
        resume = 0 if m == 0 else (m if m < n else m - 1)
        p = resume
        while p < n:
            c = min(UBATCH, n - p)
            assert s.append(toks, p, c)
            p += c
        st, rq = s.stats(), s.req()
        crc = zlib.crc32(np.ascontiguousarray(s.slots(n), np.uint32).tobytes())
        rows.append([m - forked, md, forked, resume, st["hit_tokens"], st["computed_tokens"],
                     st["evictions"], st["allocations"], st["clock"], rq["n_free"], crc])
        if between is not None:
            between(r, caches)
    return np.array(rows, dtype=np.uint64), caches


def main():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not O.ref_available():
        raise SystemExit("build the compiled reference first: make -C oracle")
    rows, _ = replay(O.RefKv, lambda c, t: c.lookup_len(t), requests())
    np.savez_compressed(os.path.join(HERE, "config3_trace.npz"), rows=rows)
    print("config3_trace.npz:", rows.shape, "evictions", rows[-2:, 6].tolist())


if __name__ == "__main__":
    main()
