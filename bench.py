"""Benchmark of the KV-cache hot path on one MI355X.

Workload (the north star): Llama-3-8B-shaped KV —
32 layers, 32 q-heads, 8 kv-heads, head_dim 128, f16 cache, 1 slot, slot
table as a fresh prefix cache assigns it (position i -> slot i).

  1. append      64 chunks x 512 rows of RoPE'd K/V appended to every layer
                 (tl_kv_append; the append tok/s figure)
  2. prefill     chunked-prefill attention of the same 64 chunks on every
                 layer (tl_attn_noappend, MFMA kernel; TFLOP/s vs MFMA peak)
  3. decode      `--steps` decode steps; one step = OP_ATTN (fused append of
                 the new row + GQA decode attention over the whole cache) on
                 each of the 32 layers.  `value` is its throughput in GB/s of
                 algorithmic bytes.

Inputs are seeded N(0,1) f32 (torch generator on the device) with RoPE NORM
(theta 5e5) applied to Q and K before they are handed over.

One JSON line is printed; besides the contract fields:
  roofline      the decode attention launch (one kernel; its key splits are
                merged by the last workgroup of each group inside the launch):
                algorithmic bytes per launch / average launch time, the timed
                region's HIP-event time on the launch stream over its K x 32
                back-to-back launches
  cpu_baseline  op_attn as the C restatement oracle/oracle.c runs it (the
                reference's own objects do not travel to the GPU box) timed on
                a bounded sample of the same decode step, single thread
  prefill, append, hbm_read_ceiling   the other measured rows
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tinyllama.c_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

CFG4 = dict(L=32, Hq=32, Hkv=8, d=128, ctx=32768, ub=512, theta=500000.0, rope_neox=0)


def decode_bytes(c, P):
    """Algorithmic bytes of one decode OP_ATTN on one layer with P visible keys:
    f16 K+V rows read, q read (f32), out written (f32), the new K/V row read
    (f32) and written (f16)."""
    B = 2 * c["Hkv"] * c["d"] * 2
    return P * B + c["Hq"] * c["d"] * 4 * 2 + c["Hkv"] * c["d"] * 2 * (4 + 2)


def decode_bytes_q8(c, P):
    """Algorithmic bytes of one decode OP_ATTN over a Q8_0 cache with P visible
    keys (rows already appended): int8 K+V rows and their f16 scales (one per
    32 values) read, q read (f32), out written (f32)."""
    B = 2 * c["Hkv"] * (c["d"] + c["d"] // 32 * 2)
    return P * B + c["Hq"] * c["d"] * 4 * 2


def prefill_flops(c, p0, n):
    """QK^T + PV flops of one layer's chunk of n rows at positions p0.. (causal)."""
    keys = n * p0 + n * (n + 1) // 2
    return 4 * c["Hq"] * c["d"] * keys


def _port_cache(c, P, rng):
    import oracle as O
    C = O.Cache(P, c["Hkv"], c["d"], f16=False)
    C.k = rng.standard_normal((c["Hkv"], P, c["d"]), dtype=np.float32)
    C.v = rng.standard_normal((c["Hkv"], P, c["d"]), dtype=np.float32)
    return C


def cpu_baseline(c, P, n_layers_sample):
    """op_attn (src/backend/cpu/cpu_op.c:964-1064) as the C restatement
    oracle/oracle.c runs it (pinned against the compiled reference; it is the
    only baseline that travels), f32 cache, one thread, on `n_layers_sample`
    layers of one decode step at P keys."""
    import oracle as O
    rng = np.random.default_rng(7)
    kd = c["Hkv"] * c["d"]
    C = _port_cache(c, P, rng)
    slots = np.arange(P, dtype=np.uint32)
    secs = 0.0
    for _ in range(n_layers_sample):
        q = rng.standard_normal((1, c["Hq"] * c["d"]), dtype=np.float32)
        k = rng.standard_normal((1, kd), dtype=np.float32)
        v = rng.standard_normal((1, kd), dtype=np.float32)
        t0 = time.perf_counter()
        O.attn(C, q, k, v, slots, P - 1, 1, c["Hq"])
        secs += time.perf_counter() - t0
    per_layer = secs / n_layers_sample
    gbs = decode_bytes(c, P) / per_layer / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n_layers_sample} layer calls of one decode step at P={P} "
                      f"(op_attn restated in C, oracle/oracle.c, over an f32 cache, single "
                      f"thread, {os.cpu_count()} host cores present), {per_layer * 1e3:.1f} ms "
                      f"per layer; GB/s counts the f16 workload's algorithmic bytes"}


def cpu_baseline_sessions(c, P, n_sessions, calls):
    """op_attn (the C restatement) for `n_sessions` concurrent sessions, one
    host thread each (the CPU server's -np N), `calls` decode-layer calls per
    session at P keys; aggregate GB/s of the f16 workload's algorithmic bytes
    over the wall time of the parallel section (ctypes releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor
    import oracle as O
    kd = c["Hkv"] * c["d"]
    slots = np.arange(P, dtype=np.uint32)
    data = []
    for i in range(n_sessions):
        rng = np.random.default_rng(100 + i)
        data.append((_port_cache(c, P, rng),
                     rng.standard_normal((calls, c["Hq"] * c["d"]), dtype=np.float32),
                     rng.standard_normal((calls, kd), dtype=np.float32)))

    def work(i):
        C, q, k = data[i]
        for j in range(calls):
            O.attn(C, q[j:j + 1], k[j:j + 1], k[j:j + 1], slots, P - 1, 1, c["Hq"])

    with ThreadPoolExecutor(n_sessions) as ex:
        t0 = time.perf_counter()
        list(ex.map(work, range(n_sessions)))
        secs = time.perf_counter() - t0
    gbs = n_sessions * calls * decode_bytes(c, P) / secs / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": n_sessions, "kind": "port",
            "sample": f"{n_sessions} sessions on {n_sessions} threads, {calls} decode-layer "
                      f"op_attn calls each at P={P} (C restatement, f32 cache; "
                      f"{os.cpu_count()} host cores present), {secs * 1e3:.0f} ms wall"}


def profiled_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/attn_decode_llama3-8b-32k_hbm_traffic.md)."""
    path = os.path.join(ROOT, "profiles", "attn_decode_llama3-8b-32k_hbm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def hbm_read_ceiling(torch, tlkv, lib, sh):
    """Best streaming-read rate of a plain 16-byte-load kernel over 4 GiB."""
    x = torch.empty(2 * 1024 ** 3, dtype=torch.float16, device="cuda")
    sink = torch.empty(8192 * 256, dtype=torch.int32, device="cuda")
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    best = 0.0
    for blocks, depth in ((2048, 1), (8192, 8)):
        def f():
            tlkv.check(lib.tl_probe_read(tlkv.ptr(x), x.numel() * 2, tlkv.ptr(sink), blocks,
                                         depth, sh))
        f()
        e0.record()
        for _ in range(5):
            f()
        e1.record()
        torch.cuda.synchronize()
        best = max(best, x.numel() * 2 * 5 / (e0.elapsed_time(e1) / 1e3) / 1e9)
    del x, sink
    return best


def mfma_ceiling(torch, tlkv, lib, sh):
    """Best dense f16 MFMA rate of a register-only v_mfma_f32_32x32x16_f16
    loop (TFLOP/s): 2048 workgroups of 4 waves, 4 chains per wave."""
    blocks, iters = 2048, 20000
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    flops = blocks * 4 * iters * 4 * 2 * 32 * 32 * 16
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    tlkv.check(lib.tl_probe_mfma(iters, blocks, tlkv.ptr(sink), sh))
    best = 0.0
    for _ in range(3):
        e0.record()
        tlkv.check(lib.tl_probe_mfma(iters, blocks, tlkv.ptr(sink), sh))
        e1.record()
        torch.cuda.synchronize()
        best = max(best, flops / (e0.elapsed_time(e1) / 1e3) / 1e12)
    del sink
    return best


def host_radix_cost(tlkv, n=32768, ub=512):
    """The host prefix cache alone (libtlkv's kv_cache_*, C): config 4's
    prefill bookkeeping -- a miss match, then kv_cache_append of n tokens in
    ub-token chunks -- and a full-hit match of the same n tokens afterwards."""
    toks = np.random.default_rng(4).integers(0, 128256, size=n, dtype=np.uint32)
    C = tlkv.KvCache(n + 64)
    t0 = time.perf_counter()
    C.match(toks)
    for p in range(0, n, ub):
        if not C.append(toks, p, ub):
            raise RuntimeError("kv_cache_append failed")
    t1 = time.perf_counter()
    hit = C.match(toks)
    t2 = time.perf_counter()
    C.close()
    return {"append_ms": round((t1 - t0) * 1e3, 3),
            "ns_per_token": round((t1 - t0) * 1e9 / n, 1),
            "hit_match_ms": round((t2 - t1) * 1e3, 3), "hit_tokens": hit,
            "note": f"{n} tokens in {ub}-token kv_cache_append calls (one host thread), "
                    "then kv_cache_match of all of them"}


# ---- the other BASELINE configs (reported beside the north star) -------------

def _gbs(nbytes, ms):
    return nbytes / (ms / 1e3) / 1e9


def run_config1(torch, tlkv, lib, sh, gen):
    """Config 1, Llama-3.2-1B KV (L16 Hq32 Hkv8 d64), 1 slot: one 512-row
    OP_ATTN chunk (MFMA prefill with fused append), then 256 decode steps of
    OP_ATTN (fused append + attention) per layer.  RoPE NORM theta 5e5."""
    c = dict(L=16, Hq=32, Hkv=8, d=64, theta=500000.0)
    L, Hq, Hkv, d = c["L"], c["Hq"], c["Hkv"], c["d"]
    kd, qd, ub, steps = Hkv * d, Hq * d, 512, 256
    cap = ub + steps
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    layers = [tlkv.Layer(cap, Hkv, d) for _ in range(L)]
    slots = torch.arange(cap, dtype=torch.int32, device="cuda")
    q = torch.randn((L, ub, qd), generator=gen, device="cuda")
    k = torch.randn((L, ub, kd), generator=gen, device="cuda")
    v = torch.randn((L, ub, kd), generator=gen, device="cuda")
    out = torch.empty((L, ub, qd), device="cuda")
    for l in range(L):
        tlkv.check(lib.tl_rope(tlkv.ptr(q[l]), ub, qd, Hq, d, d, 0, c["theta"], 0, sh))
        tlkv.check(lib.tl_rope(tlkv.ptr(k[l]), ub, kd, Hkv, d, d, 0, c["theta"], 0, sh))
    e0, e1, e2, e3 = (torch.cuda.Event(enable_timing=True) for _ in range(4))
    e0.record(stream)
    for l in range(L):
        a = tlkv.attn_args(q[l], k[l], v[l], out[l], slots, 0, ub, Hq, d, Hkv, 0, scale)
        tlkv.check(lib.tl_attn(layers[l].desc, a, sh))
    e1.record(stream)
    torch.cuda.synchronize()
    args_l = [tlkv.attn_args(q[l, :1], k[l, :1], v[l, :1], out[l, :1], slots, 0, 1, Hq, d,
                             Hkv, 0, scale) for l in range(L)]
    e2.record(stream)
    nbytes = 0
    for s in range(steps):
        pos = ub + s
        for l in range(L):
            args_l[l].pos = pos
            tlkv.check(lib.tl_attn(layers[l].desc, args_l[l], sh))
        nbytes += L * decode_bytes(c, pos + 1)
    e3.record(stream)
    torch.cuda.synchronize()
    pf_ms, dec_ms = e0.elapsed_time(e1), e2.elapsed_time(e3)
    pf_flops = L * prefill_flops(c, 0, ub)
    return {"workload": "config 1: L16 Hq32 Hkv8 d64, 512-row OP_ATTN chunk then 256 decode "
                        "steps (fused append + attention)",
            "prefill_TFLOPs": round(pf_flops / (pf_ms / 1e3) / 1e12, 2),
            "prefill_ms": round(pf_ms, 3),
            "decode_GBs": round(_gbs(nbytes, dec_ms), 1),
            "decode_hbm_frac": round(_gbs(nbytes, dec_ms) / HBM_PEAK_GBS, 4),
            "decode_us_per_step": round(dec_ms * 1e3 / steps, 2),
            "decode_us_per_layer_launch": round(dec_ms * 1e3 / steps / L, 2),
            "note": "P = 513..768 keys: each launch reads ~1.5 MB, so decode is "
                    "launch-latency-bound, not HBM-bound"}


def _fill(torch, tlkv, lib, sh, layer, kd, n, gen, ring=0):
    """Append n seeded rows (positions 0..n-1; a ring layer keeps the last
    `ring`) in chunks of at most 4096 rows."""
    CH = 4096
    buf_k = torch.randn((CH, kd), generator=gen, device="cuda")
    buf_v = torch.randn((CH, kd), generator=gen, device="cuda")
    p0 = max(0, n - ring) if ring else 0
    p = p0
    while p < n:
        m = min(CH, n - p)
        tlkv.check(lib.tl_kv_append(layer.desc, tlkv.ptr(buf_k), tlkv.ptr(buf_v), kd, None,
                                    p, m, sh))
        p += m


def run_config2(torch, tlkv, lib, sh, gen, steps=512):
    """Config 2, Qwen2.5-7B KV (L28 Hq28 Hkv4 d128, gqa 7): 8 sessions, each
    with an 8192-row cache, `steps` batched decode steps: one
    tl_attn_decode_batch launch per layer serves all 8 sessions (fused
    one-row append each).  RoPE NEOX theta 1e6 on the step's q/k."""
    L, Hq, Hkv, d, n_seq, P0 = 28, 28, 4, 128, 8, 8192
    kd, qd = Hkv * d, Hq * d
    c = dict(Hq=Hq, Hkv=Hkv, d=d)
    cap = P0 + steps + 8
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    keep = []
    layers = [[tlkv.Layer(cap, Hkv, d) for _ in range(L)] for _ in range(n_seq)]
    for sl in layers:
        for lay in sl:
            _fill(torch, tlkv, lib, sh, lay, kd, P0, gen)
    slots = torch.arange(cap, dtype=torch.int32, device="cuda")
    q = torch.randn((n_seq, L, qd), generator=gen, device="cuda")
    k = torch.randn((n_seq, L, kd), generator=gen, device="cuda")
    v = torch.randn((n_seq, L, kd), generator=gen, device="cuda")
    out = torch.empty((n_seq, L, qd), device="cuda")
    for i in range(n_seq):
        tlkv.check(lib.tl_rope(tlkv.ptr(q[i]), L, qd, Hq, d, d, P0, 1e6, 1, sh))
        tlkv.check(lib.tl_rope(tlkv.ptr(k[i]), L, kd, Hkv, d, d, P0, 1e6, 1, sh))
    batches = []
    for l in range(L):
        seqs = [tlkv.DecodeSeq(layers[i][l].desc, slots.data_ptr(), P0, 0, q[i, l].data_ptr(),
                               k[i, l].data_ptr(), v[i, l].data_ptr(), out[i, l].data_ptr())
                for i in range(n_seq)]
        batches.append((tlkv.DecodeSeq * n_seq)(*seqs))
    keep.append(batches)

    def step(pos):
        for arr in batches:
            for i in range(n_seq):
                arr[i].pos = pos
            rc = lib.tl_attn_decode_batch(arr, n_seq, Hq, 0, scale, sh)
            if rc:
                tlkv.check(rc)

    for w in range(4):
        step(P0 + w)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    nbytes = 0
    for s in range(steps):
        pos = P0 + 4 + s
        step(pos)
        nbytes += n_seq * L * decode_bytes(c, pos + 1)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    del layers, batches
    keep.clear()
    torch.cuda.empty_cache()
    q8 = run_config2_q8(torch, tlkv, lib, sh, gen, q, k, v, out, min(steps, 128))
    return {"workload": f"config 2: L28 Hq28 Hkv4 d128 (gqa 7), 8 sessions x 8192-row cache, "
                        f"{steps} batched decode steps (one launch per layer for all 8)",
            "q8_0_cache": q8,
            "GBs": round(_gbs(nbytes, ms), 1), "hbm_frac": round(_gbs(nbytes, ms) / HBM_PEAK_GBS, 4),
            "ms_per_step": round(ms / steps, 4),
            "tok_s": round(n_seq * steps / (ms / 1e3), 1),
            "us_per_layer_launch": round(ms * 1e3 / steps / L, 2)}


def run_config2_q8(torch, tlkv, lib, sh, gen, q, k, v, out, steps):
    """Config 2 over Q8_0 caches: the same 8 sessions x 8192 rows (quantized
    from N(0,1) rows), `steps` batched decode steps of tl_attn_decode_batch_q8
    (one launch per layer: the decode launch quantizes and writes the new
    rows itself)."""
    L, Hq, Hkv, d, n_seq, P0 = 28, 28, 4, 128, 8, 8192
    kd = Hkv * d
    cap = P0 + steps + 8
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    layers = [[tlkv.LayerQ8(cap, Hkv, d) for _ in range(L)] for _ in range(n_seq)]
    rows = torch.empty((P0, kd), device="cuda")
    for sl in layers:
        for lay in sl:
            rows.normal_(generator=gen)
            tlkv.check(lib.tl_kv_append_q8(lay.desc, tlkv.ptr(rows), tlkv.ptr(rows), kd, None, 0,
                                           P0, sh))
    batches = []
    for l in range(L):
        seqs = [tlkv.DecodeSeqQ8(layers[i][l].desc, None, P0, 0, q[i, l].data_ptr(),
                                 k[i, l].data_ptr(), v[i, l].data_ptr(), out[i, l].data_ptr())
                for i in range(n_seq)]
        batches.append((tlkv.DecodeSeqQ8 * n_seq)(*seqs))

    def step(pos):
        for arr in batches:
            for i in range(n_seq):
                arr[i].pos = pos
            rc = lib.tl_attn_decode_batch_q8(arr, n_seq, Hq, 0, scale, sh)
            if rc:
                tlkv.check(rc)

    for w in range(4):
        step(P0 + w)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    nbytes = 0
    c = dict(Hq=Hq, Hkv=Hkv, d=d)
    for s in range(steps):
        pos = P0 + 4 + s
        step(pos)
        nbytes += n_seq * L * decode_bytes_q8(c, pos + 1)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    del layers, batches
    return {"GBs": round(_gbs(nbytes, ms), 1), "steps": steps,
            "us_per_layer": round(ms * 1e3 / steps / L, 2),
            "tok_s": round(n_seq * steps / (ms / 1e3), 1),
            "note": "Q8_0 bytes (int8 rows + f16 scales); per layer one decode launch for "
                    "the 8 sessions that also quantizes and writes their new rows"}


def run_config5(torch, tlkv, lib, sh, gen, steps=512):
    """Config 5, Gemma-3-4B KV (L34 Hq8 Hkv4 d256): 2 sessions at 16384 keys;
    layers with l % 6 == 5 are global (full cache, theta 1e6), the other 29
    are local (window 1024 on a ring of 1024 + 512 - 1 rows, theta 1e4).
    One tl_attn_decode_batch launch per layer serves both sessions."""
    L, Hq, Hkv, d, n_seq, P0, W = 34, 8, 4, 256, 2, 16384, 1024
    ring = W + 512 - 1
    kd, qd = Hkv * d, Hq * d
    c = dict(Hq=Hq, Hkv=Hkv, d=d)
    cap = P0 + steps + 8
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    glob = [l % 6 == 5 for l in range(L)]
    layers = [[tlkv.Layer(cap if glob[l] else ring, Hkv, d, ring=0 if glob[l] else ring)
               for l in range(L)] for _ in range(n_seq)]
    for sl in layers:
        for l, lay in enumerate(sl):
            _fill(torch, tlkv, lib, sh, lay, kd, P0, gen, ring=0 if glob[l] else ring)
    q = torch.randn((n_seq, L, qd), generator=gen, device="cuda")
    k = torch.randn((n_seq, L, kd), generator=gen, device="cuda")
    v = torch.randn((n_seq, L, kd), generator=gen, device="cuda")
    out = torch.empty((n_seq, L, qd), device="cuda")
    for i in range(n_seq):
        for l in range(L):
            th = 1e6 if glob[l] else 1e4
            tlkv.check(lib.tl_rope(tlkv.ptr(q[i, l]), 1, qd, Hq, d, d, P0, th, 1, sh))
            tlkv.check(lib.tl_rope(tlkv.ptr(k[i, l]), 1, kd, Hkv, d, d, P0, th, 1, sh))
    batches = []
    for l in range(L):
        seqs = [tlkv.DecodeSeq(layers[i][l].desc, None, P0, 0, q[i, l].data_ptr(),
                               k[i, l].data_ptr(), v[i, l].data_ptr(), out[i, l].data_ptr())
                for i in range(n_seq)]
        batches.append(((tlkv.DecodeSeq * n_seq)(*seqs), 0 if glob[l] else W))

    def step(pos):
        for arr, win in batches:
            for i in range(n_seq):
                arr[i].pos = pos
            rc = lib.tl_attn_decode_batch(arr, n_seq, Hq, win, scale, sh)
            if rc:
                tlkv.check(rc)

    for w in range(4):
        step(P0 + w)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    nbytes = 0
    B = 2 * Hkv * d * 2
    small = Hq * d * 4 * 2 + Hkv * d * 2 * (4 + 2)
    for s in range(steps):
        pos = P0 + 4 + s
        step(pos)
        nbytes += n_seq * (5 * (pos + 1) * B + 29 * W * B + L * small)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    return {"workload": f"config 5: L34 Hq8 Hkv4 d256, 2 sessions at 16384 keys, 29 local "
                        f"layers (window 1024, ring) + 5 global, {steps} decode steps",
            "GBs": round(_gbs(nbytes, ms), 1), "hbm_frac": round(_gbs(nbytes, ms) / HBM_PEAK_GBS, 4),
            "ms_per_step": round(ms / steps, 4),
            "us_per_layer_launch": round(ms * 1e3 / steps / L, 2),
            "note": "local layers read 4 MB per launch: launch-latency-bound"}


def run_config3(torch, tlkv, lib, sh, gen):
    """Config 3, prefix reuse on the Qwen2.5-7B KV shape (L28 Hkv4 d128): 64
    requests = one of 8 seeded prefixes (U[256,4096] tokens, vocab 151936) +
    a unique suffix (U[32,512]).  Two sessions (-np 2) of 9216 rows each
    (together 4 requests' worth, 18432 rows) take requests alternately:
    kv_prepare_from forks a prefix that only the other session holds
    (tl_kv_copy_between), the rest is appended (K/V write-through on all
    layers); LRU eviction happens on demand, and every 16 requests each pool
    is trimmed to 3/4 and compacted (one tl_kv_copy launch).  Bytes: 172032
    per appended token, 114688 per forked or compacted row."""
    L, Hq, Hkv, d, pool, vocab = 28, 28, 4, 128, 9216, 151936
    kd = Hkv * d
    rng = np.random.default_rng(0x9E3779B97F4A7C15 ^ 3)
    prefixes = [rng.integers(0, vocab, size=int(rng.integers(256, 4097))).astype(np.uint32)
                for _ in range(8)]
    reqs = []
    for r in range(64):
        suf = rng.integers(0, vocab, size=int(rng.integers(32, 513))).astype(np.uint32)
        reqs.append(np.concatenate([prefixes[int(rng.integers(8))], suf]))
    stream = torch.cuda.current_stream()
    sess = [tlkv.Session(L, Hq, Hkv, d, pool, 512, stream=sh) for _ in range(2)]
    kbuf = torch.randn((4608, kd), generator=gen, device="cuda")
    vbuf = torch.randn((4608, kd), generator=gen, device="cuda")
    klist, vlist = [kbuf] * L, [vbuf] * L
    appended = forked = compacted = evicted_trim = hits = 0
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for r, toks in enumerate(reqs):
        S, other = sess[r % 2], sess[1 - r % 2]
        m, resume, f = S.kv_prepare_from(other, toks)
        forked += f
        hits += m - f
        S.append(toks[resume:], klist, vlist, kd)
        appended += len(toks) - resume
        if r % 16 == 15:
            for X in sess:
                ev, mv = X.compact(keep=pool * 3 // 4)
                evicted_trim += ev
                compacted += mv
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    nbytes = appended * 172032 + (forked + compacted) * 114688
    L_ = tlkv._kv_sigs()
    stats = [L_.tl_kv_cache_stats(X.radix).contents for X in sess]
    return {"workload": "config 3: L28 Hkv4 d128, 64 requests (8 shared prefixes 256..4096 + "
                        "unique suffix 32..512, vocab 151936), 2 sessions x 9216 rows, fork from "
                        "the other session, LRU eviction, trim+compaction every 16 requests",
            "GBs": round(_gbs(nbytes, ms), 1), "ms": round(ms, 2), "wall_s": round(wall, 3),
            "appended_tokens": appended, "forked_rows": forked, "compacted_rows": compacted,
            "local_hit_tokens": hits,
            "radix_hit_tokens": int(sum(x.hit_tokens for x in stats)),
            "evictions": int(sum(x.evictions for x in stats)),
            "trim_evictions": evicted_trim,
            "note": "time includes the host prefix cache (match, append, eviction, compaction "
                    "planning) between launches; bytes are algorithmic"}


def run_prefill_fused(torch, tlkv, lib, sh, gen, c, layers, slots, pf_ms, app_ms, pf_flops):
    """The 64 config-4 chunks again (fresh rows, after the decode rows are
    measured), as the executor issues them: one OP_ATTN per layer and chunk
    (tl_attn: the prefill launch writes the chunk's rows itself), against
    the separate tl_kv_append + tl_attn_noappend launches of phases 1-2.
    The append's cost inside the fused launch is the fused time minus the
    attention-only time of phase 2 (a difference of two timings)."""
    L, Hq, Hkv, d, ub = c["L"], c["Hq"], c["Hkv"], c["d"], c["ub"]
    kd, qd = Hkv * d, Hq * d
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    n_chunks = c["ctx"] // ub
    ck = torch.empty((L, ub, kd), dtype=torch.float32, device="cuda")
    cv = torch.empty((L, ub, kd), dtype=torch.float32, device="cuda")
    cq = torch.empty((L, ub, qd), dtype=torch.float32, device="cuda")
    co = torch.empty((L, ub, qd), dtype=torch.float32, device="cuda")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ms = 0.0
    for ci in range(n_chunks):
        p0 = ci * ub
        ck.normal_(generator=gen)
        cv.normal_(generator=gen)
        cq.normal_(generator=gen)
        e0.record(stream)
        for l in range(L):
            a = tlkv.attn_args(cq[l], ck[l], cv[l], co[l], slots, p0, ub, Hq, d, Hkv, 0, scale)
            tlkv.check(lib.tl_attn(layers[l].desc, a, sh))
        e1.record(stream)
        torch.cuda.synchronize()
        ms += e0.elapsed_time(e1)
    tokens = n_chunks * ub
    extra = ms - pf_ms
    return {"ms": round(ms, 2), "TFLOPs": round(pf_flops / (ms / 1e3) / 1e12, 2),
            "separate_ms": round(pf_ms + app_ms, 2),
            "append_extra_ms": round(extra, 2),
            "append_tok_s": round(tokens / (extra / 1e3), 1) if extra > 0.05 * pf_ms else None,
            "note": "OP_ATTN per layer and chunk with the append inside the prefill launch "
                    "(no kv_append_kernel launches) vs append + attention launches "
                    "(separate_ms = append.ms + prefill.ms); append_extra_ms = ms - prefill.ms, "
                    "the append's cost inside the fused launch; append_tok_s = chunk tokens / "
                    "append_extra_ms, reported only when that difference is above 5% of "
                    "prefill.ms (below it is run-to-run noise)"}


def run_q8(torch, tlkv, lib, sh, gen, c, steps):
    """Config 4 over a Q8_0 cache: the same 64 x 512-row chunks quantized into
    every layer (tl_kv_append_q8) with chunked-prefill attention over them
    (tl_attn_noappend_q8, MFMA kernel dequantizing its tiles), then decode
    steps over the contiguous cache at P = ctx + 1 keys: attention alone
    (tl_attn_noappend_q8, one launch) and OP_ATTN with the new row
    (tl_attn_q8: one launch that also quantizes and writes the new row)."""
    L, Hq, Hkv, d, ub = c["L"], c["Hq"], c["Hkv"], c["d"], c["ub"]
    kd, qd = Hkv * d, Hq * d
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    cap = c["ctx"] + steps + 8
    layers = [tlkv.LayerQ8(cap, Hkv, d) for _ in range(L)]
    descs = [x.desc for x in layers]
    n_chunks = c["ctx"] // ub
    ck = torch.empty((L, ub, kd), dtype=torch.float32, device="cuda")
    cv = torch.empty((L, ub, kd), dtype=torch.float32, device="cuda")
    cq = torch.empty((L, ub, qd), dtype=torch.float32, device="cuda")
    co = torch.empty((L, ub, qd), dtype=torch.float32, device="cuda")
    app_ms = pf_ms = 0.0
    pf_flops = 0
    e = [ev(), ev(), ev()]
    for ci in range(n_chunks):
        p0 = ci * ub
        ck.normal_(generator=gen)
        cv.normal_(generator=gen)
        cq.normal_(generator=gen)
        e[0].record(stream)
        for l in range(L):
            tlkv.check(lib.tl_kv_append_q8(descs[l], tlkv.ptr(ck[l]), tlkv.ptr(cv[l]), kd,
                                           None, p0, ub, sh))
        e[1].record(stream)
        for l in range(L):
            a = tlkv.attn_args(cq[l], None, None, co[l], None, p0, ub, Hq, d, Hkv, 0, scale)
            tlkv.check(lib.tl_attn_noappend_q8(descs[l], a, sh))
        pf_flops += L * prefill_flops(c, p0, ub)
        e[2].record(stream)
        torch.cuda.synchronize()
        app_ms += e[0].elapsed_time(e[1])
        pf_ms += e[1].elapsed_time(e[2])
    del ck, cv, cq, co
    q = torch.randn((L, 1, qd), generator=gen, device="cuda")
    k = torch.randn((L, 1, kd), generator=gen, device="cuda")
    v = torch.randn((L, 1, kd), generator=gen, device="cuda")
    out = torch.empty((L, 1, qd), dtype=torch.float32, device="cuda")
    P = c["ctx"]
    a_no = [tlkv.attn_args(q[l], None, None, out[l], None, P, 1, Hq, d, Hkv, 0, scale)
            for l in range(L)]
    noapp = lib.tl_attn_noappend_q8
    # the row at position P (read by the no-append launches)
    for l in range(L):
        tlkv.check(lib.tl_kv_append_q8(descs[l], tlkv.ptr(k[l]), tlkv.ptr(v[l]), kd, None,
                                       P, 1, sh))
        tlkv.check(noapp(descs[l], a_no[l], sh))
    torch.cuda.synchronize()
    n_st = min(128, steps)
    c0, c1 = ev(), ev()
    c0.record(stream)
    for _ in range(n_st):
        for l in range(L):
            rc = noapp(descs[l], a_no[l], sh)
            if rc:
                tlkv.check(rc)
    c1.record(stream)
    torch.cuda.synchronize()
    us = c0.elapsed_time(c1) * 1e3 / (n_st * L)
    nbytes = decode_bytes_q8(c, P + 1)
    f16_bytes = decode_bytes(c, P + 1) - Hkv * d * 2 * 6
    # OP_ATTN with the new row (quantized and written by the decode launch)
    a_ap = [tlkv.attn_args(q[l], k[l], v[l], out[l], None, P + 1, 1, Hq, d, Hkv, 0, scale)
            for l in range(L)]
    attn = lib.tl_attn_q8
    c2, c3 = ev(), ev()
    c2.record(stream)
    for s in range(n_st):
        for l in range(L):
            a = a_ap[l]
            a.pos = P + 1 + s
            rc = attn(descs[l], a, sh)
            if rc:
                tlkv.check(rc)
    c3.record(stream)
    torch.cuda.synchronize()
    us_app = c2.elapsed_time(c3) * 1e3 / (n_st * L)
    tf = pf_flops / (pf_ms / 1e3) / 1e12
    del layers
    return {
        "decode": {"us_per_layer_launch": round(us, 3),
                   "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                   "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                   "f16_equivalent_GBs": round(f16_bytes / (us * 1e-6) / 1e9, 1),
                   "steps": n_st, "keys": P + 1,
                   "kernel": "attn_decode_ring_kernel<128,4,false,true,true>",
                   "note": "tl_attn_noappend_q8 over the contiguous Q8_0 cache; GBs counts "
                           "int8 rows + f16 scales, f16_equivalent_GBs the bytes of the same "
                           "keys in the f16 cache"},
        "decode_with_append_us_per_layer": round(us_app, 3),
        "append_tok_s": round(n_chunks * ub / (app_ms / 1e3), 1),
        "prefill_TFLOPs": round(tf, 2),
        "prefill_frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
    }


def run_state_snapshot(torch, tlkv, lib, sh):
    """Recurrent-state snapshot save + load (tl_state_copy) for a hybrid arch's
    state: 36 Gated-DeltaNet-style layers x (32 heads x 128 x 128 f32 state +
    a 4 x 8192 f32 conv ring) = 74.2 MB in 72 device buffers, against the
    reference's way (graph_state_save: one device-to-host copy per buffer,
    src/graph.c:368-388) timed on the same buffers into pinned host memory."""
    segs_t = []
    for _ in range(36):
        segs_t.append(torch.randn(32 * 128 * 128, device="cuda"))
        segs_t.append(torch.randn(4 * 8192, device="cuda"))
    total = sum(t.numel() * 4 for t in segs_t)
    segs = (tlkv.StateSeg * len(segs_t))(*[tlkv.StateSeg(t.data_ptr(), t.numel() * 4) for t in segs_t])
    snap = torch.empty(total // 4, device="cuda")
    stream = torch.cuda.current_stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    for d in (tlkv.TL_STATE_SAVE, tlkv.TL_STATE_LOAD):
        tlkv.check(lib.tl_state_copy(segs, len(segs_t), tlkv.ptr(snap), d, sh))
    torch.cuda.synchronize()
    reps = 20
    out = {}
    for name, d in (("save", tlkv.TL_STATE_SAVE), ("load", tlkv.TL_STATE_LOAD)):
        e0, e1 = ev(), ev()
        e0.record(stream)
        for _ in range(reps):
            tlkv.check(lib.tl_state_copy(segs, len(segs_t), tlkv.ptr(snap), d, sh))
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        out[f"{name}_us"] = round(us, 1)
        out[f"{name}_GBs"] = round(2 * total / (us * 1e-6) / 1e9, 1)   # read + write
    host = torch.empty(total // 4, dtype=torch.float32, pin_memory=True)
    e0, e1 = ev(), ev()
    e0.record(stream)
    for _ in range(3):
        o = 0
        for t in segs_t:
            host[o:o + t.numel()].copy_(t, non_blocking=True)
            o += t.numel()
    e1.record(stream)
    torch.cuda.synchronize()
    out["reference_style_d2h_save_us"] = round(e0.elapsed_time(e1) * 1e3 / 3, 1)
    out["bytes"] = total
    out["note"] = ("tl_state_copy (one launch, device snapshot) vs one device-to-host copy "
                   "per buffer into pinned memory (graph_state_save's pattern)")
    return out


DECODE_KERNEL = "attn_decode_ring_kernel<128, 4, false, false, true>"


def split_trace(path, warmup, steps):
    """The config-4 decode launches of a profiled run, by variant: they are
    the first dispatches of DECODE_KERNEL, in the order main() issues them —
    (warmup + steps) x 32 OP_ATTN launches (identity slot table, fused
    append), then 32 + min(128, steps) x 32 over the contiguous cache
    (without the slot table or append), then 32 + min(128, steps) x 32
    through the permuted slot table; the first 32 of the last two are
    untimed warm-ups.  Prints one markdown table of average durations."""
    import csv
    L = CFG4["L"]
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r.get("Kernel_Name", "")
            if DECODE_KERNEL.replace(" ", "") in name.replace(" ", ""):
                rows.append((int(r["Dispatch_Id"]), int(r["Start_Timestamp"]),
                             int(r["End_Timestamp"])))
    rows.sort()
    n_main, n_side = (warmup + steps) * L, min(128, steps) * L
    phases = [("identity slot table + fused append (the timed `value` loop)", warmup * L,
               n_main),
              ("contiguous cache, no append (decode_contiguous)", n_main + L, n_main + L + n_side),
              ("permuted slot table, no append (decode_permuted_slots)", n_main + 2 * L + n_side,
               n_main + 2 * L + 2 * n_side)]
    print("| variant | launches | avg us | min us | max us | avg start-to-start us |")
    print("|---|---|---|---|---|---|")
    for nm, a, b in phases:
        seg = rows[a:b]
        if not seg:
            continue
        d = np.array([(e - s_) / 1e3 for _, s_, e in seg])
        st = np.array([s_ for _, s_, _ in seg], dtype=np.float64)
        gap = np.diff(st).mean() / 1e3 if len(st) > 1 else float("nan")
        print(f"| {nm} | {len(seg)} | {d.mean():.2f} | {d.min():.2f} | {d.max():.2f} | "
              f"{gap:.2f} |")


def split_counters(root, warmup, steps):
    """Counter values of a profiled run (`rocprofv3 --pmc ...` CSVs under
    `root`, any counters): the mean per dispatch of every kernel, and
    DECODE_KERNEL's dispatches split by the order main() issues them (as
    split_trace, then the decode_multi_row launches: 32 + min(64, steps) x 32
    folded, the same one row per group).  Prints markdown tables."""
    import csv
    import glob
    from collections import defaultdict
    L = CFG4["L"]
    acc = defaultdict(lambda: [0, 0.0])
    per = defaultdict(list)
    for path in glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"].replace("void ", "").split("(")[0].strip()
                key = (name, r["Counter_Name"])
                acc[key][0] += 1
                acc[key][1] += float(r["Counter_Value"])
                if DECODE_KERNEL.replace(" ", "") in name.replace(" ", ""):
                    per[r["Counter_Name"]].append((int(r["Dispatch_Id"]),
                                                   float(r["Counter_Value"])))
    print("| kernel | counter | dispatches | mean per dispatch |")
    print("|---|---|---|---|")
    for (kn, cn), (n, tot) in sorted(acc.items()):
        print(f"| `{kn}` | {cn} | {n} | {tot / n:.1f} |")
    n_main, n_side, n_mr = (warmup + steps) * L, min(128, steps) * L, min(64, steps) * L
    c0 = n_main + 2 * (L + n_side)
    phases = [("identity slot table + fused append (the timed `value` loop)", warmup * L, n_main),
              ("contiguous cache, no append", n_main + L, n_main + L + n_side),
              ("permuted slot table, no append", n_main + 2 * L + n_side, c0),
              ("4 batch rows folded into one group (decode_multi_row)", c0 + L, c0 + L + n_mr),
              ("4 batch rows, one row per group", c0 + 2 * L + n_mr, c0 + 2 * (L + n_mr))]
    for cn, vals in sorted(per.items()):
        vals.sort()
        print(f"\n`{DECODE_KERNEL}`, {cn} by bench row:\n")
        print("| row | dispatches | mean per dispatch |")
        print("|---|---|---|")
        for nm, a, b in phases:
            seg = [v for _, v in vals[a:b]]
            if seg:
                print(f"| {nm} | {len(seg)} | {sum(seg) / len(seg):.1f} |")


def long_context_sweep(reps=50):
    """Single-row decode (tl_attn_noappend, identity slot table) of the
    Llama-3-8B shape at 66K-131K keys, past the point where the 2048-key
    chunk limit needs more than one round of workgroups.  One JSON line per
    key count (us per launch, GB/s of K/V bytes)."""
    import torch
    import tlkv
    lib = tlkv.lib()
    tlkv.check(lib.tl_init(0))
    n_head, n_kv, hd = CFG4["Hq"], CFG4["Hkv"], CFG4["d"]
    kd, qd = n_kv * hd, n_head * hd
    for P in (66000, 80000, 100000, 131000):
        cap = P + 64
        L = tlkv.Layer(cap, n_kv, hd)
        rows = torch.randn((4096, kd), device="cuda")
        for p0 in range(0, P, 4096):
            tlkv.check(lib.tl_kv_append(L.desc, tlkv.ptr(rows), tlkv.ptr(rows), kd, None, p0,
                                        min(4096, P - p0), None))
        slots = torch.arange(cap, dtype=torch.int32, device="cuda")
        q = torch.randn((1, qd), device="cuda")
        o = torch.empty((1, qd), device="cuda")
        res = {}
        for name, sl in (("slot_table", slots), ("contiguous", None)):
            a = tlkv.attn_args(q, None, None, o, sl, P - 1, 1, n_head, hd, n_kv, 0, 1 / hd ** 0.5)
            for _ in range(5):
                tlkv.check(lib.tl_attn_noappend(L.desc, a, None))
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                lib.tl_attn_noappend(L.desc, a, None)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            res[name] = {"us_per_launch": round(us, 2),
                         "GBs": round(P * kd * 4 / (us * 1e-6) / 1e9, 1)}
        print(json.dumps({"keys": P, **res}), flush=True)
        del L, rows, slots


def decode_tile_sweep(P=32768, reps=50):
    """Decode of 1-8 batch rows of one session at P keys (rows in the cache,
    no append) over f16 and Q8_0 caches of several shapes, per tile variant:
    the automatic choice, the vector tile, the matrix tile with one row per
    group and with the rows folded into its columns.  Prints one JSON line
    per shape (us per launch)."""
    import torch
    import tlkv
    lib = tlkv.lib()
    tlkv.check(lib.tl_init(0))
    variants = (("auto", 0, 0), ("vector", 1, 0), ("matrix_1row", 2, 1), ("matrix_fold", 2, 0))
    for q8 in (False, True):
        for n_head, n_kv, hd in ((8, 8, 128), (32, 8, 128), (16, 4, 128), (8, 4, 256),
                                 (16, 8, 256), (8, 8, 64), (32, 8, 64)):
            kd, qd = n_kv * hd, n_head * hd
            L = (tlkv.LayerQ8 if q8 else tlkv.Layer)(P + 64, n_kv, hd)
            rows = torch.randn((4096, kd), device="cuda")
            app = lib.tl_kv_append_q8 if q8 else lib.tl_kv_append
            for p0 in range(0, P, 4096):
                tlkv.check(app(L.desc, tlkv.ptr(rows), tlkv.ptr(rows), kd, None, p0, 4096, None))
            fn = lib.tl_attn_noappend_q8 if q8 else lib.tl_attn_noappend
            for n in (1, 2, 4, 8):
                q = torch.randn((n, qd), device="cuda")
                o = torch.empty((n, qd), device="cuda")
                a = tlkv.attn_args(q, None, None, o, None, P - n, n, n_head, hd, n_kv, 0,
                                   1.0 / hd ** 0.5)
                res = {}
                for name, mf, rr in variants:
                    with tlkv.tuning(tlkv.TUNE_DECODE_MFMA, mf), \
                            tlkv.tuning(tlkv.TUNE_DECODE_ROWS, rr):
                        for _ in range(5):
                            tlkv.check(fn(L.desc, a, None))
                        torch.cuda.synchronize()
                        e0 = torch.cuda.Event(enable_timing=True)
                        e1 = torch.cuda.Event(enable_timing=True)
                        e0.record()
                        for _ in range(reps):
                            fn(L.desc, a, None)
                        e1.record()
                        torch.cuda.synchronize()
                        res[name] = round(e0.elapsed_time(e1) * 1e3 / reps, 2)
                print(json.dumps({"cache": "q8_0" if q8 else "f16", "n_head": n_head,
                                  "n_kv_head": n_kv, "head_dim": hd, "rows": n, "keys": P,
                                  "us_per_launch": res}), flush=True)
            del L, rows


def attn_kernel_sweep(reps=30):
    """OP_ATTN (tl_attn: append + attention) of 16-64 rows at 1K-16K keys,
    as planned and on the decode kernel alone (TL_TUNE_NO_PREFILL = 1): the
    crossover between the decode and the prefill kernel.  One JSON line per
    shape and key count (us per launch)."""
    import torch
    import tlkv
    lib = tlkv.lib()
    tlkv.check(lib.tl_init(0))
    for P in (1024, 2048, 4096, 8192, 16384):
        for n_head, n_kv, hd in ((32, 8, 128), (28, 4, 128), (32, 8, 64), (8, 4, 256)):
            kd, qd = n_kv * hd, n_head * hd
            L = tlkv.Layer(P + 128, n_kv, hd)
            rows = torch.randn((4096, kd), device="cuda")
            for p0 in range(0, P, 4096):
                tlkv.check(lib.tl_kv_append(L.desc, tlkv.ptr(rows), tlkv.ptr(rows), kd, None, p0,
                                            min(4096, P - p0), None))
            res = {}
            for n in (16, 24, 32, 48, 64):
                q = torch.randn((n, qd), device="cuda")
                k = torch.randn((n, kd), device="cuda")
                o = torch.empty((n, qd), device="cuda")
                a = tlkv.attn_args(q, k, k, o, None, P, n, n_head, hd, n_kv, 0, 1.0 / hd ** 0.5)
                for name, nopf in (("planned", 0), ("decode_kernel", 1)):
                    with tlkv.tuning(tlkv.TUNE_NO_PREFILL, nopf):
                        for _ in range(3):
                            tlkv.check(lib.tl_attn(L.desc, a, None))
                        torch.cuda.synchronize()
                        e0 = torch.cuda.Event(enable_timing=True)
                        e1 = torch.cuda.Event(enable_timing=True)
                        e0.record()
                        for _ in range(reps):
                            lib.tl_attn(L.desc, a, None)
                        e1.record()
                        torch.cuda.synchronize()
                        res.setdefault(f"rows{n}", {})[name] = round(
                            e0.elapsed_time(e1) * 1e3 / reps, 2)
            print(json.dumps({"n_head": n_head, "n_kv_head": n_kv, "head_dim": hd, "keys": P,
                              "us_per_launch": res}), flush=True)
            del L, rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-layers", type=int, default=96,
                    help="decode-layer calls timed for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-q8", action="store_true", help="skip the Q8_0-cache rows")
    ap.add_argument("--no-prefill-attn", action="store_true",
                    help="fill the cache with appends only (skips phase 2)")
    ap.add_argument("--ctx", type=int, default=CFG4["ctx"])
    ap.add_argument("--configs", default="1,2,3,5",
                    help="other BASELINE configs to measure after the north star ('' = none)")
    ap.add_argument("--split-trace", metavar="CSV",
                    help="no run: split a rocprofv3 kernel-trace CSV of a run with the same "
                         "--steps/--warmup into the config-4 decode variants, print markdown")
    ap.add_argument("--split-counters", metavar="DIR",
                    help="no run: summarise the rocprofv3 --pmc CSVs under DIR of a run with the "
                         "same --steps/--warmup (per kernel, and the config-4 decode by bench row)")
    ap.add_argument("--decode-tile-sweep", action="store_true",
                    help="no run: time decode tile variants over 1-8 batch rows and several "
                         "shapes at 32K keys, one JSON line per shape")
    ap.add_argument("--long-context-sweep", action="store_true",
                    help="no run: single-row decode at 66K-131K keys, one JSON line per key count")
    ap.add_argument("--attn-kernel-sweep", action="store_true",
                    help="no run: time OP_ATTN of 16-64 rows at 1K-16K keys as planned and on "
                         "the decode kernel alone, one JSON line per shape")
    args = ap.parse_args()
    if args.long_context_sweep:
        long_context_sweep()
        return
    if args.attn_kernel_sweep:
        attn_kernel_sweep()
        return
    if args.decode_tile_sweep:
        decode_tile_sweep()
        return
    if args.split_trace:
        split_trace(args.split_trace, args.warmup, args.steps)
        return
    if args.split_counters:
        split_counters(args.split_counters, args.warmup, args.steps)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; runs on several GPUs "
                                   "are not part of it"}))
        sys.exit(2)

    import torch
    import tlkv
    c = dict(CFG4)
    c["ctx"] = args.ctx
    lib = tlkv.lib()
    tlkv.check(lib.tl_init(0))
    L, Hq, Hkv, d, ub = c["L"], c["Hq"], c["Hkv"], c["d"], c["ub"]
    kd, qd = Hkv * d, Hq * d
    cap = c["ctx"] + args.warmup + args.steps + 72   # + the RoPE comparison steps
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    sh = tlkv.stream_handle(stream)
    ev = lambda: torch.cuda.Event(enable_timing=True)

    ceiling = hbm_read_ceiling(torch, tlkv, lib, sh)
    mfma_ceil = mfma_ceiling(torch, tlkv, lib, sh)

    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x9E3779B9 ^ 4)
    layers = [tlkv.Layer(cap, Hkv, d) for _ in range(L)]
    slots = torch.arange(cap, dtype=torch.int32, device="cuda")

    # ---- 1. appends + 2. chunked prefill, 64 chunks of 512 rows -------------
    n_chunks = c["ctx"] // ub
    ck = torch.empty((L, ub, kd), dtype=torch.float32, device="cuda")
    cv = torch.empty((L, ub, kd), dtype=torch.float32, device="cuda")
    cq = torch.empty((L, ub, qd), dtype=torch.float32, device="cuda")
    co = torch.empty((L, ub, qd), dtype=torch.float32, device="cuda")
    app_ms = 0.0
    pf_ms = 0.0
    pf_flops = 0
    e = [ev(), ev(), ev()]
    for ci in range(n_chunks):
        p0 = ci * ub
        ck.normal_(generator=gen)
        cv.normal_(generator=gen)
        cq.normal_(generator=gen)
        for l in range(L):
            tlkv.check(lib.tl_rope(tlkv.ptr(ck[l]), ub, kd, Hkv, d, d, p0, c["theta"],
                                   c["rope_neox"], sh))
            tlkv.check(lib.tl_rope(tlkv.ptr(cq[l]), ub, qd, Hq, d, d, p0, c["theta"],
                                   c["rope_neox"], sh))
        e[0].record(stream)
        for l in range(L):
            tlkv.check(lib.tl_kv_append(layers[l].desc, tlkv.ptr(ck[l]), tlkv.ptr(cv[l]),
                                        kd, tlkv.ptr(slots), p0, ub, sh))
        e[1].record(stream)
        if not args.no_prefill_attn:
            for l in range(L):
                a = tlkv.attn_args(cq[l], ck[l], cv[l], co[l], slots, p0, ub, Hq, d, Hkv, 0,
                                   scale)
                tlkv.check(lib.tl_attn_noappend(layers[l].desc, a, sh))
            pf_flops += L * prefill_flops(c, p0, ub)
        e[2].record(stream)
        torch.cuda.synchronize()
        app_ms += e[0].elapsed_time(e[1])
        pf_ms += e[1].elapsed_time(e[2])
    del ck, cv, cq, co
    app_tok_s = n_chunks * ub / (app_ms / 1e3)
    app_bytes = n_chunks * ub * L * kd * 2 * (4 + 2)
    # the same chunks written through all layers per call (tl_kv_append_layers,
    # the session's write-through: launches of 16 layers), rows rewritten with
    # new values at the same positions
    bk = torch.randn((L, ub, kd), generator=gen, device="cuda")
    bv = torch.randn((L, ub, kd), generator=gen, device="cuda")
    arr = (tlkv.KvLayer * L)(*[x.desc for x in layers])
    kp = (ctypes.c_void_p * L)(*[bk[l].data_ptr() for l in range(L)])
    vp_ = (ctypes.c_void_p * L)(*[bv[l].data_ptr() for l in range(L)])
    torch.cuda.synchronize()
    e[0].record(stream)
    for ci in range(n_chunks):
        tlkv.check(lib.tl_kv_append_layers(arr, L, kp, vp_, kd, tlkv.ptr(slots), ci * ub, ub, sh))
    e[1].record(stream)
    torch.cuda.synchronize()
    appl_ms = e[0].elapsed_time(e[1])
    del bk, bv

    # ---- 3. decode ---------------------------------------------------------
    q = torch.randn((L, 1, qd), generator=gen, device="cuda")
    k = torch.randn((L, 1, kd), generator=gen, device="cuda")
    v = torch.randn((L, 1, kd), generator=gen, device="cuda")
    out = torch.empty((L, 1, qd), dtype=torch.float32, device="cuda")
    for l in range(L):
        tlkv.check(lib.tl_rope(tlkv.ptr(q[l]), 1, qd, Hq, d, d, c["ctx"], c["theta"],
                               c["rope_neox"], sh))
        tlkv.check(lib.tl_rope(tlkv.ptr(k[l]), 1, kd, Hkv, d, d, c["ctx"], c["theta"],
                               c["rope_neox"], sh))
    args_l = [tlkv.attn_args(q[l], k[l], v[l], out[l], slots, 0, 1, Hq, d, Hkv, 0, scale)
              for l in range(L)]
    descs = [layers[l].desc for l in range(L)]
    attn = lib.tl_attn

    def step(pos):
        for l in range(L):
            a = args_l[l]
            a.pos = pos
            rc = attn(descs[l], a, sh)
            if rc:
                tlkv.check(rc)

    pos = c["ctx"]
    for _ in range(args.warmup):
        step(pos)
        pos += 1
    torch.cuda.synchronize()

    K = args.steps
    t_start, t_end = ev(), ev()
    pos0 = pos
    torch.cuda.synchronize()
    t_start.record(stream)
    for s in range(K):
        step(pos)
        pos += 1
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    # one OP_ATTN launch per layer and step, back to back on `stream`
    avg_launch_us = total_ms * 1e3 / (K * L)
    launch_bytes = sum(decode_bytes(c, pos0 + s + 1) for s in range(K)) / K
    achieved = launch_bytes / (avg_launch_us * 1e-6) / 1e9
    bytes_total = sum(L * decode_bytes(c, pos0 + s + 1) for s in range(K))
    value = bytes_total / (total_ms / 1e3) / 1e9

    # the same decode over the contiguous cache (no slot table: the layout the
    # reference's device backend uses, graph.c:860-870 builds the radix map
    # only for CPU layers); the slots above are the identity, so the rows are
    # the same
    cont_steps = min(128, K)
    args_c = [tlkv.attn_args(q[l], None, None, out[l], None, pos - 1, 1, Hq, d, Hkv, 0, scale)
              for l in range(L)]
    noapp = lib.tl_attn_noappend
    for l in range(L):
        tlkv.check(noapp(descs[l], args_c[l], sh))
    torch.cuda.synchronize()
    c0, c1 = ev(), ev()
    c0.record(stream)
    for _ in range(cont_steps):
        for l in range(L):
            rc = noapp(descs[l], args_c[l], sh)
            if rc:
                tlkv.check(rc)
    c1.record(stream)
    torch.cuda.synchronize()
    cont_us = c0.elapsed_time(c1) * 1e3 / (cont_steps * L)
    cont_bytes = decode_bytes(c, pos) - Hkv * d * 2 * 6     # no appended row
    decode_contiguous = {"us_per_layer_launch": round(cont_us, 3),
                         "GBs": round(cont_bytes / (cont_us * 1e-6) / 1e9, 1),
                         "hbm_frac": round(cont_bytes / (cont_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "steps": cont_steps,
                         "note": "OP_ATTN without the slot table (contiguous cache, the "
                                 "reference's device layout) and without the fused append, "
                                 f"P = {pos} keys"}

    # the same decode through a randomly permuted slot table (the layout
    # after prefix reuse and eviction: every key's row is somewhere else in
    # the pool); the rows hold the same kind of random data, so only the
    # order of the reads changes
    perm_steps = min(128, K)
    g2 = torch.Generator(device="cpu")
    g2.manual_seed(0x51A7)
    perm = torch.randperm(cap, generator=g2).to(torch.int32).cuda()
    args_p = [tlkv.attn_args(q[l], None, None, out[l], perm, pos - 1, 1, Hq, d, Hkv, 0, scale)
              for l in range(L)]
    for l in range(L):
        tlkv.check(noapp(descs[l], args_p[l], sh))
    torch.cuda.synchronize()
    p0e, p1e = ev(), ev()
    p0e.record(stream)
    for _ in range(perm_steps):
        for l in range(L):
            rc = noapp(descs[l], args_p[l], sh)
            if rc:
                tlkv.check(rc)
    p1e.record(stream)
    torch.cuda.synchronize()
    perm_us = p0e.elapsed_time(p1e) * 1e3 / (perm_steps * L)
    perm_bytes = cont_bytes + pos * 4                   # + the slot-table reads
    decode_permuted = {"us_per_layer_launch": round(perm_us, 3),
                       "GBs": round(perm_bytes / (perm_us * 1e-6) / 1e9, 1),
                       "hbm_frac": round(perm_bytes / (perm_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "steps": perm_steps,
                       "note": "OP_ATTN (no append) through a random permutation of the "
                               f"{cap}-row pool as slot table, P = {pos} keys; bytes include "
                               "the slot-table reads"}
    del perm

    # several batch rows of one session per OP_ATTN (a multi-token decode
    # step: speculative or draft tokens): the matrix-core tile folds the
    # rows of a group into its MFMA columns, so the K/V bytes are read once
    # for all of them; timed against one row per workgroup group
    # (TL_TUNE_DECODE_ROWS = 1), on rows already in the cache (no append)
    mr_n, mr_steps = 4, min(64, K)
    q4 = torch.randn((mr_n, qd), generator=gen, device="cuda")
    o4 = torch.empty((mr_n, qd), dtype=torch.float32, device="cuda")
    a4 = [tlkv.attn_args(q4, None, None, o4, None, pos - mr_n, mr_n, Hq, d, Hkv, 0, scale)
          for l in range(L)]
    mr_us = {}
    for rows in (0, 1):
        with tlkv.tuning(tlkv.TUNE_DECODE_ROWS, rows):
            for l in range(L):
                tlkv.check(noapp(descs[l], a4[l], sh))
            torch.cuda.synchronize()
            e0, e1 = ev(), ev()
            e0.record(stream)
            for _ in range(mr_steps):
                for l in range(L):
                    rc = noapp(descs[l], a4[l], sh)
                    if rc:
                        tlkv.check(rc)
            e1.record(stream)
            torch.cuda.synchronize()
        mr_us["folded" if rows == 0 else "row_per_group"] = e0.elapsed_time(e1) * 1e3 / (mr_steps * L)
    mr_bytes = cont_bytes + (mr_n - 1) * Hq * d * 8     # K/V once; q and out per row
    decode_multi_row = {"rows": mr_n,
                        "us_per_layer_launch": {k_: round(v_, 3) for k_, v_ in mr_us.items()},
                        "GBs_folded": round(mr_bytes / (mr_us["folded"] * 1e-6) / 1e9, 1),
                        "steps": mr_steps,
                        "note": f"OP_ATTN of {mr_n} batch rows of one session at P = {pos} "
                                "keys (contiguous cache, no append): the rows folded into one "
                                "matrix-core group (K/V read once) vs one row per group "
                                "(TL_DECODE_ROWS=1); GBs_folded counts K/V once"}
    del q4, o4

    # decode step with RoPE on q and the new k row (the reference's OP_ROPE x2
    # + OP_ATTN): three launches per layer (tl_rope, tl_rope, tl_attn) vs one
    # (tl_attn_rope), on raw (un-rotated) q/k rows; cache rows written past
    # the timed region's positions, so they never affect `value`
    rope_steps = min(64, K)
    rp = tlkv.RopeParams(d, c["theta"], c["rope_neox"])
    qs = torch.randn((L, 1, qd), generator=gen, device="cuda")
    ks = torch.randn((L, 1, kd), generator=gen, device="cuda")
    def step_rope(pos, fused):
        for l in range(L):
            a = args_l[l]
            a.pos = pos
            if fused:
                a.q, a.k = qs[l].data_ptr(), ks[l].data_ptr()
                tlkv.check(lib.tl_attn_rope(descs[l], a, rp, sh))
            else:
                tlkv.check(lib.tl_rope(tlkv.ptr(q[l]), 1, qd, Hq, d, d, pos, c["theta"],
                                       c["rope_neox"], sh))
                tlkv.check(lib.tl_rope(tlkv.ptr(k[l]), 1, kd, Hkv, d, d, pos, c["theta"],
                                       c["rope_neox"], sh))
                a.q, a.k = q[l].data_ptr(), k[l].data_ptr()
                tlkv.check(attn(descs[l], a, sh))
    rope_us = {}
    for fused in (False, True):
        step_rope(pos, fused)
        torch.cuda.synchronize()
        e0, e1 = ev(), ev()
        e0.record(stream)
        for s in range(rope_steps):
            step_rope(pos + s, fused)
        e1.record(stream)
        torch.cuda.synchronize()
        rope_us["fused" if fused else "separate"] = round(
            e0.elapsed_time(e1) * 1e3 / (rope_steps * L), 2)
    for l in range(L):
        args_l[l].q, args_l[l].k = q[l].data_ptr(), k[l].data_ptr()

    res = {
        "metric": "decode KV-attn GB/s (%HBM peak) + append tok/s, Llama-3-8B shape @32K ctx",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) f32 Q/K/V (device generator), RoPE NORM theta 5e5",
        "config": {"workload": "config 4: Llama-3-8B-shaped KV (L32 Hq32 Hkv8 d128, f16 "
                               f"cache), 1 slot, {c['ctx']}-token cache from 64 x 512-row "
                               f"chunked prefill, then {K} decode steps",
                   "n_layer": L, "n_head": Hq, "n_kv_head": Hkv, "head_dim": d,
                   "ctx": c["ctx"], "slots": 1},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "hbm_read_ceiling_GBs": round(ceiling, 1),
        "host_radix": host_radix_cost(tlkv),
        "decode": {"us_per_layer_launch": round(avg_launch_us, 3),
                   "tok_s": round(K / (total_ms / 1e3), 1),
                   "frac_of_measured_ceiling": round(value / ceiling, 4)},
        "decode_contiguous": decode_contiguous,
        "decode_permuted_slots": decode_permuted,
        "decode_multi_row": decode_multi_row,
        "decode_with_rope_us_per_layer": {**rope_us, "steps": rope_steps,
                                          "note": "RoPE on q and the new k row each step: "
                                                  "tl_rope x2 + tl_attn vs tl_attn_rope"},
        "append_layers": {"tok_s": round(n_chunks * ub / (appl_ms / 1e3), 1),
                          "GBs": round(app_bytes / (appl_ms / 1e3) / 1e9, 1),
                          "note": "the same 64 x 512-row chunks, each written through all 32 "
                                  "layers by one tl_kv_append_layers call (launches of 16 "
                                  "layers), as the session's write-through does"},
        "append": {"tok_s": round(app_tok_s, 1), "GBs": round(app_bytes / (app_ms / 1e3) / 1e9, 1),
                   "note": "64 x 512-row tl_kv_append per layer; a token counts once "
                           "for all 32 layers; decode appends are fused into the decode "
                           "launch (decode.tok_s)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, read "
                                       "from profiles/attn_decode_llama3-8b-32k_hbm_traffic.md "
                                       "(not measured in this run)",
                     "kernel": "attn_decode_ring_kernel<128,4,false,false,true> (one OP_ATTN launch, "
                               "split merge inside)"},
    }
    if not args.no_prefill_attn:
        tf = pf_flops / (pf_ms / 1e3) / 1e12
        res["prefill"] = {"TFLOPs": round(tf, 2), "frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                          "mfma_ceiling_TFLOPs": round(mfma_ceil, 1),
                          "frac_of_measured_mfma_ceiling": round(tf / mfma_ceil, 4),
                          "ms": round(pf_ms, 2), "flops": pf_flops,
                          "kernel": "attn_prefill_kernel<128,4> (+ split merge)"}
        res["prefill_fused_append"] = run_prefill_fused(torch, tlkv, lib, sh, gen, c, layers,
                                                        slots, pf_ms, app_ms, pf_flops)
    del layers, slots, q, k, v, out
    torch.cuda.empty_cache()
    if not args.no_q8:
        res["q8_0_cache"] = run_q8(torch, tlkv, lib, sh, gen, c, K)
        torch.cuda.empty_cache()
    res["state_snapshot"] = run_state_snapshot(torch, tlkv, lib, sh)
    torch.cuda.empty_cache()
    others = {}
    runners = {"1": run_config1, "2": run_config2, "3": run_config3, "5": run_config5}
    for cid in [x for x in args.configs.split(",") if x]:
        others[f"config{cid}"] = runners[cid](torch, tlkv, lib, sh, gen)
        torch.cuda.empty_cache()
    if others:
        res["other_configs"] = others
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(c, c["ctx"] + 1, args.cpu_layers)
        if "config2" in others:
            c2 = dict(Hq=28, Hkv=4, d=128)
            others["config2"]["cpu_baseline"] = cpu_baseline_sessions(c2, 8193, 8, 28)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
