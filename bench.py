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
  roofline      the decode attention launch (decode kernel + split merge):
                algorithmic bytes per launch / average launch time, measured
                with HIP events on the launch stream on every 8th step
  cpu_baseline  the reference's own op_attn (oracle/_ref, compiled from the
                reference sources) timed on a bounded sample of the same
                decode step, single thread
  prefill, append, hbm_read_ceiling   the other measured rows
"""
import argparse
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


def prefill_flops(c, p0, n):
    """QK^T + PV flops of one layer's chunk of n rows at positions p0.. (causal)."""
    keys = n * p0 + n * (n + 1) // 2
    return 4 * c["Hq"] * c["d"] * keys


def cpu_baseline(c, P, n_layers_sample):
    """The reference op_attn (compiled reference, f32 cache, one thread) on
    `n_layers_sample` layers of one decode step at P keys."""
    import oracle as O
    rng = np.random.default_rng(7)
    kind = "reference" if O.ref_available() else "port"
    kd = c["Hkv"] * c["d"]
    kc = rng.standard_normal((c["Hkv"], P, c["d"]), dtype=np.float32)
    vc = rng.standard_normal((c["Hkv"], P, c["d"]), dtype=np.float32)
    slots = np.arange(P, dtype=np.uint32)
    secs = 0.0
    for _ in range(n_layers_sample):
        q = rng.standard_normal((1, c["Hq"] * c["d"]), dtype=np.float32)
        k = rng.standard_normal((1, kd), dtype=np.float32)
        v = rng.standard_normal((1, kd), dtype=np.float32)
        t0 = time.perf_counter()
        if kind == "reference":
            O.ref_attn(kc, vc, q, k, v, slots, P - 1, 1, c["Hq"])
        else:
            C = O.Cache(P, c["Hkv"], c["d"], f16=False)
            C.k, C.v = kc, vc
            O.attn(C, q, k, v, slots, P - 1, 1, c["Hq"])
        secs += time.perf_counter() - t0
    per_layer = secs / n_layers_sample
    gbs = decode_bytes(c, P) / per_layer / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{n_layers_sample} layer calls of one decode step at P={P} "
                      f"(op_attn over an f32 cache, single thread, {os.cpu_count()} host "
                      f"cores present), {per_layer * 1e3:.1f} ms per layer; GB/s counts "
                      f"the f16 workload's algorithmic bytes"}


def profiled_traffic():
    """HBM bytes per decode launch pair from the committed rocprofv3 FETCH_SIZE /
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-layers", type=int, default=96,
                    help="decode-layer calls timed for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill-attn", action="store_true",
                    help="fill the cache with appends only (skips phase 2)")
    ap.add_argument("--ctx", type=int, default=CFG4["ctx"])
    args = ap.parse_args()
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
    cap = c["ctx"] + args.warmup + args.steps
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    sh = tlkv.stream_handle(stream)
    ev = lambda: torch.cuda.Event(enable_timing=True)

    ceiling = hbm_read_ceiling(torch, tlkv, lib, sh)

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

    def step(pos, evs=None):
        for l in range(L):
            a = args_l[l]
            a.pos = pos
            if evs is not None:
                evs[0][l].record(stream)
            rc = attn(descs[l], a, sh)
            if rc:
                tlkv.check(rc)
            if evs is not None:
                evs[1][l].record(stream)

    pos = c["ctx"]
    for _ in range(args.warmup):
        step(pos)
        pos += 1
    torch.cuda.synchronize()

    K = args.steps
    SAMPLE = 8
    sampled = {s: [[ev() for _ in range(L)], [ev() for _ in range(L)]]
               for s in range(0, K, SAMPLE)}
    t_start, t_end = ev(), ev()
    pos0 = pos
    torch.cuda.synchronize()
    t_start.record(stream)
    for s in range(K):
        step(pos, sampled.get(s))
        pos += 1
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)

    launch_ms, launch_bytes, n_launch = 0.0, 0.0, 0
    for s, (ea, eb) in sampled.items():
        for l in range(L):
            launch_ms += ea[l].elapsed_time(eb[l])
            launch_bytes += decode_bytes(c, pos0 + s + 1)
            n_launch += 1
    avg_launch_us = launch_ms * 1e3 / n_launch
    achieved = launch_bytes / n_launch / (avg_launch_us * 1e-6) / 1e9
    bytes_total = sum(L * decode_bytes(c, pos0 + s + 1) for s in range(K))
    value = bytes_total / (total_ms / 1e3) / 1e9

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
        "decode": {"us_per_layer_launch": round(avg_launch_us, 3),
                   "tok_s": round(K / (total_ms / 1e3), 1),
                   "frac_of_measured_ceiling": round(value / ceiling, 4)},
        "append": {"tok_s": round(app_tok_s, 1), "GBs": round(app_bytes / (app_ms / 1e3) / 1e9, 1),
                   "note": "64 x 512-row tl_kv_append per layer; a token counts once "
                           "for all 32 layers; decode appends are fused into the decode "
                           "launch (decode.tok_s)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "kernel": "attn_decode_kernel<128,4> + attn_merge_kernel<128> "
                               "(one OP_ATTN launch pair)"},
    }
    if not args.no_prefill_attn:
        tf = pf_flops / (pf_ms / 1e3) / 1e12
        res["prefill"] = {"TFLOPs": round(tf, 2), "frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                          "ms": round(pf_ms, 2), "flops": pf_flops,
                          "kernel": "attn_prefill_kernel<128,4> (+ split merge)"}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(c, c["ctx"] + 1, args.cpu_layers)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
