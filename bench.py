"""Benchmark of the KV-cache hot path on one MI355X.

Workload (the north star): Llama-3-8B-shaped KV —
32 layers, 32 q-heads, 8 kv-heads, head_dim 128, f16 cache, 1 slot.  A
32 768-token cache is filled by 64 chunked-prefill OP_ATTN calls of 512 rows
(append + MFMA prefill attention), then decode steps run: one step = for each
of the 32 layers, the one-token append and the GQA decode attention over the
whole cache (OP_ATTN).  Inputs are seeded N(0,1) f32 with RoPE (NORM, theta
5e5) applied to Q and K once at set-up.

One JSON line is printed:
  value      decode KV-attention throughput, GB/s of algorithmic bytes
             (f16 K+V rows read, q read, out written, appended rows)
  roofline   the decode attention kernel: algorithmic bytes per launch over
             its average HIP-event duration, against 8 TB/s
  cpu_baseline  the reference's own op_attn (oracle/_ref, compiled from the
             reference sources) — or the oracle port when _ref is absent —
             timed on a bounded sample of the same decode step
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

CFG4 = dict(name="llama3-8b-kv@32k", L=32, Hq=32, Hkv=8, d=128, ctx=32768,
            ub=512, theta=500000.0, rope_neox=0)


def decode_bytes(c, P):
    """Algorithmic bytes of one decode OP_ATTN on one layer with P visible keys:
    f16 K+V rows read, q read (f32), out written (f32), the new K/V row read
    (f32) and written (f16)."""
    B = 2 * c["Hkv"] * c["d"] * 2
    return P * B + c["Hq"] * c["d"] * 4 * 2 + c["Hkv"] * c["d"] * 2 * (4 + 2)


def cpu_baseline(c, P, n_layers_sample):
    """Time the reference op_attn (compiled reference, f32 cache, single thread)
    on `n_layers_sample` layers of one decode step at P keys."""
    import oracle as O
    rng = np.random.default_rng(7)
    kind = "reference" if O.ref_available() else "port"
    kd = c["Hkv"] * c["d"]
    cap = P
    kc = rng.standard_normal((c["Hkv"], cap, c["d"]), dtype=np.float32)
    vc = rng.standard_normal((c["Hkv"], cap, c["d"]), dtype=np.float32)
    slots = np.arange(cap, dtype=np.uint32)
    secs = 0.0
    for l in range(n_layers_sample):
        q = rng.standard_normal((1, c["Hq"] * c["d"]), dtype=np.float32)
        k = rng.standard_normal((1, kd), dtype=np.float32)
        v = rng.standard_normal((1, kd), dtype=np.float32)
        t0 = time.perf_counter()
        if kind == "reference":
            O.ref_attn(kc, vc, q, k, v, slots, P - 1, 1, c["Hq"])
        else:
            C = O.Cache(cap, c["Hkv"], c["d"], f16=False)
            C.k, C.v = kc, vc
            O.attn(C, q, k, v, slots, P - 1, 1, c["Hq"])
        secs += time.perf_counter() - t0
    per_layer = secs / n_layers_sample
    gbs = decode_bytes(c, P) / per_layer / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{n_layers_sample} layers of one decode step at P={P} "
                      f"(op_attn over an f32 cache, single thread), "
                      f"{per_layer * 1e3:.1f} ms/layer; bytes counted as the "
                      f"f16 workload's algorithmic bytes"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-layers", type=int, default=128,
                    help="layers of one decode step timed for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ctx", type=int, default=CFG4["ctx"])
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs "
                                   "are not part of it (see DESIGN.md)"}))
        sys.exit(2)

    import torch
    import tlkv
    c = dict(CFG4)
    c["ctx"] = args.ctx
    T = torch
    lib = tlkv.lib()
    tlkv.check(lib.tl_init(0))
    dev = "cuda"
    L, Hq, Hkv, d, ub = c["L"], c["Hq"], c["Hkv"], c["d"], c["ub"]
    kd, qd = Hkv * d, Hq * d
    cap = c["ctx"] + args.warmup + args.steps
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    stream = torch.cuda.current_stream()
    sh = tlkv.stream_handle(stream)

    gen = torch.Generator(device=dev)
    gen.manual_seed(0x9E3779B9 ^ 4)
    layers = [tlkv.Layer(cap, Hkv, d, device=dev) for _ in range(L)]
    slots = torch.arange(cap, dtype=torch.int32, device=dev)  # fresh pool: slot i for pos i

    # ---- prefill: 64 chunked appends of 512 rows per layer -------------------
    n_chunks = c["ctx"] // ub
    ck = torch.empty((L, ub, kd), dtype=torch.float32, device=dev)
    cv = torch.empty((L, ub, kd), dtype=torch.float32, device=dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    app_ms = 0.0
    for ci in range(n_chunks):
        ck.normal_(generator=gen)
        cv.normal_(generator=gen)
        for l in range(L):
            tlkv.check(lib.tl_rope(tlkv.ptr(ck[l]), ub, kd, Hkv, d, d, ci * ub,
                                   c["theta"], c["rope_neox"], sh))
        ev[0].record(stream)
        for l in range(L):
            tlkv.check(lib.tl_kv_append(layers[l].desc, tlkv.ptr(ck[l]), tlkv.ptr(cv[l]),
                                        kd, tlkv.ptr(slots), ci * ub, ub, sh))
        ev[1].record(stream)
        torch.cuda.synchronize()
        app_ms += ev[0].elapsed_time(ev[1])
    prefill_tokens = n_chunks * ub
    prefill_append_tok_s = prefill_tokens / (app_ms / 1e3)

    # ---- decode inputs --------------------------------------------------------
    q = torch.randn((L, 1, qd), generator=gen, device=dev)
    k = torch.randn((L, 1, kd), generator=gen, device=dev)
    v = torch.randn((L, 1, kd), generator=gen, device=dev)
    out = torch.empty((L, 1, qd), dtype=torch.float32, device=dev)
    for l in range(L):
        tlkv.check(lib.tl_rope(tlkv.ptr(q[l]), 1, qd, Hq, d, d, c["ctx"], c["theta"],
                               c["rope_neox"], sh))
        tlkv.check(lib.tl_rope(tlkv.ptr(k[l]), 1, kd, Hkv, d, d, c["ctx"], c["theta"],
                               c["rope_neox"], sh))
    args_l = [tlkv.attn_args(q[l], k[l], v[l], out[l], slots, 0, 1, Hq, d, Hkv, 0, scale)
              for l in range(L)]

    def step(pos, evs=None):
        # one OP_ATTN per layer: append of the new row + decode attention
        for l in range(L):
            a = args_l[l]
            a.pos = pos
            if evs is not None:
                evs[0][l].record(stream)
            tlkv.check(lib.tl_attn(layers[l].desc, a, sh))
            if evs is not None:
                evs[1][l].record(stream)

    pos = c["ctx"]
    for _ in range(args.warmup):
        step(pos)
        pos += 1
    torch.cuda.synchronize()

    K = args.steps
    evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(L)] for _ in range(2)]
           for _ in range(K)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    pos0 = pos
    torch.cuda.synchronize()
    t_start.record(stream)
    for s in range(K):
        step(pos, evs[s])
        pos += 1
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)

    attn_ms = 0.0
    for s in range(K):
        for l in range(L):
            attn_ms += evs[s][0][l].elapsed_time(evs[s][1][l])
    n_launch = K * L
    bytes_total = sum(L * decode_bytes(c, pos0 + s + 1) for s in range(K))
    kv_bytes_launch = sum(decode_bytes(c, pos0 + s + 1) for s in range(K)) / K
    avg_attn_us = attn_ms * 1e3 / n_launch
    achieved = kv_bytes_launch / (avg_attn_us * 1e-6) / 1e9
    value = bytes_total / (total_ms / 1e3) / 1e9
    ms_per_step = total_ms / K
    gap_us = (total_ms - attn_ms) * 1e3 / n_launch  # host-side gaps between launches

    res = {
        "metric": "decode KV-attn GB/s (%HBM peak) + append tok/s, Llama-3-8B shape @32K ctx",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) f32 Q/K/V, RoPE NORM theta 5e5",
        "config": {"workload": "config 4: Llama-3-8B-shaped KV (L32 Hq32 Hkv8 d128), "
                               f"1 slot, {c['ctx']}-token cache, {K} decode steps",
                   "n_layer": L, "n_head": Hq, "n_kv_head": Hkv, "head_dim": d,
                   "ctx": c["ctx"], "slots": 1},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "append_tok_s": {"prefill": round(prefill_append_tok_s, 1),
                         "decode": round(K / (total_ms / 1e3), 1),
                         "note": "tokens appended to all 32 layers per second; prefill: "
                                 "512-row append kernels alone; decode: whole fused "
                                 "append+attention steps"},
        "decode_attn_us_per_layer": round(avg_attn_us, 3),
        "gap_us_per_layer": round(gap_us, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "attn_decode_kernel<128,4> (+ attn_merge_kernel<128>)"},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(c, c["ctx"] + 1, args.cpu_layers)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
