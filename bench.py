#!/usr/bin/env python3
"""Packed-prefill attention throughput on one MI355X.

A step is one pass of the hot path over the workload's packed suffix with
every input resident in HBM: K1 (QK RMSNorm + RoPE with per-block position
restart) then K2 (packed attention over the cached prefix and the suffix
blocks).  The default workload is the 32k-prefix packed-prefill shape: a
Qwen3-8B-shaped layer (Hq=32, Hkv=8, d=128, bf16) with 64 suffix blocks x 64
tokens after a 32768-token cached prefix.

Prints one JSON line: query tokens/s (value), TFLOP/s, the roofline record of
K2 (its average launch time from HIP events on its stream) and the CPU
baseline (the oracle's candle-op restatement on a bounded sample, timed on
this host's cores).
"""
import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "rust-cev_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "packed-prefill attn query tok/s, TFLOP/s and % MFMA/HBM peak on 1 MI355X"
PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}   # dense MFMA at 2.4 GHz
PEAK_HBM_GBPS = 8000.0


def traffic_from_profiles(workload: str):
    """HBM bytes per K2 launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by a copy-kernel calibration), if recorded."""
    path = os.path.join(ROOT, "profiles", "packed_attn_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic\[%s\]\s*=\s*([0-9.]+)" % re.escape(workload), open(path).read())
    return float(m.group(1)) if m else None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, np_inputs, target_s: float = 3.0):
    """The oracle's restatement of the reference's CPU path (candle op order:
    q/k RMSNorm + RoPE, repeat_kv, dense q.k^T over every key, additive
    engine mask, softmax, bf16 rounding points, p.v) on the rows of the first
    n blocks.  The dense mask is built once outside the timed region."""
    import numpy as np

    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    pk, pv, q, k, v, wq, wk = np_inputs
    bf, d = w.bf16, w.d
    pos = w.positions()
    cos, sin = oracle.rope_table(w.theta, w.rotary_dim, w.n_pos(), bf)
    kr = oracle.rope(oracle.rms_norm(k, wk, w.eps, bf, plus_one=w.plus_one), pos, cos, sin, w.rotary_dim, bf)
    kall = np.concatenate([pk, kr.transpose(1, 0, 2)], axis=1) if w.prefix else np.ascontiguousarray(kr.transpose(1, 0, 2))
    vall = np.concatenate([pv, v.transpose(1, 0, 2)], axis=1) if w.prefix else np.ascontiguousarray(v.transpose(1, 0, 2))
    t_mask = time.perf_counter()
    plans, items = w.plans_items()
    mask = oracle.engine_pass(plans, items)["mask"]
    mask_s = time.perf_counter() - t_mask

    def run(nb):
        rows = int(sum(w.blocks[:nb]))
        t0 = time.perf_counter()
        qs = oracle.rope(oracle.rms_norm(q[:rows, :, :d], wq, w.eps, bf, plus_one=w.plus_one), pos[:rows], cos, sin, w.rotary_dim, bf)
        oracle.attend(np.ascontiguousarray(qs.transpose(1, 0, 2)), kall, vall, mask[:rows], bf)
        return rows, time.perf_counter() - t0

    _, t1 = run(1)  # warm-up, sizes the sample
    nb = int(max(1, min(len(w.blocks), round(target_s / max(t1, 1e-3)))))
    times, rows = [], 0
    for _ in range(5):
        rows, dt = run(nb)
        times.append(dt)
    med = statistics.median(times)
    return {
        "value": rows / med,
        "unit": "query tok/s",
        "cores": oracle.threads(),
        "kind": "port",
        "sample": (f"rows of the first {nb} of {len(w.blocks)} suffix blocks ({rows} query rows x {w.hq} heads) through the oracle's "
                   f"candle-op restatement over all {w.prefix + w.t} keys with the dense engine mask; median of 5 runs after a warm-up; "
                   f"dense mask build {mask_s * 1e3:.0f} ms excluded; CPU: {cpu_model()}"),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c3", choices=["c1", "c3", "c4", "c5a", "hbm"])
    ap.add_argument("--cpu-baseline", type=int, default=1, help="0 skips the CPU baseline leg")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the workload, run `steps` device copies of MIB MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings into bytes)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}): this build has no multi-GPU path; "
              "the layer would shard by KV-head group with no exchange inside attention.", file=sys.stderr)
        sys.exit(2)

    import torch

    from cev_hip import configs, device_info
    from cev_hip.layer import AttentionLayer

    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n, "launches": args.warmup + args.steps}), flush=True)
        return
    w = configs.WORKLOADS[args.workload]()
    layer = AttentionLayer(w, dev)
    for _ in range(args.warmup):
        layer.forward()
    torch.cuda.synchronize()

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record()
        layer.qknorm()
        ev[i][1].record()
        layer.attend()
        ev[i][2].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    k1_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in ev)
    k2_ms = statistics.mean(e[1].elapsed_time(e[2]) for e in ev)

    dtype = "bf16" if w.bf16 else "f32"
    flops = w.useful_flops()
    alg = w.alg_bytes()
    intensity = flops / alg
    ridge = PEAK_TFLOPS[dtype] * 1e12 / (PEAK_HBM_GBPS * 1e9)
    if intensity >= ridge:
        roof = {"bound": "mfma", "achieved": flops / (k2_ms * 1e-3) / 1e12, "peak": PEAK_TFLOPS[dtype], "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": alg / (k2_ms * 1e-3) / 1e9, "peak": PEAK_HBM_GBPS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = traffic_from_profiles(w.name)
    roof["kernel"] = "attn_bf16_kernel" if w.bf16 else "attn_f32_kernel"
    roof["kernel_ms"] = k2_ms
    roof["alg_bytes"] = alg
    roof["useful_flop"] = flops

    res = {
        "metric": METRIC,
        "value": w.t / (ms_step * 1e-3),
        "unit": "query tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded N(0,1) q/k/v and prefix K/V, QK-norm weights 1 + 0.1 N(0,1))",
        "config": {
            "workload": f"{w.name}: {w.notes}",
            "hq": w.hq, "hkv": w.hkv, "head_dim": w.d, "prefix": w.prefix,
            "suffix_blocks": len(w.blocks), "block_len": w.blocks[0], "query_tokens": w.t,
            "causal": w.causal, "gated": w.gated,
        },
        "tflops": flops / (ms_step * 1e-3) / 1e12,
        "k1_ms": k1_ms,
        "k2_ms": k2_ms,
        "roofline": roof,
        "device": device_info().name,
    }
    if args.cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w, layer.np_inputs)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
