#!/usr/bin/env python3
"""Packed-prefill attention throughput on one MI355X.

A step is one pass of the hot path over the workload's packed suffix with
every input resident in HBM: K1 (QK RMSNorm + RoPE with per-block position
restart) then K2 (packed attention over the cached prefix and the suffix
blocks), and for the d3 workload (c4) the readout of the last position.  The default workload is the 32k-prefix packed-prefill shape: a
Qwen3-8B-shaped layer (Hq=32, Hkv=8, d=128, bf16) with 64 suffix blocks x 64
tokens after a 32768-token cached prefix.

Prints one JSON line: query tokens/s (value), TFLOP/s, the roofline record of
K2 (its average launch time from HIP events on its stream), the CPU baseline
(the oracle's candle-op restatement on a bounded sample, timed on this
host's cores) and, for the default workload, K2 on the HBM-bound
32k-prefix x 16-token shape under hbm_shape and K2 on config 4's d = 256
bidirectional row under c4_shape (both outside the timed steps).
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


# Kernel source each workload's measured traffic depends on.
TRAFFIC_SOURCES = {"c5gdn": "gdn.hip", "c5gdnrows": "gdn.hip"}


def source_sha16(name: str) -> str:
    """First 16 hex digits of the SHA-256 of rust-cev_amd/csrc/<name>."""
    import hashlib
    with open(os.path.join(ROOT, "rust-cev_amd", "csrc", name), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def traffic_from_profiles(workload: str):
    """HBM bytes per K2 launch (or per GDN forward call) measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by a copy-kernel calibration), if recorded for the kernel source in the tree:
    each recorded value names the SHA-256 prefix of the source it was measured on, and a value
    measured on another version of the kernel is not reported (None)."""
    path = os.path.join(ROOT, "profiles", "packed_attn_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic\[%s\]\s*=\s*([0-9.]+)\s+src=([0-9a-f]{16})" % re.escape(workload), open(path).read())
    if not m:
        return None
    src = TRAFFIC_SOURCES.get(workload, "packed_attn.hip")
    return float(m.group(1)) if m.group(2) == source_sha16(src) else None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _sample_rows(run, total: int, step: int, target_s: float):
    """Times run(rows) once on `step` rows (warm-up), sizes a sample of about
    target_s seconds in multiples of `step`, and returns (rows, median s of 5)."""
    _, t1 = run(step)
    n = int(max(1, min(total // step, round(target_s / max(t1, 1e-3)))))
    times, rows = [], 0
    for _ in range(5):
        rows, dt = run(n * step)
        times.append(dt)
    return rows, statistics.median(times)


def cpu_baseline(w, np_inputs, target_s: float = 3.0):
    """The oracle's restatement of the reference's CPU path on the first rows
    of the suffix, in candle's op order: q/k RMSNorm + RoPE, repeat_kv, dense
    q.k^T over every key, the additive mask the reference builds for this
    layer (the engine's packed mask for causal blocks, the bidirectional row
    mask otherwise), softmax, bf16 rounding points, p.v and, for a gated
    layer, the sigmoid gate.  The two products run as register-blocked
    AVX2/FMA kernels, as a BLAS-backed CPU path computes them.  Masks are
    built once outside the timed region."""
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
    if w.causal:
        plans, items = w.plans_items()
        mask, mask_kind = oracle.engine_pass(plans, items)["mask"], "engine packed mask"
    else:
        assert len(w.blocks) == 1 and not w.prefix
        mask, mask_kind = oracle.bidirectional_mask(w.t, [w.lengths[0]])[0], "bidirectional row mask"
    mask_s = time.perf_counter() - t_mask

    def run(rows):
        t0 = time.perf_counter()
        qs = oracle.rope(oracle.rms_norm(q[:rows, :, :d], wq, w.eps, bf, plus_one=w.plus_one), pos[:rows], cos, sin,
                         w.rotary_dim, bf)
        out = oracle.attend_blocked(np.ascontiguousarray(qs.transpose(1, 0, 2)), kall, vall, mask[:rows], bf)
        if w.gated:
            o = np.ascontiguousarray(out[0].transpose(1, 0, 2)).reshape(rows, -1)
            oracle.sigmoid_gate(o, np.ascontiguousarray(q[:rows, :, d:]).reshape(rows, -1), bf)
        return rows, time.perf_counter() - t0

    step = w.blocks[0] if w.causal else 64
    rows, med = _sample_rows(run, w.t, step, target_s)
    return {
        "value": rows / med,
        "unit": "query tok/s",
        "cores": oracle.threads(),
        "kind": "port",
        "sample": (f"the first {rows} of {w.t} suffix query rows x {w.hq} heads through the oracle's candle-op restatement "
                   f"over all {w.prefix + w.t} keys with the dense {mask_kind}, its q.k^T and p.v as register-blocked AVX2/FMA "
                   f"products over cache blocks of keys (oracle/cpu_attend.c); median of 5 runs after a warm-up; mask build "
                   f"{mask_s * 1e3:.0f} ms excluded; CPU: {cpu_model()}"),
    }


def cpu_baseline_gdn(w, inp, target_s: float = 3.0):
    """The oracle's restatement of GatedDeltaNet::forward between the input
    projections and out_proj (conv + SiLU, gates, chunk_gated_delta_rule,
    gated RMSNorm) on the first tokens of row 0."""
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()

    def run(n):
        t0 = time.perf_counter()
        oracle.gdn_layer(inp["mixed"][:1, :n], inp["z"][:1, :n], inp["b"][:1, :n], inp["a"][:1, :n], inp["conv_w"],
                         inp["neg_a"], inp["dt_bias"], inp["norm_w"], w.nk, w.nv, w.dk, w.dv, w.eps, w.bf16)
        return n, time.perf_counter() - t0

    n, med = _sample_rows(run, w.t, 64, target_s)
    return {
        "value": n / med,
        "unit": "tok/s",
        "cores": oracle.threads(),
        "kind": "port",
        "sample": (f"the first {n} of {w.t} tokens of one row ({w.nv} value heads) through the oracle's restatement of the "
                   f"layer (conv + SiLU, gates, 64-token chunked delta rule, gated RMSNorm); median of 5 runs after a "
                   f"warm-up; CPU: {cpu_model()}"),
    }


def roofline(flops: float, alg: int, ms: float, dtype: str, kernel: str, traffic):
    intensity = flops / alg
    ridge = PEAK_TFLOPS[dtype] * 1e12 / (PEAK_HBM_GBPS * 1e9)
    if intensity >= ridge:
        roof = {"bound": "mfma", "achieved": flops / (ms * 1e-3) / 1e12, "peak": PEAK_TFLOPS[dtype], "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": alg / (ms * 1e-3) / 1e9, "peak": PEAK_HBM_GBPS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = traffic
    roof["kernel"] = kernel
    roof["kernel_ms"] = ms
    roof["alg_bytes"] = alg
    roof["useful_flop"] = flops
    return roof


def capture(fns):
    """One HIP graph per callable: every kernel the callable launches on the
    current stream is recorded once and replayed without host work."""
    import torch
    graphs = []
    for f in fns:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            f()
        graphs.append(g)
    torch.cuda.synchronize()
    return graphs


SETTLE = {"ms": 0.0, "launches": 0}


def settle(step, ms: float):
    """Runs `step` back to back until about `ms` of wall clock has passed,
    before the warm-up steps.  A card that was idle runs its first launches
    slow while its clocks ramp up (the 2 ms packed-prefill step takes 2.20 ms
    at first and settles at 1.98 ms after about 8 steps), so the timed steps
    start at the steady clock.  Nothing from these launches is timed or kept;
    the totals go into the JSON line as "settle"."""
    import torch
    if ms <= 0:
        return
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            step()
        n += 4
        torch.cuda.synchronize()
    SETTLE["ms"] += (time.perf_counter() - t0) * 1e3
    SETTLE["launches"] += n


def calibrate_gemm(n: int, steps: int, warmup: int):
    """The practical bf16 MFMA ceiling on this card: hipBLASLt's n^3 GEMM
    (torch.matmul) on random N(0,1) operands and on all-zero operands.  The
    gap between the two is the power limit that random data hits."""
    import torch
    dev = torch.device("cuda:0")
    out = {"calibrate_gemm": n}
    for name, make in (("random", torch.randn), ("zeros", torch.zeros)):
        a = make((n, n), dtype=torch.bfloat16, device=dev)
        b = make((n, n), dtype=torch.bfloat16, device=dev)
        for _ in range(warmup):
            torch.matmul(a, b)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            torch.matmul(a, b)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        out[name] = {"ms": ms, "tflops": 2.0 * n ** 3 / (ms * 1e-3) / 1e12}
    print(json.dumps(out), flush=True)


def bench_gdn(args, w, dev, traffic_key: str):
    """One step = the GatedDeltaNet layer core (four kernels) over the batch."""
    import numpy as np
    import torch

    import cev_hip
    from cev_hip import configs, device_info
    inp = w.inputs()
    mdt = torch.bfloat16 if w.bf16 else torch.float32

    def d(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(mdt)

    def f(x):
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)

    layer = cev_hip.GatedDeltaNet(w.batch, w.t, w.nk, w.nv, w.dk, w.dv, w.kernel, w.eps, dtype=mdt, device=dev)
    xs = [d(inp[k]) for k in ("mixed", "z", "b", "a", "conv_w")] + [f(inp[k]) for k in ("neg_a", "dt_bias", "norm_w")]
    s_in = conv_in = None
    prefill = None
    if w.batch > 1:
        # The rows continue from config 5's 4096-token prefill (hybrid.rs:554-617):
        # its conv tail and recurrent state, computed once here outside the
        # timed steps, are read by every row through batch stride 0.
        pw = configs.c5_gdn()
        pinp = pw.inputs()
        player = cev_hip.GatedDeltaNet(1, pw.t, pw.nk, pw.nv, pw.dk, pw.dv, pw.kernel, pw.eps, dtype=mdt, device=dev)
        pxs = [d(pinp[k]) for k in ("mixed", "z", "b", "a")] + [xs[4]] + xs[5:]
        _, pconv, pstate = player(*pxs)
        conv_in = pconv.expand(w.batch, -1, -1)
        s_in = pstate.expand(w.batch, -1, -1, -1)
        prefill = f"state from the {pw.t}-token prefill ({pw.name}), computed once before the timed steps"
        del player
    y = torch.empty((w.batch, w.t, w.nv * w.dv), dtype=mdt, device=dev)
    conv_out = torch.empty((w.batch, w.conv_dim, w.kernel - 1), dtype=mdt, device=dev)
    s_out = torch.empty((w.batch, w.nv, w.dk, w.dv), dtype=torch.float32, device=dev)
    def fwd():
        layer(*xs, conv_in=conv_in, s_in=s_in, y=y, conv_out=conv_out, s_out=s_out)

    settle(fwd, args.settle_ms)
    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    if args.graph:
        (g,) = capture([fwd])
        fwd = g.replay
        for _ in range(args.warmup):
            fwd()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        fwd()
        b.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    layer_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    esz = 2 if w.bf16 else 4
    tok = w.batch * w.t
    # inputs and y once per token, every row's new state and conv tail, and
    # the one broadcast initial state and tail the rows read
    state, tail = w.nv * w.dk * w.dv * 4, w.conv_dim * (w.kernel - 1) * esz
    alg = (tok * (w.conv_dim + 2 * w.nv * w.dv + 2 * w.nv) * esz + w.batch * (state + tail)
           + ((state + tail) if s_in is not None else 0))
    res = {
        "metric": "Gated DeltaNet layer core tok/s and % f32 MFMA peak on 1 MI355X",
        "value": tok / (ms_step * 1e-3),
        "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded projection outputs; beta uniform in (0,1), decay log-uniform in [1e-3, 1])",
        "config": {"workload": f"{w.name}: Gated DeltaNet layer, batch {w.batch} x {w.t} tokens, Hk={w.nk} Hv={w.nv} "
                               f"dk={w.dk} dv={w.dv}, conv kernel {w.kernel}, 64-token chunks, "
                               f"{'bf16' if w.bf16 else 'f32'} inputs, f32 chunk rule",
                   "launch": "hip graph replay" if args.graph else "direct launches",
                   **({"initial_state": prefill} if prefill else {})},
        "roofline": roofline(w.flops(), alg, layer_ms, "f32", "gdn conv + prep + scan + norm (one forward call)",
                             traffic_from_profiles(traffic_key)),
        "device": device_info().name,
        "settle": dict(SETTLE),
    }
    if args.cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_gdn(w, inp)
    print(json.dumps(res), flush=True)


def cpu_baseline_stack(w, target_layers: int = 1):
    """The oracle's restatement of one decoder layer of the packed pass
    (f32 BLAS GEMMs with the model dtype's rounding points, the pinned
    QK-norm + RoPE and candle-op attention with the engine mask, SwiGLU),
    scaled by the layer count."""
    import numpy as np

    import oracle
    from cev_hip import configs
    from oracle.qwen3_stack import Qwen3Oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    w1 = configs.Qwen3StackWorkload(w.name, w.seed, w.bf16, n_layers=target_layers, vocab=4096)
    o = Qwen3Oracle(w1, w1.weights())
    state, qs, _ = w1.ids()
    o.prefill(state[: w1.head_tokens], w1.prefill_chunk)
    plans, items = w1.plans_items()
    tokens = np.concatenate([state[w1.head_tokens:], qs.reshape(-1)])
    ep = oracle.engine_pass(plans, items)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        o._layers(tokens, ep["pos"], ep["mask"])
        times.append(time.perf_counter() - t0)
    per_layer = statistics.median(times) / target_layers
    return {
        "value": w1.pass_tokens / (per_layer * w.n_layers),
        "unit": "query tok/s",
        "cores": oracle.threads(),
        "kind": "port",
        "sample": (f"{target_layers} decoder layer(s) of the packed pass ({w1.pass_tokens} tokens over a {w1.head_tokens}-token "
                   f"cached head) through the oracle's restatement, scaled to {w.n_layers} layers; median of 3; CPU: {cpu_model()}"),
    }


def bench_stack(args, w, dev):
    """Config 2: one step = one packed pass (the 512-token tail plus 64
    question blocks of 48 tokens) through all 28 layers over the prefilled
    1536-token head; the prefill is timed once beside it."""
    import numpy as np
    import torch

    from cev_hip import BlockTable, device_info
    from cev_hip.qwen3 import Qwen3Stack
    dtype = torch.bfloat16 if w.bf16 else torch.float32
    stack = Qwen3Stack(w, w.device_weights(dev, dtype), dev, capacity=w.state_tokens + w.questions * w.q_len)
    torch.cuda.empty_cache()
    state, qs, codes = w.ids()
    # the head is prefilled into slots [0, head) (engine.rs:247-256); the
    # pass computes the tail into [head, state) and the questions into the
    # slots after it
    stack.prefill(0, state[: w.head_tokens], w.prefill_chunk)  # warm-up (library GEMM selection)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    stack.prefill(0, state[: w.head_tokens], w.prefill_chunk)
    e1.record()
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    items = [(0, w.q_len, w.state_tokens + k * w.q_len) for k in range(w.questions)]
    table, pos, slots, gather = BlockTable.from_slots([(0, w.state_tokens, w.head_tokens)], items, stack.capacity)
    tokens = np.concatenate([state[w.head_tokens:], qs.reshape(-1)])

    def step():
        # one packed pass (the tail lands in its slots again, with the same
        # values) and the code-head logits
        return stack.code_logits(stack.hidden(stack.run(tokens, pos, slots, table), gather), codes)

    settle(step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        step()
        b.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    pass_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    fl = w.flops()
    dt = "bf16" if w.bf16 else "f32"
    res = {
        "metric": METRIC,
        "value": w.pass_tokens / (ms_step * 1e-3),
        "unit": "query tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic (random token ids; weights N(0, 0.02) drawn on the device, norm weights 1)",
        "config": {"workload": f"c2: Qwen3-1.7B-shaped stack ({w.n_layers} layers, hidden {w.hidden}, Hq={w.hq}, Hkv={w.hkv}, "
                               f"d={w.d}, intermediate {w.inter}, vocab {w.vocab}), one packed pass of {w.pass_tokens} tokens "
                               f"(tail {w.state_tokens - w.head_tokens} + {w.questions} x {w.q_len}) over a {w.head_tokens}-token "
                               f"prefilled head, code-head logits over {w.n_codes} codes",
                   "launch": "direct launches"},
        "tflops": fl["pass"] / (ms_step * 1e-3) / 1e12,
        "pass_ms": pass_ms,
        "prefill_ms": prefill_ms,
        "prefill_tflops": fl["prefill"] / (prefill_ms * 1e-3) / 1e12,
        "roofline": roofline(fl["pass"], 1, pass_ms, dt, "whole pass (library GEMMs + K1 + K2 + norms + SwiGLU)", None),
        "device": device_info().name,
        "settle": dict(SETTLE),
    }
    res["roofline"]["alg_bytes"] = None
    if args.cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_stack(w)
    print(json.dumps(res), flush=True)


MALL_EVICT_BYTES = 512 << 20  # twice the 256 MB memory-side cache (MALL) in front of HBM


def mall_evictor(dev):
    """Returns a function that reads a 512 MiB buffer, so that what the
    previous step left in the 256 MB MALL is evicted with clean lines (a
    write would leave dirty lines whose write-backs then compete with the
    next step's reads).  In a pass through many layers each layer's K/V
    comes cold from HBM; back-to-back steps of one layer would otherwise
    read part of a 134 MB prefix from the MALL."""
    import torch
    buf = torch.ones(MALL_EVICT_BYTES // 8, dtype=torch.int64, device=dev)
    acc = torch.zeros((), dtype=torch.int64, device=dev)

    def evict():
        acc.add_(buf.sum())
    return evict


def time_layer(layer, steps: int, warmup: int, graph: bool, settle_ms: float = 0.0, evict=None):
    """Times `steps` steps of one attention layer: K1, K2 and, for a d3
    workload, the readout of the last position, each bracketed by HIP events
    on the stream they launch on.  With `evict`, it runs before each timed
    step, outside the events, and the step time is the sum of the parts'
    event means instead of the host clock.  Returns (ms per step, mean K1 ms,
    mean K2 ms, mean readout ms or None)."""
    import torch
    parts = [layer.qknorm, layer.attend] + ([layer.read_out] if layer.readout is not None else [])

    def one_step():
        for f in parts:
            f()

    settle(one_step, settle_ms)
    for _ in range(warmup):
        for f in parts:
            f()
    torch.cuda.synchronize()
    if graph:
        parts = [g.replay for g in capture(parts)]
        for _ in range(warmup):
            for f in parts:
                f()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        if evict is not None:
            evict()
        ev[i][0].record()
        for j, f in enumerate(parts):
            f()
            ev[i][j + 1].record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    means = [statistics.mean(e[j].elapsed_time(e[j + 1]) for e in ev) for j in range(len(parts))]
    if evict is not None:
        ms_step = sum(means)
    return ms_step, means[0], means[1], (means[2] if len(means) > 2 else None)


def hbm_shape_record(dev, steps: int, warmup: int, settle_ms: float):
    """K2 on the long-prefix short-suffix shape (the 32768-key prefix with one
    16-token block), where the kernel streams K/V and HBM bandwidth bounds
    it: its mean time and the fraction of the 8 TB/s peak, with the MALL
    evicted before each step (the K/V comes from HBM, as in a pass through
    many layers), and the same with the MALL left warm by the previous step
    under "warm_mall"."""
    from cev_hip import configs
    from cev_hip.layer import AttentionLayer
    w = configs.hbm(1)
    layer = AttentionLayer(w, dev)
    _, k1_ms, k2_ms, _ = time_layer(layer, steps, warmup, False, settle_ms, evict=mall_evictor(dev))
    _, k1w_ms, k2w_ms, _ = time_layer(layer, steps, warmup, False, 0.0)
    gbps, gbps_w = (w.alg_bytes() / (ms * 1e-3) / 1e9 for ms in (k2_ms, k2w_ms))
    return {"workload": f"{w.name}: {w.notes}", "k1_ms": k1_ms, "k2_ms": k2_ms, "alg_bytes": w.alg_bytes(),
            "achieved_gbps": gbps, "peak_gbps": PEAK_HBM_GBPS, "frac": gbps / PEAK_HBM_GBPS, "settle_ms": settle_ms,
            "mall": "evicted before each step (a 512 MiB read outside the timed events)",
            "warm_mall": {"k1_ms": k1w_ms, "k2_ms": k2w_ms, "achieved_gbps": gbps_w, "frac": gbps_w / PEAK_HBM_GBPS},
            "kernel": "attn_kernel_pipe<bf16,128> (split) + attn_merge_kernel"}


def c4_shape_record(dev, steps: int, warmup: int, settle_ms: float):
    """K2 on config 4 (the Qwen3.5-style gated layer, d = 256, one
    bidirectional 8192-token row): the d = 256 kernel's mean time, useful
    TFLOP/s and fraction of the bf16 MFMA peak.  K1 and the d3 readout are
    timed with it and reported beside."""
    from cev_hip import configs
    from cev_hip.layer import AttentionLayer
    w = configs.c4()
    _, k1_ms, k2_ms, k3_ms = time_layer(AttentionLayer(w, dev), steps, warmup, False, settle_ms)
    roof = roofline(w.useful_flops(), w.alg_bytes(), k2_ms, "bf16", "attn_kernel_wide<bf16,256>", traffic_from_profiles(w.name))
    return {"workload": f"{w.name}: {w.notes}", "k1_ms": k1_ms, "k2_ms": k2_ms, "readout_ms": k3_ms,
            "useful_flop": roof["useful_flop"], "achieved_tflops": roof["achieved"], "peak_tflops": roof["peak"],
            "frac": roof["frac"], "settle_ms": settle_ms, "kernel": roof["kernel"]}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c3", choices=["c1", "c2", "c3", "c4", "c5a", "hbm", "c5gdn", "c5gdnrows"],
                    help="c3 (default): the 32k-prefix packed-prefill attention; c2: the Qwen3-1.7B-shaped stack's packed "
                         "pass; c5gdn / c5gdnrows: the Gated DeltaNet layer core over one 4096-token row / 32 rows of 64 tokens")
    ap.add_argument("--cpu-baseline", type=int, default=1, help="0 skips the CPU baseline leg")
    ap.add_argument("--hbm-shape", type=int, default=1,
                    help="with the default c3 workload, also time K2 on the 32k-prefix x 16-token shape (HBM-bound) "
                         "and report it under hbm_shape; 0 skips it")
    ap.add_argument("--c4-shape", type=int, default=1,
                    help="with the default c3 workload, also time K2 on config 4 (d = 256, bidirectional 8192-token "
                         "gated row, MFMA-bound) and report it under c4_shape; 0 skips it")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="run the step untimed for this long before the warm-up steps, so that timing starts at the "
                         "card's steady clock (0 skips it)")
    ap.add_argument("--evict-mall", type=int, default=-1,
                    help="1: read a 512 MiB buffer before each timed step (outside the events) so the step's data "
                         "comes from HBM, not the 256 MB MALL; 0: leave the MALL as the previous step left it; "
                         "-1 (default): evict for --workload hbm only (the default line's hbm_shape always reports both)")
    ap.add_argument("--graph", type=int, default=0,
                    help="1: capture each timed call once in a HIP graph and replay it; 0 (default): launch directly (graph launch costs more than it saves here)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the workload, run `steps` device copies of MIB MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings into bytes)")
    ap.add_argument("--kv-data", default="random", choices=["random", "integer", "zero"],
                    help="diagnostic: the workload's cached prefix K/V as drawn (random, the default and the only "
                         "setting for reported figures), rounded to integers, or zero.  Same kernels and shapes, less "
                         "switching in the matrix cores: it shows how much of K2's time the card's power management sets. "
                         "The CPU baseline is skipped for the other settings")
    ap.add_argument("--calibrate-gemm", type=int, default=0, metavar="N",
                    help="instead of the workload, time torch.matmul bf16 N^3 on random and on zero operands")
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
    if args.calibrate_gemm:
        calibrate_gemm(args.calibrate_gemm, args.steps, args.warmup)
        return
    if args.workload == "c5gdn":
        bench_gdn(args, configs.c5_gdn(), dev, "c5gdn")
        return
    if args.workload == "c2":
        bench_stack(args, configs.c2(True), dev)
        return
    if args.workload == "c5gdnrows":
        bench_gdn(args, configs.c5_gdn_rows(), dev, "c5gdnrows")
        return
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
    if args.kv_data != "random" and w.prefix:
        for t in (layer.pk, layer.pv):
            t.copy_(torch.round(t.float()).to(t.dtype) if args.kv_data == "integer" else torch.zeros_like(t))
        torch.cuda.synchronize()
    evict = args.evict_mall == 1 or (args.evict_mall < 0 and args.workload == "hbm")
    ms_step, k1_ms, k2_ms, k3_ms = time_layer(layer, args.steps, args.warmup, args.graph, args.settle_ms,
                                              evict=mall_evictor(dev) if evict else None)

    dtype = "bf16" if w.bf16 else "f32"
    flops = w.useful_flops()
    kernel = {(True, 128): "attn_kernel_pipe<bf16,128>", (True, 256): "attn_kernel_wide<bf16,256>"}.get(
        (w.bf16, w.d), f"attn_kernel_seq<{dtype},{w.d}>")
    roof = roofline(flops, w.alg_bytes(), k2_ms, dtype, kernel, traffic_from_profiles(w.name))

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
        "data": ("synthetic (seeded N(0,1) q/k/v and prefix K/V, QK-norm weights 1 + 0.1 N(0,1))" if args.kv_data == "random"
                 else f"diagnostic: seeded N(0,1) q/k/v, prefix K/V {'rounded to integers' if args.kv_data == 'integer' else 'zero'}"),
        "config": {
            "workload": f"{w.name}: {w.notes}",
            "hq": w.hq, "hkv": w.hkv, "head_dim": w.d, "prefix": w.prefix,
            "suffix_blocks": len(w.blocks), "block_len": w.blocks[0], "query_tokens": w.t,
            "causal": w.causal, "gated": w.gated,
            "launch": "hip graph replay (K1 and K2 each one graph)" if args.graph else "direct launches",
            "mall": ("evicted before each step (a 512 MiB read outside the timed events; ms_per_step is the sum of "
                     "the parts' HIP event means)") if evict else "as the previous step left it",
        },
        "tflops": flops / (ms_step * 1e-3) / 1e12,
        "k1_ms": k1_ms,
        "k2_ms": k2_ms,
        "roofline": roof,
        "device": device_info().name,
        "settle": dict(SETTLE),
    }
    if k3_ms is not None:
        hidden, codes, temp = w.readout
        res["readout_ms"] = k3_ms
        res["config"]["readout"] = (f"d3 Kind::Matrix at the last position: o_proj ({w.hq * w.d} -> {hidden}), f32, "
                                    f"{codes} x {hidden} readout / temperature {temp}")
    if args.workload == "c3" and args.hbm_shape:
        res["hbm_shape"] = hbm_shape_record(dev, args.steps, args.warmup, args.settle_ms)
    if args.workload == "c3" and args.c4_shape:
        res["c4_shape"] = c4_shape_record(dev, args.steps, args.warmup, args.settle_ms)
    if args.cpu_baseline and args.kv_data == "random":
        res["cpu_baseline"] = cpu_baseline(w, layer.np_inputs)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
