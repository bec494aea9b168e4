"""GPU parity of the Gated DeltaNet layer core (cev_gdn_forward through the C
ABI) against the oracle's restatement of GatedDeltaNet::forward
(qwen35.rs:414-453, chunk rule qwen35.rs:301-368).

Bars: the chunk rule is f32 in the reference and is checked to 1e-4 max |d|
(the reference's own chunked-vs-recurrence test allows 2e-4,
qwen35.rs:776-822; the GPU sums in another order).  In bf16 the layer output
is cast to bf16 once at the end and is checked to the 2e-2 bf16 bar; the new
conv state is a copy and must match bit for bit.  At the 4096-token size the
oracle runs on a prefix of the sequence, and the split-sequence property
(T1 then T2 with the carried states == T1 + T2 at once) covers the rest.
"""
import numpy as np
import pytest

import cev_hip
from cev_hip import configs
from helpers import to_dev, to_np

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2


def _say(msg):
    print(msg, flush=True)


def _run_gpu(w, inp, device, conv_in=None, s_in=None, t=None, t0=0):
    """The layer on tokens [t0, t0 + t) of the workload's inputs."""
    import torch
    t = w.t if t is None else t
    sl = slice(t0, t0 + t)
    dev = lambda x: to_dev(np.ascontiguousarray(x), w.bf16, device)
    f32 = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(device)
    layer = cev_hip.GatedDeltaNet(w.batch, t, w.nk, w.nv, w.dk, w.dv, w.kernel, w.eps,
                                  dtype=torch.bfloat16 if w.bf16 else torch.float32, device=device)
    y, conv_out, s_out = layer(dev(inp["mixed"][:, sl]), dev(inp["z"][:, sl]), dev(inp["b"][:, sl]), dev(inp["a"][:, sl]),
                               dev(inp["conv_w"]), f32(inp["neg_a"]), f32(inp["dt_bias"]), f32(inp["norm_w"]),
                               conv_in=conv_in, s_in=s_in)
    torch.cuda.synchronize()
    return y, conv_out, s_out


def _run_oracle(orc, w, inp, t=None, conv_in=None, s_in=None):
    t = w.t if t is None else t
    return orc.gdn_layer(inp["mixed"][:, :t], inp["z"][:, :t], inp["b"][:, :t], inp["a"][:, :t], inp["conv_w"], inp["neg_a"],
                         inp["dt_bias"], inp["norm_w"], w.nk, w.nv, w.dk, w.dv, w.eps, w.bf16, conv_in=conv_in, s_in=s_in)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("t", [1, 64, 150])
def test_gdn_small_vs_oracle(gpu, orc, bf16, t):
    w = configs.GdnWorkload("gdn-small", 11, bf16, 2, t, nk=2, nv=4)
    _say(f"test gdn small: bf16={bf16} B={w.batch} T={t} nk={w.nk} nv={w.nv}")
    inp = w.inputs()
    y, co, so = _run_gpu(w, inp, gpu)
    ry, rco, rso = _run_oracle(orc, w, inp)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"  max|d| y {ey:.3g}  state {es:.3g}")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= (BF16_TOL if bf16 else F32_TOL)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("nk,nv", [(2, 2), (1, 4), (1, 8)])
def test_gdn_head_groups_vs_oracle(gpu, orc, bf16, nk, nv):
    """Value heads per key head 1, 4 and 8 over several chunks and an odd
    batch: the bf16 records keep each key head's q / k rows once, in the
    group's first value head, and the scan maps a group's heads to one XCD."""
    w = configs.GdnWorkload("gdn-groups", 14, bf16, 3, 200, nk=nk, nv=nv)
    _say(f"test gdn head groups: bf16={bf16} B={w.batch} T={w.t} nk={nk} nv={nv}")
    inp = w.inputs()
    y, co, so = _run_gpu(w, inp, gpu)
    ry, rco, rso = _run_oracle(orc, w, inp)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"  max|d| y {ey:.3g}  state {es:.3g}")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= (BF16_TOL if bf16 else F32_TOL)


def test_gdn_conv_silu_outside_table(gpu, orc):
    """bf16 conv outputs outside the SiLU table (|v| >= 128 and |v| < 2^-16):
    q/k channels scaled by 400 and by 1e-6, so every token of the q/k waves
    takes the per-element SiLU while the v waves use the table.  l2norm
    removes the scale, so the bars are those of the other cases."""
    w = configs.GdnWorkload("gdn-silu-range", 12, True, 1, 150, nk=2, nv=4)
    _say(f"test gdn silu range: B={w.batch} T={w.t}")
    inp = w.inputs()
    qk = 2 * w.nk * w.dk
    m = inp["mixed"].copy()
    m[..., : qk // 3] *= 400.0
    m[..., qk // 3: 2 * qk // 3] *= 1e-6
    inp["mixed"] = cev_hip.synth.round_bf16(m)
    y, co, so = _run_gpu(w, inp, gpu)
    ry, rco, rso = _run_oracle(orc, w, inp)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"  max|dy| {ey:.3g} max|dS| {es:.3g}")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= BF16_TOL


@pytest.mark.parametrize("bf16", [False, True])
def test_gdn_carried_state_vs_oracle(gpu, orc, bf16):
    """conv_in / s_in given (a prefix already consumed), one state broadcast
    to both rows through batch stride 0 (LayerState::broadcast,
    decoder.rs:74-88, without the copy)."""
    import torch
    w = configs.GdnWorkload("gdn-state", 12, bf16, 2, 90, nk=2, nv=4)
    inp = w.inputs()
    rng = np.random.default_rng(3)
    conv_in = rng.standard_normal((1, w.conv_dim, w.kernel - 1)).astype(np.float32)
    s_in = (0.3 * rng.standard_normal((1, w.nv, w.dk, w.dv))).astype(np.float32)
    if bf16:
        conv_in = cev_hip.synth.round_bf16(conv_in)
    ci = to_dev(conv_in, bf16, gpu).expand(w.batch, -1, -1)
    si = torch.from_numpy(s_in).to(gpu).expand(w.batch, -1, -1, -1)
    y, co, so = _run_gpu(w, inp, gpu, conv_in=ci, s_in=si)
    ry, rco, rso = _run_oracle(orc, w, inp, conv_in=np.repeat(conv_in, 2, 0), s_in=np.repeat(s_in, 2, 0))
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"gdn carried state bf16={bf16}: max|d| y {ey:.3g} state {es:.3g}")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= (BF16_TOL if bf16 else F32_TOL)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("kernel", [2, 3, 5, 7, 8])
def test_gdn_conv_widths_vs_oracle(gpu, orc, bf16, kernel):
    """Every conv width the library builds a kernel for besides 4 (widths 7
    and 8 run 512-thread workgroups), with a carried conv state and a
    sequence that ends inside a chunk and inside a conv run."""
    w = configs.GdnWorkload("gdn-width", 13, bf16, 2, 133, nk=2, nv=4, kernel=kernel)
    _say(f"test gdn conv width {kernel}: bf16={bf16} T={w.t}")
    inp = w.inputs()
    rng = np.random.default_rng(4 + kernel)
    conv_in = rng.standard_normal((w.batch, w.conv_dim, kernel - 1)).astype(np.float32)
    if bf16:
        conv_in = cev_hip.synth.round_bf16(conv_in)
    y, co, so = _run_gpu(w, inp, gpu, conv_in=to_dev(conv_in, bf16, gpu))
    ry, rco, rso = _run_oracle(orc, w, inp, conv_in=conv_in)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"  max|d| y {ey:.3g}  state {es:.3g}")
    assert to_np(co).shape == (w.batch, w.conv_dim, kernel - 1)
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= (BF16_TOL if bf16 else F32_TOL)


@pytest.mark.parametrize("bf16", [False, True])
def test_gdn_strided_views_vs_oracle(gpu, orc, bf16):
    """z as a column slice of a wider tensor (odd row stride, a view into a
    fused projection output) and y written into such a view: the
    element-wise norm path.  mixed with rows that are not 16-byte aligned is
    refused (the conv reads 8-element vectors)."""
    import torch
    w = configs.GdnWorkload("gdn-strided", 13, bf16, 2, 70, nk=2, nv=4)
    inp = w.inputs()
    dt = torch.bfloat16 if bf16 else torch.float32
    wide = lambda x: torch.cat([torch.zeros(x.shape[:-1] + (1,), dtype=dt, device=gpu), to_dev(np.ascontiguousarray(x), bf16, gpu)], -1)
    mixed = to_dev(inp["mixed"], bf16, gpu)
    z = wide(inp["z"])[..., 1:]
    assert z.stride(1) % 2 == 1
    f32 = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu)
    layer = cev_hip.GatedDeltaNet(w.batch, w.t, w.nk, w.nv, w.dk, w.dv, w.kernel, w.eps, dtype=dt, device=gpu)
    y_wide = torch.zeros(w.batch, w.t, w.nv * w.dv + 3, dtype=dt, device=gpu)
    y, co, so = layer(mixed, z, to_dev(inp["b"], bf16, gpu), to_dev(inp["a"], bf16, gpu), to_dev(inp["conv_w"], bf16, gpu),
                      f32(inp["neg_a"]), f32(inp["dt_bias"]), f32(inp["norm_w"]), y=y_wide[..., 3:])
    torch.cuda.synchronize()
    ry, rco, rso = _run_oracle(orc, w, inp)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"gdn strided views bf16={bf16}: max|d| y {ey:.3g} state {es:.3g}")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= (BF16_TOL if bf16 else F32_TOL)
    assert not to_np(y_wide[..., :3]).any()
    with pytest.raises(cev_hip.CevError, match="8-element aligned"):
        layer(wide(inp["mixed"])[..., 1:], z, to_dev(inp["b"], bf16, gpu), to_dev(inp["a"], bf16, gpu),
              to_dev(inp["conv_w"], bf16, gpu), f32(inp["neg_a"]), f32(inp["dt_bias"]), f32(inp["norm_w"]))


def test_gdn_c5_heads_vs_oracle(gpu, orc):
    """Config 5's head layout (Hk 16 -> Hv 32) on the first 256 tokens."""
    w = configs.c5_gdn(t=256)
    _say(f"test gdn c5 heads: T={w.t} nk={w.nk} nv={w.nv}")
    inp = w.inputs()
    y, co, so = _run_gpu(w, inp, gpu)
    ry, rco, rso = _run_oracle(orc, w, inp)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"  max|d| y {ey:.3g}  state {es:.3g}")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert ey <= BF16_TOL


def _bf16_close(got, ref):
    """Each bf16 output within the 2e-2 bar plus one bf16 ulp of its own
    magnitude (2^-7 |ref|): y is rounded to bf16 once at the end, so a value
    near a rounding boundary may land one ulp apart, and over 4096 tokens y
    reaches magnitudes where one ulp exceeds 2e-2."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= BF16_TOL + 2.0 ** -7 * np.abs(ref)))


def test_gdn_c5_prefill_then_rows_vs_oracle(gpu, orc):
    """Config 5's GDN half end to end at its own shape (hybrid.rs:554-617):
    the 4096-token prefill (Hk 16 -> Hv 32) against the oracle in full (y,
    conv tail and recurrent state), then 32 rows of 64 tokens that continue
    from that prefilled state (LayerState::broadcast, decoder.rs:74-88; the
    GPU reads one state through batch stride 0) against the oracle's rows
    continuing from its own prefill."""
    import torch
    w = configs.c5_gdn()
    inp = w.inputs()
    _say(f"test gdn c5 prefill: T={w.t} nk={w.nk} nv={w.nv}")
    y, co, so = _run_gpu(w, inp, gpu)
    ry, rco, rso = _run_oracle(orc, w, inp)
    ey = float(np.abs(to_np(y) - ry).max())
    es = float(np.abs(to_np(so) - rso).max())
    _say(f"  prefill: max|d| y {ey:.3g} (max|y| {np.abs(ry).max():.3g}), state {es:.3g} (max|S| {np.abs(rso).max():.3g})")
    assert np.array_equal(to_np(co), rco)
    assert es <= F32_TOL
    assert _bf16_close(to_np(y), ry)
    rows = configs.c5_gdn_rows()
    rinp = rows.inputs()
    _say(f"test gdn c5 rows: {rows.batch} x {rows.t} after the prefill")
    yr, cor, sor = _run_gpu(rows, rinp, gpu, conv_in=co.expand(rows.batch, -1, -1), s_in=so.expand(rows.batch, -1, -1, -1))
    ryr, rcor, rsor = _run_oracle(orc, rows, rinp, conv_in=np.repeat(rco, rows.batch, 0), s_in=np.repeat(rso, rows.batch, 0))
    ey = float(np.abs(to_np(yr) - ryr).max())
    es = float(np.abs(to_np(sor) - rsor).max())
    _say(f"  rows: max|d| y {ey:.3g} (max|y| {np.abs(ryr).max():.3g}), state {es:.3g}")
    assert np.array_equal(to_np(cor), rcor)
    assert np.isfinite(to_np(yr)).all()
    assert es <= F32_TOL
    assert _bf16_close(to_np(yr), ryr)
    # the rows' GPU result from the oracle's prefilled state too: what is
    # left of the difference is the rows' own arithmetic
    yr2, _, sor2 = _run_gpu(rows, rinp, gpu, conv_in=to_dev(rco, True, gpu).expand(rows.batch, -1, -1),
                            s_in=torch.from_numpy(rso).to(gpu).expand(rows.batch, -1, -1, -1))
    assert float(np.abs(to_np(sor2) - rsor).max()) <= F32_TOL
    assert _bf16_close(to_np(yr2), ryr)


def test_gdn_c5_split_sequence(gpu):
    """4096 tokens at once == 2048 + 2048 with the carried conv and recurrent
    state (size-independent continuation property at the full 4096-token, 32-head size)."""
    w = configs.c5_gdn()
    inp = w.inputs()
    _say(f"test gdn c5 split: T={w.t}")
    y, co, so = _run_gpu(w, inp, gpu)
    h = w.t // 2
    y1, co1, so1 = _run_gpu(w, inp, gpu, t=h)
    y2, co2, so2 = _run_gpu(w, inp, gpu, t=h, t0=h, conv_in=co1, s_in=so1)
    full, parts = to_np(y), np.concatenate([to_np(y1), to_np(y2)], 1)
    es = float(np.abs(to_np(so) - to_np(so2)).max())
    ey = float(np.abs(full - parts).max())
    _say(f"  max|d| y {ey:.3g}  state {es:.3g}")
    assert np.array_equal(to_np(co), to_np(co2))
    assert np.isfinite(full).all() and np.isfinite(to_np(so)).all()
    assert es <= F32_TOL
    assert ey <= BF16_TOL


def test_gdn_long_sequence_split(gpu):
    """65,536 tokens at once (1,024 chunks per head, a 4.8 GB record
    workspace, 32,768 prep workgroups) == the same tokens in two halves with
    the carried conv and recurrent state.  The halves meet at a chunk
    boundary, so every chunk is computed the same way in both runs.  Inputs
    are drawn on the device with the 4096-token workload's distributions (beta uniform in
    (0, 1), decay e^g log-uniform in [1e-3, 1])."""
    import torch
    T, nk, nv, d, K = 1 << 16, 16, 32, 128, 4
    conv_dim = 2 * nk * d + nv * d
    gen = torch.Generator(device=gpu)
    gen.manual_seed(21)
    bf = torch.bfloat16
    rnd = lambda *shape: torch.randn(shape, generator=gen, device=gpu)  # noqa: E731
    uni = lambda *shape: torch.rand(shape, generator=gen, device=gpu).clamp(1e-4, 1 - 1e-4)  # noqa: E731
    mixed, z = rnd(1, T, conv_dim).to(bf), rnd(1, T, nv * d).to(bf)
    u = uni(1, T, nv)
    b = torch.log(u / (1 - u)).to(bf)
    g = torch.log(torch.tensor(1e-3, device=gpu)) * uni(1, T, nv)
    a = torch.log(torch.expm1(torch.clamp(-g, min=1e-6))).to(bf)
    conv_w = (0.5 * rnd(conv_dim, K)).to(bf)
    neg_a, dt_bias = -torch.ones(nv, device=gpu), torch.zeros(nv, device=gpu)
    norm_w = 1.0 + 0.1 * rnd(d)
    _say(f"test gdn long sequence: T={T}")

    def run(t0, t, conv_in=None, s_in=None):
        layer = cev_hip.GatedDeltaNet(1, t, nk, nv, d, d, K, 1e-6, dtype=bf, device=gpu)
        sl = slice(t0, t0 + t)
        out = layer(mixed[:, sl], z[:, sl], b[:, sl], a[:, sl], conv_w, neg_a, dt_bias, norm_w, conv_in=conv_in, s_in=s_in)
        torch.cuda.synchronize()
        del layer
        return out

    y, co, so = run(0, T)
    h = T // 2
    y1, co1, so1 = run(0, h)
    y2, co2, so2 = run(h, h, conv_in=co1, s_in=so1)
    full, parts = to_np(y), np.concatenate([to_np(y1), to_np(y2)], 1)
    es = float(np.abs(to_np(so) - to_np(so2)).max())
    ey = float(np.abs(full - parts).max())
    _say(f"  max|d| y {ey:.3g}  state {es:.3g}")
    assert np.array_equal(to_np(co), to_np(co2))
    assert np.isfinite(full).all() and np.isfinite(to_np(so)).all()
    # same chunks, same kernels, the state handed over in f32: bit for bit
    assert es == 0.0 and ey == 0.0


def test_gdn_graph_replay_matches_eager(gpu):
    """The four GDN kernels captured once in a HIP graph give the eager
    result on every replay (eager work and synchronisations in between)."""
    import torch
    w = configs.GdnWorkload("gdn-graph", 13, True, 2, 150, nk=2, nv=4)
    inp = w.inputs()
    dev = lambda x: to_dev(np.ascontiguousarray(x), True, gpu)
    f32 = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu)
    layer = cev_hip.GatedDeltaNet(w.batch, w.t, w.nk, w.nv, w.dk, w.dv, w.kernel, w.eps, dtype=torch.bfloat16, device=gpu)
    xs = [dev(inp[k]) for k in ("mixed", "z", "b", "a", "conv_w")] + [f32(inp[k]) for k in ("neg_a", "dt_bias", "norm_w")]
    y = torch.empty((w.batch, w.t, w.nv * w.dv), dtype=torch.bfloat16, device=gpu)
    co = torch.empty((w.batch, layer.conv_dim, w.kernel - 1), dtype=torch.bfloat16, device=gpu)
    so = torch.empty((w.batch, w.nv, w.dk, w.dv), dtype=torch.float32, device=gpu)
    layer(*xs, y=y, conv_out=co, s_out=so)
    torch.cuda.synchronize()
    want = [to_np(t).copy() for t in (y, co, so)]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer(*xs, y=y, conv_out=co, s_out=so)
    for i in range(3):
        for t in (y, co, so):
            t.fill_(float("nan"))
        layer.workspace.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, ref in zip((y, co, so), want):
            assert np.array_equal(to_np(got), ref), f"replay {i}"
