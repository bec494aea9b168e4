"""GPU parity of the HIP path (through the C ABI) against the oracle.

Bars (from the path's contract): attention output max |delta| <= 1e-5 in f32
and <= 2e-2 in bf16 against the candle-op restatement on identical seeded
inputs; every bf16 comparison is also held relative to the largest reference
value (tests/bars.py: 3e-2 against the candle-op restatement, 2e-2 against
exact attention), which a dropped key chunk, a shifted position or a missing
gate would miss at these output scales.  The QK-norm + RoPE prologue is checked bit for bit.  c1, c3 and c5a
are compared in full, and c4's 8192-token row against the candle-op
restatement in full; the f64 textbook covers every c1 and c5a block, three c3
blocks and 512 c4 rows.  Size-independent properties (packed == each block
alone, poisoned keys, equivariances) cover the rest.
"""
import numpy as np
import pytest

import cev_hip
from cev_hip import configs
from bars import BF16_ABS, F32_ABS, assert_bf16, assert_f32, errors
from helpers import GpuLayer, OracleLayer, default_table, to_dev, to_np

pytestmark = pytest.mark.gpu

F32_TOL = F32_ABS
BF16_TOL = BF16_ABS


def _say(msg):
    print(msg, flush=True)


def _check_blocks(gl, ol, blocks, tol, rows=None):
    import torch
    torch.cuda.synchronize()
    out = to_np(gl.out)
    worst = worst64 = rel = rel64 = 0.0
    for b in blocks:
        r0 = int(gl.w.block_starts()[b])
        L = gl.w.blocks[b]
        sel = slice(None) if rows is None else slice(rows[0], rows[0] + rows[1])
        got = out[r0:r0 + L][sel]
        want = ol.block(b, rows=rows)[sel]
        w64 = ol.block(b, rows=rows, f64=True)[sel]
        assert np.isfinite(got).all()
        e, r = errors(got, want)
        e64, r64 = errors(got, w64)
        worst, worst64, rel, rel64 = max(worst, e), max(worst64, e64), max(rel, r), max(rel64, r64)
        # The same bars hold against exact attention (f64, no model-dtype
        # rounding): the reference's own bf16 rounding moves it by well
        # under them at these shapes.
        if gl.w.bf16:
            assert_bf16(got, candle=want, exact=w64, what=f"{gl.w.name} block {b}")
        else:
            assert_f32(got, want, f"{gl.w.name} block {b}")
            assert_f32(got, w64, f"{gl.w.name} block {b} vs f64")
    _say(f"{gl.w.name}: max|d| vs candle-op oracle {worst:.3g} ({rel:.3g} of max|ref|), vs f64 textbook {worst64:.3g} "
         f"({rel64:.3g})")
    assert worst <= tol and worst64 <= tol, (worst, worst64)
    return worst


def test_c1_f32_end_to_end(gpu, orc):
    w = configs.c1()
    _say(f"test c1: t={w.t} P={w.prefix} hq={w.hq} hkv={w.hkv}")
    gl = GpuLayer(w, gpu)
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    # K1 reproduces the reference op order exactly
    assert np.array_equal(to_np(gl.q), ol.q)
    assert np.array_equal(to_np(gl.k), ol.k)
    _check_blocks(gl, ol, range(len(w.blocks)), F32_TOL)


def test_c3_bf16_sampled_blocks(gpu, orc):
    w = configs.c3()
    _say(f"test c3: t={w.t} P={w.prefix} hq={w.hq} hkv={w.hkv}")
    gl = GpuLayer(w, gpu)
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    assert np.array_equal(to_np(gl.q), ol.q)
    assert np.array_equal(to_np(gl.k), ol.k)
    _check_blocks(gl, ol, [0, 37, 63], BF16_TOL)


def test_c3_bf16_every_block_every_head(gpu, orc):
    """All 64 blocks and all 32 query heads of the full c3 layer against the
    candle-op oracle over [prefix || block] (the f64 textbook check runs on
    the sampled blocks above)."""
    import torch
    w = configs.c3()
    _say(f"test c3 every block: {len(w.blocks)} blocks x {w.hq} heads")
    gl = GpuLayer(w, gpu)
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    torch.cuda.synchronize()
    out = to_np(gl.out)
    worst = rel = 0.0
    for b in range(len(w.blocks)):
        r0, L = int(w.block_starts()[b]), w.blocks[b]
        got = out[r0:r0 + L]
        want = ol.block(b)
        e, r = errors(got, want)
        worst, rel = max(worst, e), max(rel, r)
        assert_bf16(got, candle=want, what=f"c3 block {b}")
    _say(f"  {len(w.blocks)} blocks: max|d| {worst:.3g} ({rel:.3g} of max|ref|)")


def test_c4_bidirectional_gated_full_row(gpu, orc):
    """Every row and head of the 8192-token bidirectional gated row against
    the candle-op oracle; eight 64-row windows (the first and the last rows
    among them) also against the f64 textbook."""
    import torch
    w = configs.c4()
    _say(f"test c4: t={w.t} hq={w.hq} hkv={w.hkv} d={w.d}")
    gl = GpuLayer(w, gpu)
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    torch.cuda.synchronize()
    assert np.array_equal(to_np(gl.q), ol.q)
    assert np.array_equal(to_np(gl.k), ol.k)
    got = to_np(gl.out)
    want = ol.block(0)
    err, rel = errors(got, want)
    _say(f"c4 all {w.t} rows: max|d| vs candle-op oracle {err:.3g} ({rel:.3g} of max|ref|)")
    assert_bf16(got, candle=want, what="c4 row")
    for r0 in (0, 1000, 2047, 3333, 4000, 5555, 7000, 8128):
        _check_blocks(gl, ol, [0], BF16_TOL, rows=(r0, 64))


def _d3_check(gpu, orc, w, tol):
    """GPU: K1 + K2 over the whole row, then o_proj of the last position and
    the readout (D3Readout through cev_linear / cev_gather_rows).  Oracle:
    the same chain from the same inputs (attention of the last row by the
    candle-op restatement, its gate, oracle.readout.d3_readout)."""
    import torch
    from oracle.readout import d3_readout
    gl = GpuLayer(w, gpu)
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    torch.cuda.synchronize()
    got = to_np(gl.logits)[0]
    r = w.t - 1
    o_last = ol.block(0, rows=(r, 1))[r].reshape(1, -1)
    wo, wr = w.readout_weights()
    want = d3_readout(o_last, wo, wr, w.readout[2], w.bf16)[0]
    err = float(np.abs(got - want).max())
    # the readout arithmetic alone, on the GPU's own attention row
    own = d3_readout(to_np(gl.out)[r].reshape(1, -1), wo, wr, w.readout[2], w.bf16)[0]
    err_own = float(np.abs(got - own).max())
    scale = float(np.abs(want).max())
    _say(f"{w.name} d3 readout: {got.size} logits, max|logit| {scale:.3g}, max|d| end to end {err:.3g}, "
         f"readout alone {err_own:.3g}")
    assert got.shape == (w.readout[1],) and np.isfinite(got).all()
    assert err <= tol and err_own <= tol
    if w.bf16:
        assert_bf16(got, candle=want, what=f"{w.name} d3 logits")
        assert_bf16(got, candle=own, what=f"{w.name} d3 logits, readout alone")
    return err


def test_c4_d3_readout_full_row(gpu, orc):
    """Config 4's observable: the 255 d3 logits at the last position of the
    full 8192-token bidirectional gated row (hybrid.rs:657), bf16 bar."""
    _d3_check(gpu, orc, configs.c4(), BF16_TOL)


def test_d3_readout_f32_small(gpu, orc):
    _d3_check(gpu, orc, configs.d3_f32(), F32_TOL)


def test_linear_shapes_against_numpy(gpu, orc):
    """cev_linear on both paths (own kernel for m <= 8, hipBLASLt above) and
    both dtypes, with strided rows, against f64 products rounded once."""
    import torch
    from oracle.readout import linear as ref_linear
    rng = np.random.default_rng(3)
    for bf, m, n, k, out32 in ((True, 1, 2048, 4096, False), (True, 5, 300, 264, True), (False, 1, 255, 2048, True),
                               (False, 8, 64, 512, True), (True, 96, 512, 1024, False), (False, 64, 8, 2048, True),
                               (True, 3584, 4096, 2048, False)):
        x = rng.standard_normal((m, k + 8)).astype(np.float32)[:, :k]
        wt = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
        if bf:
            x, wt = orc.round_bf16(x), orc.round_bf16(wt)
        xd = to_dev(np.ascontiguousarray(np.pad(x, ((0, 0), (0, 8)))), bf, gpu)[:, :k]
        wd = to_dev(wt, bf, gpu)
        got = to_np(cev_hip.linear(xd, wd, alpha=0.5, out_dtype=torch.float32 if out32 else None))
        want = ref_linear(x, wt, bf and not out32) * np.float32(0.5)
        if bf and not out32:
            want = orc.round_bf16(ref_linear(x, wt, False) * np.float32(0.5))
        err = float(np.abs(got - want).max() / max(1e-30, np.abs(want).max()))
        _say(f"linear bf16={bf} m={m} n={n} k={k} f32 out={out32}: max rel err {err:.3g}")
        assert err <= (1e-2 if bf and not out32 else 1e-5)
    # the config-2 projection shapes with an offline-measured algorithm pick
    # (contiguous operands: the layout the picks apply to), bf16 out
    for m, n, k in ((3584, 4096, 2048), (3584, 2048, 2048), (3584, 2048, 6144)):
        x = orc.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
        wt = orc.round_bf16((0.02 * rng.standard_normal((n, k))).astype(np.float32))
        got = to_np(cev_hip.linear(to_dev(x, True, gpu), to_dev(wt, True, gpu)))
        want = orc.round_bf16(ref_linear(x, wt, False))
        err = float(np.abs(got - want).max() / max(1e-30, np.abs(want).max()))
        _say(f"linear bf16 picked shape m={m} n={n} k={k}: max rel err {err:.3g}")
        assert err <= 1e-2
    # gather with conversion and an out-of-range id
    tab = torch.randn(10, 16, device=gpu).to(torch.bfloat16)
    ids = torch.tensor([3, 0, 9, 10], dtype=torch.int32, device=gpu)
    g = to_np(cev_hip.gather_rows(tab, ids, out_dtype=torch.float32))
    ref = to_np(tab)
    assert np.array_equal(g[:3], ref[[3, 0, 9]]) and np.isnan(g[3]).all()


def test_c5_gated_rows_continue_prefix(gpu, orc):
    w = configs.c5_attention()
    _say(f"test c5a: rows={len(w.blocks)} x {w.blocks[0]} P={w.prefix}")
    tab = cev_hip.BlockTable.from_rows(len(w.blocks), w.blocks[0], w.prefix, causal=True)
    gl = GpuLayer(w, gpu, table=tab)
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    _check_blocks(gl, ol, range(len(w.blocks)), BF16_TOL)


SMALL = [
    # (bf16, hq, hkv, d, plans, items)
    (False, 8, 8, 128, [(37, 37, 37)], [(0, 5), (0, 1), (0, 70)]),
    (False, 16, 8, 128, [(20, 50, 20), (64, 64, 64)], [(0, 9), (1, 33), (0, 2), (1, 64)]),
    (False, 16, 4, 128, [(0, 30, 0)], [(0, 12), (0, 100)]),
    (False, 16, 2, 128, [(130, 130, 130)], [(0, 65)]),
    (True, 8, 8, 128, [(37, 37, 37)], [(0, 5), (0, 1), (0, 70)]),
    (True, 16, 8, 128, [(20, 50, 20), (64, 64, 64)], [(0, 9), (1, 33), (0, 2), (1, 64)]),
    (True, 32, 8, 128, [(300, 300, 300)], [(0, 48)] * 5),
    (True, 16, 2, 128, [(130, 130, 130)], [(0, 65)]),
    # every tile starts with a prefix of one chunk or less (a whole and a
    # partial chunk), then the local keys of two 64-token blocks
    (True, 16, 8, 128, [(64, 64, 64)], [(0, 64)] * 4),
    (True, 16, 8, 128, [(40, 40, 40)], [(0, 64)] * 4),
    (True, 16, 4, 256, [(100, 140, 100)], [(0, 17), (0, 64), (0, 3)]),
    (True, 8, 8, 256, [(33, 33, 33)], [(0, 40)]),
    (True, 16, 2, 256, [(0, 5, 0)], [(0, 31)]),
]


@pytest.mark.parametrize("case", range(len(SMALL)))
def test_small_packed_passes(gpu, orc, case):
    """Multi-plan passes with tails, ragged blocks, every GQA group size and
    both head dims, against the oracle over the reference's dense mask."""
    bf, hq, hkv, d, plans, items = SMALL[case]
    _say(f"small case {case}: bf16={bf} hq={hq} hkv={hkv} d={d} plans={plans} items={items}")
    rng = np.random.default_rng(100 + case)
    ep = orc.engine_pass(plans, items)
    tab, pos, _ = cev_hip.BlockTable.from_plans(plans, items)
    t, s_cache = ep["n"], ep["past_total"]
    rnd = (lambda x: orc.round_bf16(x)) if bf else (lambda x: x)
    q = rnd(rng.standard_normal((t, hq, d)).astype(np.float32))
    kn = rnd(rng.standard_normal((t, hkv, d)).astype(np.float32))
    vn = rnd(rng.standard_normal((t, hkv, d)).astype(np.float32))
    kc = rnd(rng.standard_normal((hkv, max(s_cache, 1), d)).astype(np.float32))[:, :s_cache]
    vc = rnd(rng.standard_normal((hkv, max(s_cache, 1), d)).astype(np.float32))[:, :s_cache]
    out = cev_hip.packed_attention(to_dev(q, bf, gpu), to_dev(kn, bf, gpu), to_dev(vn, bf, gpu), tab,
                                   k_cache=to_dev(kc, bf, gpu) if s_cache else None, v_cache=to_dev(vc, bf, gpu) if s_cache else None)
    got = to_np(out)
    kall = np.concatenate([kc, kn.transpose(1, 0, 2)], axis=1)
    vall = np.concatenate([vc, vn.transpose(1, 0, 2)], axis=1)
    want = orc.attend(q.transpose(1, 0, 2), kall, vall, ep["mask"], bf)[0].transpose(1, 0, 2)
    want64 = orc.attend_f64(q.transpose(1, 0, 2), kall, vall, ep["mask"])[0].transpose(1, 0, 2)
    err, rel = errors(got, want)
    _say(f"  max|d| {err:.3g} ({rel:.3g} of max|ref|)")
    if bf:
        assert_bf16(got, candle=want, exact=want64, what=f"small case {case}")
    else:
        assert_f32(got, want, f"small case {case}")
        assert_f32(got, want64, f"small case {case} vs f64")


@pytest.mark.parametrize("shape", ["ramp", "spike", "low", "unseen_first"])
@pytest.mark.parametrize("max_splits", [1, 0])
def test_softmax_max_moves(gpu, orc, shape, max_splits):
    """Scores far from the first key tile's: the kernels move a row's max
    lazily, so these drive every move (d = 128 and 256, bf16 and f32).
    ramp: scores climb by about 100 (base 2) over the prefix, so the row max
    moves many times and unmoved probabilities would overflow; spike: one key
    about 60 above the rest, late in the stream; low: every score near -150,
    where probabilities against a max of 0 would underflow; unseen_first: a
    causal block with no prefix, split so that parts start on keys some rows
    cannot see.  bf16 is held to exact (f64) attention: at these score
    magnitudes the candle-op restatement's own bf16 rounding of the scores
    moves its result by more than the bar; f32 is held to both."""
    rng = np.random.default_rng(7)
    for bf, d, hq, hkv in [(True, 128, 8, 2), (True, 256, 8, 2), (False, 128, 4, 2)]:
        P, L = (0, 300) if shape == "unseen_first" else (2048, 40)
        u = rng.standard_normal(d).astype(np.float32)
        u /= np.linalg.norm(u)
        q = (0.2 * rng.standard_normal((L, hq, d)) + 8.0 * u).astype(np.float32)
        kc = 0.2 * rng.standard_normal((hkv, P, d)).astype(np.float32)
        if shape == "ramp":
            kc += (np.linspace(-2.0, 100.0, P, dtype=np.float32)[None, :, None] * u)
        elif shape == "spike":
            kc[:, 1500] += 60.0 * u
        elif shape == "low":
            kc -= 150.0 * u
        vc = rng.standard_normal((hkv, P, d)).astype(np.float32)
        kn = (0.2 * rng.standard_normal((L, hkv, d)) + rng.uniform(-3, 3, (L, 1, 1)) * u).astype(np.float32)
        vn = rng.standard_normal((L, hkv, d)).astype(np.float32)
        rnd = (lambda x: orc.round_bf16(x)) if bf else (lambda x: x)
        q, kc, vc, kn, vn = map(rnd, (q, kc, vc, kn, vn))
        tab = cev_hip.BlockTable.from_rows(1, L, P, causal=True)
        dev = lambda x: to_dev(x, bf, gpu)  # noqa: E731
        out = cev_hip.packed_attention(dev(q), dev(kn), dev(vn), tab, k_cache=dev(kc) if P else None,
                                       v_cache=dev(vc) if P else None, max_splits=max_splits)
        got = to_np(out)
        kall = np.concatenate([kc, kn.transpose(1, 0, 2)], axis=1)
        vall = np.concatenate([vc, vn.transpose(1, 0, 2)], axis=1)
        mask = orc.branch_mask(L, P)
        want = orc.attend(q.transpose(1, 0, 2), kall, vall, mask, bf)[0].transpose(1, 0, 2)
        want64 = orc.attend_f64(q.transpose(1, 0, 2), kall, vall, mask)[0].transpose(1, 0, 2)
        assert np.isfinite(got).all()
        err, err64 = float(np.abs(got - want).max()), float(np.abs(got - want64).max())
        _say(f"{shape} bf16={bf} d={d} splits={max_splits}: max|d| {err:.3g} (f64 {err64:.3g}), max|out| {np.abs(want).max():.3g}")
        if bf:
            assert_bf16(got, exact=want64, what=f"{shape} d={d}")
        else:
            assert_f32(got, want, f"{shape} d={d}")
            assert_f32(got, want64, f"{shape} d={d} vs f64")


def test_packed_equals_each_block_alone_on_gpu(gpu):
    """qwen3.rs:13-17: packing is exactly asking each question alone.  The
    kernel visits the same key tiles in the same order either way (unsplit),
    so the outputs agree bit for bit at the full c3 shape."""
    w = configs.c3()
    gl = GpuLayer(w, gpu)
    gl.forward()
    packed = to_np(gl.out)
    for b in (0, 41):
        r0, L = int(w.block_starts()[b]), w.blocks[b]
        tab = cev_hip.BlockTable.from_rows(1, L, w.prefix, causal=True)
        alone = cev_hip.packed_attention(gl.q[r0:r0 + L], gl.k[r0:r0 + L], gl.v[r0:r0 + L], tab, k_cache=gl.pk, v_cache=gl.pv,
                                         max_splits=1)
        assert np.array_equal(to_np(alone), packed[r0:r0 + L])


def test_packed_rows_equal_each_row_alone_d256(gpu):
    """The same for the d = 256 kernel on the gated-rows layer: unsplit, each
    of the 32 rows run alone over [prefix || row] matches its packed rows
    bit for bit."""
    w = configs.c5_attention()
    tab = cev_hip.BlockTable.from_rows(len(w.blocks), w.blocks[0], w.prefix, causal=True)
    gl = GpuLayer(w, gpu, table=tab)
    gl.forward()
    packed = cev_hip.packed_attention(gl.q, gl.k, gl.v, tab, k_cache=gl.pk, v_cache=gl.pv, max_splits=1)
    packed = to_np(packed)
    assert np.isfinite(packed).all()
    for b in (0, 13, 31):
        r0, L = int(w.block_starts()[b]), w.blocks[b]
        one = cev_hip.BlockTable.from_rows(1, L, w.prefix, causal=True)
        alone = cev_hip.packed_attention(gl.q[r0:r0 + L], gl.k[r0:r0 + L], gl.v[r0:r0 + L], one, k_cache=gl.pk, v_cache=gl.pv,
                                         max_splits=1)
        assert np.array_equal(to_np(alone), packed[r0:r0 + L])


@pytest.mark.parametrize("d", [128, 256])
def test_poisoned_invisible_keys_are_never_read(gpu, orc, d):
    """A row never reads another plan's K/V.  Per plan p: NaN in every other
    plan's past (cache keys), in the K/V of every new token another plan
    owns, and in keys past the end of the cache must leave plan p's rows
    bit-identical to a clean run (same plan, same key tiles).  Tiles never
    mix plans (their blocks' span lists differ), so none of those keys is
    ever loaded for plan p.  Keys of the plan's own other questions are not
    poisoned: a tile may hold several of its questions and load each one's
    keys masked for the others (p = 0 times V)."""
    import torch
    bf = True
    plans, items = [(40, 40, 40), (50, 60, 50), (0, 20, 0)], [(0, 7), (1, 9), (0, 3), (2, 5), (1, 70)]
    ep = orc.engine_pass(plans, items)
    tab, _, _ = cev_hip.BlockTable.from_plans(plans, items)
    t, s = ep["n"], ep["past_total"]
    owner = ep["owner"]
    past_off = np.cumsum([0] + [p_[0] for p_ in plans])
    hq, hkv = 16, 4
    rng = np.random.default_rng(5)
    q = orc.round_bf16(rng.standard_normal((t, hq, d)).astype(np.float32))
    kn = orc.round_bf16(rng.standard_normal((t, hkv, d)).astype(np.float32))
    vn = orc.round_bf16(rng.standard_normal((t, hkv, d)).astype(np.float32))
    pad = 64  # keys after the cache end, inside the cache view's row stride
    kc = orc.round_bf16(rng.standard_normal((hkv, s + pad, d)).astype(np.float32))
    vc = orc.round_bf16(rng.standard_normal((hkv, s + pad, d)).astype(np.float32))
    qd = to_dev(q, bf, gpu)
    clean = to_np(cev_hip.packed_attention(qd, to_dev(kn, bf, gpu), to_dev(vn, bf, gpu), tab,
                                           k_cache=to_dev(kc, bf, gpu)[:, :s], v_cache=to_dev(vc, bf, gpu)[:, :s]))
    assert np.isfinite(clean).all()
    for p in range(len(plans)):
        kcp, vcp, knp, vnp = kc.copy(), vc.copy(), kn.copy(), vn.copy()
        for o in range(len(plans)):
            if o != p:
                kcp[:, past_off[o]:past_off[o + 1]] = np.nan
                vcp[:, past_off[o]:past_off[o + 1]] = np.nan
        other = owner != p
        knp[other] = np.nan
        vnp[other] = np.nan
        kcp[:, s:] = np.nan
        vcp[:, s:] = np.nan
        got = to_np(cev_hip.packed_attention(qd, to_dev(knp, bf, gpu), to_dev(vnp, bf, gpu), tab,
                                             k_cache=to_dev(kcp, bf, gpu)[:, :s], v_cache=to_dev(vcp, bf, gpu)[:, :s]))
        torch.cuda.synchronize()
        mine = owner == p
        _say(f"poisoned run for plan {p}, d={d}: {int(mine.sum())} rows checked")
        assert np.isfinite(got[mine]).all()
        assert np.array_equal(got[mine], clean[mine])


def test_stale_device_plan_gives_nan_not_stale_rows(gpu):
    """A device plan that is not a copy of the host plan the launch was
    validated with (another table of the same shape) is never followed: the
    whole output becomes NaN and the call still returns CEV_OK."""
    import torch
    t, hq, hkv, d, s = 64, 8, 2, 128, 100
    B = cev_hip.BlockTable.block
    tab_a = cev_hip.BlockTable([B(0, 32, s, spans=[(0, s)]), B(32, 32, s + 32, spans=[(0, s)])], t, s)
    tab_b = cev_hip.BlockTable([B(0, 64, s, spans=[(0, 50)])], t, s)
    q = torch.randn(t, hq, d, device=gpu).to(torch.bfloat16)
    k = torch.randn(t, hkv, d, device=gpu).to(torch.bfloat16)
    kc = torch.randn(hkv, s, d, device=gpu).to(torch.bfloat16)
    op_a = cev_hip.PackedAttention(q, k, tab_a, k_cache=kc, s_cache=s, v_new=k, v_cache=kc)
    op_b = cev_hip.PackedAttention(q, k, tab_b, k_cache=kc, s_cache=s, v_new=k, v_cache=kc)
    good = op_a(q, k, k, kc, kc)
    assert torch.isfinite(good.float()).all()
    op_a.plan.dev = op_b.plan.dev  # host plan A, device plan B
    out = torch.zeros_like(q)
    op_a(q, k, k, kc, kc, out=out)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


def test_rows_outside_every_block_are_untouched(gpu):
    import torch
    t, hq, hkv, d, s = 100, 8, 2, 128, 30
    B = cev_hip.BlockTable.block
    tab = cev_hip.BlockTable([B(10, 20, s + 10, spans=[(0, s)]), B(60, 5, s + 60, spans=[(0, s)])], t, s)
    q = torch.randn(t, hq, d, device=gpu).to(torch.bfloat16)
    k = torch.randn(t, hkv, d, device=gpu).to(torch.bfloat16)
    kc = torch.randn(hkv, s, d, device=gpu).to(torch.bfloat16)
    out = torch.full((t, hq, d), 7.0, device=gpu, dtype=torch.bfloat16)
    cev_hip.packed_attention(q, k, k, tab, k_cache=kc, v_cache=kc, out=out)
    o = to_np(out)
    assert (o[:10] == 7).all() and (o[30:60] == 7).all() and (o[65:] == 7).all()
    assert not (o[10:30] == 7).all()


def test_split_plan_with_rows_outside_every_block(gpu):
    """A split plan whose tiles skip rows: the merge finds its rows through
    the tile table.  Covered rows equal the unsplit result, and rows outside
    every block keep what the output held."""
    import torch
    t, hq, hkv, d, s = 48, 32, 8, 128, 32768
    B = cev_hip.BlockTable.block
    tab = cev_hip.BlockTable([B(8, 16, s + 8, spans=[(0, s)]), B(40, 4, s + 40, spans=[(0, s)])], t, s)
    g = torch.Generator(device="cpu").manual_seed(5)
    rnd = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16).to(gpu)  # noqa: E731
    q, kn, vn, kc, vc = rnd(t, hq, d), rnd(t, hkv, d), rnd(t, hkv, d), rnd(hkv, s, d), rnd(hkv, s, d)
    op = cev_hip.PackedAttention(q, kn, tab, k_cache=kc, s_cache=s, v_new=vn, v_cache=vc)
    assert op.plan.n_splits > 1
    out = torch.full((t, hq, d), 7.0, device=gpu, dtype=torch.bfloat16)
    op(q, kn, vn, kc, vc, out=out)
    whole = cev_hip.packed_attention(q, kn, vn, tab, k_cache=kc, v_cache=vc, max_splits=1)
    o, w = to_np(out), to_np(whole)
    covered = np.zeros(t, bool)
    covered[8:24] = covered[40:44] = True
    assert (o[~covered] == 7).all()
    err = np.abs(o[covered] - w[covered]).max()
    _say(f"split plan with gaps: parts {op.plan.n_splits}, max|split - unsplit| {err:.3g}")
    assert err <= 1e-2


def test_stale_device_plan_split_gives_nan(gpu):
    """As the stale-plan test above, for split plans: the attention kernel
    fills the output with NaN and the merge, whose record loads go out
    before its header check, stores nothing over it."""
    import torch
    t, hq, hkv, d, s = 16, 32, 8, 128, 32768
    B = cev_hip.BlockTable.block
    tab_a = cev_hip.BlockTable([B(0, 16, s, spans=[(0, s)])], t, s)
    tab_b = cev_hip.BlockTable([B(0, 16, s, spans=[(0, s - 64)])], t, s)
    g = torch.Generator(device="cpu").manual_seed(6)
    rnd = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16).to(gpu)  # noqa: E731
    q, kn, vn, kc, vc = rnd(t, hq, d), rnd(t, hkv, d), rnd(t, hkv, d), rnd(hkv, s, d), rnd(hkv, s, d)
    op_a = cev_hip.PackedAttention(q, kn, tab_a, k_cache=kc, s_cache=s, v_new=vn, v_cache=vc)
    op_b = cev_hip.PackedAttention(q, kn, tab_b, k_cache=kc, s_cache=s, v_new=vn, v_cache=vc)
    assert op_a.plan.n_splits > 1 and op_a.plan.n_splits == op_b.plan.n_splits
    assert torch.isfinite(op_a(q, kn, vn, kc, vc).float()).all()
    op_a.plan.dev = op_b.plan.dev  # host plan A, device plan B
    out = torch.zeros_like(q)
    op_a(q, kn, vn, kc, vc, out=out)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


def test_bidirectional_padded_rows(gpu, orc):
    bf, t, hq, hkv, d = True, 40, 8, 2, 256
    lengths = [40, 17, 1, 0]
    tab = cev_hip.BlockTable.from_rows(len(lengths), t, 0, causal=False, lengths=lengths)
    rng = np.random.default_rng(9)
    n = len(lengths) * t
    q = orc.round_bf16(rng.standard_normal((n, hq, d)).astype(np.float32))
    k = orc.round_bf16(rng.standard_normal((n, hkv, d)).astype(np.float32))
    v = orc.round_bf16(rng.standard_normal((n, hkv, d)).astype(np.float32))
    got = to_np(cev_hip.packed_attention(to_dev(q, bf, gpu), to_dev(k, bf, gpu), to_dev(v, bf, gpu), tab))
    mask = orc.bidirectional_mask(t, lengths)
    for r in range(len(lengths)):
        sl = slice(r * t, (r + 1) * t)
        want = orc.attend(q[sl].transpose(1, 0, 2), k[sl].transpose(1, 0, 2), v[sl].transpose(1, 0, 2), mask[r], bf)[0]
        assert_bf16(got[sl], candle=want.transpose(1, 0, 2), what=f"padded row {r} (length {lengths[r]})")


def test_kernel_repeats_bitwise(gpu):
    w = configs.c1()
    gl = GpuLayer(w, gpu)
    gl.forward()
    a = to_np(gl.out).copy()
    gl.forward()
    assert np.array_equal(a, to_np(gl.out))


@pytest.mark.parametrize("blocks", [1, 4])
def test_long_prefix_short_suffix_split(gpu, orc, blocks):
    """The HBM-bound shape: c3's 32768-key prefix with 16-token blocks.  The
    planner splits each tile's key stream; the merged result matches the
    oracle and the unsplit kernel."""
    w = configs.hbm(blocks)
    _say(f"test {w.name}: t={w.t} P={w.prefix}")
    gl = GpuLayer(w, gpu)
    assert gl.attn.plan.n_splits > 1
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    _check_blocks(gl, ol, range(len(w.blocks)), BF16_TOL)
    split = to_np(gl.out).copy()
    whole = cev_hip.packed_attention(gl.q, gl.k, gl.v, gl.table, k_cache=gl.pk, v_cache=gl.pv, max_splits=1)
    assert np.abs(to_np(whole) - split).max() <= 4e-3


def test_million_key_prefix_many_parts(gpu):
    """A 2^20-key cached prefix (256 MiB of K per head) with one 16-token
    causal block, g = 8: the planner cuts the single tile's key stream into
    the most parts it allows, and the merge combines them over several
    batches.  Sampled rows and heads are held to exact attention computed in
    f64 over all 2^20 + 16 keys, and the split result to the unsplit one."""
    import torch
    P, t, hq, hkv, d = 1 << 20, 16, 8, 1, 128
    _say(f"test 1M-key prefix: P={P} t={t} hq={hq} hkv={hkv}")
    rng = np.random.default_rng(20)
    f = lambda *shape: torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(gpu).to(torch.bfloat16)  # noqa: E731
    q, kn, vn = f(t, hq, d), f(t, hkv, d), f(t, hkv, d)
    kc, vc = f(hkv, P, d), f(hkv, P, d)
    # Random keys alone give a near-uniform softmax over 2^20 keys and
    # outputs near zero; a few planted keys aligned with each sampled query
    # (at the start, the middle and the end of the prefix) carry most of its
    # weight, so the outputs are O(1) and every part of the split matters.
    samples = [(0, 0, (5, 524_301, P - 3)), (7, 3, (77_777, 600_000, P - 9)), (15, 7, (1, 300_000, 1_000_003))]
    for i, h, where in samples:
        for pos in where:
            kc[0, pos] = (1.5 * q[i, h].float()).to(torch.bfloat16)
    tab = cev_hip.BlockTable.from_rows(1, t, P, causal=True)
    attn = cev_hip.PackedAttention(q, kn, tab, k_cache=kc, s_cache=P, v_new=vn, v_cache=vc)
    assert attn.plan.n_splits >= 128, attn.plan.n_splits
    out = to_np(attn(q, kn, vn, kc, vc))
    whole = to_np(cev_hip.packed_attention(q, kn, vn, tab, k_cache=kc, v_cache=vc, max_splits=1))
    assert np.isfinite(out).all()
    # two bf16 ulps at the planted rows' magnitude (|out| < 2): the parts
    # sum in another order than the single stream
    assert np.abs(whole - out).max() <= 2 * 2.0 ** -7
    k_all = np.concatenate([to_np(kc)[0], to_np(kn)[:, 0]]).astype(np.float64)
    v_all = np.concatenate([to_np(vc)[0], to_np(vn)[:, 0]]).astype(np.float64)
    qn = to_np(q).astype(np.float64)
    worst = 0.0
    for i, h, _ in samples:
        keys = P + i + 1  # the prefix and the block's own keys up to row i
        sc = k_all[:keys] @ qn[i, h] / np.sqrt(d)
        pr = np.exp(sc - sc.max())
        ref = (pr @ v_all[:keys]) / pr.sum()
        worst = max(worst, float(np.abs(out[i, h] - ref).max()))
        assert_bf16(out[i, h], exact=ref, what=f"row {i} head {h}")
    _say(f"  parts {attn.plan.n_splits}, max|d| vs exact f64 {worst:.3g}")


def test_long_prefix_many_parts_d256(gpu):
    """The d = 256 kernel and merge with many parts: a 2^17-key cached prefix
    with one 16-token causal block, g = 4.  Sampled rows and heads are held
    to exact attention in f64 over every key (planted keys aligned with
    each sampled query carry most of the weight), and the split result to
    the unsplit one."""
    import torch
    P, t, hq, hkv, d = 1 << 17, 16, 16, 4, 256
    _say(f"test long prefix d=256: P={P} t={t} hq={hq} hkv={hkv}")
    rng = np.random.default_rng(21)
    f = lambda *shape: torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(gpu).to(torch.bfloat16)  # noqa: E731
    q, kn, vn = f(t, hq, d), f(t, hkv, d), f(t, hkv, d)
    kc, vc = f(hkv, P, d), f(hkv, P, d)
    samples = [(0, 0, (3, 65_537, P - 2)), (9, 6, (40_000, 100_001, P - 7)), (15, 15, (0, 77_777, 131_000))]
    for i, h, where in samples:
        for pos in where:
            kc[h // (hq // hkv), pos] = (0.75 * q[i, h].float()).to(torch.bfloat16)
    tab = cev_hip.BlockTable.from_rows(1, t, P, causal=True)
    attn = cev_hip.PackedAttention(q, kn, tab, k_cache=kc, s_cache=P, v_new=vn, v_cache=vc)
    assert attn.plan.n_splits >= 16, attn.plan.n_splits
    out = to_np(attn(q, kn, vn, kc, vc))
    whole = to_np(cev_hip.packed_attention(q, kn, vn, tab, k_cache=kc, v_cache=vc, max_splits=1))
    assert np.isfinite(out).all()
    assert np.abs(whole - out).max() <= 2 * 2.0 ** -7
    qn = to_np(q).astype(np.float64)
    worst = 0.0
    for i, h, _ in samples:
        kvh = h // (hq // hkv)
        keys = P + i + 1
        k_all = np.concatenate([to_np(kc)[kvh], to_np(kn)[:, kvh]]).astype(np.float64)[:keys]
        v_all = np.concatenate([to_np(vc)[kvh], to_np(vn)[:, kvh]]).astype(np.float64)[:keys]
        sc = k_all @ qn[i, h] / np.sqrt(d)
        pr = np.exp(sc - sc.max())
        ref = (pr @ v_all) / pr.sum()
        worst = max(worst, float(np.abs(out[i, h] - ref).max()))
        assert_bf16(out[i, h], exact=ref, what=f"row {i} head {h}")
    _say(f"  parts {attn.plan.n_splits}, max|d| vs exact f64 {worst:.3g}, split vs whole {np.abs(whole - out).max():.3g}")


def test_split_f32_matches_unsplit(gpu):
    w = configs.c1()
    gl = GpuLayer(w, gpu)
    gl.forward()
    assert gl.attn.plan.n_splits > 1
    split = to_np(gl.out).copy()
    whole = cev_hip.packed_attention(gl.q, gl.k, gl.v, gl.table, k_cache=gl.pk, v_cache=gl.pv, max_splits=1)
    assert np.abs(to_np(whole) - split).max() <= 1e-6


def test_split_gated_rows(gpu, orc):
    """Gate epilogue in the merge pass (c5a splits its 128 workgroups)."""
    w = configs.c5_attention()
    tab = cev_hip.BlockTable.from_rows(len(w.blocks), w.blocks[0], w.prefix, causal=True)
    gl = GpuLayer(w, gpu, table=tab)
    assert gl.attn.plan.n_splits > 1
    ol = OracleLayer(orc, w, gl.np_inputs)
    gl.forward()
    _check_blocks(gl, ol, [3, 17], BF16_TOL)


@pytest.mark.parametrize("name", ["c1", "hbm", "c5a"])
def test_graph_replay_matches_eager(gpu, name):
    """K1 + K2 captured once in a HIP graph: every replay, with eager work and
    synchronisations between replays, gives the eager result bit for bit
    (split plans included: the merge pass is part of the graph)."""
    import torch
    w = configs.WORKLOADS[name]()
    table = cev_hip.BlockTable.from_rows(len(w.blocks), w.blocks[0], w.prefix, causal=True) if name == "c5a" else None
    gl = GpuLayer(w, gpu, table=table)
    _say(f"test graph replay {w.name}: n_splits={gl.attn.plan.n_splits}")
    gl.forward()
    torch.cuda.synchronize()
    want = to_np(gl.out).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gl.qknorm()
        gl.attend()
    for i in range(3):
        gl.out.fill_(float("nan"))
        gl.q.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_np(gl.out), want), f"replay {i}"


def _same_bits(a, b):
    """Bit equality of two f32 arrays (so -0 != +0), NaN matching NaN."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


@pytest.mark.parametrize("repeat", [1, 30], ids=["quad", "lane"])
@pytest.mark.parametrize("bf16,d,rot,plus_one,inplace", [(True, 128, 128, False, False), (True, 256, 64, True, False),
                                                         (False, 128, 128, False, False), (True, 128, 128, False, True),
                                                         (True, 128, 32, False, False)])
def test_qknorm_rope_bit_exact_on_extreme_values(gpu, orc, bf16, d, rot, plus_one, inplace, repeat):
    """A call with few vectors gives each vector a DPP quad of lanes (576
    vectors here); a larger one (the same tokens 30 times, 17,280 vectors)
    gives each vector one lane.  A wave whose vectors are all in the fast
    division's range divides by reciprocal + FMA correction, any other wave
    uses IEEE division.  Vectors with zeros, -0, elements below 2^-96, huge
    elements and ordinary ones (both kinds of waves, and waves that mix
    them) must all match the oracle bit for bit, the sign of zero included;
    the in-place form (q_out = q_in) too."""
    import torch
    from cev_hip import synth
    t, hq, hkv, eps, theta = 96, 4, 2, 1e-6, 1e6
    dt = torch.bfloat16 if bf16 else torch.float32
    rng = np.random.default_rng(7)
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((t, hkv, d)).astype(np.float32)
    # tokens 0..15 (first wave of q): ordinary; 16..31: a tiny element in
    # some vectors; 32..47: zero and -0 vectors; 48..63: huge elements;
    # 64..95: scattered -0 and tiny elements in k
    q[16:32:3, 1, 5] = 2.0 ** -100
    q[17:32:5, 2, 70] = -(2.0 ** -110)
    q[32:40] = 0.0
    q[40:48] = -0.0
    q[48:64:4, 0, 3] = 2.0 ** 70
    q[50, 3, 9] = 2.0 ** 66
    k[64:96:2, 0, ::7] = -0.0
    k[65:96:4, 1, 11] = 2.0 ** -98
    if bf16:
        q, k = synth.round_bf16(q), synth.round_bf16(k)
    wq = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32) - (1.0 if plus_one else 0.0)
    wk = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32) - (1.0 if plus_one else 0.0)
    if bf16:
        wq, wk = synth.round_bf16(wq), synth.round_bf16(wk)
    pos = (np.arange(t) % 40 + 3).astype(np.int32)
    q, k, pos = np.tile(q, (repeat, 1, 1)), np.tile(k, (repeat, 1, 1)), np.tile(pos, repeat)
    n_pos = 64
    rotary = cev_hip.Rotary(theta, rot, n_pos, dt, gpu)
    dq, dk = to_dev(q, bf16, gpu), to_dev(k, bf16, gpu)
    kw = dict(q_out=dq, k_out=dk) if inplace else {}
    qo, ko = cev_hip.qknorm_rope(dq, dk, to_dev(wq, bf16, gpu), to_dev(wk, bf16, gpu), torch.from_numpy(pos).to(gpu), rotary, eps,
                                 plus_one=plus_one, **kw)
    torch.cuda.synchronize()
    cos, sin = orc.rope_table(theta, rot, n_pos, bf16)
    rq = orc.rope(orc.rms_norm(q, wq, eps, bf16, plus_one=plus_one), pos, cos, sin, rot, bf16)
    rk = orc.rope(orc.rms_norm(k, wk, eps, bf16, plus_one=plus_one), pos, cos, sin, rot, bf16)
    gq, gk = to_np(qo), to_np(ko)
    for name, got, want in (("q", gq, rq), ("k", gk, rk)):
        bad = ~((np.isnan(got) & np.isnan(want)) | (got.view(np.uint32) == want.view(np.uint32)))
        if bad.any():
            idx = np.argwhere(bad)[:5]
            _say(f"{name} mismatches at {idx.tolist()}: got {got[tuple(idx.T)]}, want {want[tuple(idx.T)]}")
        assert _same_bits(got, want), name


def test_split_records_are_never_stale(gpu):
    """Split parts write partial records that the merge pass reads.  A
    second call on the same plan and workspace with new K/V in the same
    buffers must merge the new records, not the first call's: each call is
    compared with an unsplit run of its own inputs (the merge may differ
    from it only in the last bits).  hkv = 4 puts the parts of one tile on
    two XCDs."""
    import torch
    for prefix, t, hq, hkv, d, dtype, gated in ((32768, 16, 32, 8, 128, torch.bfloat16, False),
                                                (4096, 128, 16, 4, 256, torch.bfloat16, True),
                                                (256, 32, 16, 8, 128, torch.float32, False)):
        g = torch.Generator(device="cpu").manual_seed(t)
        rnd = lambda *s: torch.randn(*s, generator=g).to(dtype).to(gpu)  # noqa: E731
        q, kn, vn = rnd(t, hq, d), rnd(t, hkv, d), rnd(t, hkv, d)
        kc, vc = rnd(hkv, prefix, d), rnd(hkv, prefix, d)
        gate = rnd(t, hq, d) if gated else None
        tab = cev_hip.BlockTable.from_rows(1, t, prefix, causal=True)
        op = cev_hip.PackedAttention(q, kn, tab, k_cache=kc, s_cache=prefix, v_new=vn, v_cache=vc, has_gate=gated, gate=gate)
        ref = cev_hip.PackedAttention(q, kn, tab, k_cache=kc, s_cache=prefix, v_new=vn, v_cache=vc, has_gate=gated, gate=gate,
                                      max_splits=1)
        assert op.plan.n_splits > 1 and ref.plan.n_splits == 1
        for call in range(3):
            got = op(q, kn, vn, kc, vc, gate).float()
            want = ref(q, kn, vn, kc, vc, gate).float()
            err = float((got - want).abs().max())
            _say(f"stale check hkv={hkv} d={d} {dtype} parts={op.plan.n_splits} call {call}: max|split - unsplit| {err:.3g}")
            assert err <= (1e-5 if dtype == torch.float32 else 1e-2)
            kc.copy_(rnd(hkv, prefix, d))  # new keys and values in place
            vc.copy_(rnd(hkv, prefix, d) * (call + 2))
