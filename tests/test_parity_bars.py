"""The bf16 parity bars (tests/bars.py) discriminate at the configs' own
output scales.  On the CPU, at c3's and c4's full shapes, a reference built
wrong on purpose from the oracle must miss the bars against the correct
references (each bar on its own), while the candle-op restatement itself,
a correct computation with its own bf16 rounding, passes against exact
attention.  Planted mistakes: one 64-key chunk of the key stream dropped,
RoPE positions of the query rows shifted by one, and (c4) the sigmoid output
gate left out."""
import numpy as np
import pytest

from bars import BF16_REL_CANDLE, BF16_REL_EXACT, bf16_failures, errors
from cev_hip import configs
from helpers import OracleLayer


def _inputs(w):
    pk, pv = w.prefix_kv()
    q, k, v = w.suffix_qkv()
    wq, wk = w.norm_weights()
    return pk, pv, q, k, v, wq, wk


def _block_operands(orc, ol, w, b, inputs, pos_shift=0):
    """(q, k, v) of block b over [prefix || block] as the oracle layer builds
    them, with the block's query positions moved by pos_shift."""
    pk, pv, q, k, v, wq, wk = inputs
    r0, L, d = int(w.block_starts()[b]), w.blocks[b], w.d
    qb = ol.q[r0:r0 + L]
    if pos_shift:
        cos, sin = orc.rope_table(w.theta, w.rotary_dim, w.n_pos() + pos_shift, w.bf16)
        qn = orc.rms_norm(q[r0:r0 + L, :, :d], wq, w.eps, w.bf16, plus_one=w.plus_one)
        qb = orc.rope(qn, w.positions()[r0:r0 + L] + pos_shift, cos, sin, w.rotary_dim, w.bf16)
    kb, vb = ol.k[r0:r0 + L].transpose(1, 0, 2), ol.v[r0:r0 + L].transpose(1, 0, 2)
    if w.prefix:
        kb = np.concatenate([ol.pk, kb], axis=1)
        vb = np.concatenate([ol.pv, vb], axis=1)
    return np.ascontiguousarray(qb.transpose(1, 0, 2)), np.ascontiguousarray(kb), np.ascontiguousarray(vb)


def _check(name, refs, planted):
    candle, exact = refs
    legit = bf16_failures(candle, exact=exact)
    _, rel_ce = errors(candle, exact)
    print(f"{name}: max|ref| {np.abs(exact).max():.3g}; candle-op vs exact rel {rel_ce:.3g} (bar {BF16_REL_EXACT})", flush=True)
    assert not legit, legit
    for what, out in planted.items():
        _, rc = errors(out, candle)
        _, re = errors(out, exact)
        print(f"  planted '{what}': rel vs candle-op {rc:.3g} (bar {BF16_REL_CANDLE}), vs exact {re:.3g} (bar {BF16_REL_EXACT})",
              flush=True)
        assert bf16_failures(out, candle=candle), what
        assert bf16_failures(out, exact=exact), what


@pytest.fixture(scope="module")
def c3_case(orc):
    w = configs.c3()
    inputs = _inputs(w)
    return w, inputs, OracleLayer(orc, w, inputs)


def test_bars_reject_planted_mistakes_c3(orc, c3_case):
    w, inputs, ol = c3_case
    b, rows = 20, (0, 32)
    q, k, v = _block_operands(orc, ol, w, b, inputs)
    mask = ol.mask(b)
    sel = slice(rows[0], rows[0] + rows[1])
    candle = orc.attend(q, k, v, mask, True, rows=rows)[0].transpose(1, 0, 2)[sel]
    exact = orc.attend_f64(q, k, v, mask, rows=rows)[0].transpose(1, 0, 2)[sel]
    dropped = mask.copy()
    dropped[:, w.prefix // 2: w.prefix // 2 + 64] = -np.inf
    planted = {
        "64-key prefix chunk dropped": orc.attend(q, k, v, dropped, True, rows=rows)[0].transpose(1, 0, 2)[sel],
        "positions shifted by one": orc.attend(_block_operands(orc, ol, w, b, inputs, pos_shift=1)[0], k, v, mask, True,
                                               rows=rows)[0].transpose(1, 0, 2)[sel],
    }
    _check("c3 block 20, rows 0-31", (candle, exact), planted)


def test_bars_reject_planted_mistakes_c4(orc):
    w = configs.c4()
    inputs = _inputs(w)
    ol = OracleLayer(orc, w, inputs)
    rows = (4000, 32)
    sel = slice(rows[0], rows[0] + rows[1])
    q, k, v = _block_operands(orc, ol, w, 0, inputs)
    mask = np.zeros((w.t, w.t), np.float32)  # one full-length bidirectional row: every key visible
    assert np.array_equal(mask[sel], orc.bidirectional_mask(w.t, [w.t])[0][sel])
    gate = ol.gate[sel]

    def gated(out):
        o = np.ascontiguousarray(out[sel])
        return orc.sigmoid_gate(o.reshape(o.shape[0], -1), np.ascontiguousarray(gate).reshape(o.shape[0], -1),
                                True).reshape(o.shape)

    raw = orc.attend(q, k, v, mask, True, rows=rows)[0].transpose(1, 0, 2)
    candle = gated(raw)
    exact = ol.block(0, rows=rows, f64=True)[sel]
    dropped = mask.copy()
    dropped[:, 4096:4160] = -np.inf
    planted = {
        "64-key chunk dropped": gated(orc.attend(q, k, v, dropped, True, rows=rows)[0].transpose(1, 0, 2)),
        "positions shifted by one": gated(orc.attend(_block_operands(orc, ol, w, 0, inputs, pos_shift=1)[0], k, v, mask, True,
                                                     rows=rows)[0].transpose(1, 0, 2)),
        "output gate left out": np.ascontiguousarray(raw[sel]),
    }
    _check("c4 rows 4000-4031", (candle, exact), planted)
