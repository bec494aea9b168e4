"""Pass bars of the attention parity tests.

The contract's bars are absolute: attention output max |delta| <= 1e-5 in
f32 and <= 2e-2 in bf16.  At the bf16 configs' output scales (c3's outputs
average N(0,1) values over about 32k keys and peak near 0.04) an absolute
2e-2 cannot tell a good kernel from one that drops part of the key stream,
so every bf16 comparison also holds the error relative to the largest
reference value of that comparison:

- against exact attention (f64 over the same bf16 inputs): 2e-2 of max|ref|
  (a gated layer's output is rounded to bf16 through the gate's own bf16
  ops, about 2^-8 of each value, so exact agreement stops near 1e-2);
- against the candle-op restatement (which rounds scores and probabilities
  to bf16 on its own): 3e-2 of max|ref|.

tests/test_parity_bars.py shows on the CPU, at c3's and c4's scale, that
these bars reject references built wrong on purpose (a 64-key chunk of the
prefix dropped, RoPE positions shifted by one, the output gate left out)
while the candle-op restatement itself passes against exact attention.
"""
from __future__ import annotations

import numpy as np

F32_ABS = 1e-5
BF16_ABS = 2e-2
BF16_REL_EXACT = 2e-2
BF16_REL_CANDLE = 3e-2


def errors(got, ref):
    """(max |got - ref|, that divided by max |ref|)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    return err, (err / scale if scale > 0 else (0.0 if err == 0 else float("inf")))


def bf16_failures(got, candle=None, exact=None):
    """The bf16 bars `got` misses against the candle-op reference and/or exact
    attention, as a list of strings (empty: it passes)."""
    bad = []
    for name, ref, rel_bar in (("candle-op", candle, BF16_REL_CANDLE), ("exact", exact, BF16_REL_EXACT)):
        if ref is None:
            continue
        if not np.isfinite(np.asarray(got, np.float64)).all():
            bad.append(f"non-finite output vs {name}")
            continue
        err, rel = errors(got, ref)
        if not err <= BF16_ABS:
            bad.append(f"max|d| {err:.3g} vs {name} > {BF16_ABS}")
        if not rel <= rel_bar:
            bad.append(f"max|d|/max|ref| {rel:.3g} vs {name} > {rel_bar}")
    return bad


def assert_bf16(got, candle=None, exact=None, what=""):
    bad = bf16_failures(got, candle, exact)
    assert not bad, f"{what}: " + "; ".join(bad)


def assert_f32(got, ref, what=""):
    err, _ = errors(got, ref)
    assert np.isfinite(np.asarray(got)).all() and err <= F32_ABS, f"{what}: max|d| {err:.3g} > {F32_ABS}"
