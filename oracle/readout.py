"""CPU oracle of the d3 readout (test infrastructure: loaded by tests/ only,
never by the product path).

Kind::Matrix reads a d3 package out as `answers.matmul(weight.t()) /
temperature` (crates/cev-model/src/hybrid.rs:657) with the (codes, hidden)
weight converted to f32 at load (crates/cev-model/src/load.rs:424).  Over one
Qwen3.5 gated-attention layer the answer row is that layer's o_proj output
(crates/cev-model/src/qwen35.rs:556-560: the gated attention output through
`self.o`, a bias-free Linear in the model dtype) at the last position,
converted to f32.

linear() is candle's matmul as the oracle states it: exact products summed
in f64, rounded once to f32 and, for bf16, once more to bf16 (candle's bf16
matmul rounds its f32 accumulator once; the gemm crate's f32 summation order
is unpinned and sits inside the tolerances).  Division by the temperature is
candle's `Tensor / f64`, an affine multiply by 1 / temperature in f32.
"""
from __future__ import annotations

import numpy as np

from . import round_bf16


def linear(x, w, bf16: bool) -> np.ndarray:
    """x (m, k) . w (n, k)^T in the model dtype (f32 values, bf16-exact for bf16)."""
    y = (np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32)
    return round_bf16(y) if bf16 else y


def inv_temperature(temperature: float) -> np.float32:
    """The f32 multiplier of `t / temperature as f64`: 1 / f64(f32(temperature))."""
    return np.float32(1.0 / np.float64(np.float32(temperature)))


def d3_readout(o_rows, wo, wr, temperature: float, bf16: bool) -> np.ndarray:
    """Logits (rows, codes) f32 of the attention output rows (rows, hq d)."""
    h = linear(o_rows, wo, bf16)            # o_proj in the model dtype
    z = linear(h.astype(np.float32), wr, False)  # answers (f32) . weight^T
    return (z * inv_temperature(temperature)).astype(np.float32)
