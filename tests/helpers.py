"""Shared pipelines for the parity tests: the GPU path through the C ABI and
the oracle path on the same seeded inputs."""
from __future__ import annotations

import numpy as np

import cev_hip
from cev_hip import configs
from cev_hip.layer import AttentionLayer, default_table  # noqa: F401


def to_dev(x: np.ndarray, bf16: bool, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(device)
    return t.to(torch.bfloat16) if bf16 else t


def to_np(t) -> np.ndarray:
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


GpuLayer = AttentionLayer


class OracleLayer:
    """The same layer through the oracle: rms_norm -> rope -> attend per block
    over [prefix || block] (packed equivalence makes this the reference's
    packed result row for row) -> gate."""

    def __init__(self, orc, w: configs.AttnWorkload, inputs):
        self.orc, self.w = orc, w
        pk, pv, q, k, v, wq, wk = inputs
        bf = w.bf16
        d = w.d
        cos, sin = orc.rope_table(w.theta, w.rotary_dim, w.n_pos(), bf)
        qn = orc.rms_norm(q[:, :, :d], wq, w.eps, bf, plus_one=w.plus_one)
        kn = orc.rms_norm(k, wk, w.eps, bf, plus_one=w.plus_one)
        pos = w.positions()
        self.q = orc.rope(qn, pos, cos, sin, w.rotary_dim, bf)
        self.k = orc.rope(kn, pos, cos, sin, w.rotary_dim, bf)
        self.v = v
        self.gate = q[:, :, d:] if w.gated else None
        self.pk, self.pv = pk, pv
        self._masks = {}

    def mask(self, b: int) -> np.ndarray:
        """Additive mask of block b, built once (an 8192-token bidirectional
        mask takes seconds)."""
        if b not in self._masks:
            w, orc, L = self.w, self.orc, self.w.blocks[b]
            self._masks[b] = (orc.branch_mask(L, w.prefix) if w.causal else
                              orc.bidirectional_mask(L, [w.lengths[b]])[0])
        return self._masks[b]

    def block(self, b: int, rows=None, f64: bool = False):
        """Attention output (L, hq, d) of block b (rows=(r0, n) within it)."""
        w, orc = self.w, self.orc
        r0 = int(w.block_starts()[b])
        L = w.blocks[b]
        qb = self.q[r0:r0 + L].transpose(1, 0, 2)
        kb = self.k[r0:r0 + L].transpose(1, 0, 2)
        vb = self.v[r0:r0 + L].transpose(1, 0, 2)
        if w.prefix:
            kb = np.concatenate([self.pk, kb], axis=1)
            vb = np.concatenate([self.pv, vb], axis=1)
        mask = self.mask(b)
        if f64:
            out = orc.attend_f64(qb, kb, vb, mask, rows=rows)[0].transpose(1, 0, 2)
        else:
            out = orc.attend(qb, kb, vb, mask, w.bf16, rows=rows)[0].transpose(1, 0, 2)
        if self.gate is not None and not f64:
            g = self.gate[r0:r0 + L]
            sel = slice(None) if rows is None else slice(rows[0], rows[0] + rows[1])
            o = out[sel]
            out = out.copy()
            out[sel] = orc.sigmoid_gate(o.reshape(o.shape[0], -1), np.ascontiguousarray(g[sel]).reshape(o.shape[0], -1),
                                        w.bf16).reshape(o.shape)
        elif self.gate is not None:
            g = self.gate[r0:r0 + L].astype(np.float64)
            out = out * (1.0 / (1.0 + np.exp(-g)))
        return out
