"""Shared pipelines for the parity tests: the GPU path through the C ABI and
the oracle path on the same seeded inputs."""
from __future__ import annotations

import numpy as np

import cev_hip
from cev_hip import configs


def to_dev(x: np.ndarray, bf16: bool, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(device)
    return t.to(torch.bfloat16) if bf16 else t


def to_np(t) -> np.ndarray:
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


class GpuLayer:
    """K1 (QK-norm + RoPE) then K2 (packed attention) for a workload, inputs
    resident on the device."""

    def __init__(self, w: configs.AttnWorkload, device, table=None, inputs=None):
        import torch
        self.w = w
        self.dev = device
        bf = w.bf16
        self.dtype = torch.bfloat16 if bf else torch.float32
        if inputs is None:
            pk, pv = w.prefix_kv()
            q, k, v = w.suffix_qkv()
            wq, wk = w.norm_weights()
        else:
            pk, pv, q, k, v, wq, wk = inputs
        self.np_inputs = (pk, pv, q, k, v, wq, wk)
        self.pk = to_dev(pk, bf, device) if w.prefix else None
        self.pv = to_dev(pv, bf, device) if w.prefix else None
        self.qp = to_dev(q, bf, device)             # (t, hq, d) or gated (t, hq, 2d)
        self.k_in = to_dev(k, bf, device)
        self.v = to_dev(v, bf, device)
        self.wq = to_dev(wq, bf, device)
        self.wk = to_dev(wk, bf, device)
        self.pos = torch.from_numpy(w.positions()).to(device)
        self.rot = cev_hip.Rotary(w.theta, w.rotary_dim, w.n_pos(), self.dtype, device)
        d = w.d
        self.q_in = self.qp[:, :, :d]
        self.gate = self.qp[:, :, d:] if w.gated else None
        self.q = torch.empty((w.t, w.hq, d), dtype=self.dtype, device=device)
        self.k = torch.empty((w.t, w.hkv, d), dtype=self.dtype, device=device)
        self.out = torch.empty((w.t, w.hq, d), dtype=self.dtype, device=device)
        if table is None:
            table = default_table(w)
        self.table = table
        self.attn = cev_hip.PackedAttention(self.q, self.k, table, k_cache=self.pk, s_cache=w.prefix, has_gate=w.gated,
                                            out=self.out, gate=self.gate, v_new=self.v, v_cache=self.pv)

    def qknorm(self):
        cev_hip.qknorm_rope(self.q_in, self.k_in, self.wq, self.wk, self.pos, self.rot, self.w.eps, plus_one=self.w.plus_one,
                            q_out=self.q, k_out=self.k)

    def attend(self):
        return self.attn(self.q, self.k, self.v, self.pk, self.pv, self.gate, self.out)

    def forward(self):
        self.qknorm()
        return self.attend()


def default_table(w: configs.AttnWorkload) -> cev_hip.BlockTable:
    if w.causal:
        if w.prefix == 0:
            return cev_hip.BlockTable.from_rows(len(w.blocks), w.blocks[0], 0, causal=True)
        plans, items = w.plans_items()
        tab, pos, _ = cev_hip.BlockTable.from_plans(plans, items)
        assert np.array_equal(pos, w.positions())
        return tab
    assert len(set(w.blocks)) == 1
    return cev_hip.BlockTable.from_rows(len(w.blocks), w.blocks[0], 0, causal=False, lengths=w.lengths)


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
        if w.causal:
            mask = orc.branch_mask(L, w.prefix)
        else:
            mask = orc.bidirectional_mask(L, [w.lengths[b]])[0]
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
