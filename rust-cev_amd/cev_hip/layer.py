"""One attention layer's hot path with its inputs resident in device memory:
K1 (QK-norm + RoPE, qwen3.rs:193-196 / qwen35.rs:529-539) then K2 (packed
attention, qwen3.rs:206-220 / qwen35.rs:563-579), both through the C ABI."""
from __future__ import annotations

import numpy as np

from . import BlockTable, D3Readout, PackedAttention, Rotary, qknorm_rope
from .configs import AttnWorkload


def _to_dev(x: np.ndarray, bf16: bool, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x)).to(device)
    return t.to(torch.bfloat16) if bf16 else t


def default_table(w: AttnWorkload) -> BlockTable:
    """The table the reference's engines build for a workload: the packed
    pass of engine.rs for causal blocks after a cached prefix, batch rows of
    hybrid.rs otherwise."""
    if w.causal:
        if w.prefix == 0:
            return BlockTable.from_rows(len(w.blocks), w.blocks[0], 0, causal=True)
        plans, items = w.plans_items()
        tab, pos, _ = BlockTable.from_plans(plans, items)
        if not np.array_equal(pos, w.positions()):
            raise AssertionError("engine positions disagree with the workload")
        return tab
    if len(set(w.blocks)) != 1:
        raise ValueError("bidirectional rows must share one length")
    return BlockTable.from_rows(len(w.blocks), w.blocks[0], 0, causal=False, lengths=w.lengths)


class AttentionLayer:
    def __init__(self, w: AttnWorkload, device, table: BlockTable = None, inputs=None):
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
        self.pk = _to_dev(pk, bf, device) if w.prefix else None
        self.pv = _to_dev(pv, bf, device) if w.prefix else None
        self.qp = _to_dev(q, bf, device)  # (t, hq, d) or the gated q_proj output (t, hq, 2d)
        self.k_in = _to_dev(k, bf, device)
        self.v = _to_dev(v, bf, device)
        self.wq = _to_dev(wq, bf, device)
        self.wk = _to_dev(wk, bf, device)
        self.pos = torch.from_numpy(w.positions()).to(device)
        self.rot = Rotary(w.theta, w.rotary_dim, w.n_pos(), self.dtype, device)
        d = w.d
        self.q_in = self.qp[:, :, :d]
        self.gate = self.qp[:, :, d:] if w.gated else None
        self.q = torch.empty((w.t, w.hq, d), dtype=self.dtype, device=device)
        self.k = torch.empty((w.t, w.hkv, d), dtype=self.dtype, device=device)
        self.out = torch.empty((w.t, w.hq, d), dtype=self.dtype, device=device)
        self.table = default_table(w) if table is None else table
        self.attn = PackedAttention(self.q, self.k, self.table, k_cache=self.pk, s_cache=w.prefix, has_gate=w.gated, out=self.out,
                                    gate=self.gate, v_new=self.v, v_cache=self.pv)
        # d3 workloads read the last position out through o_proj and the
        # readout matrix (hybrid.rs:657)
        self.readout = None
        self.logits = None
        if w.readout is not None:
            wo, wr = w.readout_weights()
            self.readout = D3Readout(wo, wr, w.readout[2], device, self.dtype)

    def qknorm(self):
        qknorm_rope(self.q_in, self.k_in, self.wq, self.wk, self.pos, self.rot, self.w.eps, plus_one=self.w.plus_one, q_out=self.q,
                    k_out=self.k)

    def attend(self):
        return self.attn(self.q, self.k, self.v, self.pk, self.pv, self.gate, self.out)

    def read_out(self):
        """Logits (1, codes) f32 of the last position (hybrid.rs:634, :657)."""
        w = self.w
        self.logits = self.readout(self.out[w.t - 1: w.t].view(1, w.hq * w.d))
        return self.logits

    def forward(self):
        self.qknorm()
        out = self.attend()
        if self.readout is not None:
            self.read_out()
        return out
