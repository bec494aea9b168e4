"""A device-resident Qwen3 decoder stack around the packed attention path.

The host mirror of Qwen3::prefill and Qwen3::forward_packed
(crates/cev-model/src/qwen3.rs:346-401) with everything on the GPU:
  - the projections are library GEMMs (torch.matmul -> hipBLASLt), q/k/v
    fused into one and gate/up into another;
  - K1 (cev_qknorm_rope) writes normalised, rotated q and k, and k lands
    straight in this pass's slots of the layer's device K cache;
  - K2 (cev_packed_attention) reads the cache as (past, new) through two
    base pointers and the block table: no mask, no repeat_kv, no cat;
  - the norms, residual adds and SwiGLU are cev_rms_norm / cev_swiglu.
The per-layer K/V caches are preallocated (hkv, capacity, d) device tensors:
a chunked prefill appends in place, and a packed pass's tail slots become
part of the cached prefix without a copy (engine.rs:445-461 concatenates
instead).
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from . import BlockTable, PackedAttention, Rotary, qknorm_rope, rms_norm, swiglu


class Qwen3Stack:
    def __init__(self, w, weights: dict, device, capacity: int, dtype=None, max_splits: int = 0):
        """w: a Qwen3StackWorkload (shapes); weights: {name: array} as made
        by w.weights() (numpy) or w.device_weights() (torch); capacity: K/V
        cache slots per layer."""
        import torch
        self.w, self.device = w, device
        self.dtype = dtype if dtype is not None else (torch.bfloat16 if w.bf16 else torch.float32)

        def dev(x):
            if not isinstance(x, torch.Tensor):
                x = torch.from_numpy(np.ascontiguousarray(x))
            return x.to(device=device, dtype=self.dtype).contiguous()

        cat = lambda *xs: torch.cat([dev(x) for x in xs])  # noqa: E731
        self.embed = dev(weights["embed"])
        self.layers = []
        for i in range(w.n_layers):
            p = f"l{i}."
            self.layers.append(dict(
                wqkv=cat(weights[p + "wq"], weights[p + "wk"], weights[p + "wv"]),
                wo=dev(weights[p + "wo"]),
                wgu=cat(weights[p + "gate"], weights[p + "up"]),
                wdown=dev(weights[p + "down"]),
                q_norm=dev(weights[p + "q_norm"]), k_norm=dev(weights[p + "k_norm"]),
                ln1=dev(weights[p + "ln1"]), ln2=dev(weights[p + "ln2"]),
                k=torch.zeros((w.hkv, capacity, w.d), dtype=self.dtype, device=device),
                v=torch.zeros((w.hkv, capacity, w.d), dtype=self.dtype, device=device),
            ))
        self.norm = dev(weights["norm"])
        self.capacity = capacity
        self.rot = Rotary(w.theta, w.d, capacity, self.dtype, device)
        self.cached = 0  # tokens in the K/V caches
        self.max_splits = max_splits  # split policy of the attention plans (0: the planner's)

    def _run(self, tokens, pos, table: BlockTable, keep: bool) -> "torch.Tensor":
        """All layers over the packed new tokens; their K/V land in cache
        slots [cached, cached + t).  Returns the last residual stream (t, H)."""
        import torch
        w = self.w
        t, s0 = len(tokens), self.cached
        if table.t != t or table.s_cache != s0:
            raise ValueError(f"table is for t={table.t}, s_cache={table.s_cache}; pass has t={t}, cached={s0}")
        if s0 + t > self.capacity:
            raise ValueError(f"cache capacity {self.capacity} < {s0 + t} tokens")
        H, hq, hkv, d = w.hidden, w.hq, w.hkv, w.d
        ids = torch.as_tensor(np.asarray(tokens, np.int64), device=self.device)
        pos_d = torch.as_tensor(np.asarray(pos, np.int32), device=self.device)
        x = self.embed.index_select(0, ids)
        y = torch.empty_like(x)
        q = torch.empty((t, hq, d), dtype=self.dtype, device=self.device)
        o = torch.empty((t, hq, d), dtype=self.dtype, device=self.device)
        act = torch.empty((t, w.inter), dtype=self.dtype, device=self.device)
        attn: Optional[PackedAttention] = None
        for i, L in enumerate(self.layers):
            # ln1: the first layer's input is the embedding; later ones come
            # fused with the previous layer's MLP residual add below
            if i == 0:
                rms_norm(x, L["ln1"], w.eps, y=y)
            qkv = torch.matmul(y, L["wqkv"].t())
            q_in = qkv[:, : hq * d].view(t, hq, d)
            k_in = qkv[:, hq * d: (hq + hkv) * d].view(t, hkv, d)
            v_in = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
            k_new = L["k"][:, s0: s0 + t].transpose(0, 1)  # (t, hkv, d) view of the cache slots
            v_new = L["v"][:, s0: s0 + t].transpose(0, 1)
            qknorm_rope(q_in, k_in, L["q_norm"], L["k_norm"], pos_d, self.rot, w.eps, q_out=q, k_out=k_new)
            v_new.copy_(v_in)
            kc, vc = L["k"][:, :s0], L["v"][:, :s0]
            if attn is None:
                attn = PackedAttention(q, k_new, table, k_cache=kc if s0 else None, s_cache=s0, out=o, v_new=v_new,
                                       v_cache=vc if s0 else None, max_splits=self.max_splits)
            attn(q, k_new, v_new, kc if s0 else None, vc if s0 else None, None, o)
            h = torch.matmul(o.view(t, hq * d), L["wo"].t())
            rms_norm(x, L["ln2"], w.eps, h=h, x_out=x, y=y)  # x += h; y = ln2(x)
            gu = torch.matmul(y, L["wgu"].t())
            swiglu(gu[:, : w.inter], gu[:, w.inter:], out=act)
            h = torch.matmul(act, L["wdown"].t())
            nxt = self.layers[i + 1]["ln1"] if i + 1 < len(self.layers) else None
            if nxt is not None:
                rms_norm(x, nxt, w.eps, h=h, x_out=x, y=y)  # x += h; y = next ln1(x)
            else:
                x.add_(h)
        if keep:
            self.cached = s0 + t
        return x

    def prefill(self, tokens, chunk: int):
        """Qwen3::prefill (qwen3.rs:346-362): chunks seeing the cache and
        themselves causally, appended to the cache in place."""
        for c0 in range(0, len(tokens), max(1, chunk)):
            part = tokens[c0: c0 + chunk]
            n = len(part)
            table = BlockTable.from_segment_ids(np.zeros(n, np.uint32), past=self.cached)
            self._run(part, np.arange(self.cached, self.cached + n, dtype=np.int32), table, keep=True)

    def forward_packed(self, tokens, pos, table: BlockTable, gather, keep_tokens: int = 0):
        """Qwen3::forward_packed (qwen3.rs:364-401): the final-normed hidden
        state (f32) at the gather rows.  The first keep_tokens new tokens
        (a plan's tail) stay in the cache; later slots are reused."""
        import torch
        x = self._run(tokens, pos, table, keep=False)
        g = torch.as_tensor(np.asarray(gather, np.int64), device=self.device)
        xg = x.index_select(0, g)
        hidden = rms_norm(xg, self.norm, self.w.eps).to(torch.float32)
        self.cached += keep_tokens
        return hidden

    def code_logits(self, hidden, code_ids):
        """hidden . code_head^T with code_head = the tied head's rows for the
        code tokens, in f32 (engine.rs:155, :463)."""
        import torch
        head = self.embed.index_select(0, torch.as_tensor(np.asarray(code_ids, np.int64), device=self.device)).to(torch.float32)
        return torch.matmul(hidden, head.t())


def softmax64(z) -> np.ndarray:
    """math::softmax (crates/cev-core/src/math.rs:7-12): f32 logits, f64 math."""
    z = np.asarray(z, np.float32)
    m = z.max(axis=-1, keepdims=True).astype(np.float64)
    e = np.exp(z.astype(np.float64) - m)
    return e / e.sum(axis=-1, keepdims=True)
