"""A device-resident Qwen3 decoder stack around the packed attention path.

The host mirror of Qwen3::prefill and Qwen3::forward_packed
(crates/cev-model/src/qwen3.rs:346-401) with everything on the GPU and every
compute call through the C ABI (torch only holds device memory):
  - embedding rows, the answer-row gather and the f32 conversion are
    cev_gather_rows (qwen3.rs:288-293, :399-400);
  - the projections are cev_linear (hipBLASLt GEMMs), q/k/v fused into one
    and gate/up into another (qwen3.rs:175-178, :229-233);
  - K1 (cev_qknorm_rope_kv) writes normalised, rotated q, and stores k and v
    straight into their slots of the layer's device caches;
  - K2 (cev_packed_attention) reads every key from those caches through the
    slot-addressed block table: no mask, no repeat_kv, no cat;
  - the norms, residual adds and SwiGLU are cev_rms_norm / cev_swiglu.
Every layer owns one (hkv, capacity, d) K cache and one V cache with the
same slot numbering; a cev_prefix_store (cev_hip.PrefixStore) decides which
slots hold which cached prefix (cev_hip.engine.DeviceEngine).
"""
from __future__ import annotations

import numpy as np

from . import (BlockTable, PackedAttention, Rotary, gather_rows, linear, qknorm_rope_kv, rms_norm, swiglu)


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
        self.rot = Rotary(w.theta, w.d, capacity + w.questions * w.q_len + 1, self.dtype, device)
        self.max_splits = max_splits  # split policy of the attention plans (0: the planner's)
        self._heads = {}

    def run(self, tokens, pos, slots, table: BlockTable):
        """All layers over the packed new tokens (Qwen3::forward_packed's
        layer loop, qwen3.rs:389-398); token i's K/V land in cache slot
        slots[i] of every layer.  The table is slot-addressed (s_cache =
        capacity).  Returns (x, h): the residual stream before the last
        layer's MLP residual add and that MLP output (t, H)."""
        import torch
        w = self.w
        t = len(tokens)
        if table.t != t or table.s_cache != self.capacity:
            raise ValueError(f"table is for t={table.t}, s_cache={table.s_cache}; pass has t={t}, capacity={self.capacity}")
        H, hq, hkv, d = w.hidden, w.hq, w.hkv, w.d
        i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a, np.int32), device=self.device)  # noqa: E731
        ids, pos_d, slots_d = i32(tokens), i32(pos), i32(slots)
        x = gather_rows(self.embed, ids)
        y = torch.empty_like(x)
        q = torch.empty((t, hq, d), dtype=self.dtype, device=self.device)
        o = torch.empty((t, hq, d), dtype=self.dtype, device=self.device)
        act = torch.empty((t, w.inter), dtype=self.dtype, device=self.device)
        qkv = torch.empty((t, (hq + 2 * hkv) * d), dtype=self.dtype, device=self.device)
        gu = torch.empty((t, 2 * w.inter), dtype=self.dtype, device=self.device)
        h = torch.empty_like(x)
        L0 = self.layers[0]
        # every key is a cache slot: the "new" K/V views are never read
        attn = PackedAttention(q, L0["k"].transpose(0, 1), table, k_cache=L0["k"], s_cache=self.capacity, out=o,
                               v_new=L0["v"].transpose(0, 1), v_cache=L0["v"], max_splits=self.max_splits)
        for i, L in enumerate(self.layers):
            # ln1: the first layer's input is the embedding; later ones come
            # fused with the previous layer's MLP residual add below
            if i == 0:
                rms_norm(x, L["ln1"], w.eps, y=y)
            linear(y, L["wqkv"], out=qkv)
            q_in = qkv[:, : hq * d].view(t, hq, d)
            k_in = qkv[:, hq * d: (hq + hkv) * d].view(t, hkv, d)
            v_in = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
            kt, vt = L["k"].transpose(0, 1), L["v"].transpose(0, 1)  # (capacity, hkv, d) views
            qknorm_rope_kv(q_in, k_in, v_in, L["q_norm"], L["k_norm"], pos_d, self.rot, w.eps, q, kt, vt, slots=slots_d,
                           n_slots=self.capacity)
            attn(q, kt, vt, L["k"], L["v"], None, o)
            linear(o.view(t, hq * d), L["wo"], out=h)
            rms_norm(x, L["ln2"], w.eps, h=h, x_out=x, y=y)  # x += h; y = ln2(x)
            linear(y, L["wgu"], out=gu)
            swiglu(gu[:, : w.inter], gu[:, w.inter:], out=act)
            linear(act, L["wdown"], out=h)
            if i + 1 < len(self.layers):
                rms_norm(x, self.layers[i + 1]["ln1"], w.eps, h=h, x_out=x, y=y)  # x += h; y = next ln1(x)
        return x, h

    def hidden(self, xh, gather):
        """The last residual add and the final norm at the gather rows, as
        f32 (qwen3.rs:397-400): rows are independent, so the add runs on the
        gathered rows only."""
        import torch
        x, h = xh
        g = torch.as_tensor(np.ascontiguousarray(gather, np.int32), device=self.device)
        xg, hg = gather_rows(x, g), gather_rows(h, g)
        y = rms_norm(xg, self.norm, self.w.eps, h=hg, x_out=xg)
        return gather_rows(y, out_dtype=torch.float32)

    def prefill(self, begin: int, tokens, chunk: int):
        """Qwen3::prefill (qwen3.rs:346-362) into slots begin .. begin +
        len(tokens): 512-token chunks that see the slots before them and
        themselves causally (segment_mask, qwen3.rs:157-169)."""
        n = len(tokens)
        for c0 in range(0, n, max(1, chunk)):
            part = tokens[c0: c0 + chunk]
            tab, pos, slots, _ = BlockTable.from_slots([(begin, c0 + len(part), c0)], [], self.capacity)
            self.run(part, pos, slots, tab)

    def code_head(self, code_ids):
        """The code rows of the tied head as f32 (engine.rs:155)."""
        import torch
        key = tuple(int(c) for c in code_ids)
        if key not in self._heads:
            ids = torch.as_tensor(np.asarray(key, np.int32), device=self.device)
            self._heads[key] = gather_rows(self.embed, ids, out_dtype=torch.float32)
        return self._heads[key]

    def code_logits(self, hidden, code_ids):
        """hidden . code_head^T in f32 (engine.rs:463)."""
        return linear(hidden, self.code_head(code_ids))


def softmax64(z) -> np.ndarray:
    """math::softmax (crates/cev-core/src/math.rs:7-12): f32 logits, f64 math."""
    z = np.asarray(z, np.float32)
    m = z.max(axis=-1, keepdims=True).astype(np.float64)
    e = np.exp(z.astype(np.float64) - m)
    return e / e.sum(axis=-1, keepdims=True)
