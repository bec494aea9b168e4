"""Host side of the MI355X packed-prefill attention path, over libcev_hip.so.

This mirrors what the reference's attention call needs from its tensor layer
(crates/cev-model/src/qwen3.rs:187-220, crates/cev-model/src/qwen35.rs:526-579)
with the block-offset table in place of the dense mask builders
(crates/cev-model/src/engine.rs:389-442, qwen3.rs:153-169, qwen35.rs:469-498).
Every compute call goes through the C ABI; torch is used only to hold device
memory and to name the current stream.  There is no CPU fallback: without the
built library every call raises.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import synth  # noqa: F401  (re-exported)
from ._abi import (CEV_BF16, CEV_F32, CEV_LINEAR_WORKSPACE_BYTES, CEV_MAX_SPANS, AttnDesc, Block, CevError, GdnDesc, QkNormDesc, Span,
                   check, lib)

__all__ = [
    "GatedDeltaNet",
    "CEV_BF16", "CEV_F32", "CevError", "Block", "Span", "BlockTable", "AttnPlan", "PackedAttention",
    "packed_attention", "qknorm_rope", "rope_table", "Rotary", "device_info", "synth",
    "Blas", "linear", "gather_rows", "D3Readout", "PrefixStore", "qknorm_rope_kv",
]


def _torch():
    import torch
    return torch


def _dtype_code(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return CEV_F32
    if t.dtype == torch.bfloat16:
        return CEV_BF16
    raise CevError(-2, f"dtype {t.dtype} not supported (float32, bfloat16)")


def _stream_ptr(stream):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


# ---------------------------------------------------------------------------
# Block-offset table


class BlockTable:
    """A list of cev_block rows: which keys each packed query row sees."""

    def __init__(self, blocks: Sequence[Block], t: int, s_cache: int):
        self.blocks = list(blocks)
        self.t = int(t)
        self.s_cache = int(s_cache)

    def __len__(self):
        return len(self.blocks)

    def array(self):
        arr = (Block * max(1, len(self.blocks)))()
        for i, b in enumerate(self.blocks):
            arr[i] = b
        return arr

    @staticmethod
    def block(q_begin, q_len, local_begin, spans=(), causal=True, valid_len=None) -> Block:
        b = Block()
        b.q_begin, b.q_len, b.local_begin = int(q_begin), int(q_len), int(local_begin)
        b.causal = 1 if causal else 0
        b.valid_len = int(q_len if valid_len is None else valid_len)
        if len(spans) > CEV_MAX_SPANS:
            raise CevError(-1, f"{len(spans)} spans > {CEV_MAX_SPANS}")
        b.n_spans = len(spans)
        for i, (s0, sl) in enumerate(spans):
            b.spans[i] = Span(int(s0), int(sl))
        return b

    @classmethod
    def from_plans(cls, plans, items):
        """engine.rs:365-442.  plans: [(past_len, prefix_len, tail_start)];
        items: [(plan, question_len)].  Returns (table, pos, gather)."""
        L = lib()
        n_pl = len(plans)
        a = lambda xs: (C.c_int32 * max(1, len(xs)))(*[int(x) for x in xs])  # noqa: E731
        past, pre, ts = a([p[0] for p in plans]), a([p[1] for p in plans]), a([p[2] for p in plans])
        ip, il = a([i[0] for i in items]), a([i[1] for i in items])
        nb, nt = C.c_int32(), C.c_int32()
        check(L.cev_table_from_plans(n_pl, past, pre, ts, len(items), ip, il, None, 0, C.byref(nb), None, 0, C.byref(nt), None))
        blocks = (Block * max(1, nb.value))()
        pos = (C.c_int32 * max(1, nt.value))()
        gather = (C.c_int32 * max(1, len(items)))()
        check(L.cev_table_from_plans(n_pl, past, pre, ts, len(items), ip, il, blocks, nb.value, C.byref(nb), pos, nt.value,
                                     C.byref(nt), gather))
        s_cache = int(sum(p[0] for p in plans))
        tab = cls([blocks[i] for i in range(nb.value)], nt.value, s_cache)
        return tab, np.frombuffer(pos, np.int32)[: nt.value].copy(), np.frombuffer(gather, np.int32)[: len(items)].copy()

    @classmethod
    def from_slots(cls, plans, items, capacity: int):
        """engine.rs:365-442 over slot-addressed caches.  plans: [(kv_begin,
        prefix_len, tail_start)]; items: [(plan, question_len, first_slot)].
        Returns (table with s_cache = capacity, pos, slots, gather)."""
        L = lib()
        a = lambda xs: (C.c_int32 * max(1, len(xs)))(*[int(x) for x in xs])  # noqa: E731
        kb, pre, ts = a([p[0] for p in plans]), a([p[1] for p in plans]), a([p[2] for p in plans])
        ip, il, isl = a([i[0] for i in items]), a([i[1] for i in items]), a([i[2] for i in items])
        nb, nt = C.c_int32(), C.c_int32()
        check(L.cev_table_from_slots(len(plans), kb, pre, ts, len(items), ip, il, isl, int(capacity), None, 0, C.byref(nb), None, None,
                                     0, C.byref(nt), None))
        blocks = (Block * max(1, nb.value))()
        pos = (C.c_int32 * max(1, nt.value))()
        slots = (C.c_int32 * max(1, nt.value))()
        gather = (C.c_int32 * max(1, len(items)))()
        check(L.cev_table_from_slots(len(plans), kb, pre, ts, len(items), ip, il, isl, int(capacity), blocks, nb.value, C.byref(nb), pos,
                                     slots, nt.value, C.byref(nt), gather))
        tab = cls([blocks[i] for i in range(nb.value)], nt.value, int(capacity))
        as_np = lambda x, n: np.frombuffer(x, np.int32)[:n].copy()  # noqa: E731
        return tab, as_np(pos, nt.value), as_np(slots, nt.value), as_np(gather, len(items))

    @classmethod
    def from_rows(cls, b: int, t: int, past: int = 0, causal: bool = True, lengths=None):
        """HybridEngine::rows (hybrid.rs:592-617): b rows of t tokens."""
        blocks = (Block * max(1, b))()
        ln = None if lengths is None else (C.c_int32 * max(1, b))(*[int(x) for x in lengths])
        check(lib().cev_table_from_rows(b, t, past, 1 if causal else 0, ln, blocks, b))
        return cls([blocks[i] for i in range(b)], b * t, past)

    @classmethod
    def from_segment_ids(cls, seg, past: int = 0):
        """segment_mask (qwen3.rs:157-169) for contiguous segments."""
        seg = np.ascontiguousarray(seg, np.uint32)
        n = seg.size
        nb = C.c_int32()
        sp = seg.ctypes.data_as(C.POINTER(C.c_uint32))
        check(lib().cev_table_from_segment_ids(sp, n, past, None, 0, C.byref(nb)))
        blocks = (Block * max(1, nb.value))()
        check(lib().cev_table_from_segment_ids(sp, n, past, blocks, nb.value, C.byref(nb)))
        return cls([blocks[i] for i in range(nb.value)], n, past)

    @classmethod
    def from_dense_mask(cls, mask: np.ndarray, s_cache: int):
        mask = np.ascontiguousarray(mask, np.float32)
        t = mask.shape[0]
        assert mask.shape == (t, s_cache + t)
        nb = C.c_int32()
        check(lib().cev_table_from_dense_mask(C.c_void_p(mask.ctypes.data), t, s_cache, None, 0, C.byref(nb)))
        blocks = (Block * max(1, nb.value))()
        check(lib().cev_table_from_dense_mask(C.c_void_p(mask.ctypes.data), t, s_cache, blocks, nb.value, C.byref(nb)))
        return cls([blocks[i] for i in range(nb.value)], t, s_cache)

    def to_dense_mask(self) -> np.ndarray:
        m = np.empty((self.t, self.s_cache + self.t), np.float32)
        check(lib().cev_table_to_dense_mask(self.array(), len(self.blocks), self.t, self.s_cache, C.c_void_p(m.ctypes.data)))
        return m


# ---------------------------------------------------------------------------
# Attention


def attn_desc(dtype: int, hq: int, hkv: int, d: int, t: int, s_cache: int, has_gate: bool = False, scale: Optional[float] = None,
              **strides) -> AttnDesc:
    desc = AttnDesc()
    check(lib().cev_attn_desc_init(C.byref(desc), dtype, hq, hkv, d, t, s_cache, 1 if has_gate else 0))
    if scale is not None:
        desc.scale = float(scale)
    for k, v in strides.items():
        setattr(desc, k, int(v))
    return desc


class AttnPlan:
    """A table compiled for one descriptor: host bytes plus a device copy."""

    def __init__(self, desc: AttnDesc, table: BlockTable, device=None):
        L = lib()
        arr = table.array()
        size = C.c_size_t()
        check(L.cev_attn_plan_size(C.byref(desc), arr, len(table), C.byref(size)))
        raw = np.zeros(size.value + 16, np.uint8)
        off = (-raw.ctypes.data) % 16
        self.host = raw[off: off + size.value]
        check(L.cev_attn_plan_build(C.byref(desc), arr, len(table), C.c_void_p(self.host.ctypes.data), size.value))
        hdr = self.header()
        self.n_tiles = int(hdr[2])
        self.n_segs = int(hdr[3])
        self.tile_rows = int(hdr[6])
        self.n_splits = int(hdr[15])
        self.block_n = int(hdr[16])
        self.nbytes = size.value
        ws = C.c_size_t()
        check(L.cev_attn_workspace_size(C.c_void_p(self.host.ctypes.data), C.byref(ws)))
        self.workspace_bytes = ws.value
        self.dev = None
        self.workspace = None
        if device is not None:
            torch = _torch()
            self.dev = torch.from_numpy(self.host.copy()).to(device)
            if self.workspace_bytes:
                self.workspace = torch.empty(self.workspace_bytes, dtype=torch.uint8, device=device)

    def header(self) -> np.ndarray:
        return self.host[:80].view(np.int32)

    def tiles(self) -> np.ndarray:
        """(n_tiles, 8): row_begin, row_count, seg_begin, seg_count, n_chunks, 0, 0, 0."""
        hdr = self.header()
        return self.host.view(np.int32)[hdr[11]: hdr[11] + 8 * self.n_tiles].reshape(-1, 8)

    def segs(self) -> np.ndarray:
        hdr = self.header()
        return self.host.view(np.int32)[hdr[12]: hdr[12] + 4 * self.n_segs].reshape(-1, 4)

    def rows(self) -> np.ndarray:
        hdr = self.header()
        return self.host.view(np.int32)[hdr[13]: hdr[13] + 4 * int(hdr[4])].reshape(-1, 4)


class PackedAttention:
    """Packed-prefill attention over fixed shapes: Attention::attend
    (qwen3.rs:206-220) with K/V given as (cache, new) and a block table.

    Layouts: q, gate, out (t, hq, d) (any strides with unit last stride);
    k_cache / v_cache (hkv, s_cache, d); k_new / v_new (t, hkv, d)."""

    def __init__(self, q, k_new, table: BlockTable, k_cache=None, s_cache: int = 0, has_gate: bool = False,
                 scale: Optional[float] = None, out=None, gate=None, v_new=None, v_cache=None, max_splits: int = 0):
        t, hq, d = q.shape
        hkv = k_new.shape[1]
        if table.t != t or table.s_cache != s_cache:
            raise CevError(-1, f"table is for t={table.t}, s_cache={table.s_cache}; call has t={t}, s_cache={s_cache}")
        self.dtype = _dtype_code(q)
        self.desc = attn_desc(self.dtype, hq, hkv, d, t, s_cache, has_gate, scale)
        self.desc.max_splits = int(max_splits)
        self._set_strides(q, k_new, v_new if v_new is not None else k_new, k_cache, v_cache if v_cache is not None else k_cache,
                          out if out is not None else q, gate)
        self.plan = AttnPlan(self.desc, table, device=q.device)

    def _set_strides(self, q, kn, vn, kc, vc, out, gate):
        D = self.desc
        for t_ in (q, kn, vn, kc, vc, out, gate):
            if t_ is not None and t_.stride(-1) != 1:
                raise CevError(-2, "last dimension must be contiguous")
        D.q_stride_t, D.q_stride_h = q.stride(0), q.stride(1)
        D.kn_stride_t, D.kn_stride_h = kn.stride(0), kn.stride(1)
        D.vn_stride_t, D.vn_stride_h = vn.stride(0), vn.stride(1)
        if kc is not None:
            D.kc_stride_h, D.kc_stride_s = kc.stride(0), kc.stride(1)
            D.vc_stride_h, D.vc_stride_s = vc.stride(0), vc.stride(1)
        D.o_stride_t, D.o_stride_h = out.stride(0), out.stride(1)
        if gate is not None:
            D.g_stride_t, D.g_stride_h = gate.stride(0), gate.stride(1)

    def __call__(self, q, k_new, v_new, k_cache=None, v_cache=None, gate=None, out=None, stream=None):
        torch = _torch()
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        self._set_strides(q, k_new, v_new, k_cache, v_cache, out, gate)
        check(lib().cev_packed_attention(C.byref(self.desc), C.c_void_p(self.plan.host.ctypes.data), _ptr(self.plan.dev), _ptr(q),
                                         _ptr(k_cache), _ptr(v_cache), _ptr(k_new), _ptr(v_new), _ptr(gate), _ptr(out),
                                         _ptr(self.plan.workspace), self.plan.workspace_bytes, _stream_ptr(stream)))
        return out


def packed_attention(q, k_new, v_new, table: BlockTable, k_cache=None, v_cache=None, gate=None, scale=None, out=None, stream=None,
                     max_splits: int = 0):
    s_cache = 0 if k_cache is None else k_cache.shape[1]
    op = PackedAttention(q, k_new, table, k_cache=k_cache, s_cache=s_cache, has_gate=gate is not None, scale=scale, out=out,
                         gate=gate, v_new=v_new, v_cache=v_cache, max_splits=max_splits)
    return op(q, k_new, v_new, k_cache, v_cache, gate, out, stream)


# ---------------------------------------------------------------------------
# QK-norm + RoPE


def rope_table(theta: float, rotary_dim: int, n_pos: int, dtype: int):
    """Rotary::new (qwen3.rs:107-118) on the host: (cos, sin) as numpy
    arrays (n_pos, rotary_dim/2), float32 or uint16 bf16 bits."""
    half = rotary_dim // 2
    npdt = np.float32 if dtype == CEV_F32 else np.uint16
    c = np.empty((n_pos, half), npdt)
    s = np.empty((n_pos, half), npdt)
    check(lib().cev_rope_table(float(theta), int(rotary_dim), int(n_pos), int(dtype), C.c_void_p(c.ctypes.data),
                               C.c_void_p(s.ctypes.data)))
    return c, s


class Rotary:
    """Device-resident cos/sin table in the model dtype."""

    def __init__(self, theta: float, rotary_dim: int, n_pos: int, dtype, device):
        torch = _torch()
        code = CEV_F32 if dtype == torch.float32 else CEV_BF16
        c, s = rope_table(theta, rotary_dim, n_pos, code)
        if code == CEV_BF16:
            c = torch.from_numpy(c.view(np.int16)).view(torch.bfloat16)
            s = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
        else:
            c, s = torch.from_numpy(c), torch.from_numpy(s)
        self.cos = c.to(device)
        self.sin = s.to(device)
        self.rotary_dim = rotary_dim
        self.n_pos = n_pos


def qknorm_rope(q_in, k_in, w_q, w_k, pos, rot: Rotary, eps: float, plus_one: bool = False, q_out=None, k_out=None, stream=None):
    """RMSNorm + RoPE of q (t, hq, d) and k (t, hkv, d) views (qwen3.rs:193-196,
    qwen35.rs:529-539).  q_in may be a strided view of a gated q_proj output."""
    torch = _torch()
    t, hq, d = q_in.shape
    hkv = k_in.shape[1]
    code = _dtype_code(q_in)
    if q_out is None:
        q_out = torch.empty((t, hq, d), dtype=q_in.dtype, device=q_in.device)
    if k_out is None:
        k_out = torch.empty((t, hkv, d), dtype=k_in.dtype, device=k_in.device)
    desc = QkNormDesc()
    check(lib().cev_qknorm_desc_init(C.byref(desc), code, hq, hkv, d, t, rot.rotary_dim, rot.n_pos, 1 if plus_one else 0, float(eps), 0))
    for t_ in (q_in, k_in, q_out, k_out):
        if t_.stride(-1) != 1:
            raise CevError(-2, "last dimension must be contiguous")
    desc.qi_stride_t, desc.qi_stride_h = q_in.stride(0), q_in.stride(1)
    desc.ki_stride_t, desc.ki_stride_h = k_in.stride(0), k_in.stride(1)
    desc.qo_stride_t, desc.qo_stride_h = q_out.stride(0), q_out.stride(1)
    desc.ko_stride_t, desc.ko_stride_h = k_out.stride(0), k_out.stride(1)
    if pos.dtype != torch.int32:
        raise CevError(-1, "positions must be int32")
    check(lib().cev_qknorm_rope(C.byref(desc), _ptr(q_in), _ptr(k_in), _ptr(w_q), _ptr(w_k), _ptr(pos), _ptr(rot.cos), _ptr(rot.sin),
                                _ptr(q_out), _ptr(k_out), _stream_ptr(stream)))
    return q_out, k_out


def qknorm_rope_kv(q_in, k_in, v_in, w_q, w_k, pos, rot: Rotary, eps: float, q_out, k_out, v_out, slots=None, n_slots: int = 0,
                   plus_one: bool = False, stream=None):
    """qknorm_rope plus the cache store of the new tokens in one launch: k
    (normalised, rotated) and v (copied) of token i land in row slots[i] of
    k_out / v_out (row i without slots), e.g. (t_or_capacity, hkv, d) views
    of head-major caches."""
    torch = _torch()
    t, hq, d = q_in.shape
    hkv = k_in.shape[1]
    code = _dtype_code(q_in)
    desc = QkNormDesc()
    check(lib().cev_qknorm_desc_init(C.byref(desc), code, hq, hkv, d, t, rot.rotary_dim, rot.n_pos, 1 if plus_one else 0, float(eps), 0))
    for t_ in (q_in, k_in, v_in, q_out, k_out, v_out):
        if t_.stride(-1) != 1:
            raise CevError(-2, "last dimension must be contiguous")
    desc.qi_stride_t, desc.qi_stride_h = q_in.stride(0), q_in.stride(1)
    desc.ki_stride_t, desc.ki_stride_h = k_in.stride(0), k_in.stride(1)
    desc.qo_stride_t, desc.qo_stride_h = q_out.stride(0), q_out.stride(1)
    desc.ko_stride_t, desc.ko_stride_h = k_out.stride(0), k_out.stride(1)
    if pos.dtype != torch.int32 or (slots is not None and slots.dtype != torch.int32):
        raise CevError(-1, "positions and slots must be int32")
    check(lib().cev_qknorm_rope_kv(C.byref(desc), _ptr(q_in), _ptr(k_in), _ptr(v_in), v_in.stride(0), v_in.stride(1), _ptr(w_q),
                                   _ptr(w_k), _ptr(pos), _ptr(rot.cos), _ptr(rot.sin), _ptr(slots), int(n_slots), _ptr(q_out),
                                   _ptr(k_out), _ptr(v_out), v_out.stride(0), v_out.stride(1), _stream_ptr(stream)))
    return q_out, k_out, v_out


def rms_norm(x, w, eps: float, h=None, x_out=None, y=None, plus_one: bool = False, stream=None, sequential: bool = False):
    """candle_nn RmsNorm over the last dim of a (rows, hidden) view in the
    model dtype (qwen3.rs:254-255, :400); with h, the residual add before it
    (qwen3.rs:261, :358, :397): x_out = x + h is written (x_out may be x)
    and normalised.  sequential=True sums the squares in element order
    (cev_rms_norm_seq, candle's CPU order bit for bit) instead of tree order.
    Returns y."""
    torch = _torch()
    rows, hidden = x.shape
    if y is None:
        y = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
    if h is not None and x_out is None:
        x_out = x
    for t_ in (x, y, w) + ((h, x_out) if h is not None else ()):
        if t_.stride(-1) != 1 or t_.dtype != x.dtype:
            raise CevError(-2, "rms_norm: tensors must share the dtype and have a contiguous last dim")
    fn = lib().cev_rms_norm_seq if sequential else lib().cev_rms_norm
    check(fn(_dtype_code(x), rows, hidden, _ptr(x), x.stride(0), _ptr(h), h.stride(0) if h is not None else 0,
                             _ptr(x_out), x_out.stride(0) if x_out is not None else 0, _ptr(w), float(eps), 1 if plus_one else 0,
                             _ptr(y), y.stride(0), _stream_ptr(stream)))
    return y


def swiglu(gate, up, out=None, stream=None):
    """silu(gate) * up in the model dtype (Mlp::forward, qwen3.rs:230-233);
    gate and up are (rows, inter) views sharing a row stride."""
    torch = _torch()
    rows, inter = gate.shape
    if up.shape != gate.shape or up.stride(0) != gate.stride(0):
        raise CevError(-1, "swiglu: gate and up must have the same shape and row stride")
    if out is None:
        out = torch.empty((rows, inter), dtype=gate.dtype, device=gate.device)
    check(lib().cev_swiglu(_dtype_code(gate), rows, inter, _ptr(gate), _ptr(up), gate.stride(0), _ptr(out), out.stride(0),
                           _stream_ptr(stream)))
    return out


def debias_scores(logits, order, span_begin, span_len, n_options, calib=None, stream=None):
    """Debiased option scores on the device (Service::run_debiased's
    averaging, service.rs:330-345; math::log_softmax in f64, math.rs:14-18).
    logits / calib: (variants, ld) f32; order, span_begin, span_len,
    n_options: int32 device tensors.  Returns (questions, ld) f32."""
    torch = _torch()
    n_var, ld = logits.shape
    n_q = span_begin.shape[0]
    for name, t, dt in (("logits", logits, torch.float32), ("order", order, torch.int32), ("span_begin", span_begin, torch.int32),
                        ("span_len", span_len, torch.int32), ("n_options", n_options, torch.int32)) + \
            ((("calib", calib, torch.float32),) if calib is not None else ()):
        if t.dtype != dt or not t.is_contiguous():
            raise CevError(-1, f"debias_scores: {name} must be contiguous {dt}")
    if order.shape != logits.shape or (calib is not None and calib.shape != logits.shape):
        raise CevError(-1, "debias_scores: order / calib must match logits' shape")
    if span_len.shape[0] != n_q or n_options.shape[0] != n_q:
        raise CevError(-1, "debias_scores: one span and option count per question")
    scores = torch.empty((n_q, ld), dtype=torch.float32, device=logits.device)
    check(lib().cev_debias_scores(n_q, n_var, _ptr(span_begin), _ptr(span_len), _ptr(n_options), _ptr(logits),
                                  _ptr(calib) if calib is not None else None, _ptr(order), ld, _ptr(scores), _stream_ptr(stream)))
    return scores


# ---------------------------------------------------------------------------
# Linear layers, row gathers and the d3 readout


class Blas:
    """A cev_blas context (hipBLASLt, cached algorithms) and its workspace on
    one device; Blas.on(device) keeps one per device."""
    _per_device: dict = {}

    def __init__(self, device):
        torch = _torch()
        h = C.c_void_p()
        check(lib().cev_blas_create(C.byref(h)))
        self.handle = h
        self.workspace = torch.empty(CEV_LINEAR_WORKSPACE_BYTES, dtype=torch.uint8, device=device)

    @classmethod
    def on(cls, device) -> "Blas":
        torch = _torch()
        key = torch.device(device).index or 0
        if key not in cls._per_device:
            cls._per_device[key] = cls(device)
        return cls._per_device[key]

    def __del__(self):
        if getattr(self, "handle", None) is not None:
            try:
                lib().cev_blas_destroy(self.handle)
            except Exception:  # interpreter shutdown
                pass


def linear(x, w, out=None, alpha: float = 1.0, out_dtype=None, blas: Optional[Blas] = None, stream=None):
    """out = out_dtype(alpha * x @ w.T) for x (m, k), w (n, k): candle's bias-free
    Linear::forward (qwen3.rs:175-178, :229-233), the code head (engine.rs:463)
    and the d3 readout (hybrid.rs:657, alpha = 1 / temperature)."""
    torch = _torch()
    m, k = x.shape
    n = w.shape[0]
    code = _dtype_code(x)
    if w.dtype != x.dtype or w.shape[1] != k:
        raise CevError(-1, "linear: w must be (n, k) in x's dtype")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    for t_ in (x, w, out):
        if t_.stride(-1) != 1:
            raise CevError(-2, "linear: last dimension must be contiguous")
    blas = Blas.on(x.device) if (blas is None and m > 8) else blas
    ws = blas.workspace if blas is not None else None
    check(lib().cev_linear(blas.handle if blas is not None else None, code, _dtype_code(out), m, n, k, _ptr(x), x.stride(0), _ptr(w),
                           w.stride(0), float(alpha), _ptr(out), out.stride(0), _ptr(ws), ws.numel() if ws is not None else 0,
                           _stream_ptr(stream)))
    return out


def gather_rows(table, ids=None, out=None, out_dtype=None, stream=None):
    """out[i] = table[ids[i]] converted to out_dtype (Embedding rows,
    qwen3.rs:288-293; index_select of answer rows, qwen3.rs:399;
    to_dtype(F32), qwen3.rs:400, with ids None)."""
    torch = _torch()
    rows, width = table.shape
    n = rows if ids is None else ids.shape[0]
    if ids is not None and (ids.dtype != torch.int32 or not ids.is_contiguous()):
        raise CevError(-1, "gather_rows: ids must be contiguous int32")
    out_dtype = table.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((n, width), dtype=out_dtype, device=table.device)
    check(lib().cev_gather_rows(_dtype_code(table), _dtype_code(out), n, width, _ptr(table), table.stride(0), rows, _ptr(ids), _ptr(out),
                                out.stride(0), _stream_ptr(stream)))
    return out


class D3Readout:
    """Kind::Matrix (hybrid.rs:59-63, :657) over one Qwen3.5 gated-attention
    layer: the answer rows of the gated attention output go through o_proj
    (qwen35.rs:560, model dtype), are converted to f32 and multiplied by the
    (codes, hidden) f32 readout matrix, then divided by the temperature
    (candle's affine by 1 / temperature in f32)."""

    def __init__(self, wo, wr, temperature: float, device, dtype):
        torch = _torch()
        dev = lambda x, dt: torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dt)  # noqa: E731
        self.wo = dev(wo, dtype)
        self.wr = dev(wr, torch.float32)
        self.alpha = float(np.float32(1.0 / np.float64(np.float32(temperature))))
        self.h = torch.empty((1, self.wo.shape[0]), dtype=dtype, device=device)
        self.h32 = torch.empty((1, self.wo.shape[0]), dtype=torch.float32, device=device)
        self.logits = torch.empty((1, self.wr.shape[0]), dtype=torch.float32, device=device)

    def __call__(self, rows, stream=None):
        """rows: (r, hq d) answer rows of the attention output (r <= 8 reuse
        the preallocated buffers); returns (r, codes) f32 logits."""
        torch = _torch()
        r = rows.shape[0]
        if r != self.h.shape[0]:
            self.h = torch.empty((r, self.wo.shape[0]), dtype=self.wo.dtype, device=rows.device)
            self.h32 = torch.empty((r, self.wo.shape[0]), dtype=torch.float32, device=rows.device)
            self.logits = torch.empty((r, self.wr.shape[0]), dtype=torch.float32, device=rows.device)
        linear(rows, self.wo, out=self.h, stream=stream)
        gather_rows(self.h, out=self.h32, stream=stream)
        return linear(self.h32, self.wr, out=self.logits, alpha=self.alpha, stream=stream)


class PrefixStore:
    """cev_prefix_store: PrefixCache (engine.rs:474-503) over slot ranges of
    the per-layer device caches."""

    def __init__(self, capacity: int, budget: int):
        h = C.c_void_p()
        check(lib().cev_prefix_store_create(int(capacity), int(budget), C.byref(h)))
        self.handle, self.capacity, self.budget = h, int(capacity), int(budget)

    def __del__(self):
        if getattr(self, "handle", None) is not None:
            try:
                lib().cev_prefix_store_destroy(self.handle)
            except Exception:  # interpreter shutdown
                pass

    @staticmethod
    def _ids(tokens):
        arr = np.ascontiguousarray(tokens, np.uint32)
        return arr, arr.ctypes.data_as(C.POINTER(C.c_uint32))

    def get(self, tokens) -> Optional[int]:
        """First slot of the cached prefix `tokens` (now held), or None."""
        arr, p = self._ids(tokens)
        b, f = C.c_int32(), C.c_int32()
        check(lib().cev_prefix_store_get(self.handle, p, arr.size, C.byref(b), C.byref(f)))
        return b.value if f.value else None

    def reserve(self, n: int) -> int:
        b = C.c_int32()
        check(lib().cev_prefix_store_reserve(self.handle, int(n), C.byref(b)))
        return b.value

    def put(self, tokens, begin: int) -> None:
        arr, p = self._ids(tokens)
        check(lib().cev_prefix_store_put(self.handle, p, arr.size, int(begin)))

    def release(self, begin: int) -> None:
        check(lib().cev_prefix_store_release(self.handle, int(begin)))

    def stats(self):
        e, c, u = C.c_int32(), C.c_int64(), C.c_int32()
        check(lib().cev_prefix_store_stats(self.handle, C.byref(e), C.byref(c), C.byref(u)))
        return dict(entries=e.value, cached_tokens=c.value, used_slots=u.value)

    def entries(self):
        """[(first slot, length)] in LRU order (oldest first)."""
        out = []
        for i in range(self.stats()["entries"]):
            b, n = C.c_int32(), C.c_int32()
            check(lib().cev_prefix_store_entry(self.handle, i, C.byref(b), C.byref(n)))
            out.append((b.value, n.value))
        return out


@dataclass
class DeviceInfo:
    name: str
    n_cus: int
    hbm_bytes: int
    clock_mhz: int


def device_info(device: int = 0) -> DeviceInfo:
    name = C.create_string_buffer(128)
    cus, hbm, clk = C.c_int32(), C.c_int64(), C.c_int32()
    check(lib().cev_device_info(device, name, 128, C.byref(cus), C.byref(hbm), C.byref(clk)))
    return DeviceInfo(name.value.decode(), cus.value, hbm.value, clk.value)


# ---------------------------------------------------------------------------
# Gated DeltaNet layer core


class GatedDeltaNet:
    """The part of GatedDeltaNet::forward (qwen35.rs:414-453) between the input
    projections and out_proj, on the device: conv + SiLU with its state,
    l2norm / sigmoid / softplus gates, chunk_gated_delta_rule and the gated
    RMSNorm.  The projections stay the caller's GEMMs.

    Tensors: mixed (B, T, 2 nk dk + nv dv), z (B, T, nv dv), b, a (B, T, nv)
    and conv_w (conv_dim, K) in the model dtype; neg_a = -exp(A_log), dt_bias
    and norm_w f32; conv_in (B, conv_dim, K-1) in the model dtype and s_in
    (B, nv, dk, dv) f32, either may have batch stride 0 (one state for every
    row) or be None (zero state).  Returns (y (B, T, nv dv), conv_out, s_out)."""

    def __init__(self, batch: int, t: int, n_k_heads: int, n_v_heads: int, head_k_dim: int = 128, head_v_dim: int = 128,
                 conv_kernel: int = 4, eps: float = 1e-6, dtype=None, device=None):
        torch = _torch()
        dtype = torch.bfloat16 if dtype is None else dtype
        self.dtype, self.device = dtype, device
        self.desc = GdnDesc()
        code = CEV_BF16 if dtype == torch.bfloat16 else CEV_F32
        check(lib().cev_gdn_desc_init(C.byref(self.desc), code, batch, t, n_k_heads, n_v_heads, head_k_dim, head_v_dim,
                                      conv_kernel, float(eps)))
        n = C.c_size_t(0)
        check(lib().cev_gdn_workspace_size(C.byref(self.desc), C.byref(n)))
        self.workspace = torch.empty(n.value, dtype=torch.uint8, device=device)
        self.conv_dim = 2 * n_k_heads * head_k_dim + n_v_heads * head_v_dim
        self.shape = (batch, t, n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel)

    def __call__(self, mixed, z, b, a, conv_w, neg_a, dt_bias, norm_w, conv_in=None, s_in=None, y=None, conv_out=None,
                 s_out=None, stream=None):
        torch = _torch()
        B, T, nk, nv, dk, dv, K = self.shape
        D = self.desc
        for name, x in (("mixed", mixed), ("z", z), ("b", b), ("a", a)):
            if x.stride(-1) != 1 or x.dtype != self.dtype:
                raise ValueError(f"{name} must be {self.dtype} with unit channel stride")
        D.mixed_stride_b, D.mixed_stride_t = mixed.stride(0), mixed.stride(1)
        D.z_stride_b, D.z_stride_t = z.stride(0), z.stride(1)
        if a.stride() != b.stride():
            raise ValueError("a and b must share strides")
        D.ab_stride_b, D.ab_stride_t = a.stride(0), a.stride(1)
        if conv_in is not None:
            if conv_in.stride(1) != K - 1 or conv_in.stride(2) != 1:
                raise ValueError("conv_in must be (B, conv_dim, K-1) with contiguous rows")
            D.conv_in_stride_b = conv_in.stride(0)
        if s_in is not None:
            if s_in.dtype != torch.float32 or tuple(s_in.stride()[1:]) != (dk * dv, dv, 1):
                raise ValueError("s_in must be f32 (B, nv, dk, dv) with contiguous heads")
            D.s_in_stride_b = s_in.stride(0)
        if y is None:
            y = torch.empty((B, T, nv * dv), dtype=self.dtype, device=mixed.device)
        D.y_stride_b, D.y_stride_t = y.stride(0), y.stride(1)
        if conv_out is None:
            conv_out = torch.empty((B, self.conv_dim, K - 1), dtype=self.dtype, device=mixed.device)
        if s_out is None:
            s_out = torch.empty((B, nv, dk, dv), dtype=torch.float32, device=mixed.device)
        check(lib().cev_gdn_forward(C.byref(D), _ptr(mixed), _ptr(z), _ptr(b), _ptr(a), _ptr(conv_w), _ptr(neg_a), _ptr(dt_bias),
                                    _ptr(norm_w), _ptr(conv_in), _ptr(s_in), _ptr(y), _ptr(conv_out), _ptr(s_out),
                                    _ptr(self.workspace), self.workspace.numel(), _stream_ptr(stream)))
        return y, conv_out, s_out
