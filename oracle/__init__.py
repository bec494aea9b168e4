"""CPU oracle for cev's packed-prefill attention path (test infrastructure).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check results against (or as
the timed CPU baseline).  The product path never calls it.

The arithmetic lives in ``cev_oracle.c`` / ``gdn_oracle.c`` (built by the
Makefile next to this file into ``oracle/build/liboracle.so``); this module is
a thin numpy wrapper.  Each wrapper names the reference function it restates
(paths relative to the reference checkout).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")

# Planted mistakes, see cev_oracle.c.  Used only by the oracle's own pinning tests.
MUT_NONE = 0
MUT_ROPE_SIN_SIGN = 1
MUT_ATTN_KV_MODULO = 2
MUT_ATTN_NO_SCALE = 3
MUT_ATTN_V_SHIFT = 4
MUT_MASK_NO_DIAG = 5
MUT_NORM_DIM_M1 = 6
MUT_TABLE_POS = 7
MUT_GDN_NO_DECAY = 8

_lib = None


def build() -> str:
    """Compile the oracle with make (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


def _declare(L):
    i, i64, f, d, v = C.c_int, C.c_int64, C.c_float, C.c_double, None
    sig = {
        "orc_set_mutation": (v, [i]),
        "orc_get_mutation": (i, []),
        "orc_num_threads": (i, []),
        "orc_set_num_threads": (v, [i]),
        "orc_round_bf16": (v, [_f32p, _f32p, i64]),
        "orc_rope_table": (v, [d, i, i, i, _f32p, _f32p]),
        "orc_rms_norm": (v, [_f32p, i64, i, _f32p, i, f, i, _f32p]),
        "orc_rope": (v, [_f32p, i, i, i, i, _i32p, _f32p, _f32p, i]),
        "orc_segment_mask": (v, [_u32p, i, i, _f32p]),
        "orc_engine_pass": (i, [i, _i32p, _i32p, _i32p, i, _i32p, _i32p, _i32p, _i32p, _i32p, _i32p, C.c_void_p]),
        "orc_branch_mask": (v, [i, i, _f32p]),
        "orc_bidirectional_mask": (v, [i, _i32p, i, _f32p]),
        "orc_attend": (v, [_f32p, _f32p, _f32p, _f32p, i, i, i, i, i, i, i64, i64, i64, i, i, i, _f32p]),
        "orc_attend_blocked": (v, [_f32p, _f32p, _f32p, _f32p, i, i, i, i, i, i, i64, i64, i64, i, i, i, _f32p]),
        "orc_attend_f64": (v, [_f32p, _f32p, _f32p, _f32p, i, i, i, i, i, i, i64, i64, i64, i, i, _f64p]),
        "orc_sigmoid_gate": (v, [_f32p, _f32p, i64, i]),
        "orc_l2norm": (v, [_f32p, i64, i, _f32p]),
        "orc_softplus": (f, [f]),
        "orc_inv_unit_lower": (v, [_f32p, i, i, _f32p]),
        "orc_chunk_gated_delta_rule": (v, [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_void_p, i, i, i, i, i, _f32p, _f32p]),
        "orc_gdn_recurrence": (v, [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_void_p, i, i, i, i, _f32p, _f32p]),
        "orc_conv_silu": (v, [_f32p, C.c_void_p, _f32p, i, i, i, i, _f32p, _f32p]),
        "orc_gated_rmsnorm": (v, [_f32p, _f32p, _f32p, i64, i, f, i, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _c(x, dtype=np.float32):
    return np.ascontiguousarray(x, dtype=dtype)


class mutation:
    """Context manager planting one of the MUT_* mistakes in the oracle."""

    def __init__(self, m: int):
        self.m = m

    def __enter__(self):
        self.prev = lib().orc_get_mutation()
        lib().orc_set_mutation(self.m)
        return self

    def __exit__(self, *exc):
        lib().orc_set_mutation(self.prev)


def set_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def threads() -> int:
    return int(lib().orc_num_threads())


def round_bf16(x) -> np.ndarray:
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_round_bf16(x.reshape(-1), y.reshape(-1), x.size)
    return y


def rope_table(theta: float, rot: int, n_pos: int, bf16: bool):
    """Rotary::new, qwen3.rs:107-118 (and qwen35.rs:188-228 for text)."""
    half = rot // 2
    c = np.empty((n_pos, half), np.float32)
    s = np.empty((n_pos, half), np.float32)
    lib().orc_rope_table(float(theta), int(rot), int(n_pos), int(bf16), c, s)
    return c, s


def rms_norm(x, w, eps: float, bf16: bool, plus_one: bool = False) -> np.ndarray:
    """candle_nn::ops::rms_norm over the last dim (qwen3.rs:193-194, qwen35.rs:160-176)."""
    x = _c(x)
    d = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rms_norm(x.reshape(-1), x.size // d, d, _c(w), int(plus_one), float(eps), int(bf16), y.reshape(-1))
    return y


def rope(x, pos, cos, sin, rot: int, bf16: bool) -> np.ndarray:
    """Rotate-half RoPE on x (t, heads, d) at positions pos (t) (qwen3.rs:121-123)."""
    x = _c(x).copy()
    t, h, d = x.shape
    lib().orc_rope(x.reshape(-1), t, h, d, int(rot), _c(pos, np.int32), _c(cos), _c(sin), int(bf16))
    return x


def segment_mask(segments, past: int) -> np.ndarray:
    """qwen3.rs:157-169."""
    seg = _c(segments, np.uint32)
    n = seg.size
    m = np.empty((n, past + n), np.float32)
    lib().orc_segment_mask(seg, n, int(past), m)
    return m


def engine_pass(plans, batch, with_mask: bool = True):
    """The packed-pass builder of engine.rs:365-442.

    plans: list of (past_len, prefix_len, tail_start); batch: list of
    (plan index, question length).  Returns dict(pos, gather, owner, seg, mask,
    n, past_total).
    """
    n_plans = len(plans)
    past = _c([p[0] for p in plans] or [0], np.int32)
    pre = _c([p[1] for p in plans] or [0], np.int32)
    ts = _c([p[2] for p in plans] or [0], np.int32)
    ip = _c([b[0] for b in batch] or [0], np.int32)
    il = _c([b[1] for b in batch] or [0], np.int32)
    n = int(sum(max(p[1] - p[2], 0) for p in plans) + sum(b[1] for b in batch))
    past_total = int(sum(p[0] for p in plans))
    pos = np.zeros(max(n, 1), np.int32)
    owner = np.zeros(max(n, 1), np.int32)
    seg = np.zeros(max(n, 1), np.int32)
    gather = np.zeros(max(len(batch), 1), np.int32)
    mask = np.zeros((n, past_total + n), np.float32) if with_mask else None
    got = lib().orc_engine_pass(n_plans, past, pre, ts, len(batch), ip, il, pos, gather, owner, seg,
                                mask.ctypes.data if mask is not None else None)
    assert got == n
    return dict(pos=pos[:n], gather=gather[: len(batch)], owner=owner[:n], seg=seg[:n], mask=mask, n=n,
                past_total=past_total)


def branch_mask(t: int, past: int) -> np.ndarray:
    """qwen35.rs:471-479."""
    m = np.empty((t, past + t), np.float32)
    lib().orc_branch_mask(int(t), int(past), m)
    return m


def bidirectional_mask(t: int, lengths) -> np.ndarray:
    """qwen35.rs:483-498, (b, t, t)."""
    ln = _c(lengths, np.int32)
    m = np.empty((ln.size, t, t), np.float32)
    lib().orc_bidirectional_mask(int(t), ln, ln.size, m)
    return m


def _attend_shapes(q, k, mask):
    if q.ndim == 3:
        q = q[None]
    if k.ndim == 3:
        k = k[None]
    if mask.ndim == 2:
        mask = mask[None]
    return q, k, mask


def attend(q, k, v, mask, bf16: bool, rows=None) -> np.ndarray:
    """The candle op sequence of Attention::attend (qwen3.rs:206-220, qwen35.rs:563-579).

    q (b?, hq, t, d), k/v (b?, hkv, s, d) (b=1 broadcasts), mask (b?, t, s) additive.
    rows=(row0, nrows) restricts the computation to those query rows; the
    other rows of the output are left as NaN.
    """
    q, k, mask = _attend_shapes(_c(q), _c(k), _c(mask))
    v = _c(v)
    if v.ndim == 3:
        v = v[None]
    b = max(q.shape[0], k.shape[0], mask.shape[0])
    hq, t, d = q.shape[1:]
    hkv, s = k.shape[1], k.shape[2]
    assert mask.shape[-2:] == (t, s), (mask.shape, t, s)
    q_bs = 0 if q.shape[0] == 1 and b > 1 else hq * t * d
    if q.shape[0] != b:
        q = np.ascontiguousarray(np.broadcast_to(q, (b,) + q.shape[1:]))
        q_bs = hq * t * d
    kv_bs = 0 if k.shape[0] == 1 else hkv * s * d
    m_bs = 0 if mask.shape[0] == 1 else t * s
    row0, nrows = (0, t) if rows is None else rows
    out = np.full((b, hq, t, d), np.nan, np.float32)
    lib().orc_attend(q.reshape(-1), k.reshape(-1), v.reshape(-1), mask.reshape(-1), b, hq, hkv, t, s, d, q_bs, kv_bs, m_bs,
                     int(bf16), int(row0), int(nrows), out.reshape(-1))
    return out


def attend_blocked(q, k, v, mask, bf16: bool, rows=None) -> np.ndarray:
    """attend's op sequence with register-blocked FMA products over a packed
    K^T (oracle/cpu_attend.c): the CPU baseline's timed path.  Same shapes and
    result layout as attend; d a multiple of 32."""
    q, k, mask = _attend_shapes(_c(q), _c(k), _c(mask))
    v = _c(v)
    if v.ndim == 3:
        v = v[None]
    b = max(q.shape[0], k.shape[0], mask.shape[0])
    hq, t, d = q.shape[1:]
    hkv, s = k.shape[1], k.shape[2]
    assert mask.shape[-2:] == (t, s) and d % 32 == 0
    if q.shape[0] != b:
        q = np.ascontiguousarray(np.broadcast_to(q, (b,) + q.shape[1:]))
    kv_bs = 0 if k.shape[0] == 1 else hkv * s * d
    m_bs = 0 if mask.shape[0] == 1 else t * s
    row0, nrows = (0, t) if rows is None else rows
    out = np.full((b, hq, t, d), np.nan, np.float32)
    lib().orc_attend_blocked(q.reshape(-1), k.reshape(-1), v.reshape(-1), mask.reshape(-1), b, hq, hkv, t, s, d, hq * t * d, kv_bs,
                             m_bs, int(bf16), int(row0), int(nrows), out.reshape(-1))
    return out


def attend_f64(q, k, v, mask, rows=None) -> np.ndarray:
    """Textbook softmax attention in f64 over the keys the mask leaves visible."""
    q, k, mask = _attend_shapes(_c(q), _c(k), _c(mask))
    v = _c(v)
    if v.ndim == 3:
        v = v[None]
    b = max(q.shape[0], k.shape[0], mask.shape[0])
    if q.shape[0] != b:
        q = np.ascontiguousarray(np.broadcast_to(q, (b,) + q.shape[1:]))
    hq, t, d = q.shape[1:]
    hkv, s = k.shape[1], k.shape[2]
    kv_bs = 0 if k.shape[0] == 1 else hkv * s * d
    m_bs = 0 if mask.shape[0] == 1 else t * s
    row0, nrows = (0, t) if rows is None else rows
    out = np.full((b, hq, t, d), np.nan, np.float64)
    lib().orc_attend_f64(q.reshape(-1), k.reshape(-1), v.reshape(-1), mask.reshape(-1), b, hq, hkv, t, s, d, hq * t * d, kv_bs,
                         m_bs, int(row0), int(nrows), out.reshape(-1))
    return out


def sigmoid_gate(out, gate, bf16: bool) -> np.ndarray:
    """out * sigmoid(gate) in the model dtype (qwen35.rs:556-558)."""
    o = _c(out).copy()
    g = _c(gate)
    assert o.shape == g.shape
    lib().orc_sigmoid_gate(o.reshape(-1), g.reshape(-1), o.size, int(bf16))
    return o


def l2norm(x) -> np.ndarray:
    x = _c(x)
    y = np.empty_like(x)
    d = x.shape[-1]
    lib().orc_l2norm(x.reshape(-1), x.size // d, d, y.reshape(-1))
    return y


def softplus(x: float) -> float:
    return float(lib().orc_softplus(float(x)))


def inv_unit_lower(m) -> np.ndarray:
    """qwen35.rs:266-296 over the last two dims."""
    m = _c(m)
    n = m.shape[-1]
    out = np.empty_like(m)
    lib().orc_inv_unit_lower(m.reshape(-1), m.size // (n * n), n, out.reshape(-1))
    return out


def chunk_gated_delta_rule(q, k, v, g, beta, s0=None, chunk: int = 64):
    """qwen35.rs:301-368 for (h, t, ·) inputs; returns (out (h,t,dv), state (h,dk,dv))."""
    q, k, v, g, beta = (_c(x) for x in (q, k, v, g, beta))
    h, t, dk = q.shape
    dv = v.shape[-1]
    out = np.empty((h, t, dv), np.float32)
    st = np.empty((h, dk, dv), np.float32)
    s0c = None if s0 is None else _c(s0)
    lib().orc_chunk_gated_delta_rule(q.reshape(-1), k.reshape(-1), v.reshape(-1), g.reshape(-1), beta.reshape(-1),
                                     None if s0c is None else s0c.ctypes.data, h, t, dk, dv, int(chunk), out.reshape(-1),
                                     st.reshape(-1))
    return out, st


def gdn_recurrence(qn, kn, v, g, beta, s0=None):
    """The token recurrence of qwen35.rs:796-821 on normalised q, k."""
    qn, kn, v, g, beta = (_c(x) for x in (qn, kn, v, g, beta))
    h, t, dk = qn.shape
    dv = v.shape[-1]
    out = np.empty((h, t, dv), np.float32)
    st = np.empty((h, dk, dv), np.float32)
    s0c = None if s0 is None else _c(s0)
    lib().orc_gdn_recurrence(qn.reshape(-1), kn.reshape(-1), v.reshape(-1), g.reshape(-1), beta.reshape(-1),
                             None if s0c is None else s0c.ctypes.data, h, t, dk, dv, out.reshape(-1), st.reshape(-1))
    return out, st


def conv_silu(x, tail, w, bf16: bool):
    """Depthwise conv over [tail || x] + SiLU and the new tail (qwen35.rs:428-430)."""
    x = _c(x)
    c, t = x.shape
    kw = w.shape[-1]
    y = np.empty_like(x)
    nt = np.empty((c, kw - 1), np.float32)
    tc = None if tail is None else _c(tail)
    lib().orc_conv_silu(x.reshape(-1), None if tc is None else tc.ctypes.data, _c(w).reshape(-1), c, t, kw, int(bf16),
                        y.reshape(-1), nt.reshape(-1))
    return y, nt


def gated_rmsnorm(core, z, w, eps: float, bf16: bool):
    """qwen35.rs:447-451: core / sqrt(mean core^2 + eps) * w * silu(z), rows of dv."""
    core, z, w = _c(core), _c(z), _c(w)
    dv = core.shape[-1]
    y = np.empty_like(core)
    lib().orc_gated_rmsnorm(core.reshape(-1), z.reshape(-1), w, core.size // dv, dv, float(eps), int(bf16), y.reshape(-1))
    return y


def softplus_vec(x):
    return np.array([softplus(float(v)) for v in np.asarray(x, np.float32).reshape(-1)], np.float32).reshape(np.shape(x))


def gdn_layer(mixed, z, b, a, conv_w, neg_a, dt_bias, norm_w, nk: int, nv: int, dk: int, dv: int, eps: float, bf16: bool,
              conv_in=None, s_in=None):
    """GatedDeltaNet::forward (qwen35.rs:414-453) from the projection outputs on:
    mixed (B, T, 2 nk dk + nv dv), z (B, T, nv dv), b / a (B, T, nv) as f32 arrays
    holding model-dtype values; conv_w (C, K); neg_a = -exp(A_log), dt_bias,
    norm_w f32; conv_in (B, C, K-1) or None; s_in (B, nv, dk, dv) or None.
    Returns y (B, T, nv dv) before out_proj, the new conv tail and state."""
    B, T, Cd = mixed.shape
    kd = nk * dk
    ys, tails, states = [], [], []
    for r in range(B):
        x = np.ascontiguousarray(mixed[r].T)  # (C, T)
        conved, tail = conv_silu(x, None if conv_in is None else conv_in[r], conv_w, bf16)
        conved = conved.T  # (T, C)
        q = conved[:, :kd].reshape(T, nk, dk).transpose(1, 0, 2)
        k = conved[:, kd:2 * kd].reshape(T, nk, dk).transpose(1, 0, 2)
        v = conved[:, 2 * kd:].reshape(T, nv, dv).transpose(1, 0, 2)
        rep = nv // nk
        q = np.repeat(q, rep, axis=0)
        k = np.repeat(k, rep, axis=0)
        beta = (1.0 / (1.0 + np.exp(-b[r].astype(np.float32)))).astype(np.float32).T  # (nv, T)
        g = (softplus_vec(a[r].astype(np.float32) + dt_bias[None, :]) * neg_a[None, :]).astype(np.float32).T
        core, s = chunk_gated_delta_rule(q, k, v, g, beta, None if s_in is None else s_in[r])
        core = core.transpose(1, 0, 2).reshape(T * nv, dv)
        y = gated_rmsnorm(core, z[r].reshape(T * nv, dv), norm_w, eps, bf16).reshape(T, nv * dv)
        ys.append(y)
        tails.append(tail)
        states.append(s)
    return np.stack(ys), np.stack(tails), np.stack(states)
