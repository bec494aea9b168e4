"""CPU oracle for the Qwen3 decoder stack (test infrastructure: loaded by
tests/ and the golden-fixture script only, never by the product path).

Restates Qwen3::prefill and Qwen3::forward_packed
(crates/cev-model/src/qwen3.rs:346-401) with the layer of qwen3.rs:187-262:
  x = embed[tokens]
  per layer:  y = ln1(x)                       rms_norm (the pinned C restatement)
              q, k, v = y W^T                  f32 GEMM, rounded once to the dtype
              q, k = rope(rms_norm(q|k))       the pinned QK-norm + RoPE (qwen3.rs:193-196)
              a = attend(q, [past k | k], ...) the pinned candle-op attention + dense mask
              x = dtype(x + a W_o^T)           (qwen3.rs:397)
              x = dtype(x + down(silu(g) * u)) with g, u = ln2(x) W^T (qwen3.rs:229-262)
  out = final_norm(x[gather]) as f32           (qwen3.rs:399-400)
The GEMMs use numpy's BLAS (f32 accumulation; candle's gemm summation order
is unpinned and sits inside the tolerances), bf16 results rounded once as
candle's bf16 matmul rounds its f32 accumulator.  SiLU in bf16 rounds each
op (exp, 1 + e, v / den) as in the device kernel and the GDN oracle.
"""
from __future__ import annotations

import numpy as np

from . import attend, engine_pass, rms_norm, rope, rope_table, round_bf16, segment_mask


def _rnd(x, bf16: bool):
    return round_bf16(x) if bf16 else np.ascontiguousarray(x, np.float32)


def _silu_mul(g, u, bf16: bool):
    g = g.astype(np.float32)
    if bf16:
        e = round_bf16(np.exp(-g))
        den = round_bf16(np.float32(1.0) + e)
        s = round_bf16(g / den)
        return round_bf16(s * u)
    return (g / (np.float32(1.0) + np.exp(-g))) * u


class Qwen3Oracle:
    def __init__(self, w, weights: dict):
        self.w, self.W = w, weights
        self.bf = w.bf16
        self.past = [(np.zeros((w.hkv, 0, w.d), np.float32), np.zeros((w.hkv, 0, w.d), np.float32)) for _ in range(w.n_layers)]
        self.cos, self.sin = rope_table(w.theta, w.d, w.state_tokens + w.questions * w.q_len + 1, self.bf)

    def _layers(self, tokens, pos, mask, past=None):
        """All layers over new tokens with the dense additive mask (t, past + t)
        over `past` (per layer (k, v), default the oracle's own cache).
        Returns the last residual stream and each layer's new (k, v)."""
        w, W, bf = self.w, self.W, self.bf
        past = self.past if past is None else past
        t = len(tokens)
        H, hq, hkv, d = w.hidden, w.hq, w.hkv, w.d
        x = W["embed"][np.asarray(tokens, np.int64)].astype(np.float32)
        new_kv = []
        for i in range(w.n_layers):
            p = f"l{i}."
            y = rms_norm(x, W[p + "ln1"], w.eps, bf)
            q = _rnd(y @ W[p + "wq"].T, bf).reshape(t, hq, d)
            k = _rnd(y @ W[p + "wk"].T, bf).reshape(t, hkv, d)
            v = _rnd(y @ W[p + "wv"].T, bf).reshape(t, hkv, d)
            q = rope(rms_norm(q, W[p + "q_norm"], w.eps, bf), pos, self.cos, self.sin, d, bf)
            k = rope(rms_norm(k, W[p + "k_norm"], w.eps, bf), pos, self.cos, self.sin, d, bf)
            kt, vt = k.transpose(1, 0, 2), v.transpose(1, 0, 2)
            pk, pv = past[i]
            kall = np.ascontiguousarray(np.concatenate([pk, kt], axis=1))
            vall = np.ascontiguousarray(np.concatenate([pv, vt], axis=1))
            a = attend(np.ascontiguousarray(q.transpose(1, 0, 2)), kall, vall, mask, bf)[0]  # (hq, t, d)
            a = np.ascontiguousarray(a.transpose(1, 0, 2)).reshape(t, hq * d)
            x = _rnd(x + _rnd(a @ W[p + "wo"].T, bf), bf)
            y = rms_norm(x, W[p + "ln2"], w.eps, bf)
            g = _rnd(y @ W[p + "gate"].T, bf)
            u = _rnd(y @ W[p + "up"].T, bf)
            x = _rnd(x + _rnd(_silu_mul(g, u, bf) @ W[p + "down"].T, bf), bf)
            new_kv.append((np.ascontiguousarray(kt), np.ascontiguousarray(vt)))
        return x, new_kv

    def prefill(self, tokens, chunk: int):
        """Qwen3::prefill (qwen3.rs:346-362): causal chunks over the cache."""
        for c0 in range(0, len(tokens), max(1, chunk)):
            part = tokens[c0: c0 + chunk]
            n, past = len(part), self.past[0][0].shape[1]
            mask = segment_mask(np.zeros(n, np.uint32), past)
            _, kv = self._layers(part, np.arange(past, past + n, dtype=np.int32), mask)
            self.past = [(np.concatenate([pk, k], 1), np.concatenate([pv, v], 1)) for (pk, pv), (k, v) in zip(self.past, kv)]

    def forward_packed(self, plans, items, tokens):
        """Engine::pass (engine.rs:365-442) + forward_packed: the final-normed
        hidden state (f32) at the gather rows; the plan's tail joins the cache."""
        ep = engine_pass(plans, items)
        x, kv = self._layers(tokens, ep["pos"], ep["mask"])
        hid = rms_norm(x[ep["gather"]], self.W["norm"], self.w.eps, self.bf).astype(np.float32)
        tail = plans[0][1] - plans[0][2]
        self.past = [(np.concatenate([pk, k[:, :tail]], 1), np.concatenate([pv, v[:, :tail]], 1))
                     for (pk, pv), (k, v) in zip(self.past, kv)]
        return hid

    def prefill_kv(self, tokens, chunk: int):
        """Qwen3::prefill from an empty cache, returned as per-layer (k, v)
        instead of kept (the PrefixKv the engine caches, engine.rs:251-254)."""
        kv = [(np.zeros((self.w.hkv, 0, self.w.d), np.float32),) * 2 for _ in range(self.w.n_layers)]
        for c0 in range(0, len(tokens), max(1, chunk)):
            part = tokens[c0: c0 + chunk]
            n, past = len(part), kv[0][0].shape[1]
            mask = segment_mask(np.zeros(n, np.uint32), past)
            _, new = self._layers(part, np.arange(past, past + n, dtype=np.int32), mask, past=kv)
            kv = [(np.concatenate([pk, k], 1), np.concatenate([pv, v], 1)) for (pk, pv), (k, v) in zip(kv, new)]
        return kv

    def code_logits(self, hidden, code_ids):
        head = self.W["embed"][np.asarray(code_ids, np.int64)].astype(np.float32)
        return hidden @ head.T


def softmax64(z) -> np.ndarray:
    """math::softmax (crates/cev-core/src/math.rs:7-12): f32 logits, f64 math."""
    z = np.asarray(z, np.float32)
    m = z.max(axis=-1, keepdims=True).astype(np.float64)
    e = np.exp(z.astype(np.float64) - m)
    return e / e.sum(axis=-1, keepdims=True)


def log_softmax64(z) -> np.ndarray:
    """math::log_softmax (crates/cev-core/src/math.rs:14-18): the f32 max as
    f64, lse = m + ln(sum e^(z - m)) with the sum taken in position order
    (the reference's iterator), z - lse in f64."""
    z = np.asarray(z, np.float32)
    m = np.float64(z.max())
    e = np.exp(z.astype(np.float64) - m)
    s = np.cumsum(e)[-1]  # sequential, left to right
    return z.astype(np.float64) - (m + np.log(s))


def rotation_shifts(k: int, max_permutations: int):
    """Debias::shifts for Permute / Full (crates/cev-core/src/compile.rs:127-136):
    at most max_permutations rotations of k options, evenly spread."""
    if k < 2:
        return [0]
    n = min(k, max(max_permutations, 1))
    out = []
    for i in range(n):
        s = i * k // n
        if not out or out[-1] != s:
            out.append(s)
    return out


def rotated_order(order, shift: int):
    """CompiledQuestion::rotated (crates/cev-core/src/compile.rs:67-73): the
    option shown at position j is order[(j + shift) % k]."""
    k = len(order)
    return [order[(j + shift) % k] for j in range(k)]


def debias_scores(logits, order, span_begin, span_len, n_options, calib=None) -> np.ndarray:
    """Service::run_debiased's averaging (crates/cev-runtime/src/service.rs:
    330-345): score[order[v][p]] += (lp_v[p] - base_v[p]) / n over the
    question's variants v in order, f64, stored as f32."""
    logits = np.asarray(logits, np.float32)
    q_n, ld = len(span_begin), logits.shape[1]
    out = np.zeros((q_n, ld), np.float32)
    for q in range(q_n):
        k, b, n = int(n_options[q]), int(span_begin[q]), int(span_len[q])
        score = np.zeros(k, np.float64)
        for v in range(b, b + n):
            lp = log_softmax64(logits[v, :k])
            base = log_softmax64(calib[v, :k]) if calib is not None else np.zeros(k)
            for pos in range(k):
                score[int(order[v][pos])] += (lp[pos] - base[pos]) / n
        out[q, :k] = score.astype(np.float32)
    return out


def run_config(w, weights=None):
    """The whole Qwen3-1.7B-shaped packed-pass flow on the oracle: prefill the head, one packed
    pass (tail + questions), code-head probabilities.  Returns
    (probabilities (questions, n_codes) f64, hidden (questions, H) f32)."""
    weights = w.weights() if weights is None else weights
    state, qs, codes = w.ids()
    o = Qwen3Oracle(w, weights)
    o.prefill(state[: w.head_tokens], w.prefill_chunk)
    plans, items = w.plans_items()
    tokens = np.concatenate([state[w.head_tokens:], qs.reshape(-1)])
    hid = o.forward_packed(plans, items, tokens)
    return softmax64(o.code_logits(hid, codes)), hid
