"""The synthetic workloads of this path as concrete shapes and seeded inputs.

Every tensor comes from cev_hip.synth with seed = workload number and its own
stream id, so the GPU run and the CPU oracle see identical values.  Arrays
are f32 (holding bf16-exact values for bf16 workloads).

  c1  Qwen3-0.6B-shaped attention layer, f32: cached prefix P=256 (Hkv=8,
      d=128, post-RoPE K/V), 4 questions x 3 rotations = 12 blocks x 32 tokens,
      Hq=16, positions restart at 256 per block (engine.rs:411).
  c3  Qwen3-8B-shaped layer, bf16: P=32768, 64 blocks x 64 tokens, Hq=32,
      Hkv=8, d=128, positions restart at 32768.
  c4  Qwen3.5-style gated layer, bf16, bidirectional (d3): one 8192-token row,
      Hq=16, Hkv=4, d=256, rotary 64 of 256 dims (theta 1e7), weight 1 + w,
      sigmoid output gate; read out at the last position through o_proj
      (hidden 2048) and a random 255 x 2048 f32 readout matrix at
      temperature 0.8 (d3's Kind::Matrix, hybrid.rs:657).
  c5a the gated-attention half of the hybrid pair: 32 rows right-padded to
      64 tokens continue a 4096-token prefix (Hq=16, Hkv=4, d=256).
  hbm the long-prefix short-suffix shape: c3 with 1 block x 16 tokens.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from . import synth

# stream ids
S_PK, S_PV, S_Q, S_K, S_V, S_WQ, S_WK, S_GATE, S_LEN, S_WO, S_WR = range(1, 12)


@dataclass
class AttnWorkload:
    name: str
    seed: int
    bf16: bool
    hq: int
    hkv: int
    d: int
    prefix: int                     # cached keys (post-RoPE prefix K/V)
    blocks: List[int]               # suffix block lengths (packed in order)
    theta: float
    rotary_dim: int
    causal: bool = True
    gated: bool = False
    plus_one: bool = False          # Qwen3.5 RMSNorm weight 1 + w
    eps: float = 1e-6
    lengths: Optional[List[int]] = None   # real tokens per row (padded rows)
    pos0: Optional[int] = None      # first suffix position (default: prefix)
    readout: Optional[Tuple[int, int, float]] = None  # d3 readout: (hidden, codes, temperature)
    notes: str = ""

    @property
    def t(self) -> int:
        return int(sum(self.blocks))

    @property
    def g(self) -> int:
        return self.hq // self.hkv

    def positions(self) -> np.ndarray:
        p0 = self.prefix if self.pos0 is None else self.pos0
        return np.concatenate([p0 + np.arange(L, dtype=np.int32) for L in self.blocks]).astype(np.int32)

    def n_pos(self) -> int:
        return int(self.positions().max()) + 1

    def block_starts(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.blocks)[:-1]]).astype(np.int64)

    def useful_pairs(self) -> int:
        """Unmasked (query row, key) pairs per query head."""
        tot = 0
        for i, L in enumerate(self.blocks):
            if self.causal:
                tot += L * self.prefix + L * (L + 1) // 2
            else:
                v = L if self.lengths is None else self.lengths[i]
                tot += L * self.prefix + v * L + (L - v)
        return tot

    def useful_flops(self) -> float:
        """Unmasked pairs x 4d (QK^T and PV) over all query heads."""
        return 4.0 * self.d * self.hq * self.useful_pairs()

    def alg_bytes(self) -> int:
        """Q, K/V (prefix + new), O and the gate, each once, in the config dtype."""
        e = 2 if self.bf16 else 4
        t = self.t
        n = t * self.hq * self.d * 2 + 2 * (self.prefix + t) * self.hkv * self.d
        if self.gated:
            n += t * self.hq * self.d
        return n * e

    # ---- inputs -------------------------------------------------------
    def prefix_kv(self, kv_heads: Optional[Tuple[int, int]] = None):
        """(hkv, P, d) post-RoPE cached K and V."""
        shape = (self.hkv, self.prefix, self.d)
        return (synth.tensor(self.seed, S_PK, shape, self.bf16), synth.tensor(self.seed, S_PV, shape, self.bf16))

    def suffix_qkv(self):
        """Pre-norm q (t, hq, d) [or the gated (t, hq, 2d) q_proj output], k and v (t, hkv, d)."""
        t = self.t
        qd = 2 * self.d if self.gated else self.d
        q = synth.tensor(self.seed, S_Q, (t, self.hq, qd), self.bf16)
        k = synth.tensor(self.seed, S_K, (t, self.hkv, self.d), self.bf16)
        v = synth.tensor(self.seed, S_V, (t, self.hkv, self.d), self.bf16)
        return q, k, v

    def norm_weights(self):
        """QK-norm weights: 1 + 0.1 N(0,1) as stored (Qwen3), or 0.1 N(0,1)
        as stored for the zero-centred form (Qwen3.5 applies 1 + w)."""
        off = 0.0 if self.plus_one else 1.0
        wq = synth.tensor(self.seed, S_WQ, (self.d,), self.bf16, scale=0.1, offset=off)
        wk = synth.tensor(self.seed, S_WK, (self.d,), self.bf16, scale=0.1, offset=off)
        return wq, wk

    def readout_weights(self):
        """d3 readout: o_proj (hidden, hq d) N(0, 0.02) in the model dtype
        and the readout matrix (codes, hidden) N(0, 0.02) in f32 (load.rs
        converts it to f32)."""
        hidden, codes, _ = self.readout
        wo = synth.tensor(self.seed, S_WO, (hidden, self.hq * self.d), self.bf16, scale=0.02)
        wr = synth.tensor(self.seed, S_WR, (codes, hidden), False, scale=0.02)
        return wo, wr

    def plans_items(self):
        """engine.rs packing: one plan whose whole prefix is cached, one
        question item per block."""
        return [(self.prefix, self.prefix, self.prefix)], [(0, L) for L in self.blocks]


def c1() -> AttnWorkload:
    return AttnWorkload("c1", 1, False, 16, 8, 128, 256, [32] * 12, 1e6, 128,
                        notes="Qwen3-0.6B-shaped layer, f32, 12 x 32 blocks after P=256")


def c3(blocks: int = 64, block_len: int = 64) -> AttnWorkload:
    return AttnWorkload("c3", 3, True, 32, 8, 128, 32768, [block_len] * blocks, 1e6, 128,
                        notes="Qwen3-8B-shaped layer, bf16, 64 x 64 blocks after P=32768")


def hbm(blocks: int = 1) -> AttnWorkload:
    w = c3(blocks, 16)
    w.name = f"hbm{blocks}x16"
    w.notes = f"c3 prefix with {blocks} x 16 suffix tokens (KV-streaming bound)"
    return w


def c4() -> AttnWorkload:
    return AttnWorkload("c4", 4, True, 16, 4, 256, 0, [8192], 1e7, 64, causal=False, gated=True, plus_one=True,
                        lengths=[8192], pos0=0, readout=(2048, 255, 0.8),
                        notes="Qwen3.5-style gated layer, bf16, bidirectional 8192-token row, d3 readout at the last position")


def d3_f32() -> AttnWorkload:
    """A small f32 case of c4's shape family for the d3 readout's f32 bar:
    one 64-token bidirectional gated row, Hq=4, Hkv=2, d=128, hidden 256."""
    return AttnWorkload("d3f32", 6, False, 4, 2, 128, 0, [64], 1e7, 32, causal=False, gated=True, plus_one=True, lengths=[64],
                        pos0=0, readout=(256, 255, 0.8), notes="f32 gated bidirectional row with a d3 readout")


def c5_attention() -> AttnWorkload:
    n_rows, t = 32, 64
    lengths = (33 + np.floor(synth.uniform(5, S_LEN, n_rows) * 32)).astype(int).tolist()
    return AttnWorkload("c5a", 5, True, 16, 4, 256, 4096, [t] * n_rows, 1e7, 64, causal=True, gated=True, plus_one=True,
                        lengths=lengths, notes="Qwen3.5 gated attention: 32 rows padded to 64 after P=4096")


WORKLOADS = {"c1": c1, "c3": c3, "c4": c4, "c5a": c5_attention, "hbm": hbm}


@dataclass
class GdnWorkload:
    """One Gated DeltaNet layer of a Qwen3.5 hybrid prefix (the 4096-token prefix's GDN
    part: Hk = 16 repeated to Hv = 32, dk = dv = 128, conv kernel 4, 64-token
    chunks).  Synthetic inputs stand for the projection outputs: q/k/v/z
    N(0,1); beta = sigmoid(b) uniform in (0, 1) and the per-token decay
    e^g log-uniform in [1e-3, 1] (b = logit(u), a = softplus^-1(-g) with
    dt_bias = 0, -e^A = -1)."""
    name: str
    seed: int
    bf16: bool
    batch: int
    t: int
    nk: int = 16
    nv: int = 32
    dk: int = 128
    dv: int = 128
    kernel: int = 4
    eps: float = 1e-6

    @property
    def conv_dim(self) -> int:
        return 2 * self.nk * self.dk + self.nv * self.dv

    def flops(self) -> float:
        """chunk_gated_delta_rule multiply-adds (x2) per head and 64-token chunk:
        k k^T, q k^T, inv v, inv k, k_cumdecay S, q S, intra v_new, k^T v_new."""
        n = -(-self.t // 64)
        per = 2 * (64 * 64 * self.dk * 2 + 64 * 64 * (self.dv + self.dk) + 64 * self.dk * self.dv * 3 + 64 * 64 * self.dv)
        return float(per) * n * self.nv * self.batch

    def inputs(self):
        from .synth import round_bf16, tensor, uniform
        B, T, s = self.batch, self.t, self.seed
        rb = round_bf16 if self.bf16 else (lambda x: x)
        mixed = tensor(s, 1, (B, T, self.conv_dim), self.bf16)
        z = tensor(s, 2, (B, T, self.nv * self.dv), self.bf16)
        u = np.clip(uniform(s, 3, B * T * self.nv), 1e-4, 1 - 1e-4).reshape(B, T, self.nv)
        b = rb(np.log(u / (1.0 - u)).astype(np.float32))
        g = (np.log(1e-3) * uniform(s, 4, B * T * self.nv)).reshape(B, T, self.nv)
        a = rb(np.log(np.expm1(np.maximum(-g, 1e-6))).astype(np.float32))
        conv_w = tensor(s, 5, (self.conv_dim, self.kernel), self.bf16, scale=0.5)
        neg_a = -np.ones(self.nv, np.float32)
        dt_bias = np.zeros(self.nv, np.float32)
        norm_w = (1.0 + 0.1 * tensor(s, 6, (self.dv,), False)).astype(np.float32)
        return dict(mixed=mixed, z=z, b=b, a=a, conv_w=conv_w, neg_a=neg_a, dt_bias=dt_bias, norm_w=norm_w)


def c5_gdn(t: int = 4096, batch: int = 1) -> GdnWorkload:
    return GdnWorkload(f"c5gdn{batch}x{t}", 5, True, batch, t)


def c5_gdn_rows() -> GdnWorkload:
    """Config 5's 32 question rows right-padded to 64 tokens through the GDN
    layer, continuing from the 4096-token prefill's state (their own seed,
    so their tokens are not the prefill's first tokens again)."""
    return GdnWorkload("c5gdn32x64", 55, True, 32, 64)


@dataclass
class Qwen3StackWorkload:
    """Config 2: a Qwen3-1.7B-shaped decoder stack (28 layers, hidden 2048,
    Hq = 16, Hkv = 8, d = 128, intermediate 6144, vocab 151936, tied
    embeddings, eps 1e-6, theta 1e6) with random weights N(0, 0.02) and norm
    weights 1.  A 2048-token state of uniform token ids: its first 1536
    tokens are prefilled in 512-token chunks (qwen3.rs:346-362), the last 512
    (the tail) ride along in one packed pass with 64 question blocks of 48
    tokens (engine.rs:236-287, :365-442); the readout is the final-normed
    hidden state at the 64 gather positions times 8 code rows of the tied
    head (engine.rs:155, :463-469).

    Weights come from numpy's PCG64, one seeded stream per tensor (the
    splitmix64 streams of the attention configs are too slow for 1.7e9
    values); token ids from PCG64 too."""
    name: str
    seed: int
    bf16: bool
    n_layers: int = 28
    hidden: int = 2048
    hq: int = 16
    hkv: int = 8
    d: int = 128
    inter: int = 6144
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1e6
    state_tokens: int = 2048
    prefill_chunk: int = 512
    questions: int = 64
    q_len: int = 48
    n_codes: int = 8
    std: float = 0.02

    @property
    def head_tokens(self) -> int:
        """Tokens prefilled before the pass: all but the last chunk (engine.rs:251-253)."""
        return self.state_tokens - min(self.state_tokens, self.prefill_chunk)

    @property
    def pass_tokens(self) -> int:
        return self.state_tokens - self.head_tokens + self.questions * self.q_len

    def _normal(self, stream: int, shape):
        g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([self.seed, stream])))
        x = g.standard_normal(int(np.prod(shape)), dtype=np.float32).reshape(shape)
        x *= np.float32(self.std)
        return x

    def weights(self, threads: int = 8) -> dict:
        """{name: f32 array} in the layout of torch / candle Linear (out, in);
        bf16 configs hold bf16-representable values."""
        from concurrent.futures import ThreadPoolExecutor

        from .synth import round_bf16
        specs = self.weight_specs()

        def make(spec):
            name, stream, shape = spec
            x = self._normal(stream, shape)
            return name, round_bf16(x) if self.bf16 else x

        with ThreadPoolExecutor(threads) as ex:
            w = dict(ex.map(make, specs))
        w.update({name: np.ones(n, np.float32) for name, n in self.norm_specs()})
        return w

    def weight_specs(self):
        """(name, PCG64 stream, shape) of every random matrix."""
        H, d = self.hidden, self.d
        specs = [("embed", 1, (self.vocab, H))]
        for i in range(self.n_layers):
            base = 100 + 16 * i
            specs += [(f"l{i}.wq", base, (self.hq * d, H)), (f"l{i}.wk", base + 1, (self.hkv * d, H)),
                      (f"l{i}.wv", base + 2, (self.hkv * d, H)), (f"l{i}.wo", base + 3, (H, self.hq * d)),
                      (f"l{i}.gate", base + 4, (self.inter, H)), (f"l{i}.up", base + 5, (self.inter, H)),
                      (f"l{i}.down", base + 6, (H, self.inter))]
        return specs

    def norm_specs(self):
        """(name, length) of every norm weight (all ones)."""
        out = []
        for i in range(self.n_layers):
            out += [(f"l{i}.q_norm", self.d), (f"l{i}.k_norm", self.d), (f"l{i}.ln1", self.hidden), (f"l{i}.ln2", self.hidden)]
        return out + [("norm", self.hidden)]

    def device_weights(self, device, dtype):
        """Random weights of the same shapes drawn on the device (torch's
        generator, not the PCG64 streams): for timing runs, where the values
        only need the right distribution."""
        import torch
        g = torch.Generator(device=device).manual_seed(self.seed)
        w = {}
        for name, _, shape in self.weight_specs():
            w[name] = (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * self.std).to(dtype)
        for name, n in self.norm_specs():
            w[name] = torch.ones(n, device=device, dtype=dtype)
        return w

    def ids(self):
        """(state ids, question ids (questions, q_len), code ids)."""
        g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([self.seed, 2])))
        state = g.integers(0, self.vocab, self.state_tokens, dtype=np.int64)
        qs = g.integers(0, self.vocab, (self.questions, self.q_len), dtype=np.int64)
        codes = g.choice(self.vocab, self.n_codes, replace=False).astype(np.int64)
        return state, qs, codes

    def plans_items(self):
        """One plan (past = head, prefix = state, tail = the rest) and its questions."""
        return [(self.head_tokens, self.state_tokens, self.head_tokens)], [(0, self.q_len)] * self.questions

    def flops(self) -> dict:
        """Useful FLOPs of the prefill and of the pass: linear layers (2 per
        multiply-add) and attention (unmasked pairs x 4d)."""
        H, I, d, L = self.hidden, self.inter, self.d, self.n_layers
        lin = 2 * (H * (self.hq + 2 * self.hkv) * d + self.hq * d * H + 3 * H * I)
        out = {}
        past, pre = 0, 0
        for n in [self.prefill_chunk] * (self.head_tokens // self.prefill_chunk) + (
                [self.head_tokens % self.prefill_chunk] if self.head_tokens % self.prefill_chunk else []):
            pre += lin * n + 4 * d * self.hq * (n * past + n * (n + 1) // 2)
            past += n
        out["prefill"] = float(pre * L)
        tail = self.state_tokens - self.head_tokens
        pairs = tail * self.head_tokens + tail * (tail + 1) // 2
        pairs += self.questions * (self.q_len * self.state_tokens + self.q_len * (self.q_len + 1) // 2)
        out["pass"] = float(L * (lin * self.pass_tokens + 4 * d * self.hq * pairs))
        return out


def c2(bf16: bool = True, **kw) -> Qwen3StackWorkload:
    return Qwen3StackWorkload("c2" if bf16 else "c2-f32", 2, bf16, **kw)
