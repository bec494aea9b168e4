"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked against something outside itself: the
reference's own unit-test vectors (qwen35.rs:758-822), closed forms, textbook
special cases, a second independent implementation (f64 brute force, torch),
or hand-derived known answers from reading the reference.  Every `*_catches`
test plants a plausible mistake in the oracle (cev_oracle.c MUT_*) and shows
that the same check then fails.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from cev_hip import synth

RNG = np.random.default_rng(12345)


# ---------------------------------------------------------------- bf16 rounding


def test_bf16_rounding_known_answers(orc):
    x = np.array([1.0, 1 + 2**-8, 1 + 3 * 2**-8, -2.5, 3.0e38, 1e-40, 0.0], np.float32)
    want = np.array([1.0, 1.0, 1 + 2**-6, -2.5], np.float32)
    got = orc.round_bf16(x)
    assert np.array_equal(got[:4], want)  # ties to even
    assert math.isinf(float(orc.round_bf16(np.array([3.4e38], np.float32))[0]))


def test_bf16_rounding_matches_torch(orc):
    x = (RNG.standard_normal(100000) * 10.0 ** RNG.integers(-6, 6, 100000)).astype(np.float32)
    t = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(orc.round_bf16(x), t)
    assert np.array_equal(synth.round_bf16(x), t)


# ---------------------------------------------------------------- RoPE table


def _table_closed_form(theta, rot, n_pos):
    half = rot // 2
    inv = np.array([np.float32(1.0) / np.float32(theta ** (2 * i / rot)) for i in range(half)], np.float32)
    ang = (np.arange(n_pos, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))


def _check_table(orc, theta=1e6, rot=128, n_pos=4096):
    c, s = orc.rope_table(theta, rot, n_pos, False)
    cw, sw = _table_closed_form(theta, rot, n_pos)
    ulp = np.spacing(np.float32(1.0))
    return (np.abs(c - cw).max() <= ulp and np.abs(s - sw).max() <= ulp and np.all(c[0] == 1.0) and np.all(s[0] == 0.0))


def test_rope_table_closed_form(orc):
    assert _check_table(orc)
    assert _check_table(orc, theta=1e7, rot=64, n_pos=8200)


def test_rope_table_catches_shifted_position(orc):
    with oracle.mutation(oracle.MUT_TABLE_POS):
        assert not _check_table(orc)


def test_rope_table_bf16_is_rounded_f32(orc):
    c, s = orc.rope_table(1e6, 128, 600, False)
    cb, sb = orc.rope_table(1e6, 128, 600, True)
    assert np.array_equal(cb, orc.round_bf16(c)) and np.array_equal(sb, orc.round_bf16(s))


# ---------------------------------------------------------------- RMSNorm


def _check_norm(orc):
    # closed form: d=2, x=(3,4), w=1 -> x / sqrt(12.5 + eps)
    y = orc.rms_norm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32), 1e-6, False)
    want = np.array([3.0, 4.0]) / math.sqrt(12.5 + 1e-6)
    ok = np.abs(y[0] - want).max() < 1e-6
    # unit RMS with w = 1
    x = RNG.standard_normal((64, 128)).astype(np.float32)
    y = orc.rms_norm(x, np.ones(128, np.float32), 1e-6, False)
    ok &= np.abs((y.astype(np.float64) ** 2).mean(-1) - 1.0).max() < 5e-6
    return bool(ok)


def test_rms_norm_closed_forms(orc):
    assert _check_norm(orc)


def test_rms_norm_catches_wrong_mean(orc):
    with oracle.mutation(oracle.MUT_NORM_DIM_M1):
        assert not _check_norm(orc)


def test_rms_norm_scale_invariance_and_weights(orc):
    x = RNG.standard_normal((32, 256)).astype(np.float32)
    w = (1 + 0.1 * RNG.standard_normal(256)).astype(np.float32)
    a = orc.rms_norm(x, w, 0.0, False)
    b = orc.rms_norm(x * np.float32(8.0), w, 0.0, False)  # eps 0 and a power of two: exact
    assert np.array_equal(a, b)
    # zero-centred weights (qwen35.rs:169): (1 + w) rounded to the dtype
    for bf in (False, True):
        xb = orc.round_bf16(x) if bf else x
        wz = orc.round_bf16(0.1 * w) if bf else (0.1 * w).astype(np.float32)
        one_plus = orc.round_bf16(wz + 1) if bf else (wz + 1).astype(np.float32)
        assert np.array_equal(orc.rms_norm(xb, wz, 1e-6, bf, plus_one=True), orc.rms_norm(xb, one_plus, 1e-6, bf))


# ---------------------------------------------------------------- RoPE


def _check_rope_basis(orc, rot=128, d=128):
    c, s = orc.rope_table(1e6, rot, 300, False)
    half = rot // 2
    ok = True
    for i in (0, 5, half - 1):
        for p in (0, 7, 299):
            x = np.zeros((1, 2, d), np.float32)
            x[0, 0, i] = 1.0          # e_i      -> (c, s) at (i, i + half)
            x[0, 1, i + half] = 1.0   # e_{i+h}  -> (-s, c)
            y = orc.rope(x, np.array([p], np.int32), c, s, rot, False)
            ok &= y[0, 0, i] == c[p, i] and y[0, 0, i + half] == s[p, i]
            ok &= y[0, 1, i] == -s[p, i] and y[0, 1, i + half] == c[p, i]
            ok &= np.count_nonzero(y[0, :, rot:]) == 0
    return bool(ok)


def test_rope_basis_vectors(orc):
    assert _check_rope_basis(orc)
    assert _check_rope_basis(orc, rot=64, d=256)


def test_rope_catches_sign(orc):
    with oracle.mutation(oracle.MUT_ROPE_SIN_SIGN):
        assert not _check_rope_basis(orc)


def test_rope_preserves_norm_and_relative_position(orc):
    c, s = orc.rope_table(1e6, 128, 512, False)
    x = RNG.standard_normal((6, 4, 128)).astype(np.float32)
    pos = np.array([0, 3, 100, 200, 300, 511], np.int32)
    y = orc.rope(x, pos, c, s, 128, False)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=2e-6)
    q = RNG.standard_normal((1, 1, 128)).astype(np.float32)
    k = RNG.standard_normal((1, 1, 128)).astype(np.float32)
    dots = []
    for shift in (0, 17, 150):  # <R(p)q, R(p')k> depends only on p - p'
        rq = orc.rope(q, np.array([40 + shift], np.int32), c, s, 128, False)
        rk = orc.rope(k, np.array([10 + shift], np.int32), c, s, 128, False)
        dots.append(float((rq.astype(np.float64) * rk).sum()))
    assert max(dots) - min(dots) < 1e-4 * (1 + abs(dots[0]))


# ---------------------------------------------------------------- attention


def _two_key_case():
    d = 8
    q = np.zeros((1, 1, d), np.float32)
    q[0, 0, :2] = [1.7, -0.4]
    k = np.zeros((1, 2, d), np.float32)
    k[0, 0, 0] = 1.0
    k[0, 1, 1] = 1.0
    v = np.zeros((1, 2, d), np.float32)
    v[0, 0, 0] = 1.0
    v[0, 1, 1] = 1.0
    mask = np.zeros((1, 2), np.float32)
    p1 = 1.0 / (1.0 + math.exp((-0.4 - 1.7) / math.sqrt(d)))
    return q, k, v, mask, p1


def _check_two_key(orc):
    q, k, v, mask, p1 = _two_key_case()
    o = orc.attend(q, k, v, mask, False)[0, 0, 0]
    return abs(o[0] - p1) < 1e-6 and abs(o[1] - (1 - p1)) < 1e-6 and np.count_nonzero(o[2:]) == 0


def test_attend_two_key_closed_form(orc):
    assert _check_two_key(orc)


@pytest.mark.parametrize("mut", [oracle.MUT_ATTN_NO_SCALE, oracle.MUT_ATTN_V_SHIFT])
def test_attend_two_key_catches(orc, mut):
    with oracle.mutation(mut):
        assert not _check_two_key(orc)


def _mask_case(orc):
    plans = [(40, 40, 40), (24, 30, 24)]
    items = [(0, 5), (1, 1), (0, 7), (1, 3)]
    return orc.engine_pass(plans, items)


def _check_identical_keys(orc):
    ep = _mask_case(orc)
    n, s = ep["n"], ep["past_total"] + ep["n"]
    mask = ep["mask"]
    q = RNG.standard_normal((2, n, 16)).astype(np.float32)
    k = np.broadcast_to(RNG.standard_normal(16).astype(np.float32), (1, s, 16)).copy()
    v = RNG.standard_normal((1, s, 16)).astype(np.float32)
    o = orc.attend(q, k, v, mask, False)[0]
    vis = (mask == 0).astype(np.float64)
    want = (vis @ v[0].astype(np.float64)) / vis.sum(1, keepdims=True)
    return bool(np.abs(o - want[None]).max() < 2e-6)


def test_attend_identical_keys_give_mean_of_visible_values(orc):
    assert _check_identical_keys(orc)


def test_attend_identical_keys_catches_value_shift(orc):
    with oracle.mutation(oracle.MUT_ATTN_V_SHIFT):
        assert not _check_identical_keys(orc)


def test_attend_zero_query_uniform_and_constant_values(orc):
    ep = _mask_case(orc)
    n, s = ep["n"], ep["past_total"] + ep["n"]
    mask = ep["mask"]
    k = RNG.standard_normal((1, s, 32)).astype(np.float32)
    v = RNG.standard_normal((1, s, 32)).astype(np.float32)
    o = orc.attend(np.zeros((1, n, 32), np.float32), k, v, mask, False)[0, 0]
    vis = (mask == 0).astype(np.float64)
    assert np.abs(o - (vis @ v[0]) / vis.sum(1, keepdims=True)).max() < 2e-6
    q = RNG.standard_normal((1, n, 32)).astype(np.float32)
    vc = np.broadcast_to(np.linspace(-2, 2, 32, dtype=np.float32), (1, s, 32)).copy()
    o = orc.attend(q, k, vc, mask, False)[0, 0]
    assert np.abs(o - vc[0, 0]).max() < 2e-6


def _check_gqa(orc):
    t, s, d = 6, 11, 16
    q = RNG.standard_normal((8, t, d)).astype(np.float32)
    k = RNG.standard_normal((2, s, d)).astype(np.float32)
    v = RNG.standard_normal((2, s, d)).astype(np.float32)
    mask = orc.branch_mask(t, s - t)
    a = orc.attend(q, k, v, mask, False)
    b = orc.attend(q, np.repeat(k, 4, axis=0), np.repeat(v, 4, axis=0), mask, False)
    return bool(np.array_equal(a, b))


def test_attend_gqa_equals_mha_with_repeated_heads(orc):
    assert _check_gqa(orc)


def test_attend_gqa_catches_head_map(orc):
    with oracle.mutation(oracle.MUT_ATTN_KV_MODULO):
        assert not _check_gqa(orc)


def test_attend_f32_matches_f64_textbook(orc):
    ep = _mask_case(orc)
    n, s = ep["n"], ep["past_total"] + ep["n"]
    q = RNG.standard_normal((4, n, 128)).astype(np.float32)
    k = RNG.standard_normal((2, s, 128)).astype(np.float32)
    v = RNG.standard_normal((2, s, 128)).astype(np.float32)
    a = orc.attend(q, k, v, ep["mask"], False)
    b = orc.attend_f64(q, k, v, ep["mask"])
    assert np.abs(a - b).max() < 2e-6
    ab = orc.attend(orc.round_bf16(q), orc.round_bf16(k), orc.round_bf16(v), ep["mask"], True)
    bb = orc.attend_f64(orc.round_bf16(q), orc.round_bf16(k), orc.round_bf16(v), ep["mask"])
    assert np.abs(ab - bb).max() < 2e-2


@pytest.mark.parametrize("bf16,hq,hkv,t,s,d,batch", [(True, 8, 2, 40, 300, 128, 1), (False, 4, 4, 33, 101, 128, 1),
                                                       (True, 4, 1, 17, 1003, 256, 1), (True, 8, 2, 9, 70, 128, 3)])
def test_attend_blocked_matches_attend(orc, bf16, hq, hkv, t, s, d, batch):
    """The CPU baseline's blocked restatement computes the same candle op
    sequence: equal to attend up to f32 summation order (f32 models) and one
    bf16 ulp of a probability or output (bf16 models), over causal masks,
    GQA, both head dims and a batch of rows sharing one K/V (stride 0)."""
    rng = np.random.default_rng(11)
    rnd = (lambda x: orc.round_bf16(x)) if bf16 else (lambda x: x)
    q = rnd(rng.standard_normal((batch, hq, t, d)).astype(np.float32))
    k = orc.round_bf16(rng.standard_normal((1, hkv, s, d)).astype(np.float32))
    v = orc.round_bf16(rng.standard_normal((1, hkv, s, d)).astype(np.float32))
    m = orc.branch_mask(t, s - t)
    want = orc.attend(q, k, v, m, bf16)
    got = orc.attend_blocked(q, k, v, m, bf16)
    assert np.isfinite(got).all()
    # bf16: a probability or an output one bf16 ulp apart moves an output by
    # at most about 2^-8 of the largest one
    tol = 2.0 ** -8 * float(np.abs(want).max()) if bf16 else 1e-5
    assert float(np.abs(got - want).max()) <= tol
    got_rows = orc.attend_blocked(q, k, v, m, bf16, rows=(3, 5))
    assert np.array_equal(got_rows[:, :, 3:8], got[:, :, 3:8]) and np.isnan(got_rows[:, :, :3]).all()


def test_attend_bidirectional_key_permutation(orc):
    t, d = 9, 32
    lengths = [9, 6]
    mask = orc.bidirectional_mask(t, lengths)
    q = RNG.standard_normal((2, 2, t, d)).astype(np.float32)
    k = RNG.standard_normal((2, 1, t, d)).astype(np.float32)
    v = RNG.standard_normal((2, 1, t, d)).astype(np.float32)
    a = orc.attend(q, k, v, mask, False)
    perm = np.array([3, 1, 4, 0, 5, 2, 6, 7, 8])  # permutes real keys of both rows
    b = orc.attend(q, k[:, :, perm], v[:, :, perm], mask[:, :, perm], False)
    assert np.abs(a - b).max() < 2e-6


# ---------------------------------------------------------------- masks


def test_engine_mask_known_answer(orc):
    # past 2, prefix 3 with a 1-token tail, one 2-token question (engine.rs:389-442)
    ep = orc.engine_pass([(2, 3, 2)], [(0, 2)])
    z, n_ = 0.0, -np.inf
    want = np.array([[z, z, z, n_, n_], [z, z, z, z, n_], [z, z, z, z, z]], np.float32)
    assert np.array_equal(ep["mask"], want)
    assert ep["pos"].tolist() == [2, 3, 4] and ep["gather"].tolist() == [2]


def test_segment_mask_is_branch_mask_for_one_segment(orc):
    for past, n in ((0, 7), (5, 4)):
        assert np.array_equal(orc.segment_mask(np.zeros(n, np.uint32), past), orc.branch_mask(n, past))


def _check_packed_equivalence(orc):
    """Packed block b == causal attention over [prefix || block b] alone (qwen3.rs:13-17)."""
    P, lens, d = 19, [5, 1, 7], 32
    ep = orc.engine_pass([(P, P, P)], [(0, L) for L in lens])
    n = ep["n"]
    q = RNG.standard_normal((2, n, d)).astype(np.float32)
    k = RNG.standard_normal((1, P + n, d)).astype(np.float32)
    v = RNG.standard_normal((1, P + n, d)).astype(np.float32)
    packed = orc.attend(q, k, v, ep["mask"], False)[0]
    ok, r0 = True, 0
    for L in lens:
        kb = np.concatenate([k[:, :P], k[:, P + r0: P + r0 + L]], axis=1)
        vb = np.concatenate([v[:, :P], v[:, P + r0: P + r0 + L]], axis=1)
        alone = orc.attend(q[:, r0: r0 + L], kb, vb, orc.branch_mask(L, P), False)[0]
        ok &= np.array_equal(packed[:, r0: r0 + L], alone)
        r0 += L
    return bool(ok)


def test_packed_equals_each_block_alone(orc):
    assert _check_packed_equivalence(orc)


def test_packed_equivalence_catches_mask(orc):
    with oracle.mutation(oracle.MUT_MASK_NO_DIAG):
        assert not _check_packed_equivalence(orc)


def test_sigmoid_gate_matches_closed_form(orc):
    o = RNG.standard_normal(1000).astype(np.float32)
    g = RNG.standard_normal(1000).astype(np.float32)
    got = orc.sigmoid_gate(o, g, False)
    assert np.abs(got - o / (1 + np.exp(-g.astype(np.float64)))).max() < 1e-6
    gb = orc.sigmoid_gate(orc.round_bf16(o), orc.round_bf16(g), True)
    assert np.abs(gb - o / (1 + np.exp(-g.astype(np.float64)))).max() < 2e-2


# ---------------------------------------------------------------- Gated DeltaNet


def _ref_gen(n, seed):
    """The deterministic generator of the reference's test (qwen35.rs:781)."""
    i = np.arange(n, dtype=np.uint64)
    return (((i + 1) * np.uint64(seed + 7919)) % np.uint64(1000)).astype(np.float32) / np.float32(500.0) - np.float32(1.0)


def _gdn_case(orc):
    b, h, t, dk, dv = 1, 2, 70, 4, 3
    q = _ref_gen(b * h * t * dk, 1).reshape(h, t, dk)
    k = _ref_gen(b * h * t * dk, 2).reshape(h, t, dk)
    v = _ref_gen(b * h * t * dv, 3).reshape(h, t, dv)
    g = (np.abs(_ref_gen(b * h * t, 4)) * np.float32(-0.5)).reshape(h, t)
    beta = (1.0 / (1.0 + np.exp(-_ref_gen(b * h * t, 5).astype(np.float64)))).astype(np.float32).reshape(h, t)
    return q, k, v, g, beta


def _check_gdn(orc):
    q, k, v, g, beta = _gdn_case(orc)
    out, s = orc.chunk_gated_delta_rule(q, k, v, g, beta)
    dk = q.shape[-1]
    qn = (orc.l2norm(q) * np.float32(dk ** -0.5)).astype(np.float32)
    kn = orc.l2norm(k)
    ro, rs = orc.gdn_recurrence(qn, kn, v, g, beta)
    return bool(np.abs(out - ro).max() < 2e-4 and np.abs(s - rs).max() < 2e-4)


def test_gdn_chunked_rule_matches_recurrence(orc):
    """qwen35.rs:776-822 with the reference's generator and tolerance."""
    assert _check_gdn(orc)


def test_gdn_catches_missing_decay(orc):
    with oracle.mutation(oracle.MUT_GDN_NO_DECAY):
        assert not _check_gdn(orc)


def test_gdn_with_initial_state_continues_the_sequence(orc):
    q, k, v, g, beta = _gdn_case(orc)
    full, s_full = orc.chunk_gated_delta_rule(q, k, v, g, beta)
    a, s_a = orc.chunk_gated_delta_rule(q[:, :40], k[:, :40], v[:, :40], g[:, :40], beta[:, :40])
    b, s_b = orc.chunk_gated_delta_rule(q[:, 40:], k[:, 40:], v[:, 40:], g[:, 40:], beta[:, 40:], s0=s_a)
    assert np.abs(np.concatenate([a, b], 1) - full).max() < 2e-4
    assert np.abs(s_b - s_full).max() < 2e-4


def test_inv_unit_lower_matches_definition(orc):
    """qwen35.rs:758-774: (I + strict_lower(m)) . inv == I."""
    n = 8
    vals = ((np.arange(n * n) * 37 % 11).astype(np.float32) - 5.0) / 7.0
    m = vals.reshape(1, n, n).astype(np.float32)
    inv = orc.inv_unit_lower(m)[0]
    a = np.tril(m[0], -1) + np.eye(n, dtype=np.float32)
    assert np.abs(a @ inv - np.eye(n)).max() < 1e-4
    assert np.abs(inv - np.linalg.inv(a.astype(np.float64))).max() < 1e-4
    big = RNG.standard_normal((3, 64, 64)).astype(np.float32) * 0.1
    inv = orc.inv_unit_lower(big)
    for i in range(3):
        a = np.tril(big[i], -1) + np.eye(64)
        assert np.abs(a @ inv[i] - np.eye(64)).max() < 1e-4


def test_softplus_closed_form(orc):
    for x in (-30.0, -2.0, 0.0, 0.5, 3.0, 40.0):
        want = math.log1p(math.exp(x)) if x < 30 else x
        assert abs(orc.softplus(x) - want) <= 1e-5 * max(1.0, abs(want))


def test_l2norm_unit_rows_and_direction(orc):
    x = RNG.standard_normal((50, 128)).astype(np.float32) * 3.0
    y = orc.l2norm(x)
    assert np.abs(np.linalg.norm(y.astype(np.float64), axis=1) - 1.0).max() < 1e-5
    assert np.abs(y * np.linalg.norm(x.astype(np.float64), axis=1, keepdims=True) - x).max() < 1e-4
    # the 1e-6 inside the root (qwen35.rs:252): a zero row stays zero, a tiny row is damped
    z = orc.l2norm(np.zeros((1, 8), np.float32))
    assert np.all(z == 0.0)


def _conv_direct(x, tail, w):
    """Depthwise causal conv + SiLU in f64 by the definition: y[c, i] =
    silu(sum_u full[c, i + u] w[c, u]) over full = [tail || x]."""
    c, t = x.shape
    kw = w.shape[1]
    full = np.concatenate([np.zeros((c, kw - 1)) if tail is None else tail, x], 1).astype(np.float64)
    y = np.zeros((c, t))
    for i in range(t):
        y[:, i] = (full[:, i:i + kw] * w).sum(1)
    return y / (1.0 + np.exp(-y)), full[:, t:t + kw - 1]


def test_conv_silu_f32_matches_direct_convolution(orc):
    c, t, kw = 6, 11, 4
    x = RNG.standard_normal((c, t)).astype(np.float32)
    tail = RNG.standard_normal((c, kw - 1)).astype(np.float32)
    # taps differ in size and sign, so a reversed or shifted kernel fails
    w = (np.array([0.1, -0.7, 0.4, 1.3], np.float32)[None, :] * (1.0 + np.arange(c, dtype=np.float32)[:, None] / 4)).astype(np.float32)
    for tl in (None, tail):
        y, nt = orc.conv_silu(x, tl, w, False)
        ry, rnt = _conv_direct(x, tl, w)
        assert np.abs(y - ry).max() < 1e-5
        assert np.array_equal(nt, rnt.astype(np.float32))
    # a short call: the new tail still reaches back into the old one
    y, nt = orc.conv_silu(x[:, :2], tail, w, False)
    ry, rnt = _conv_direct(x[:, :2], tail, w)
    assert np.abs(y - ry).max() < 1e-5 and np.array_equal(nt, rnt.astype(np.float32))


def test_conv_silu_bf16_within_rounding_of_exact(orc):
    c, t, kw = 16, 40, 4
    x = orc.round_bf16(RNG.standard_normal((c, t)).astype(np.float32))
    w = orc.round_bf16((RNG.standard_normal((c, kw)) * 0.5).astype(np.float32))
    y, _ = orc.conv_silu(x, None, w, True)
    ry, _ = _conv_direct(x, None, w)
    assert np.array_equal(y, orc.round_bf16(y))  # every output is a bf16 value
    assert np.abs(y - ry).max() <= 2e-2 * max(1.0, np.abs(ry).max())


def test_gated_rmsnorm_closed_form(orc):
    rows, dv = 40, 128
    core = RNG.standard_normal((rows, dv)).astype(np.float32)
    z = RNG.standard_normal((rows, dv)).astype(np.float32)
    w = (1.0 + 0.1 * RNG.standard_normal(dv)).astype(np.float32)
    y = orc.gated_rmsnorm(core, z, w, 1e-6, False)
    c64 = core.astype(np.float64)
    ref = c64 / np.sqrt((c64 ** 2).mean(1, keepdims=True) + 1e-6) * w * (z / (1.0 + np.exp(-z.astype(np.float64))))
    assert np.abs(y - ref).max() < 1e-5
    yb = orc.gated_rmsnorm(core, z, w, 1e-6, True)
    assert np.array_equal(yb, orc.round_bf16(yb)) and np.abs(yb - ref).max() < 2e-2 * np.abs(ref).max()


def test_gdn_layer_value_heads_follow_key_heads_in_blocks(orc):
    """Value head h reads key head h // (nv / nk) (the unsqueeze(2).expand of
    qwen35.rs:438).  Swapping the two key heads' q/k channels must swap
    value heads {0, 1} with {2, 3} and nothing else."""
    from cev_hip import configs
    nk, nv, dk, dv = 2, 4, 8, 8
    w = configs.GdnWorkload("rep", 3, False, 1, 20, nk=nk, nv=nv, dk=dk, dv=dv)
    inp = w.inputs()
    args = lambda m, z, b, a: orc.gdn_layer(m, z, b, a, inp["conv_w_p"], inp["neg_a"], inp["dt_bias"], inp["norm_w"], nk, nv,
                                            dk, dv, w.eps, False)[0]
    kd = nk * dk
    perm_c = np.concatenate([np.arange(dk, 2 * dk), np.arange(dk), kd + np.arange(dk, 2 * dk), kd + np.arange(dk),
                             2 * kd + np.arange(2 * dv, 4 * dv), 2 * kd + np.arange(2 * dv)])
    perm_h = np.array([2, 3, 0, 1])
    # conv weights must follow the channels for the swap to be a symmetry
    inp["conv_w_p"] = inp["conv_w"]
    y = args(inp["mixed"], inp["z"], inp["b"], inp["a"])
    inp["conv_w_p"] = inp["conv_w"][perm_c]
    zz = inp["z"].reshape(1, w.t, nv, dv)[:, :, perm_h].reshape(1, w.t, nv * dv)
    yp = args(inp["mixed"][:, :, perm_c], zz, inp["b"][:, :, perm_h], inp["a"][:, :, perm_h])
    want = y.reshape(1, w.t, nv, dv)[:, :, perm_h].reshape(1, w.t, nv * dv)
    assert np.abs(yp - want).max() < 1e-5
    # the tiled order (h % nk) would pair value head 1 with key head 1: not a symmetry of the layer
    assert np.abs(y.reshape(1, w.t, nv, dv)[:, :, 0] - y.reshape(1, w.t, nv, dv)[:, :, 2]).max() > 1e-3


# ---------------------------------------------------------------- debiased readout


def test_log_softmax64_closed_forms():
    """math::log_softmax: constant logits give -ln k; it equals an
    independent f64 log-softmax; shifting all logits by a constant (exactly
    representable sums) changes nothing."""
    from oracle.qwen3_stack import log_softmax64
    for k in (1, 2, 5, 64):
        assert np.allclose(log_softmax64(np.full(k, 3.25, np.float32)), -math.log(k), rtol=0, atol=1e-15)
    z = RNG.standard_normal(37).astype(np.float32) * 4
    zz = z.astype(np.float64)
    ind = zz - zz.max() - np.log(np.exp(zz - zz.max()).sum())
    assert np.allclose(log_softmax64(z), ind, rtol=0, atol=1e-13)
    z = (np.round(RNG.standard_normal(37) * 4096) / 1024).astype(np.float32)  # z + 8 is exact in f32
    assert np.allclose(log_softmax64(z), log_softmax64(z + np.float32(8.0)), rtol=0, atol=1e-12)


def test_rotation_shifts_and_orders():
    """Debias::shifts / CompiledQuestion::rotated by hand: 5 options, at most
    4 rotations -> shifts 0, 1, 2, 3; 2 options -> 0, 1; 1 option -> 0."""
    from oracle.qwen3_stack import rotated_order, rotation_shifts
    assert rotation_shifts(5, 4) == [0, 1, 2, 3]
    assert rotation_shifts(8, 4) == [0, 2, 4, 6]
    assert rotation_shifts(2, 4) == [0, 1]
    assert rotation_shifts(1, 4) == [0]
    assert rotated_order([0, 1, 2, 3, 4], 2) == [2, 3, 4, 0, 1]


def _invariant_case(rng, ks, max_perm=4):
    """Variants of a position-invariant model (the reference's own check,
    crates/cev-runtime/tests/runtime.rs:185-207): option o has the same logit
    at every position it is shown in."""
    from oracle.qwen3_stack import rotated_order, rotation_shifts
    ld = max(ks)
    rows, orders, begin, length, canon = [], [], [], [], []
    for k in ks:
        f = rng.standard_normal(k).astype(np.float32) * 2
        canon.append(f)
        begin.append(len(rows))
        shifts = rotation_shifts(k, max_perm)
        length.append(len(shifts))
        for s in shifts:
            order = rotated_order(list(range(k)), s)
            row = np.zeros(ld, np.float32)
            row[:k] = f[order]
            rows.append(row)
            orders.append(order + [0] * (ld - k))
    return np.array(rows), np.array(orders, np.int32), np.array(begin), np.array(length), np.array(ks), canon


def test_debias_rotations_map_back_to_canonical_options():
    """Averaging the rotations of a position-invariant model reproduces the
    undebiased log-probabilities per option (runtime.rs:185-207); an index
    mix-up (scoring by position instead of option) breaks it."""
    from oracle.qwen3_stack import debias_scores, log_softmax64
    rng = np.random.default_rng(5)
    logits, order, begin, length, ks, canon = _invariant_case(rng, [5, 2, 8, 3])
    got = debias_scores(logits, order, begin, length, ks)
    for q, k in enumerate(ks):
        assert np.allclose(got[q, :k], log_softmax64(canon[q]), rtol=0, atol=1e-6)
    wrong = debias_scores(logits, np.tile(np.arange(logits.shape[1], dtype=np.int32), (len(logits), 1)), begin, length, ks)
    assert not np.allclose(wrong[0, :5], got[0, :5], rtol=0, atol=1e-3)


def test_debias_calibration_against_itself_is_zero():
    from oracle.qwen3_stack import debias_scores
    rng = np.random.default_rng(6)
    logits, order, begin, length, ks, _ = _invariant_case(rng, [4, 6])
    logits = logits + rng.standard_normal(logits.shape).astype(np.float32)  # not invariant any more
    got = debias_scores(logits, order, begin, length, ks, calib=logits)
    assert np.array_equal(got, np.zeros_like(got))


# ---------------------------------------------------------------------------
# d3 readout (oracle/readout.py)


def test_readout_linear_matches_definition_and_orientation():
    """linear(x, w) is x . w^T: an elementwise f64 sum by the definition, and
    a transposed (square) weight gives a different answer."""
    from oracle.readout import linear
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 6)).astype(np.float32)
    w = rng.standard_normal((6, 6)).astype(np.float32)
    want = np.array([[sum(float(x[i, e]) * float(w[j, e]) for e in range(6)) for j in range(6)] for i in range(3)], np.float32)
    assert np.array_equal(linear(x, w, False), want)
    assert not np.allclose(linear(x, w.T, False), want)
    # bf16: the f32 result rounded once
    assert np.array_equal(linear(x, w, True), oracle.round_bf16(want))


def test_d3_readout_composition_and_temperature():
    """d3_readout = (o_rows . wo^T in the model dtype) . wr^T times the f32
    1 / temperature: a one-hot o row picks one column of wo, and halving the
    temperature doubles every logit exactly."""
    from oracle.readout import d3_readout, inv_temperature
    rng = np.random.default_rng(2)
    wo = rng.standard_normal((5, 8)).astype(np.float32)
    wr = rng.standard_normal((7, 5)).astype(np.float32)
    o = np.zeros((1, 8), np.float32)
    o[0, 3] = 1.0
    z = d3_readout(o, wo, wr, 1.0, False)
    assert np.allclose(z[0], (wr.astype(np.float64) @ wo[:, 3].astype(np.float64)), rtol=1e-6, atol=1e-6)
    assert np.array_equal(d3_readout(o, wo, wr, 0.5, False), 2 * z)
    assert inv_temperature(0.8) == np.float32(1.0 / np.float64(np.float32(0.8)))


# ---------------------------------------------------------------------------
# Packed-pass engine (oracle/engine.py)


def _tiny_stack(bf16=False):
    from cev_hip import configs
    return configs.Qwen3StackWorkload("tiny", 9, bf16, n_layers=2, hidden=256, hq=4, hkv=2, d=128, inter=512, vocab=512)


def test_oracle_engine_packing_is_asking_each_request_alone(orc):
    """README.md:47 / qwen3.rs:13-17: packing several plans and their
    questions into passes is exactly asking each one alone.  A request and
    its calibration twin in one call (two plans, two tails, 3 passes under a
    small token budget) give the same logits as each request in a call of
    its own.  The comparison is sensitive: a planted error in the pass mask
    (a question token missing its own key) moves the logits beyond it."""
    from oracle.engine import OracleEngine
    from oracle.qwen3_stack import Qwen3Oracle
    w = _tiny_stack()
    W = w.weights()
    rng = np.random.default_rng(0)
    a = (rng.integers(0, w.vocab, 700), [rng.integers(0, w.vocab, int(rng.integers(3, 20))) for _ in range(5)])
    b = (rng.integers(0, w.vocab, 90), [rng.integers(0, w.vocab, int(rng.integers(3, 20))) for _ in range(5)])
    codes = [3, 17, 99, 200]
    both = OracleEngine(Qwen3Oracle(w, W), 10_000, codes, pass_tokens=300).run_many([a, b])
    alone_a = OracleEngine(Qwen3Oracle(w, W), 10_000, codes).run_many([a])[0]
    alone_b = OracleEngine(Qwen3Oracle(w, W), 10_000, codes).run_many([b])[0]
    assert np.allclose(both[0]["logits"], alone_a["logits"], rtol=0, atol=2e-5)
    assert np.allclose(both[1]["logits"], alone_b["logits"], rtol=0, atol=2e-5)
    with oracle.mutation(oracle.MUT_MASK_NO_DIAG):
        bad = OracleEngine(Qwen3Oracle(w, W), 10_000, codes, pass_tokens=300).run_many([a, b])
    assert not np.allclose(bad[0]["logits"], alone_a["logits"], rtol=0, atol=2e-5)


def test_oracle_engine_cache_hit_reproduces_the_miss(orc):
    """A second call on a cached prefix (no prefill, no tail) gives the
    first call's logits for the same questions (parity_models.rs:60-67
    holds the reference to 1e-4 here)."""
    from oracle.engine import OracleEngine
    from oracle.qwen3_stack import Qwen3Oracle
    w = _tiny_stack()
    eng = OracleEngine(Qwen3Oracle(w, w.weights()), 10_000, [1, 2, 3])
    rng = np.random.default_rng(1)
    req = (rng.integers(0, w.vocab, 600), [rng.integers(0, w.vocab, 12) for _ in range(3)])
    first = eng.run_many([req])[0]
    second = eng.run_many([req])[0]
    assert not first["prefix_cached"] and second["prefix_cached"]
    assert np.allclose(first["logits"], second["logits"], rtol=0, atol=1e-5)


# ---------------------------------------------------------------------------
# Config 2 against HF transformers (tests/golden/make_c2_hf.py)

HF_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c2_hf_f32.npz")


@pytest.mark.skipif(not os.path.exists(HF_GOLDEN), reason="tests/golden/c2_hf_f32.npz not generated")
def test_c2_oracle_matches_hf_transformers(orc):
    """The Qwen3 stack oracle's composition (layer order, residual
    placement, QK-norm + RoPE, the engine's chunked head prefill and packed
    pass, final norm at the gather rows, tied code head) against
    Qwen3ForCausalLM asked each question alone over [state || question], on
    the Qwen3-1.7B-shaped stack's seeded weights at 2 layers: the reference's own pin of its
    f32 path (README.md:48, |dp| < 5e-5)."""
    from cev_hip import configs
    from oracle.engine import OracleEngine
    from oracle.qwen3_stack import Qwen3Oracle, softmax64
    g = np.load(HF_GOLDEN)
    w = configs.c2(False, n_layers=int(g["layers"]), vocab=int(g["vocab"]), questions=int(g["questions"]))
    state, qs, codes = w.ids()
    eng = OracleEngine(Qwen3Oracle(w, w.weights()), w.state_tokens, codes, pass_tokens=w.pass_tokens, prefill_chunk=w.prefill_chunk)
    r = eng.run_many([(state, list(qs))])[0]
    dp = float(np.abs(softmax64(r["logits"]) - g["p"]).max())
    dh = float(np.abs(r["hidden"] - g["hidden"]).max())
    print(f"oracle vs HF: |dp| {dp:.3g}, max|dhidden| {dh:.3g} (|hidden| <= {float(np.abs(g['hidden']).max()):.3g})")
    assert eng.passes == 1
    assert dp < 5e-5
    assert dh < 1e-3
