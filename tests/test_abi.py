"""CPU tests of libcev_hip.so: it loads, exports every symbol the header
declares, validates inputs before any launch, and its host table builders
reproduce the reference's dense masks exactly (the masks come from the
oracle's restatement of engine.rs:418-442, qwen3.rs:157-169,
qwen35.rs:471-498)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import cev_hip
from cev_hip import _abi
from cev_hip._abi import CEV_BF16, CEV_ERR_INVALID, CEV_ERR_SPACE, CEV_ERR_UNSUPPORTED, CEV_F32, CevError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RNG = np.random.default_rng(7)


def _header_symbols():
    src = open(os.path.join(ROOT, "include", "cev_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(cev_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_header_symbol(cev):
    syms = _header_symbols()
    assert len(syms) >= 20
    L = _abi.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert set(syms) == set(_abi.SIGNATURES), "ctypes signatures and header disagree"
    assert L.cev_abi_version() == 1


def test_desc_init_layouts(cev):
    d = cev_hip.attn_desc(CEV_BF16, 32, 8, 128, 4096, 32768)
    assert d.q_stride_t == 32 * 128 and d.q_stride_h == 128
    assert d.kc_stride_h == 32768 * 128 and d.kc_stride_s == 128
    assert d.kn_stride_t == 8 * 128 and d.kn_stride_h == 128
    assert np.float32(d.scale) == np.float32(1 / np.sqrt(128))  # f32, as qwen3.rs:207 + affine


def _plan_rc(desc, blocks):
    arr = (_abi.Block * max(1, len(blocks)))(*blocks)
    size = C.c_size_t()
    return _abi.lib().cev_attn_plan_size(C.byref(desc), arr, len(blocks), C.byref(size))


B = cev_hip.BlockTable.block


@pytest.mark.parametrize("blocks,code", [
    ([B(0, 0, 10)], CEV_ERR_INVALID),                                  # q_len 0
    ([B(0, 4, 10), B(2, 4, 14)], CEV_ERR_INVALID),                      # overlapping rows
    ([B(0, 4, 10, spans=[(0, 11)])], CEV_ERR_INVALID),                  # span overlaps own keys
    ([B(0, 4, 10, spans=[(0, 5), (4, 3)])], CEV_ERR_INVALID),           # overlapping spans
    ([B(0, 4, 10, spans=[(20, 5)])], CEV_ERR_INVALID),                  # span past S
    ([B(6, 4, 10)], CEV_ERR_INVALID),                                   # rows past t
    ([B(0, 4, 10, causal=False, valid_len=5)], CEV_ERR_INVALID),        # valid_len > q_len
    ([B(0, 4, 10, causal=True, valid_len=3)], CEV_ERR_INVALID),         # causal with padding
])
def test_malformed_tables_are_rejected(cev, blocks, code):
    d = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 8, 10)
    assert _plan_rc(d, blocks) == code
    assert _abi.lib().cev_last_error()


@pytest.mark.parametrize("blocks", [
    [B(0, 16, 2**31 - 6)],                               # local keys end past INT32_MAX
    [B(0, 16, 0, spans=[(2**31 - 6, 16)])],              # a span ending past INT32_MAX
    [B(0, 16, 0, spans=[(2**31 - 1, 2**31 - 1)])],
])
def test_table_intervals_do_not_wrap(cev, blocks):
    """Interval ends are formed in 64 bits: a begin near INT32_MAX plus a
    length must be rejected, not wrap to a small end that passes."""
    d = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 16, 0)
    assert _plan_rc(d, blocks) == CEV_ERR_INVALID
    assert "outside" in _abi.lib().cev_last_error().decode()


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=64), CEV_ERR_UNSUPPORTED),
    (dict(n_q_heads=12, n_kv_heads=4), CEV_ERR_UNSUPPORTED),   # g = 3
    (dict(n_q_heads=10, n_kv_heads=4), CEV_ERR_INVALID),       # not a multiple
    (dict(dtype=7), CEV_ERR_UNSUPPORTED),
    (dict(q_stride_h=100), CEV_ERR_UNSUPPORTED),               # misaligned rows
    (dict(t=-1), CEV_ERR_INVALID),
])
def test_unsupported_descriptors_are_rejected(cev, kw, code):
    d = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 8, 10)
    for k, v in kw.items():
        setattr(d, k, v)
    assert _plan_rc(d, [B(0, 8, 10, spans=[(0, 10)])]) == code


def test_f32_head_dim_256_is_unsupported(cev):
    d = cev_hip.attn_desc(CEV_F32, 8, 2, 256, 8, 10)
    assert _plan_rc(d, [B(0, 8, 10, spans=[(0, 10)])]) == CEV_ERR_UNSUPPORTED


def test_plan_buffer_too_small(cev):
    d = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 8, 10)
    arr = (_abi.Block * 1)(B(0, 8, 10, spans=[(0, 10)]))
    buf = np.zeros(64, np.uint8)
    off = (-buf.ctypes.data) % 16
    rc = _abi.lib().cev_attn_plan_build(C.byref(d), arr, 1, C.c_void_p(buf.ctypes.data + off), 32)
    assert rc == CEV_ERR_SPACE


def test_launch_validates_before_any_gpu_call(cev):
    d = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 8, 10)
    tab = cev_hip.BlockTable([B(0, 8, 10, spans=[(0, 10)])], 8, 10)
    plan = cev_hip.AttnPlan(d, tab)
    L = _abi.lib()
    fake = C.c_void_p(4096)
    # null plan / null buffers / a plan for other shapes: all fail before a launch
    assert L.cev_packed_attention(C.byref(d), None, None, fake, fake, fake, fake, fake, None, fake, None, 0, None) == CEV_ERR_INVALID
    hp = C.c_void_p(plan.host.ctypes.data)
    assert L.cev_packed_attention(C.byref(d), hp, fake, None, fake, fake, fake, fake, None, fake, None, 0, None) == CEV_ERR_INVALID
    d2 = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 9, 10)
    assert L.cev_packed_attention(C.byref(d2), hp, fake, fake, fake, fake, fake, fake, None, fake, None, 0, None) == CEV_ERR_INVALID
    assert L.cev_packed_attention(C.byref(d), hp, fake, fake, None, None, fake, fake, None, fake, None, 0, None) == CEV_ERR_INVALID
    d.has_gate = 1
    assert L.cev_packed_attention(C.byref(d), hp, fake, fake, fake, fake, fake, fake, None, fake, None, 0, None) == CEV_ERR_INVALID
    d.has_gate = 0
    # the launch's own strides and scale are validated, not only the plan's
    for field, value, code in (("kc_stride_s", 100, CEV_ERR_UNSUPPORTED),   # rows not 16-byte aligned
                               ("kc_stride_s", 64, CEV_ERR_UNSUPPORTED),    # row shorter than head_dim
                               ("kn_stride_t", 2**40, CEV_ERR_UNSUPPORTED), # beyond a buffer load's range
                               ("o_stride_h", -128, CEV_ERR_INVALID),
                               ("scale", float("nan"), CEV_ERR_INVALID),
                               ("scale", -0.5, CEV_ERR_INVALID)):
        bad = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 8, 10)
        setattr(bad, field, value)
        rc = L.cev_packed_attention(C.byref(bad), hp, fake, fake, fake, fake, fake, fake, None, fake, None, 0, None)
        assert rc == code, (field, value, rc)


def test_empty_table_needs_no_launch(cev):
    d = cev_hip.attn_desc(CEV_BF16, 8, 2, 128, 8, 10)
    plan = cev_hip.AttnPlan(d, cev_hip.BlockTable([], 8, 10))
    assert plan.n_tiles == 0
    hp = C.c_void_p(plan.host.ctypes.data)
    assert _abi.lib().cev_packed_attention(C.byref(d), hp, hp, None, None, None, None, None, None, None, None, 0, None) == 0


def test_qknorm_validation(cev):
    L = _abi.lib()
    d = _abi.QkNormDesc()
    assert L.cev_qknorm_desc_init(C.byref(d), CEV_BF16, 8, 2, 128, 4, 130, 10, 0, 1e-6, 0) == 0
    assert L.cev_qknorm_rope(C.byref(d), None, None, None, None, None, None, None, None, None, None) == CEV_ERR_INVALID
    d.rotary_dim = 128
    d.head_dim = 96
    assert L.cev_qknorm_rope(C.byref(d), None, None, None, None, None, None, None, None, None, None) == CEV_ERR_UNSUPPORTED


def test_layer_norm_and_swiglu_validation(cev):
    """cev_rms_norm / cev_swiglu refuse bad shapes, null and misaligned
    buffers and short strides before any launch (no GPU needed)."""
    L = _abi.lib()
    buf = (C.c_uint8 * 4096)()
    a = C.addressof(buf)
    al = a + (-a) % 16
    p = C.c_void_p(al)
    odd = C.c_void_p(al + 2)
    # dtype, hidden not a multiple of 8 (bf16) / 4 (f32), negative eps
    assert L.cev_rms_norm(7, 4, 64, p, 64, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_UNSUPPORTED
    assert L.cev_rms_norm(CEV_BF16, 4, 60, p, 64, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_F32, 4, 62, p, 64, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_BF16, 4, 64, p, 64, None, 0, None, 0, p, -1.0, 0, p, 64, None) == CEV_ERR_INVALID
    # null, misaligned, strides shorter than a row or breaking 16-byte rows
    assert L.cev_rms_norm(CEV_BF16, 4, 64, None, 64, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_BF16, 4, 64, p, 64, p, 64, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_BF16, 4, 64, odd, 64, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_BF16, 4, 64, p, 32, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_BF16, 4, 64, p, 68, None, 0, None, 0, p, 1e-6, 0, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_rms_norm(CEV_BF16, 0, 64, None, 0, None, 0, None, 0, None, 1e-6, 0, None, 0, None) == 0  # nothing to do
    assert L.cev_swiglu(CEV_BF16, 4, 60, p, p, 64, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_swiglu(CEV_BF16, 4, 64, p, None, 64, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_swiglu(CEV_BF16, 4, 64, p, odd, 64, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_swiglu(CEV_BF16, 4, 64, p, p, 40, p, 64, None) == CEV_ERR_INVALID
    assert L.cev_swiglu(CEV_BF16, 0, 64, None, None, 0, None, 0, None) == 0


def test_linear_gather_and_kv_store_validation(cev):
    """cev_linear, cev_gather_rows and the v store of cev_qknorm_rope_kv
    refuse bad dtypes, sizes, strides, null and misaligned buffers before
    any launch; a product of more than 8 rows needs a cev_blas handle."""
    L = _abi.lib()
    buf = (C.c_uint8 * 8192)()
    a = C.addressof(buf)
    al = a + (-a) % 16
    p = C.c_void_p(al)
    odd = C.c_void_p(al + 2)
    lin = lambda dt, odt, m, n, k, x, ldx, w, ldw, alpha, y, ldy, h=None: L.cev_linear(  # noqa: E731
        h, dt, odt, m, n, k, x, ldx, w, ldw, alpha, y, ldy, None, 0, None)
    assert lin(7, CEV_F32, 2, 4, 64, p, 64, p, 64, 1.0, p, 4) == CEV_ERR_UNSUPPORTED
    assert lin(CEV_F32, CEV_BF16, 2, 4, 64, p, 64, p, 64, 1.0, p, 4) == CEV_ERR_UNSUPPORTED   # f32 in, bf16 out
    assert lin(CEV_BF16, CEV_F32, -1, 4, 64, p, 64, p, 64, 1.0, p, 4) == CEV_ERR_INVALID
    assert lin(CEV_BF16, CEV_F32, 2, 4, 60, p, 64, p, 64, 1.0, p, 4) == CEV_ERR_INVALID       # k not 8-element rows
    assert lin(CEV_BF16, CEV_F32, 2, 4, 64, p, 64, p, 64, float("nan"), p, 4) == CEV_ERR_INVALID
    assert lin(CEV_BF16, CEV_F32, 2, 4, 64, None, 64, p, 64, 1.0, p, 4) == CEV_ERR_INVALID
    assert lin(CEV_BF16, CEV_F32, 2, 4, 64, p, 32, p, 64, 1.0, p, 4) == CEV_ERR_INVALID       # ldx < k
    assert lin(CEV_BF16, CEV_F32, 2, 4, 64, p, 64, p, 64, 1.0, p, 2) == CEV_ERR_INVALID       # ldy < n
    assert lin(CEV_BF16, CEV_F32, 2, 4, 64, odd, 64, p, 64, 1.0, p, 4) == CEV_ERR_INVALID
    assert lin(CEV_BF16, CEV_F32, 16, 4, 64, p, 64, p, 64, 1.0, p, 4) == CEV_ERR_INVALID      # 16 rows, no handle
    # the library GEMM path (more than 8 rows) needs y 16-byte aligned and ldy
    # a multiple of the output's 16-byte vector, checked before the handle
    assert lin(CEV_BF16, CEV_F32, 16, 4, 64, p, 64, p, 64, 1.0, odd, 4) == CEV_ERR_INVALID
    assert "y must be 16-byte aligned" in L.cev_last_error().decode()
    assert lin(CEV_BF16, CEV_F32, 16, 4, 64, p, 64, p, 64, 1.0, p, 6) == CEV_ERR_INVALID      # ldy 6 f32
    assert "y must be 16-byte aligned" in L.cev_last_error().decode()
    assert lin(CEV_BF16, CEV_BF16, 16, 8, 64, p, 64, p, 64, 1.0, p, 12) == CEV_ERR_INVALID    # ldy 12 bf16
    assert "y must be 16-byte aligned" in L.cev_last_error().decode()
    assert lin(CEV_BF16, CEV_F32, 16, 4, 64, p, 64, p, 64, 1.0, p, 8) == CEV_ERR_INVALID      # aligned: only the handle is missing
    assert "cev_blas handle" in L.cev_last_error().decode()
    assert lin(CEV_BF16, CEV_F32, 0, 4, 64, None, 0, None, 0, 1.0, None, 0) == 0               # nothing to do
    gat = lambda dt, odt, n, width, table, ldt, rows, ids, out, ldo: L.cev_gather_rows(  # noqa: E731
        dt, odt, n, width, table, ldt, rows, ids, out, ldo, None)
    assert gat(7, CEV_F32, 2, 8, p, 8, 4, None, p, 8) == CEV_ERR_UNSUPPORTED
    assert gat(CEV_BF16, 9, 2, 8, p, 8, 4, None, p, 8) == CEV_ERR_UNSUPPORTED
    assert gat(CEV_BF16, CEV_F32, -2, 8, p, 8, 4, None, p, 8) == CEV_ERR_INVALID
    assert gat(CEV_BF16, CEV_F32, 2, 8, None, 8, 4, None, p, 8) == CEV_ERR_INVALID
    assert gat(CEV_BF16, CEV_F32, 2, 8, p, 4, 4, None, p, 8) == CEV_ERR_INVALID                # ld_table < width
    assert gat(CEV_BF16, CEV_F32, 6, 8, p, 8, 4, None, p, 8) == CEV_ERR_INVALID                # 6 rows of a 4-row table
    assert gat(CEV_BF16, CEV_F32, 0, 8, None, 0, 0, None, None, 0) == 0
    d = _abi.QkNormDesc()
    assert L.cev_qknorm_desc_init(C.byref(d), CEV_BF16, 8, 2, 128, 4, 128, 10, 0, 1e-6, 0) == 0
    pos = (C.c_int32 * 4)()
    kv = lambda v_in, vi_t, v_out, vo_t: L.cev_qknorm_rope_kv(  # noqa: E731
        C.byref(d), p, p, v_in, vi_t, 128, p, p, pos, p, p, None, 0, p, p, v_out, vo_t, 128, None)
    assert kv(p, 256, None, 256) == CEV_ERR_INVALID       # v_in without v_out
    assert kv(odd, 256, p, 256) == CEV_ERR_INVALID        # misaligned v rows
    assert kv(p, 260, p, 256) == CEV_ERR_INVALID          # v row stride breaks 16-byte rows


def test_prefix_store_argument_errors(cev):
    """The store refuses empty reservations, unknown ranges and bad
    capacities with CEV_ERR_INVALID, and a reservation beyond the capacity
    with CEV_ERR_SPACE; a refused call changes nothing."""
    L = _abi.lib()
    h = C.c_void_p()
    assert L.cev_prefix_store_create(0, 10, C.byref(h)) == CEV_ERR_INVALID
    assert L.cev_prefix_store_create(10, -1, C.byref(h)) == CEV_ERR_INVALID
    store = cev_hip.PrefixStore(capacity=64, budget=64)
    for bad in (0, -3):
        with pytest.raises(CevError) as e:
            store.reserve(bad)
        assert e.value.code == CEV_ERR_INVALID
    with pytest.raises(CevError) as e:
        store.reserve(65)
    assert e.value.code == CEV_ERR_SPACE
    b = store.reserve(16)
    with pytest.raises(CevError) as e:
        store.put(list(range(8)), b)       # length differs from the reservation
    assert e.value.code == CEV_ERR_INVALID
    with pytest.raises(CevError) as e:
        store.release(b + 1)               # not the start of a held range
    assert e.value.code == CEV_ERR_INVALID
    assert store.stats()["used_slots"] == 16
    store.release(b)
    with pytest.raises(CevError) as e:
        store.release(b)                   # already released
    assert e.value.code == CEV_ERR_INVALID
    assert store.stats() == {"entries": 0, "cached_tokens": 0, "used_slots": 0}


# ---------------------------------------------------------------- table builders vs reference masks


def _random_pass(rng):
    n_plans = int(rng.integers(1, 4))
    plans = []
    for _ in range(n_plans):
        prefix = int(rng.integers(1, 40))
        mode = rng.integers(0, 3)
        if mode == 0:       # cached prefix, no tail
            plans.append((prefix, prefix, prefix))
        elif mode == 1:     # head prefilled, tail in the pass
            tail = int(rng.integers(1, prefix + 1))
            plans.append((prefix - tail, prefix, prefix - tail))
        else:               # nothing cached, whole prefix is the tail
            plans.append((0, prefix, 0))
    items = [(int(rng.integers(0, n_plans)), int(rng.integers(1, 12))) for _ in range(int(rng.integers(1, 7)))]
    return plans, items


def test_table_from_plans_reproduces_engine_mask(cev, orc):
    rng = np.random.default_rng(3)
    for _ in range(200):
        plans, items = _random_pass(rng)
        ep = orc.engine_pass(plans, items)
        tab, pos, gather = cev_hip.BlockTable.from_plans(plans, items)
        assert tab.t == ep["n"] and tab.s_cache == ep["past_total"]
        assert np.array_equal(tab.to_dense_mask(), ep["mask"])
        assert np.array_equal(pos, ep["pos"]) and np.array_equal(gather, ep["gather"])
        back = cev_hip.BlockTable.from_dense_mask(ep["mask"], ep["past_total"])
        assert np.array_equal(back.to_dense_mask(), ep["mask"])


def test_table_from_segments_reproduces_segment_mask(cev, orc):
    for past, seg in ((0, [0] * 9), (12, [0] * 5), (7, [0, 0, 1, 1, 1, 2, 3, 3])):
        tab = cev_hip.BlockTable.from_segment_ids(seg, past)
        assert np.array_equal(tab.to_dense_mask(), orc.segment_mask(seg, past))
    with pytest.raises(CevError):
        cev_hip.BlockTable.from_segment_ids([0, 1, 0], 3)


def test_table_from_rows_reproduces_qwen35_masks(cev, orc):
    b, t, past = 3, 6, 10
    tab = cev_hip.BlockTable.from_rows(b, t, past, causal=True)
    # rows of a batch each see the (broadcast) prefix and their own row causally
    dense = tab.to_dense_mask()
    br = orc.branch_mask(t, past)
    for r in range(b):
        rows = dense[r * t:(r + 1) * t]
        assert np.array_equal(rows[:, :past], br[:, :past])
        assert np.array_equal(rows[:, past + r * t: past + (r + 1) * t], br[:, past:])
        others = np.delete(rows[:, past:], np.s_[r * t:(r + 1) * t], axis=1)
        assert np.all(np.isneginf(others))
    lengths = [6, 2, 0]
    tab = cev_hip.BlockTable.from_rows(b, t, 0, causal=False, lengths=lengths)
    dense = tab.to_dense_mask()
    bd = orc.bidirectional_mask(t, lengths)
    for r in range(b):
        assert np.array_equal(dense[r * t:(r + 1) * t, r * t:(r + 1) * t], bd[r])
    back = cev_hip.BlockTable.from_dense_mask(dense, 0)
    assert np.array_equal(back.to_dense_mask(), dense)
    with pytest.raises(CevError):
        cev_hip.BlockTable.from_rows(2, 4, 5, causal=False, lengths=[4, 4])


def test_rope_table_is_the_reference_recipe(cev, orc):
    for theta, rot, n in ((1e6, 128, 3000), (1e7, 64, 9000)):
        c, s = cev_hip.rope_table(theta, rot, n, CEV_F32)
        oc, os_ = orc.rope_table(theta, rot, n, False)
        assert np.array_equal(c, oc) and np.array_equal(s, os_)
        cb, sb = cev_hip.rope_table(theta, rot, n, CEV_BF16)
        ocb, osb = orc.rope_table(theta, rot, n, True)
        assert np.array_equal((cb.astype(np.uint32) << 16).view(np.float32), ocb)
        assert np.array_equal((sb.astype(np.uint32) << 16).view(np.float32), osb)


def test_plan_tiles_cover_rows_and_keys(cev, orc):
    """The compiled plan visits exactly the keys each row may see."""
    rng = np.random.default_rng(11)
    for _ in range(60):
        plans, items = _random_pass(rng)
        tab, _, _ = cev_hip.BlockTable.from_plans(plans, items)
        for hq, hkv in ((8, 8), (8, 4), (8, 2), (8, 1)):
            d = cev_hip.attn_desc(CEV_BF16, hq, hkv, 128, tab.t, tab.s_cache)
            plan = cev_hip.AttnPlan(d, tab)
            dense = tab.to_dense_mask() == 0
            rows = plan.rows()
            seen = np.zeros_like(dense)
            for tr0, tn, s0, sn, nch, _, _, _ in plan.tiles():
                assert nch == sum(-(-(ke - kb) // plan.block_n) for kb, ke, _, _ in plan.segs()[s0:s0 + sn])
                assert tn <= plan.tile_rows
                for kb, ke, masked, _ in plan.segs()[s0:s0 + sn]:
                    assert (kb < tab.s_cache) == (ke <= tab.s_cache) or kb >= tab.s_cache
                    for r in range(tr0, tr0 + tn):
                        keys = np.arange(kb, ke)
                        if masked:
                            lo, hi, dg, _ = rows[r]
                            keys = keys[((keys >= lo) & (keys < hi)) | (keys == dg)]
                        assert not seen[r, keys].any(), "a key visited twice"
                        seen[r, keys] = True
            assert np.array_equal(seen, dense)


def test_split_policy(cev):
    """Few long-prefix rows split their key stream; full grids do not."""
    B = cev_hip.BlockTable.block
    hbm = cev_hip.BlockTable([B(0, 16, 32768, spans=[(0, 32768)])], 16, 32768)
    d = cev_hip.attn_desc(CEV_BF16, 32, 8, 128, 16, 32768)
    p = cev_hip.AttnPlan(d, hbm)
    assert p.n_splits > 1 and p.n_tiles * p.n_splits * 8 >= 256
    # one record per (row, head, part): its bf16 output values in the first
    # region, its f32 m and l in the second
    assert p.workspace_bytes == 16 * 32 * p.n_splits * (2 * 128 + 8)
    d.max_splits = 1
    assert cev_hip.AttnPlan(d, hbm).n_splits == 1 and cev_hip.AttnPlan(d, hbm).workspace_bytes == 0
    d.max_splits = 3
    assert cev_hip.AttnPlan(d, hbm).n_splits == 3
    plans, items = [(32768, 32768, 32768)], [(0, 64)] * 64
    tab, _, _ = cev_hip.BlockTable.from_plans(plans, items)
    d = cev_hip.attn_desc(CEV_BF16, 32, 8, 128, tab.t, tab.s_cache)
    assert cev_hip.AttnPlan(d, tab).n_splits == 1
    # one round of 256 workgroups: the 16-token shape takes 32 parts (8 x 32)
    d = cev_hip.attn_desc(CEV_BF16, 32, 8, 128, 16, 32768)
    assert cev_hip.AttnPlan(d, hbm).n_splits == 32
    # 224 workgroups already fill the round: splitting would add a second
    # round and the merge (the 28-layer Qwen3-1.7B-shaped pass)
    tab, _, _ = cev_hip.BlockTable.from_plans([(1536, 2048, 1536)], [(0, 48)] * 64)
    d = cev_hip.attn_desc(CEV_BF16, 16, 8, 128, tab.t, tab.s_cache)
    p = cev_hip.AttnPlan(d, tab)
    assert p.n_tiles * 8 == 224 and p.n_splits == 1
    # 128 workgroups of long rows: two parts fill the round (the gated rows)
    tab = cev_hip.BlockTable.from_rows(32, 64, 4096, causal=True)
    d = cev_hip.attn_desc(CEV_BF16, 16, 4, 256, tab.t, tab.s_cache, has_gate=True)
    assert cev_hip.AttnPlan(d, tab).n_splits == 2
    # f32 key tiles are MFMA-heavy: 12 x 32-token blocks after a 256-token
    # prefix (3 full tiles x 8 KV heads, at most half a round) get half-full
    # tiles, 6 x 8 items, whose 12-chunk key streams split into 5 parts (one
    # round); the same table in bf16 keeps full tiles
    tab = cev_hip.BlockTable.from_rows(12, 32, 256, causal=True)
    d = cev_hip.attn_desc(CEV_F32, 16, 8, 128, tab.t, tab.s_cache)
    p = cev_hip.AttnPlan(d, tab)
    assert p.n_tiles == 6 and p.n_splits == 5
    d = cev_hip.attn_desc(CEV_BF16, 16, 8, 128, tab.t, tab.s_cache)
    assert cev_hip.AttnPlan(d, tab).n_tiles == 3
    d = cev_hip.attn_desc(CEV_BF16, 16, 8, 128, tab.t, tab.s_cache)
    assert cev_hip.AttnPlan(d, tab).n_splits == 1


def test_launch_requires_workspace_for_split_plans(cev):
    B = cev_hip.BlockTable.block
    tab = cev_hip.BlockTable([B(0, 16, 4096, spans=[(0, 4096)])], 16, 4096)
    d = cev_hip.attn_desc(CEV_BF16, 32, 8, 128, 16, 4096)
    plan = cev_hip.AttnPlan(d, tab)
    assert plan.n_splits > 1
    fake = C.c_void_p(4096)
    hp = C.c_void_p(plan.host.ctypes.data)
    L = _abi.lib()
    assert L.cev_packed_attention(C.byref(d), hp, fake, fake, fake, fake, fake, fake, None, fake, None, 0, None) == CEV_ERR_INVALID
    assert L.cev_packed_attention(C.byref(d), hp, fake, fake, fake, fake, fake, fake, None, fake, fake, 16, None) == CEV_ERR_SPACE


def test_runtime_helpers_validate_before_any_gpu_call(cev):
    L = _abi.lib()
    assert L.cev_event_create(None) == CEV_ERR_INVALID
    assert L.cev_event_record(None, None) == CEV_ERR_INVALID
    assert L.cev_event_synchronize(None) == CEV_ERR_INVALID
    assert L.cev_event_elapsed_ms(None, None, None) == CEV_ERR_INVALID
    assert L.cev_malloc(None, 16) == CEV_ERR_INVALID
    assert L.cev_stream_create(None) == CEV_ERR_INVALID
