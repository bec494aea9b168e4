"""The allocation-free attention entry point (cev_packed_attention_noalloc)
against cev_packed_attention, both called through the C ABI.

The two share their kernels and plan; only where a split plan's partial
records live differs (a static device buffer instead of the caller's
workspace), so the outputs must agree bit for bit.  Two calls in a row, the
second smaller than the first, check that nothing the first call left in
the buffer leaks into the second."""
import ctypes as C

import numpy as np
import pytest

import cev_hip
from cev_hip import _abi
from cev_hip._abi import CEV_ERR_SPACE


def _say(msg):
    print(msg, flush=True)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _case(gpu, prefix, t, hq, hkv, d, seed, dtype=None):
    import torch
    dtype = torch.bfloat16 if dtype is None else dtype
    g = torch.Generator(device="cpu").manual_seed(seed)
    rnd = lambda *s: torch.randn(*s, generator=g).to(dtype).to(gpu)  # noqa: E731
    q, kn, vn = rnd(t, hq, d), rnd(t, hkv, d), rnd(t, hkv, d)
    kc, vc = rnd(hkv, prefix, d), rnd(hkv, prefix, d)
    tab = cev_hip.BlockTable.from_rows(1, t, prefix, causal=True)
    op = cev_hip.PackedAttention(q, kn, tab, k_cache=kc, s_cache=prefix, v_new=vn, v_cache=vc)
    return op, (q, kn, vn, kc, vc)


def _noalloc(op, q, kn, vn, kc, vc, out):
    import torch
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    op._set_strides(q, kn, vn, kc, vc, out, None)
    return _abi.lib().cev_packed_attention_noalloc(C.byref(op.desc), C.c_void_p(op.plan.host.ctypes.data), _ptr(op.plan.dev),
                                                   _ptr(q), _ptr(kc), _ptr(vc), _ptr(kn), _ptr(vn), None, _ptr(out), stream)


# (dtype, head dim, GQA shape, [(prefix, tokens, seed), ...]): every record
# layout of the split kernels (bf16 d = 128, bf16 d = 256, f32 d = 128),
# each as two calls in a row, the second smaller than the first
CASES = [("bf16", 128, (32, 8), [(32768, 16, 1), (4096, 16, 2)]),
         ("bf16", 256, (16, 4), [(16384, 16, 3), (2048, 16, 4)]),
         ("f32", 128, (16, 8), [(8192, 16, 5), (1024, 16, 6)])]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,d,heads,calls", CASES, ids=[f"{c[0]}-d{c[1]}" for c in CASES])
def test_noalloc_matches_workspace_entry_on_two_calls(gpu, dtype, d, heads, calls):
    import torch
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    for prefix, t, seed in calls:
        op, (q, kn, vn, kc, vc) = _case(gpu, prefix, t, heads[0], heads[1], d, seed, tdt)
        _say(f"noalloc {dtype} d={d}: prefix {prefix} x {t} tokens, {op.plan.n_splits} parts, {op.plan.workspace_bytes} record bytes")
        assert op.plan.n_splits > 1 and 0 < op.plan.workspace_bytes <= _abi.CEV_ATTN_SCRATCH_BYTES
        want = op(q, kn, vn, kc, vc)
        got = torch.full_like(q, float("nan"))
        _abi.check(_noalloc(op, q, kn, vn, kc, vc, got))
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want)


@pytest.mark.gpu
def test_noalloc_replays_from_a_graph(gpu):
    """One direct call (which resolves the scratch address), then the call
    captured in a HIP graph: every replay, with eager work and
    synchronisations in between, equals the workspace entry point bit for
    bit."""
    import torch
    op, (q, kn, vn, kc, vc) = _case(gpu, 32768, 16, 32, 8, 128, 7)
    want = op(q, kn, vn, kc, vc)
    got = torch.full_like(q, float("nan"))
    _abi.check(_noalloc(op, q, kn, vn, kc, vc, got))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = _noalloc(op, q, kn, vn, kc, vc, got)
    assert rc == 0
    small, (q2, kn2, vn2, kc2, vc2) = _case(gpu, 4096, 16, 32, 8, 128, 8)
    out2 = torch.empty_like(q2)
    for i in range(3):
        got.fill_(float("nan"))
        if i == 1:  # eager calls in between: the workspace entry point, and a direct call that rewrites the scratch
            op(q, kn, vn, kc, vc)
            _abi.check(_noalloc(small, q2, kn2, vn2, kc2, vc2, out2))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"


def test_noalloc_rejects_plans_beyond_the_scratch(cev):
    """Checked on the host before any GPU call: a plan whose split records
    exceed the static buffer fails with CEV_ERR_SPACE."""
    d = cev_hip.attn_desc(_abi.CEV_BF16, 32, 8, 128, 16, 4096)
    plan = cev_hip.AttnPlan(d, cev_hip.BlockTable.from_rows(1, 16, 4096, causal=True))
    host = plan.host.copy()
    hdr = host[:80].view(np.int32)
    hdr[4] = 1 << 20   # t
    hdr[15] = 64       # n_splits: 2^20 rows x 32 heads x 64 parts of records
    fake = C.c_void_p(4096)
    rc = _abi.lib().cev_packed_attention_noalloc(C.byref(d), C.c_void_p(host.ctypes.data), fake, fake, fake, fake, fake, fake, None,
                                                 fake, None)
    assert rc == CEV_ERR_SPACE
    assert "static scratch" in _abi.lib().cev_last_error().decode()
