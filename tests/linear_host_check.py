"""cev_linear driven the way a host without torch drives it (through the C
ABI only: cev_malloc, copies, a cev_blas handle, events), so the library
binds to ROCm's hipBLASLt: the instance the per-shape algorithm picks in
linear.hip were measured on.  Run as a script by tests/test_runtime_gpu.py
(a pytest process has torch, and with it torch's hipBLASLt, loaded).
Checks the config-2 projection shapes (the picked ones and gate/up, which
keeps the heuristic's choice) against f64 products rounded to bf16, and
prints each product's time."""
import ctypes as C
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "rust-cev_amd"))
from cev_hip import _abi  # noqa: E402
from cev_hip._abi import CEV_BF16, CEV_LINEAR_WORKSPACE_BYTES, check  # noqa: E402


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bits(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def main():
    L = _abi.lib()
    rng = np.random.default_rng(11)
    s, e0, e1, blas, ws = (C.c_void_p() for _ in range(5))
    check(L.cev_stream_create(C.byref(s)))
    check(L.cev_event_create(C.byref(e0)))
    check(L.cev_event_create(C.byref(e1)))
    check(L.cev_blas_create(C.byref(blas)))
    check(L.cev_malloc(C.byref(ws), CEV_LINEAR_WORKSPACE_BYTES))
    worst = 0.0
    for name, m, n, k in (("q/k/v", 3584, 4096, 2048), ("o_proj", 3584, 2048, 2048), ("gate/up", 3584, 12288, 2048),
                          ("down", 3584, 2048, 6144)):
        xb = bf16_bits(rng.standard_normal((m, k)))
        wb = bf16_bits(0.02 * rng.standard_normal((n, k)))
        x, w, y = C.c_void_p(), C.c_void_p(), C.c_void_p()
        for p, nbytes in ((x, xb.nbytes), (w, wb.nbytes), (y, m * n * 2)):
            check(L.cev_malloc(C.byref(p), nbytes))
        try:
            check(L.cev_memcpy_h2d(x, xb.ctypes.data, xb.nbytes, s))
            check(L.cev_memcpy_h2d(w, wb.ctypes.data, wb.nbytes, s))

            def run():
                check(L.cev_linear(blas, CEV_BF16, CEV_BF16, m, n, k, x, k, w, k, 1.0, y, n, ws, CEV_LINEAR_WORKSPACE_BYTES, s))

            for _ in range(3):
                run()
            check(L.cev_event_record(e0, s))
            for _ in range(20):
                run()
            check(L.cev_event_record(e1, s))
            check(L.cev_event_synchronize(e1))
            ms = C.c_float()
            check(L.cev_event_elapsed_ms(e0, e1, C.byref(ms)))
            yb = np.empty((m, n), np.uint16)
            check(L.cev_memcpy_d2h(yb.ctypes.data, y, yb.nbytes, s))
            check(L.cev_stream_synchronize(s))
            want = from_bits(bf16_bits(from_bits(xb).astype(np.float64) @ from_bits(wb).astype(np.float64).T))
            got = from_bits(yb)
            err = float(np.abs(got - want).max() / np.abs(want).max())
            worst = max(worst, err)
            print(f"{name} m={m} n={n} k={k}: {1000 * ms.value / 20:.2f} us, max rel err {err:.3g}", flush=True)
        finally:
            for p in (x, w, y):
                check(L.cev_free(p))
    check(L.cev_free(ws))
    check(L.cev_blas_destroy(blas))
    check(L.cev_event_destroy(e0))
    check(L.cev_event_destroy(e1))
    check(L.cev_stream_destroy(s))
    assert "torch" not in sys.modules, "this check must run without torch"
    assert worst <= 1e-2, worst
    return 0


if __name__ == "__main__":
    sys.exit(main())
