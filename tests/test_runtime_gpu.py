"""The C-ABI runtime helpers a host without a HIP binding uses (buffers,
copies, streams and timing events), driven only through the library."""
import ctypes as C

import numpy as np
import pytest

from cev_hip import _abi
from cev_hip._abi import check

pytestmark = pytest.mark.gpu


def test_buffers_copies_streams_and_events():
    L = _abi.lib()
    n = 1 << 20
    src = (np.arange(n, dtype=np.float32) * 0.5 - 7.0).astype(np.float32)
    a, b, s, e0, e1 = (C.c_void_p() for _ in range(5))
    check(L.cev_malloc(C.byref(a), n * 4))
    check(L.cev_malloc(C.byref(b), n * 4))
    check(L.cev_stream_create(C.byref(s)))
    check(L.cev_event_create(C.byref(e0)))
    check(L.cev_event_create(C.byref(e1)))
    try:
        check(L.cev_memcpy_h2d(a, src.ctypes.data, n * 4, s))
        check(L.cev_event_record(e0, s))
        for _ in range(4):
            check(L.cev_memcpy_d2d(b, a, n * 4, s))
        check(L.cev_event_record(e1, s))
        out = np.zeros_like(src)
        check(L.cev_memcpy_d2h(out.ctypes.data, b, n * 4, s))
        check(L.cev_stream_synchronize(s))
        check(L.cev_event_synchronize(e1))
        ms = C.c_float(-1.0)
        check(L.cev_event_elapsed_ms(e0, e1, C.byref(ms)))
        assert 0.0 < ms.value < 1000.0
        np.testing.assert_array_equal(out, src)
    finally:
        check(L.cev_event_destroy(e0))
        check(L.cev_event_destroy(e1))
        check(L.cev_stream_destroy(s))
        check(L.cev_free(a))
        check(L.cev_free(b))


def test_linear_from_a_host_without_torch():
    """cev_linear on the config-2 projection shapes from a process that has
    not loaded torch (so the library binds to ROCm's hipBLASLt, where its
    per-shape picks apply), against f64 products rounded to bf16."""
    import os
    import subprocess
    import sys
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "linear_host_check.py")
    r = subprocess.run([sys.executable, script], capture_output=True, text=True, timeout=150)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0
