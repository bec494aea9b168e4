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
