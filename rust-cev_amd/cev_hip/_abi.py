"""ctypes view of include/cev_hip.h (libcev_hip.so).

Struct layouts and signatures mirror the header one to one; a Rust host
binds the same symbols with `extern "C"` declarations.
"""
from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("CEV_HIP_LIB") or os.path.join(_PKG, "build", "libcev_hip.so")

CEV_OK = 0
CEV_ERR_INVALID = -1
CEV_ERR_UNSUPPORTED = -2
CEV_ERR_HIP = -3
CEV_ERR_SPACE = -4

CEV_F32 = 0
CEV_BF16 = 1
CEV_MAX_SPANS = 4
CEV_ATTN_SCRATCH_BYTES = 64 << 20
CEV_LINEAR_WORKSPACE_BYTES = 32 << 20

i32 = C.c_int32
i64 = C.c_int64


class Span(C.Structure):
    _fields_ = [("begin", i32), ("len", i32)]


class Block(C.Structure):
    _fields_ = [
        ("q_begin", i32),
        ("q_len", i32),
        ("valid_len", i32),
        ("causal", i32),
        ("local_begin", i32),
        ("n_spans", i32),
        ("spans", Span * CEV_MAX_SPANS),
    ]

    def as_tuple(self):
        return (self.q_begin, self.q_len, self.valid_len, self.causal, self.local_begin,
                tuple((self.spans[i].begin, self.spans[i].len) for i in range(self.n_spans)))


class AttnDesc(C.Structure):
    _fields_ = [
        ("dtype", i32), ("n_q_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
        ("t", i32), ("s_cache", i32), ("scale", C.c_float), ("has_gate", i32),
        ("q_stride_t", i64), ("q_stride_h", i64),
        ("kc_stride_s", i64), ("kc_stride_h", i64),
        ("vc_stride_s", i64), ("vc_stride_h", i64),
        ("kn_stride_t", i64), ("kn_stride_h", i64),
        ("vn_stride_t", i64), ("vn_stride_h", i64),
        ("g_stride_t", i64), ("g_stride_h", i64),
        ("o_stride_t", i64), ("o_stride_h", i64),
        ("max_splits", i32), ("reserved", i32),
    ]


class QkNormDesc(C.Structure):
    _fields_ = [
        ("dtype", i32), ("n_q_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
        ("t", i32), ("rotary_dim", i32), ("n_pos", i32), ("weight_plus_one", i32),
        ("eps", C.c_float),
        ("qi_stride_t", i64), ("qi_stride_h", i64),
        ("ki_stride_t", i64), ("ki_stride_h", i64),
        ("qo_stride_t", i64), ("qo_stride_h", i64),
        ("ko_stride_t", i64), ("ko_stride_h", i64),
    ]


class GdnDesc(C.Structure):
    _fields_ = [
        ("dtype", i32), ("batch", i32), ("t", i32), ("n_k_heads", i32), ("n_v_heads", i32),
        ("head_k_dim", i32), ("head_v_dim", i32), ("conv_kernel", i32), ("eps", C.c_float), ("reserved", i32),
        ("mixed_stride_b", i64), ("mixed_stride_t", i64),
        ("z_stride_b", i64), ("z_stride_t", i64),
        ("ab_stride_b", i64), ("ab_stride_t", i64),
        ("conv_in_stride_b", i64), ("s_in_stride_b", i64),
        ("y_stride_b", i64), ("y_stride_t", i64),
    ]


P = C.c_void_p
Pi32 = C.POINTER(i32)
PBlock = C.POINTER(Block)

# name -> (restype, argtypes); the exact list of symbols include/cev_hip.h declares.
SIGNATURES = {
    "cev_attn_desc_init": (i32, [C.POINTER(AttnDesc), i32, i32, i32, i32, i32, i32, i32]),
    "cev_attn_plan_size": (i32, [C.POINTER(AttnDesc), PBlock, i32, C.POINTER(C.c_size_t)]),
    "cev_attn_plan_build": (i32, [C.POINTER(AttnDesc), PBlock, i32, P, C.c_size_t]),
    "cev_attn_workspace_size": (i32, [P, C.POINTER(C.c_size_t)]),
    "cev_packed_attention": (i32, [C.POINTER(AttnDesc), P, P, P, P, P, P, P, P, P, P, C.c_size_t, P]),
    "cev_packed_attention_noalloc": (i32, [C.POINTER(AttnDesc), P, P, P, P, P, P, P, P, P, P]),
    "cev_qknorm_desc_init": (i32, [C.POINTER(QkNormDesc), i32, i32, i32, i32, i32, i32, i32, i32, C.c_float, i32]),
    "cev_qknorm_rope": (i32, [C.POINTER(QkNormDesc), P, P, P, P, P, P, P, P, P, P]),
    "cev_qknorm_rope_kv": (i32, [C.POINTER(QkNormDesc), P, P, P, i64, i64, P, P, P, P, P, P, i32, P, P, P, i64, i64, P]),
    "cev_rope_table": (i32, [C.c_double, i32, i32, i32, P, P]),
    "cev_gdn_desc_init": (i32, [C.POINTER(GdnDesc), i32, i32, i32, i32, i32, i32, i32, i32, C.c_float]),
    "cev_gdn_workspace_size": (i32, [C.POINTER(GdnDesc), C.POINTER(C.c_size_t)]),
    "cev_gdn_forward": (i32, [C.POINTER(GdnDesc), P, P, P, P, P, P, P, P, P, P, P, P, P, P, C.c_size_t, P]),
    "cev_rms_norm": (i32, [i32, i64, i32, P, i64, P, i64, P, i64, P, C.c_float, i32, P, i64, P]),
    "cev_rms_norm_seq": (i32, [i32, i64, i32, P, i64, P, i64, P, i64, P, C.c_float, i32, P, i64, P]),
    "cev_swiglu": (i32, [i32, i64, i32, P, P, i64, P, i64, P]),
    "cev_debias_scores": (i32, [i32, i32, P, P, P, P, P, P, i32, P, P]),
    "cev_blas_create": (i32, [C.POINTER(P)]),
    "cev_blas_destroy": (i32, [P]),
    "cev_linear": (i32, [P, i32, i32, i64, i64, i64, P, i64, P, i64, C.c_float, P, i64, P, C.c_size_t, P]),
    "cev_gather_rows": (i32, [i32, i32, i64, i64, P, i64, i64, P, P, i64, P]),
    "cev_table_from_plans": (i32, [i32, Pi32, Pi32, Pi32, i32, Pi32, Pi32, PBlock, i32, Pi32, Pi32, i32, Pi32, Pi32]),
    "cev_table_from_rows": (i32, [i32, i32, i32, i32, Pi32, PBlock, i32]),
    "cev_table_from_slots": (i32, [i32, Pi32, Pi32, Pi32, i32, Pi32, Pi32, Pi32, i32, PBlock, i32, Pi32, Pi32, Pi32, i32, Pi32, Pi32]),
    "cev_prefix_store_create": (i32, [i32, i64, C.POINTER(P)]),
    "cev_prefix_store_destroy": (i32, [P]),
    "cev_prefix_store_get": (i32, [P, C.POINTER(C.c_uint32), i32, Pi32, Pi32]),
    "cev_prefix_store_reserve": (i32, [P, i32, Pi32]),
    "cev_prefix_store_put": (i32, [P, C.POINTER(C.c_uint32), i32, i32]),
    "cev_prefix_store_release": (i32, [P, i32]),
    "cev_prefix_store_stats": (i32, [P, Pi32, C.POINTER(i64), Pi32]),
    "cev_prefix_store_entry": (i32, [P, i32, Pi32, Pi32]),
    "cev_table_from_segment_ids": (i32, [C.POINTER(C.c_uint32), i32, i32, PBlock, i32, Pi32]),
    "cev_table_to_dense_mask": (i32, [PBlock, i32, i32, i32, P]),
    "cev_table_from_dense_mask": (i32, [P, i32, i32, PBlock, i32, Pi32]),
    "cev_last_error": (C.c_char_p, []),
    "cev_abi_version": (i32, []),
    "cev_device_info": (i32, [i32, C.c_char_p, C.c_size_t, Pi32, C.POINTER(i64), Pi32]),
    "cev_malloc": (i32, [C.POINTER(P), C.c_size_t]),
    "cev_free": (i32, [P]),
    "cev_memcpy_h2d": (i32, [P, P, C.c_size_t, P]),
    "cev_memcpy_d2h": (i32, [P, P, C.c_size_t, P]),
    "cev_stream_create": (i32, [C.POINTER(P)]),
    "cev_stream_destroy": (i32, [P]),
    "cev_stream_synchronize": (i32, [P]),
    "cev_memcpy_d2d": (i32, [P, P, C.c_size_t, P]),
    "cev_event_create": (i32, [C.POINTER(P)]),
    "cev_event_destroy": (i32, [P]),
    "cev_event_record": (i32, [P, P]),
    "cev_event_synchronize": (i32, [P]),
    "cev_event_elapsed_ms": (i32, [P, P, C.POINTER(C.c_float)]),
}

_lib = None


class CevError(RuntimeError):
    """A failed C-ABI call: `code` is the CEV_ERR_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"cev error {code}: {msg}")
        self.code = code


def lib():
    """The loaded libcev_hip.so.  There is no fallback: without the built
    library every entry point raises."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != CEV_OK:
        raise CevError(rc, lib().cev_last_error().decode(errors="replace"))
