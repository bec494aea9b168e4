"""Runs the hipBLASLt candidate probe (csrc/gemm_probe.cpp) on torch's own
libhipblaslt.so: torch is imported first, so build/libgemm_probe.so binds to
the hipBLASLt instance that libcev_hip.so uses in a torch process.

    make gemm-probe && python3 gemm_probe.py [m ...]
"""
import ctypes
import os
import sys

import torch  # noqa: F401  (loads torch's libhipblaslt.so before the probe)


def main(argv):
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "build", "libgemm_probe.so"))
    lib.cev_gemm_probe.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
    args = (ctypes.c_char_p * max(1, len(argv)))(*[a.encode() for a in argv])
    sys.stdout.flush()
    return lib.cev_gemm_probe(len(argv), args)


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
