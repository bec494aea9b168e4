"""Writes tests/golden/c2_f32.npz: the oracle's answer-code probabilities
and final hidden state for config 2 in f32 (28 layers, full vocab), the
fixture test_qwen3_stack_gpu.py compares the device stack with.

    python tests/golden/make_c2_golden.py      (CPU only; several minutes)
"""
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "rust-cev_amd")]

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from cev_hip import configs  # noqa: E402
from oracle import qwen3_stack  # noqa: E402


def main():
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    w = configs.c2(False)
    t0 = time.time()
    weights = w.weights()
    print(f"weights: {time.time() - t0:.1f} s", flush=True)
    p, hid = qwen3_stack.run_config(w, weights)
    print(f"oracle config 2 (f32): {time.time() - t0:.1f} s; p[0] = {np.round(p[0], 5)}", flush=True)
    np.savez_compressed(os.path.join(HERE, "c2_f32.npz"), p=p, hidden=hid.astype(np.float32))


if __name__ == "__main__":
    main()
