"""Writes tests/golden/c2_f32.npz and c2_bf16.npz: the oracle's answer-code
probabilities and final hidden state of the 28-layer Qwen3-1.7B-shaped pass in f32 and in bf16 (28
layers, full vocab), the fixtures test_qwen3_stack_gpu.py compares the
device stack with.

    python tests/golden/make_c2_golden.py [f32|bf16 ...]   (CPU only; several minutes each)
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


def main(dtypes):
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    for dt in dtypes:
        w = configs.c2(dt == "bf16")
        t0 = time.time()
        weights = w.weights()
        print(f"weights: {time.time() - t0:.1f} s", flush=True)
        p, hid = qwen3_stack.run_config(w, weights)
        print(f"oracle 28-layer pass ({dt}): {time.time() - t0:.1f} s; p[0] = {np.round(p[0], 5)}", flush=True)
        np.savez_compressed(os.path.join(HERE, f"c2_{dt}.npz"), p=p, hidden=hid.astype(np.float32))


if __name__ == "__main__":
    main(sys.argv[1:] or ["f32", "bf16"])
