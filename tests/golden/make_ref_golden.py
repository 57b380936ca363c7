"""Writes tests/golden/ref_cpu_golden.npz: outputs of the reference's own FP64
oracle (kernels/matmul_iq4xs/ref_cpu.cpp:12-139, compiled unchanged by
`make -C oracle ref` into oracle/_ref/libref_cpu.so) on small seeded inputs.
These pin this repository's oracle restatement, and travel where the
reference does not.  Run: python tests/golden/make_ref_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.oracle import Oracle, RefCpu  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_cpu_golden.npz")

# (name, K, N, M, weight seed, activation seed, outliers)
CASES = [
    ("gemv_512x48", 512, 48, 1, 101, 201, False),
    ("gemv_1024x16_outliers", 1024, 16, 1, 102, 202, True),
    ("gemv_768x8_odd_superblocks", 768, 8, 1, 103, 203, False),
    ("gemm_512x16x8", 512, 16, 8, 104, 204, False),
    ("gemm_256x8x5", 256, 8, 5, 105, 205, True),
]


def main() -> None:
    orc, ref = Oracle(), RefCpu()
    arrays = {}
    for name, K, N, M, ws, xs, outl in CASES:
        W = orc.gen_weights(K, N, ws)
        arrays[f"{name}.W"] = W
        if M == 1:
            x = orc.gen_activations(K, xs, outl)
            arrays[f"{name}.x"] = x
            arrays[f"{name}.y"] = ref.gemv_fp64(W, x, K, N)
        else:
            X = orc.gen_activations(K * M, xs, outl).reshape(K, M)
            arrays[f"{name}.X_km"] = X
            arrays[f"{name}.Y"] = ref.gemm_fp64(W, X, K, N, M)
        arrays[f"{name}.dequant"] = ref.dequant(W, K, N)
        arrays[f"{name}.shape"] = np.array([K, N, M], np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
