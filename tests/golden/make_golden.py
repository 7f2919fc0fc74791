"""Writes tests/golden/small_problem.npz: a small seeded problem and the oracle's answers.

    python tests/golden/make_golden.py

It is a regression fixture of the oracle (oracle/quant.py), which is itself pinned by
tests/test_oracle.py (test_golden_small_problem_regression re-derives every array bit for bit);
the GPU tests run the op on its inputs against its y_ref (test_golden_small_problem).  The reference
ships no vector files and its Python oracle is not executed here (every function is pinned by
closed forms, hand-derived known answers and exhaustive checks instead).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import quant  # noqa: E402


def main():
    rng = np.random.default_rng(2024)
    M, N, K, G = 5, 64, 512, 64
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    scales = rng.uniform(0.002, 0.05, (K // G, N)).astype(np.float16)
    x = rng.standard_normal((M, K)).astype(np.float16)
    Wp = quant.pack_int4(q)
    Wd = quant.dequantize_w4(q, scales, G)
    y = quant.ref_gemm(x, q, scales, G)
    np.savez_compressed(os.path.join(HERE, "small_problem.npz"), M=M, N=N, K=K, G=G, q=q, scales=scales,
                        x=x, Wp=Wp, Wd=Wd, y_ref=y)


if __name__ == "__main__":
    main()
