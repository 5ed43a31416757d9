"""Writes the committed golden fixtures under tests/golden/ from the restated
reference packers (packers.py): GGUF bytes and the exactly recorded
coefficients of matrix_precision.rs:145-287 at the reference's K=512, N=33.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import packers as P  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    k, n = 512, 33
    for fmt in [P.F32, P.F16, P.BF16, P.Q4_0, P.Q4_1, P.Q8_0, P.Q4_K, P.Q5_K, P.Q6_K]:
        data, coeffs = P.dense_weights(fmt, n, k)
        np.savez_compressed(os.path.join(HERE, f"dense_{fmt}.npz"), k=k, n=n,
                            bytes=np.frombuffer(data, np.uint8),
                            coefficients=np.array([c for c, _ in coeffs]),
                            magnitudes=np.array([a for _, a in coeffs]),
                            input=P.dense_input(2, k))


if __name__ == "__main__":
    main()
