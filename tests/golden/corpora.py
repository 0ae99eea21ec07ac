"""Input corpora restated from the reference's own tests (data generators, not checks).

``float_sum_bound_corpus`` is the five-row adversarial corpus of
crates/unpopped/tests/kernel_parallel_reduction_float_sum_bound.rs:47-70 (benign positives, a
cancelling +-1e8 row, huge/tiny alternation scaled by 1e-20, 0.1 with no exact binary form,
mixed signs), drawn from the same LCG and seed, in the same per-column draw order.
"""
from __future__ import annotations

import numpy as np

MASK = (1 << 64) - 1


class Lcg:
    """kernel_parallel_reduction_float_sum_bound.rs:40-45: u = (s >> 11) / 2^53 after each step."""

    def __init__(self, state: int):
        self.s = state & MASK

    def __call__(self) -> float:
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & MASK
        return (self.s >> 11) / float(1 << 53)


def float_sum_bound_corpus(rows: int = 5, cols: int = 96) -> np.ndarray:
    lcg = Lcg(0x9E3779B97F4A7C15)
    v: list[float] = []
    for c in range(cols):
        v.append(1.0e-3 + 1.0e3 * lcg())
        big = 1.0e8 if c % 2 == 0 else -1.0e8
        v.append(1.0 + lcg() if c % 7 == 0 else big)
        huge = 1.0e30 if c % 2 == 0 else -1.0e30 * (1.0 + 1e-3 * lcg())
        v.append(huge * 1.0e-20)
        v.append(0.1)
        v.append((lcg() - 0.5) * 2.0e5)
    a = np.array(v, dtype=np.float64).reshape(cols, rows)  # pushed column by column
    return np.ascontiguousarray(a.T)


def dequant_gemm_fixture(signed: bool = True) -> dict:
    """The dequant-GEMM fixture of crates/unpopped/tests/support/dequant.rs:145-181 (R=4, K=8, C=4,
    GROUP=4): its data generators and its host answer, the fixture's own triple loop."""
    R, K, C, GROUP = 4, 8, 4, 4
    G = K // GROUP
    nib = [(r * 5 + k * 3 + 1) % 16 for r in range(R) for k in range(K)]
    packed = np.array([nib[i] | nib[i + 1] << 4 for i in range(0, len(nib), 2)], np.uint8)
    zero = np.array([(i % 3) - 1 for i in range(R * G)], np.int32)
    scale = np.array([1 + (i * 2 % 3) for i in range(R * G)], np.int32)
    x = np.array([(i * 7 % 9) - 4 for i in range(K * C)], np.int32)
    want = np.zeros((R, C), np.int64)
    for r in range(R):
        for c in range(C):
            for k in range(K):
                n = nib[r * K + k]
                n = n - 16 if signed and n >= 8 else n
                g = r * G + k // GROUP
                want[r, c] += (n - int(zero[g])) * int(scale[g]) * int(x[k * C + c])
    return {"rows": R, "k": K, "cols": C, "group": GROUP, "w_packed": packed, "zero": zero, "scale": scale,
            "x": x, "expected": want.astype(np.int32)}
