"""Seeded synthetic inputs (``csrc/synth.c``) as numpy arrays: the benchmark configurations'
distributions and seeds, generated identically for the GPU run and for the CPU checks."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

SYNTH_PATH = Path(__file__).resolve().parent / "libunpopped_synth.so"
_s = None


def _lib() -> C.CDLL:
    global _s
    if _s is None:
        if not SYNTH_PATH.exists():
            raise RuntimeError(f"{SYNTH_PATH} is not built: run unpopped_amd/build.py")
        L = C.CDLL(str(SYNTH_PATH))
        u64, i64, P, d = C.c_uint64, C.c_int64, C.c_void_p, C.c_double
        for name, args in {
            "unp_synth_uniform_pm1_f32": [u64, i64, P],
            "unp_synth_uniform_01_f32": [u64, i64, P],
            "unp_synth_int16_i32": [u64, i64, P],
            "unp_synth_normal_f32": [u64, i64, P],
            "unp_synth_normal_bf16": [u64, i64, d, P],
            "unp_synth_uniform_ids_i32": [u64, i64, i64, P],
            "unp_synth_zipf_ids_i32": [u64, i64, i64, d, P],
            "unp_synth_nibbles": [u64, i64, P],
            "unp_synth_uniform_f16": [u64, i64, d, d, P],
        }.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int if name == "unp_synth_zipf_ids_i32" else None
        _s = L
    return _s


def uniform_pm1_f32(seed: int, n: int) -> np.ndarray:
    a = np.empty(n, np.float32)
    _lib().unp_synth_uniform_pm1_f32(seed, n, a.ctypes.data)
    return a


def uniform_01_f32(seed: int, n: int) -> np.ndarray:
    a = np.empty(n, np.float32)
    _lib().unp_synth_uniform_01_f32(seed, n, a.ctypes.data)
    return a


def int16_i32(seed: int, n: int) -> np.ndarray:
    a = np.empty(n, np.int32)
    _lib().unp_synth_int16_i32(seed, n, a.ctypes.data)
    return a


def normal_f32(seed: int, n: int) -> np.ndarray:
    a = np.empty(n, np.float32)
    _lib().unp_synth_normal_f32(seed, n, a.ctypes.data)
    return a


def normal_bf16_bits(seed: int, n: int, sigma: float) -> np.ndarray:
    a = np.empty(n, np.uint16)
    _lib().unp_synth_normal_bf16(seed, n, sigma, a.ctypes.data)
    return a


def uniform_ids_i32(seed: int, n: int, rng: int) -> np.ndarray:
    a = np.empty(n, np.int32)
    _lib().unp_synth_uniform_ids_i32(seed, n, rng, a.ctypes.data)
    return a


def zipf_ids_i32(seed: int, n: int, rng: int, exponent: float) -> np.ndarray:
    a = np.empty(n, np.int32)
    if _lib().unp_synth_zipf_ids_i32(seed, n, rng, exponent, a.ctypes.data) != 0:
        raise ValueError("zipf range must be a power of two")
    return a


def nibbles(seed: int, n: int) -> np.ndarray:
    """``n`` values in [0, 16) packed two per byte, low nibble first."""
    a = np.empty((n + 1) // 2, np.uint8)
    _lib().unp_synth_nibbles(seed, n, a.ctypes.data)
    return a


def uniform_f16_bits(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    a = np.empty(n, np.uint16)
    _lib().unp_synth_uniform_f16(seed, n, lo, hi, a.ctypes.data)
    return a
