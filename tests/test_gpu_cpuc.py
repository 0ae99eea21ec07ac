"""GPU parity against the second reference: the reference's cpu-c C99 leg (restated in oracle/cpuc.*),
run on the same launched KernelFn the GPU lowers and on identical seeded inputs.

* Integer folds and scans, Max/Min, the gather, the dequant and the dequantizing GEMM: the HIP result
  equals the C99 result bit for bit.
* Float Sum: the C99 runs the launched lift's written order, the GPU its own device-class schedule; both
  are within the reference's declared bound of the exact sum (block_reduce.rs:14-24, per prefix for
  scans: kernel_parallel_scan_agrees.rs:287-300), so they differ by at most the two bounds.  On dyadic
  data every order is exact, and both equal RN32(exact) bit for bit.
* RowReduce at F32: the GPU follows the oracle (f64, one rounding per statement), the C leg rounds per
  operation: within 3 ulps plus exp's condition number, as in tests/test_cpuc.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import unpopped_amd as u
from oracle import cpuc
from oracle.cpuc import View
from unpopped_amd import expr as X
from unpopped_amd import forms as H
from unpopped_amd import synth

pytestmark = pytest.mark.gpu
LAUNCH = H.CALLER_LAUNCH
RNG = np.random.default_rng(31337)


def c_leg(k: dict, *args) -> None:
    assert cpuc.run(k, *args) == cpuc.OK


def gamma(n: int) -> float:
    uu = 2.0 ** -53
    return n * uu / (1 - n * uu)


def test_row_sum_max_matches_the_c_leg(hip_device):
    R, Cc = 48, 4096
    x = synth.normal_f32(1, R * Cc).reshape(R, Cc)
    s, m = H.reduce_rows(x, "Sum", op1="Max")
    cs, cm = np.zeros(R, np.float32), np.zeros(R, np.float32)
    c_leg(H.kernel_for(kind="row_reduce2", dtype="F32", rank=2), x, cs, cm, R, Cc)
    assert m.tobytes() == cm.tobytes()
    for r in range(R):
        a = np.abs(x[r].astype(np.float64)).sum()
        tol = 2 * gamma(Cc) * a + np.spacing(np.float32(abs(cs[r])))
        assert abs(float(s[r]) - float(cs[r])) <= tol, r
    xd = synth.uniform_pm1_f32(5, R * Cc).reshape(R, Cc)  # dyadic: every order is exact
    s, m = H.reduce_rows(xd, "Sum", op1="Max")
    c_leg(H.kernel_for(kind="row_reduce2", dtype="F32", rank=2), xd, cs, cm, R, Cc)
    assert s.tobytes() == cs.tobytes() and m.tobytes() == cm.tobytes()


@pytest.mark.parametrize("dtype", ["I32", "I64"])
def test_integer_row_folds_match_the_c_leg(hip_device, dtype):
    nt = np.int32 if dtype == "I32" else np.int64
    info = np.iinfo(nt)
    x = RNG.integers(info.min, info.max, (33, 1000), dtype=np.int64).astype(nt)
    for op in ("Sum", "Prod", "Max", "Min"):
        got = H.reduce_rows(x, op)
        want = np.zeros(33, nt)
        c_leg(H.kernel_for(kind="reduction", dtype=dtype, rank=2, op=op, reduced_from=1), x, want, 33, 1000)
        assert np.array_equal(got, want), op


@pytest.mark.parametrize("axes", [(0,), (0, 2), (1,)])
def test_axis_set_reductions_match_the_c_leg(hip_device, axes):
    x = RNG.integers(-10**6, 10**6, (24, 40, 36)).astype(np.int64)
    xf = RNG.standard_normal((24, 40, 36))
    kept = tuple(n for d, n in enumerate(x.shape) if d not in axes)
    for arr, dtype, op in ((x, "I64", "Sum"), (xf, "F64", "Max"), (xf, "F64", "Min")):
        got = H.reduce_axes(arr, axes, op)
        want = np.zeros(kept, arr.dtype)
        c_leg(H.kernel_for(kind="reduction", dtype=dtype, rank=3, op=op, axes=axes), arr, want, *arr.shape)
        assert got.tobytes() == want.tobytes(), (dtype, op)


def test_integer_scans_match_the_c_leg(hip_device):
    n = 1 << 18
    x = synth.int16_i32(2, n)
    k = H.kernel_for(kind="scan", dtype="I32", rank=2, op="Sum")
    got = H.scan_rows(x, "Sum")
    want = np.zeros(n, np.int32)
    c_leg(k, x.reshape(1, n), want.reshape(1, n), 1, n)
    assert np.array_equal(got, want)
    xl = RNG.integers(-2**40, 2**40, (4, 5000)).astype(np.int64)
    for op, exclusive, reverse in (("Max", False, False), ("Min", True, False), ("Sum", False, True)):
        got = H.scan_rows(xl, op, exclusive, reverse)
        want = np.zeros_like(xl)
        c_leg(H.kernel_for(kind="scan", dtype="I64", rank=2, op=op, exclusive=exclusive, reverse=reverse), xl, want,
              4, 5000)
        assert np.array_equal(got, want), (op, exclusive, reverse)


def test_f32_scan_matches_the_c_leg(hip_device):
    n = 1 << 16
    k = H.kernel_for(kind="scan", dtype="F32", rank=2, op="Sum")
    xd = synth.uniform_01_f32(2, n)  # dyadic
    got = H.scan_rows(xd, "Sum")
    want = np.zeros(n, np.float32)
    c_leg(k, xd.reshape(1, n), want.reshape(1, n), 1, n)
    assert got.tobytes() == want.tobytes()
    x = synth.normal_f32(3, n)
    got = H.scan_rows(x, "Sum")
    c_leg(k, x.reshape(1, n), want.reshape(1, n), 1, n)
    prefix_abs = np.cumsum(np.abs(x.astype(np.float64)))
    i = np.arange(1, n + 1)
    tol = 2 * (i * 2.0**-53 / (1 - i * 2.0**-53)) * prefix_abs + np.spacing(np.abs(want).astype(np.float32))
    assert (np.abs(got.astype(np.float64) - want) <= tol).all()


@pytest.mark.parametrize("index_dtype", ["I32", "I64", "U32"])
def test_gather_matches_the_c_leg(hip_device, index_dtype):
    V, D, N = 300, 192, 257
    table = synth.normal_bf16_bits(3, V * D, 0.02).reshape(V, D)
    nt = {"I32": np.int32, "I64": np.int64, "U32": np.uint32}[index_dtype]
    ids = RNG.integers(0, V + 40, N).astype(nt)
    for oob in ("Skip", "ZeroFill", "Clamp"):
        init = np.full((N, D), 0x1234, np.uint16)
        got = H.gather_rows(table, ids, oob, out_init=init, elem_kind="Bf16")
        want = init.copy()
        c_leg(H.kernel_for(kind="gather", dtype="Bf16", rank=2, index_dtype=index_dtype, oob=oob), table,
              View(ids, (N, D), (1, 0)), want, N, D, V)
        assert np.array_equal(got, want), oob


@pytest.mark.parametrize("q_kind,z_kind", [("U4", "U4"), ("I4", "I4")])
def test_dequant_matches_the_c_leg(hip_device, q_kind, z_kind):
    R, Cc, G = 24, 2048, 128
    q, z = synth.nibbles(4, R * Cc), synth.nibbles(41, R * Cc // G)
    s = synth.uniform_f16_bits(42, R * Cc // G, 0.001, 0.02)
    got = H.dequant4(q, s, z, R, Cc, G, q_kind, z_kind)
    want = np.zeros(R * Cc, np.uint16)
    c_leg(H.kernel_for(kind="dequant4", q_kind=q_kind, z_kind=z_kind, group=G), View(q, (R * Cc,), (1,)), s,
          View(z, (R * Cc // G,), (1,)), want, R, Cc)
    assert np.array_equal(got.ravel(), want)


@pytest.mark.parametrize("w_kind,xdt", [("U4", np.int32), ("I4", np.int8)])
def test_dequant_gemm_matches_the_c_leg(hip_device, w_kind, xdt):
    R, K, Cc, G = 70, 256, 68, 64
    w = synth.nibbles(5, R * K)
    zero = RNG.integers(-2**31, 2**31, R * K // G, dtype=np.int64).astype(np.int32)
    scale = RNG.integers(-2**31, 2**31, R * K // G, dtype=np.int64).astype(np.int32)
    info = np.iinfo(xdt)
    x = RNG.integers(info.min, info.max, K * Cc, dtype=np.int64).astype(xdt)
    got = H.dequant_gemm(w, zero, scale, x, R, K, Cc, G, w_kind=w_kind)
    want = np.zeros(R * Cc, np.int32)
    c_leg(H.kernel_for(kind="dequant_gemm", q_kind=w_kind, dtype="I32" if xdt == np.int32 else "I8", group=G),
          View(w, (R * K,), (1,)), zero, scale, x, want, R, K, Cc)
    assert np.array_equal(got.ravel(), want)


def test_softmax_matches_the_c_leg(hip_device):
    R, Cc = 16, 1000
    x = synth.normal_f32(7, R * Cc).reshape(R, Cc)
    stages, epi = X.softmax()
    got = H.row_reduce([x], stages, epi)
    want = np.zeros_like(x)
    c_leg(u.lift_row_reduce("row_reduce", "F32", 2, stages, epi, launch=LAUNCH), x, want, R, Cc)
    ia, ib = got.view(np.int32).astype(np.int64), want.view(np.int32).astype(np.int64)
    bound = 3 + np.ceil(np.abs(x - x.max(axis=1, keepdims=True)))
    assert (np.abs(ia - ib) <= bound).all()


def test_config1_data_on_the_gpu_equals_the_c_leg(hip_device):
    """BASELINE config 1's data (2^24 f32 uniform[-1,1) from seed 0): the GPU's full Sum, the C99 of the
    serial lift and the C99 of the launched lift all equal RN32 of the exact sum."""
    n = 1 << 24
    x = synth.uniform_pm1_f32(0, n)
    exact = np.float32(float(int(np.round(x.astype(np.float64) * 2.0**24).astype(np.int64).sum())) * 2.0**-24)
    assert H.reduce_all(x, "Sum") == exact
    for launch in (None, LAUNCH):
        out = np.zeros(1, np.float32)
        c_leg(u.lift_reduction("cfg1", "F32", 1, "Sum", launch=launch), x, View(out.reshape(()), (), ()), n)
        assert out[0] == exact, launch
