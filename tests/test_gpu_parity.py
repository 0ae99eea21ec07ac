"""GPU parity: every lowered form, launched through the C ABI on the MI355X, against the CPU
oracle on identical seeded inputs.

Bars (the north star's): bit-exact for integer folds and scans, gathers and the int4 dequant;
Max/Min bit-exact up to NaN payload and the sign of a zero (kernel_lift/block_reduce.rs:7-12);
float Sum/Mean within the declared bound gamma_(n-1) * sum|x| + 1/2 ulp + 4u|exact|
(kernel_lift/block_reduce.rs:14-24, tests/kernel_parallel_reduction_float_sum_bound.rs:188-214),
and bit-equal to the oracle whenever the data are dyadic (every partial sum exact in f64).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import unpopped_amd as u
from oracle import cpuc
from unpopped_amd import forms as H
from unpopped_amd import synth

RNG = np.random.default_rng(4242)

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def assert_sum_within_bound(x2d: np.ndarray, got: np.ndarray, mean=False):
    f32 = x2d.dtype == np.float32
    for r in range(x2d.shape[0]):
        xs = x2d[r].astype(np.float64)
        b = oracle.sum_bound(xs, float(got[r]), mean=mean, f32=f32)
        exact = oracle.neumaier(xs) / (xs.size if mean else 1)
        assert abs(float(got[r]) - exact) <= b, (r, float(got[r]), exact, b)


def equal_extremum(a, b):
    return np.array_equal(a, b, equal_nan=True)


# ---------------------------------------------------------------------------------------
# Row reductions
# ---------------------------------------------------------------------------------------

SHAPES = [(1, 1), (3, 5), (2, 64), (5, 255), (4, 256), (7, 1000), (3, 4096), (2, 100003), (300, 20), (0, 7), (4, 0)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["Sum", "Max", "Min", "Mean"])
def test_rowreduce_f32(hip_device, shape, op):
    H.say(f"[case] rowreduce f32 {op} {shape}")
    x = rng(1).normal(size=shape).astype(np.float32)
    got = H.reduce_rows(x, op)
    want = oracle.reduce_rows(x, op)
    if op in ("Max", "Min"):
        assert equal_extremum(got, want)
    elif shape[1] == 0:
        assert np.array_equal(got, want, equal_nan=True)
    else:
        assert_sum_within_bound(x, got, mean=(op == "Mean"))


@pytest.mark.parametrize("shape", [(3, 5), (5, 255), (7, 1000), (2, 100003)])
@pytest.mark.parametrize("op", ["Sum", "Max", "Min", "Mean"])
def test_rowreduce_f64(hip_device, shape, op):
    H.say(f"[case] rowreduce f64 {op} {shape}")
    x = rng(2).normal(size=shape)
    got = H.reduce_rows(x, op)
    want = oracle.reduce_rows(x, op)
    if op in ("Max", "Min"):
        assert equal_extremum(got, want)
    else:
        assert_sum_within_bound(x, got, mean=(op == "Mean"))


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("op", ["Sum", "Prod", "Max", "Min"])
@pytest.mark.parametrize("shape", [(3, 5), (4, 256), (7, 1001), (2, 70000)])
def test_rowreduce_int_bit_exact(hip_device, dtype, op, shape):
    H.say(f"[case] rowreduce {np.dtype(dtype).name} {op} {shape}")
    info = np.iinfo(dtype)
    x = rng(3).integers(info.min, info.max, size=shape, dtype=dtype, endpoint=True)
    x[0, 0] = info.min
    x[-1, -1] = info.max
    assert np.array_equal(H.reduce_rows(x, op), oracle.reduce_rows(x, op))


def test_rowreduce_nan_and_infinities(hip_device):
    H.say("[case] rowreduce f32 NaN/inf corpus")
    x = rng(4).normal(size=(6, 777)).astype(np.float32)
    x[0, 5] = np.nan
    x[1, 700] = np.inf
    x[2, 3] = -np.inf
    x[3, :] = np.nan
    x[4, 10] = np.inf
    x[4, 11] = -np.inf
    for op in ("Max", "Min"):
        assert equal_extremum(H.reduce_rows(x, op), oracle.reduce_rows(x, op)), op
    s = H.reduce_rows(x, "Sum")
    want = oracle.reduce_rows(x, "Sum")
    assert np.isnan(s[0]) and np.isnan(want[0])
    assert s[1] == want[1] == np.inf and s[2] == want[2] == -np.inf
    assert np.isnan(s[4]) and np.isnan(want[4])


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.int64])
@pytest.mark.parametrize("shape", [(3, 5), (7, 1000), (2, 70000), (1, 1 << 20)])
def test_sequential_only_folds_on_rows_and_whole_arrays(hip_device, dtype, shape):
    """The folds the reference lifts only sequentially: MaxNum/MinNum (NaN-ignoring) and, at the
    integers, And/Or/Xor, bit-exact against the oracle on the row schedule and the whole-array
    schedule; a float Prod in the serial lift's own order, bit-exact too."""
    is_int = dtype in (np.int32, np.int64)
    r = rng(47)
    if is_int:
        info = np.iinfo(dtype)
        x = r.integers(info.min, info.max, size=shape, dtype=dtype, endpoint=True)
        ops = ["And", "Or", "Xor", "MaxNum", "MinNum"]
    else:
        x = r.normal(size=shape).astype(dtype)
        x.ravel()[::5] = np.nan
        if shape[0] > 1:
            x[1, :] = np.nan  # a row of only NaN folds to NaN
        ops = ["MaxNum", "MinNum"] + (["Prod"] if x.size <= 70000 * 2 else [])
    for op in ops:
        H.say(f"[case] {op} rows {shape} {np.dtype(dtype).name}")
        xp = np.abs(x) + 0.5 if op == "Prod" else x  # keep the products finite and away from 0
        got = H.reduce_rows(xp, op)
        assert np.array_equal(got, oracle.reduce_rows(xp, op), equal_nan=True), op
        if x.size <= (1 << 20) and op != "Prod" or x.size <= 4096:
            H.say(f"[case] {op} all {x.size} {np.dtype(dtype).name}")
            got = H.reduce_all(np.ascontiguousarray(xp.ravel()), op)
            want = oracle.reduce_rows(np.ascontiguousarray(xp.reshape(1, -1)), op)[0]
            assert np.array_equal(np.array([got]), np.array([want]), equal_nan=True), op


def test_rowreduce_sum_max_fused_matches_two_folds(hip_device):
    H.say("[case] row_reduce2 sum+max f32 (129, 4096)")
    x = synth.normal_f32(1, 129 * 4096).reshape(129, 4096)
    s, m = H.reduce_rows(x, "Sum", op1="Max")
    assert equal_extremum(m, oracle.reduce_rows(x, "Max"))
    assert_sum_within_bound(x, s)


def test_rowreduce_dyadic_sum_is_bit_exact(hip_device):
    H.say("[case] rowreduce f32 dyadic Sum (64, 8192)")
    x = synth.uniform_pm1_f32(0, 64 * 8192).reshape(64, 8192)
    assert np.array_equal(H.reduce_rows(x, "Sum"), oracle.reduce_rows(x, "Sum"))


def test_reference_bound_corpus(hip_device):
    """The adversarial rows of the reference's bound test: cancellation, huge/tiny, mixed signs."""
    from tests.golden import corpora

    H.say("[case] rowreduce reference bound corpus")
    for dtype in (np.float32, np.float64):
        x = corpora.float_sum_bound_corpus().astype(dtype)
        for op in ("Sum", "Mean"):
            assert_sum_within_bound(x, H.reduce_rows(x, op), mean=(op == "Mean"))


# ---------------------------------------------------------------------------------------
# Full reductions (no kept axis)
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 3, 64, 1000, 65537, 1 << 20, (1 << 20) + 3])
def test_reduce_all_f32(hip_device, n):
    H.say(f"[case] reduce_all f32 n={n}")
    x = synth.uniform_pm1_f32(0, n)
    got = H.reduce_all(x, "Sum")
    assert got == oracle.reduce_rows(x.reshape(1, -1), "Sum")[0]  # dyadic: exact in any order
    for op in ("Max", "Min"):
        assert H.reduce_all(x, op) == oracle.reduce_rows(x.reshape(1, -1), op)[0]
    y = rng(5).normal(size=n).astype(np.float32)
    assert_sum_within_bound(y.reshape(1, -1), [H.reduce_all(y, "Sum")])


def test_reduce_all_int_and_f64(hip_device):
    H.say("[case] reduce_all i32/i64/f64")
    xi = rng(6).integers(-2**31, 2**31 - 1, size=300001, dtype=np.int32)
    for op in ("Sum", "Max", "Min", "Prod"):
        assert H.reduce_all(xi, op) == oracle.reduce_rows(xi.reshape(1, -1), op)[0], op
    xl = rng(7).integers(-2**63, 2**63 - 1, size=70001, dtype=np.int64)
    assert H.reduce_all(xl, "Sum") == oracle.reduce_rows(xl.reshape(1, -1), "Sum")[0]
    xd = rng(8).normal(size=123457)
    assert_sum_within_bound(xd.reshape(1, -1), [H.reduce_all(xd, "Mean")], mean=True)


def test_reduce_all_config1_full_size(hip_device):
    """Config 1's data: f32 Sum over 2^24 dyadic uniforms from seed 0: equal to RN32(exact)."""
    H.say("[case] reduce_all f32 config-1 2^24")
    x = synth.uniform_pm1_f32(0, 1 << 24)
    exact = x.astype(np.float64).sum()  # dyadic: every partial sum exact in f64
    got = H.reduce_all(x, "Sum")
    assert got == np.float32(exact)
    assert got == oracle.reduce_rows(x.reshape(1, -1), "Sum")[0]
    # launched twice: the same bits (the order is fixed by the geometry)
    assert H.reduce_all(x, "Sum") == got


# ---------------------------------------------------------------------------------------
# Scans
# ---------------------------------------------------------------------------------------

SCAN_N = [1, 2, 63, 64, 255, 256, 1023, 4096, 4097, 8191, 100000, (1 << 20) + 5]


@pytest.mark.parametrize("n", SCAN_N)
@pytest.mark.parametrize("exclusive", [False, True])
@pytest.mark.parametrize("reverse", [False, True])
def test_scan_i32_sum_bit_exact(hip_device, n, exclusive, reverse):
    H.say(f"[case] scan i32 Sum n={n} excl={exclusive} rev={reverse}")
    x = rng(9).integers(-2**31, 2**31 - 1, size=(1, n), dtype=np.int32)
    got = H.scan_rows(x, "Sum", exclusive, reverse)
    assert np.array_equal(got, oracle.scan_rows(x, "Sum", exclusive, reverse))


@pytest.mark.parametrize("op", ["Max", "Min", "Prod"])
@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_scan_int_other_folds(hip_device, op, dtype):
    H.say(f"[case] scan {np.dtype(dtype).name} {op}")
    for shape in [(1, 5000), (3, 777), (2, 65)]:
        x = rng(10).integers(-1000, 1000, size=shape, dtype=dtype)
        for excl in (False, True):
            assert np.array_equal(H.scan_rows(x, op, excl), oracle.scan_rows(x, op, excl)), (shape, excl)


@pytest.mark.parametrize("n", [1, 64, 4096, 4097, 50000, (1 << 20) + 7])
@pytest.mark.parametrize("exclusive", [False, True])
@pytest.mark.parametrize("reverse", [False, True])
def test_scan_f32_sum_dyadic_bit_exact(hip_device, n, exclusive, reverse):
    H.say(f"[case] scan f32 Sum dyadic n={n} excl={exclusive} rev={reverse}")
    x = synth.uniform_01_f32(2, n).reshape(1, n)
    got = H.scan_rows(x, "Sum", exclusive, reverse)
    assert np.array_equal(got, oracle.scan_rows(x, "Sum", exclusive, reverse))


def test_scan_f32_sum_within_bound(hip_device):
    H.say("[case] scan f32 Sum normal data, per-prefix bound")
    n = 300007
    x = rng(11).normal(size=(1, n)).astype(np.float32)
    got = H.scan_rows(x, "Sum").ravel().astype(np.float64)
    xs = x.ravel().astype(np.float64)
    exact = np.cumsum(xs)  # reference only; the bound below carries the slack
    u = 2.0 ** -53
    k = np.arange(n, dtype=np.float64)
    gamma = k * u / (1 - k * u)
    ulp = np.spacing(np.abs(got).astype(np.float32)).astype(np.float64)
    bound = gamma * np.cumsum(np.abs(xs)) + 0.5 * ulp + 4 * u * np.abs(exact) + 1e-300
    # np.cumsum in f64 has its own error; compare against the oracle's serial f64 order too
    want = oracle.scan_rows(x, "Sum").ravel().astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * bound)


def _repeat_within_bound(x, run, launches):
    """`launches` results of `run()` on the normal f32 row `x`, each checked against the declared
    per-prefix bound of the serial lift's f64 scan (kernel_parallel_scan_agrees.rs:287-300)."""
    n = x.shape[1]
    want = oracle.scan_rows(x, "Sum").ravel().astype(np.float64)
    xs = x.ravel().astype(np.float64)
    u53 = 2.0 ** -53
    k = np.arange(n, dtype=np.float64)
    gamma = k * u53 / (1 - k * u53)
    prefix_abs = np.cumsum(np.abs(xs))
    runs = []
    for _ in range(launches):
        got = run().ravel()
        g = got.astype(np.float64)
        ulp = np.spacing(np.abs(got)).astype(np.float64)
        assert np.all(np.abs(g - want) <= 2 * gamma * prefix_abs + ulp)
        runs.append(got)
    return runs


def test_scan_f32_repeat_launches_are_bit_identical(hip_device):
    """A lifted f32 Sum scan lowers the fixed schedule, whose carries fold tile aggregates in an
    association the tiling fixes: eight launches on the same normal data, over every CU, give the same
    bits (the reference's launched scan is reproducible too, kernel_lift/scan_launched.rs:22-27), each
    within the declared per-prefix bound.  On dyadic data every association is exact: the oracle's bits."""
    n = 1 << 24
    H.say(f"[case] scan f32 Sum (lower_kernel: fixed schedule), {n} normal values, 8 launches")
    x = rng(29).normal(size=(1, n)).astype(np.float32)
    runs = _repeat_within_bound(x, lambda: H.scan_rows(x, "Sum"), 8)
    assert all(r.tobytes() == runs[0].tobytes() for r in runs)
    xd = synth.uniform_pm1_f32(30, n).reshape(1, n)
    first = H.scan_rows(xd, "Sum")
    assert first.tobytes() == oracle.scan_rows(xd, "Sum").tobytes()
    for _ in range(2):
        assert H.scan_rows(xd, "Sum").tobytes() == first.tobytes()


def test_scan_f32_device_schedule_stays_within_the_bound(hip_device):
    """The device schedule, a Nondeterministic variant: its carry's association depends on how far
    each tile's look-back walked, which can change from launch to launch.  Eight launches on normal
    data are each within the declared per-prefix bound; the spread between launches is reported."""
    n = 1 << 24
    H.say(f"[case] scan f32 Sum on the device schedule, {n} normal values, 8 launches")
    x = rng(29).normal(size=(1, n)).astype(np.float32)
    ex = u.Executor(u.HipBackend().lower_form("scan", "F32", 2, "Sum", schedule="device"))
    din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(x.nbytes)

    def run():
        ex.launch(din, dout, 1, n)
        ex.check()
        return dout.download(np.float32, n)

    runs = _repeat_within_bound(x, run, 8)
    differ = max(int(np.count_nonzero(r != runs[0])) for r in runs)
    H.say(f"[case] device-schedule launches differ from the first in at most {differ} of {n} outputs")


def test_scan_f32_fixed_bits_per_entry(hip_device):
    """The fixed schedule's association is fixed by the entry's tile size, and the entry follows from
    the row's length and the buffers' alignment: the same normal values at a 16-byte-aligned address
    take the staged entry (18432-element tiles) and 4 bytes further on the register entry
    (16384-element tiles).  Each gives the same bits on every launch and stays within the bound; the
    two may differ from each other, and how many outputs do is reported."""
    n = 3 * (1 << 20)
    H.say(f"[case] fixed scan f32 Sum normal n={n}, aligned and at +4 bytes, two launches each")
    x = rng(61).normal(size=(1, n)).astype(np.float32)
    ex = H.executor(kind="scan", dtype="F32", rank=2, op="Sum")
    din, dout = u.DeviceBuffer(x.nbytes + 16), u.DeviceBuffer(x.nbytes + 16)
    got = {}
    for off in (0, 4):
        din.at(off).upload(x)

        def run():
            ex.launch(din.at(off), dout.at(off), 1, n)
            ex.check()
            return dout.at(off).download(np.float32, n)

        runs = _repeat_within_bound(x, run, 2)
        assert runs[0].tobytes() == runs[1].tobytes(), off
        got[off] = (ex.last_launch()["entry"], runs[0])
    assert got[0][0].endswith("_v") and got[4][0].endswith("_s"), (got[0][0], got[4][0])
    H.say(f"[case] the two entries differ in {int(np.count_nonzero(got[0][1] != got[4][1]))} of {n} outputs")


@pytest.mark.parametrize("op", ["Max", "Min"])
def test_scan_f32_extremum_with_nan(hip_device, op):
    H.say(f"[case] scan f32 {op} with NaN/inf")
    x = rng(12).normal(size=(2, 9000)).astype(np.float32)
    x[0, 4000] = np.nan
    x[1, 10] = np.inf
    x[1, 8000] = -np.inf
    for excl in (False, True):
        for rev in (False, True):
            assert equal_extremum(H.scan_rows(x, op, excl, rev), oracle.scan_rows(x, op, excl, rev))


@pytest.mark.parametrize("shape", [(3, 1000), (17, 4096), (5, 4097), (64, 3)])
def test_scan_multi_row(hip_device, shape):
    H.say(f"[case] scan multi-row {shape}")
    xi = rng(13).integers(0, 16, size=shape, dtype=np.int32)
    assert np.array_equal(H.scan_rows(xi, "Sum"), oracle.scan_rows(xi, "Sum"))
    xf = synth.uniform_01_f32(2, shape[0] * shape[1]).reshape(shape)
    assert np.array_equal(H.scan_rows(xf, "Sum"), oracle.scan_rows(xf, "Sum"))
    xd = rng(14).normal(size=shape)
    got = H.scan_rows(xd, "Sum")
    want = oracle.scan_rows(xd, "Sum")
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("exclusive", [False, True])
@pytest.mark.parametrize("reverse", [False, True])
def test_scan_many_tiles_several_rows(hip_device, exclusive, reverse):
    """Rows of many block tiles each: tickets run across row boundaries, look-backs stop at a
    row's first tile."""
    H.say(f"[case] scan i32 (4, 400000) excl={exclusive} rev={reverse}")
    x = rng(15).integers(-2**31, 2**31 - 1, size=(4, 400000), dtype=np.int32)
    assert np.array_equal(H.scan_rows(x, "Sum", exclusive, reverse), oracle.scan_rows(x, "Sum", exclusive, reverse))


@pytest.mark.parametrize("op", ["Sum", "Max", "Prod"])
def test_scan_eight_byte_staged(hip_device, op):
    """8-byte elements on the staged path (two status words per tile) over many tiles."""
    H.say(f"[case] scan i64/f64 {op} (2, 300000)")
    xi = rng(16).integers(-2**62, 2**62, size=(2, 300000), dtype=np.int64)
    for excl, rev in ((False, False), (True, True)):
        assert np.array_equal(H.scan_rows(xi, op, excl, rev), oracle.scan_rows(xi, op, excl, rev)), (excl, rev)
    if op == "Prod":
        return
    xf = synth.uniform_01_f32(5, 600000).astype(np.float64).reshape(2, 300000)  # dyadic: exact in f64
    for excl, rev in ((False, False), (True, True)):
        assert np.array_equal(H.scan_rows(xf, op, excl, rev), oracle.scan_rows(xf, op, excl, rev)), (excl, rev)


SCAN_AXES_CASES = [((64, 300), 0), ((3, 1000, 5), 1), ((5, 7, 300), 0), ((2, 3, 4, 5), 2), ((1000, 2), 0),
                   ((1, 4096, 64), 1), ((3, 0, 4), 1), ((6, 5), 1)]


@pytest.mark.parametrize("shape,axis", SCAN_AXES_CASES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.int64])
def test_scan_any_axis_bit_exact(hip_device, shape, axis, dtype):
    """The serial scan lift along any axis (lift_scan_opdef, kernel_lift.rs:504-519): a non-innermost
    axis, and a float Prod on any axis, run in the serial lift's own order and are bit-exact for every
    op, float Sum and Mean included; the innermost axis of the other folds takes the look-back scan."""
    is_int = dtype in (np.int32, np.int64)
    r = rng(48)
    if is_int:
        x = r.integers(-1000, 1000, size=shape, dtype=dtype)
    else:
        x = r.normal(size=shape).astype(dtype)
    inner = axis == len(shape) - 1
    for op in ("Sum", "Max", "Min", "Prod") + (() if is_int else ("Mean",)):
        for exclusive, reverse in ((False, False), (True, False), (False, True)):
            H.say(f"[case] scan axis {axis} of {shape} {np.dtype(dtype).name} {op} excl={exclusive} rev={reverse}")
            xs = (np.abs(x) * 0.5 + 0.75).astype(dtype) if op == "Prod" and not is_int else x
            got = H.scan_axis(xs, axis, op, exclusive, reverse)
            xm = np.ascontiguousarray(np.moveaxis(xs, axis, -1))
            rows = xm.reshape(-1, xm.shape[-1]) if xm.size else xm.reshape(0, max(xm.shape[-1], 0))
            want = np.moveaxis(oracle.scan_rows(rows, op, exclusive, reverse).reshape(xm.shape), -1, axis)
            if inner and not is_int and op in ("Sum", "Mean"):
                # the look-back scan: every prefix within the declared bound
                cols = xm.shape[-1]
                g2 = np.moveaxis(got, axis, -1).reshape(-1, cols).astype(np.float64)
                w2 = rows.astype(np.float64)
                for i in range(g2.shape[0]):
                    pre = np.cumsum(np.abs(w2[i][::-1] if reverse else w2[i]))
                    if exclusive:
                        pre = np.concatenate([[0.0], pre[:-1]])
                    n = np.arange(1, cols + 1, dtype=np.float64)
                    cnt = (n - 1 if exclusive else n) if op == "Mean" else np.ones(cols)
                    g = g2[i][::-1] if reverse else g2[i]
                    wv = np.moveaxis(want, axis, -1).reshape(-1, cols)[i].astype(np.float64)
                    wv = wv[::-1] if reverse else wv
                    tol = (2 * n * 2.0**-53 * pre) / np.maximum(cnt, 1) + np.spacing(np.abs(wv).astype(dtype))
                    ok = np.isnan(wv) | (np.abs(g - wv) <= tol)
                    assert ok.all(), (op, i)
            else:
                assert np.array_equal(got, want, equal_nan=True), op


def test_mean_scan_dyadic_is_bit_exact(hip_device):
    """A Mean scan on the innermost axis (the look-back scan, divided at the store): on dyadic data
    every f64 prefix is exact, so each output is the oracle's (prefix / count) rounded, bit for bit;
    an exclusive scan's first output is 0 / 0."""
    for n in (1, 4096, 50000, (1 << 20) + 3):
        x = dyadic(49, (n,), np.float32)
        for exclusive in (False, True):
            H.say(f"[case] mean scan n={n} excl={exclusive}")
            got = H.scan_rows(x, "Mean", exclusive)
            want = oracle.scan_rows(x.reshape(1, -1), "Mean", exclusive).ravel()
            assert np.array_equal(got, want, equal_nan=True)
            if exclusive:
                assert np.isnan(got[0])


def test_scan_unaligned_takes_the_register_path(hip_device):
    """A row whose extent is not a multiple of 16 bytes runs the register entry at size."""
    H.say("[case] scan i32 unaligned (1, 1000003)")
    x = rng(17).integers(-1000, 1000, size=(1, 1000003), dtype=np.int32)
    ex = H.executor(kind="scan", dtype="I32", rank=2, op="Sum")
    din = u.DeviceBuffer.from_array(x)
    dout = u.DeviceBuffer(x.nbytes)
    ex.launch(din, dout, 1, x.shape[1])
    u.synchronize()
    assert ex.last_launch()["entry"].endswith("_s")
    assert np.array_equal(dout.download(np.int32, x.size).reshape(x.shape), oracle.scan_rows(x, "Sum"))


WAIT_CASES = {
    # form, input, launch scalars from the input's shape; one launch spans every CU
    "scan_i32_staged": (dict(kind="scan", dtype="I32", rank=2, op="Sum"), lambda: rng(41).integers(
        -50, 50, size=(1, 1 << 24), dtype=np.int32), lambda x: oracle.scan_rows(x, "Sum")),
    "scan_i32_register": (dict(kind="scan", dtype="I32", rank=2, op="Max"), lambda: rng(42).integers(
        -1000, 1000, size=(1, (1 << 23) + 1), dtype=np.int32), lambda x: oracle.scan_rows(x, "Max")),
    "scan_f32_staged": (dict(kind="scan", dtype="F32", rank=2, op="Sum"),
                        lambda: synth.uniform_pm1_f32(43, 1 << 24).reshape(1, -1), lambda x: oracle.scan_rows(x, "Sum")),
    "scan_f32_register": (dict(kind="scan", dtype="F32", rank=2, op="Sum"),
                          lambda: synth.uniform_pm1_f32(47, (1 << 23) + 3).reshape(1, -1),
                          lambda x: oracle.scan_rows(x, "Sum")),
    "scan_f32_device": (dict(kind="scan", dtype="F32", rank=2, op="Sum", schedule="device"),
                        lambda: synth.uniform_pm1_f32(48, 1 << 24).reshape(1, -1), lambda x: oracle.scan_rows(x, "Sum")),
    "reduce_all": (dict(kind="reduction", dtype="I64", rank=1, op="Sum", reduced_from=0), lambda: rng(44).integers(
        -1 << 40, 1 << 40, size=1 << 22, dtype=np.int64), lambda x: np.array([oracle.reduce_rows(x.reshape(1, -1), "Sum")[0]])),
    "reduce_columns": (dict(kind="reduction", dtype="F32", rank=2, op="Max", axes=(0,)), lambda: rng(45).normal(
        size=(8192, 512)).astype(np.float32), lambda x: x.max(axis=0)),
}


@pytest.mark.parametrize("case", sorted(WAIT_CASES))
def test_a_wait_that_runs_out_is_reported_not_hung(hip_device, case):
    """Every wait of a kernel for another block is bounded.  With the bound at 0 a wait gives up at
    its first unanswered probe, so the launch still ends on the device; a launch whose output then
    differs from the oracle must have said so (``check`` raises Stalled).  With the default bound
    restored, the same executor is exact again and reports nothing."""
    form, make, want_of = WAIT_CASES[case]
    x = make()
    want = want_of(x)
    if "schedule" in form:  # a schedule the lifted kernel does not lower by default
        f = dict(form)
        ex = u.Executor(u.HipBackend().lower_form(f.pop("kind"), f.pop("dtype"), f.pop("rank"), f.pop("op"), **f))
    else:
        ex = u.Executor(H._backend.lower_kernel(H.kernel_for(**form)))
    din = u.DeviceBuffer.from_array(x)
    dout = u.DeviceBuffer(x.nbytes)
    outs = want.size

    def run():
        ex.launch(din, dout, *x.shape)
        u.synchronize()
        return dout.download(x.dtype, outs).reshape(want.shape)

    H.say(f"[case] wait bound 0: {case} {x.shape}")
    ex.set_wait_limit(0)
    for i in range(3):
        got = run()
        try:
            ex.check()
            stalled = False
        except u.UnpError as e:
            assert e.kind == "Stalled", e
            stalled = True
        exact = np.array_equal(got, want)
        H.say(f"[case] launch {i}: stalled={stalled} exact={exact}")
        assert stalled or exact
    ex.set_wait_limit(1_000_000)
    assert np.array_equal(run(), want)
    ex.check()


# ---- scans with a pre-map and a fused post ---------------------------------------------

def _eighths(seed, shape, dt=np.float32):
    """Multiples of 1/8 in [-12.5, 12.5): every product, partial sum and prefix of these stays exact,
    so every association of the fold gives the serial bits."""
    return (rng(seed).integers(-100, 100, size=shape) / 8).astype(dt)


def _scan_x_cases():
    from unpopped_amd import expr as X

    x0, x1, x2, r0 = X.input(0), X.input(1), X.input(2), X.reduced(0)
    # name: (dtype, shape, axis, op, exclusive, reverse, n_inputs, pre, post, data)
    return {
        "dev_sum_prod": (np.float32, (4, 5000), 1, "Sum", False, False, 2, x0 * x1, None, "eighths"),
        "dev_sum_excl_rev_post": (np.float32, (3, 70001), 1, "Sum", True, True, 2, x0 * x1, r0 - x0, "eighths"),
        "dev_sum_full_row": (np.float32, (1, 1 << 22), 1, "Sum", False, False, 2, x0 * x1, r0 - x0, "eighths"),
        "dev_max_three_inputs": (np.float64, (2, 33333), 1, "Max", False, False, 3, x0 * x1 + x2, r0 * x2, "normal"),
        "dev_min_sqrt_post": (np.float32, (5, 4096), 1, "Min", True, False, 2, x0 - x1, (r0 * r0).sqrt(), "normal"),
        "seq_mean_axis1": (np.float32, (6, 7, 9), 1, "Mean", False, False, 2, x0 + x1, r0 * 2.0, "normal"),
        "seq_sum_axis0": (np.float32, (300, 17), 0, "Sum", False, True, 1, x0 * x0, None, "normal"),
        "seq_prod": (np.float32, (4, 50), 1, "Prod", True, False, 1, x0 * 0.5 + 1.0, None, "normal"),
        "seq_max_f64_axis0": (np.float64, (40, 3, 5), 0, "Max", False, False, 2, x0 / x1, r0 - x1, "normal"),
    }


@pytest.mark.parametrize("case", sorted(_scan_x_cases()))
def test_scan_with_a_pre_and_a_post(hip_device, case):
    """Scans of n inputs with a pre-map and a fused post against orc_scan_x: bit-exact on every
    schedule (the data make every association of a Sum exact), Max/Min exact up to NaN payload; NaN and
    infinity from the pre (x / y with zeros) included.  The small serial cases are checked against the
    C99 leg of the same KernelFn too."""
    dt, shape, axis, op, excl, rev, n, pre, post, data = _scan_x_cases()[case]
    H.say(f"[case] scan with pre/post {case} {shape}")
    if data == "eighths":
        xs = [_eighths(60 + k, shape, dt) for k in range(n)]
    else:
        xs = [rng(60 + k).normal(size=shape).astype(dt) for k in range(n)]
        if n >= 2:
            xs[1].ravel()[::97] = 0.0  # x / 0: infinities and NaN from the pre
    got = H.scan_expr(xs, axis, op, pre, post, excl, rev)
    want = oracle.scan_expr(xs, axis, op, pre, post, excl, rev)
    assert np.array_equal(got, want, equal_nan=True)
    if case.startswith("seq") and int(np.prod(shape)) <= 4096:
        k = u.lift_scan("s", H.NP_KIND[dt], len(shape), op, axis=axis, exclusive=excl, reverse=rev, n_inputs=n,
                        pre=pre, post=post)
        out = np.zeros(shape, dt)
        assert cpuc.run(k, *xs, out, *shape) == cpuc.OK
        # C rounds each operation of a statement; the kernel evaluator once per statement
        close = np.isclose(out, want, rtol=4 * np.finfo(dt).eps, atol=0, equal_nan=True)
        assert close.all()


def test_scan_with_a_pre_within_the_bound_on_normal_data(hip_device):
    """A lifted Sum of x * y over 2^22 normal values (the fixed schedule, which lower_kernel takes for a
    float scan): every prefix within the declared per-prefix bound of the serial lift's f64 scan of the
    pre-mapped values, and four launches bit for bit the same."""
    from unpopped_amd import expr as X

    n = 1 << 22
    H.say(f"[case] scan with pre x*y, {n} normal values, 4 launches")
    x = rng(71).normal(size=(1, n)).astype(np.float32)
    y = rng(72).normal(size=(1, n)).astype(np.float32)
    first = H.scan_expr([x, y], 1, "Sum", X.input(0) * X.input(1))
    got = first.ravel().astype(np.float64)
    want = oracle.scan_expr([x, y], 1, "Sum", X.input(0) * X.input(1)).ravel().astype(np.float64)
    v = (x * y).ravel().astype(np.float64)
    k = np.arange(n, dtype=np.float64)
    gamma = k * 2.0 ** -53 / (1 - k * 2.0 ** -53)
    ulp = np.spacing(np.abs(got).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * gamma * np.cumsum(np.abs(v)) + ulp)
    for _ in range(3):
        assert H.scan_expr([x, y], 1, "Sum", X.input(0) * X.input(1)).tobytes() == first.tobytes()


def test_scan_repeated_launches_reuse_state(hip_device):
    """The look-back state is reused across launches (epoch tags): results stay exact."""
    H.say("[case] scan repeated launches")
    for i in range(5):
        n = [100000, 5000, 300000, 64, 4097][i]
        x = rng(20 + i).integers(-50, 50, size=(1, n), dtype=np.int32)
        assert np.array_equal(H.scan_rows(x, "Sum"), oracle.scan_rows(x, "Sum")), n


# ---------------------------------------------------------------------------------------
# Gather
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
@pytest.mark.parametrize("idx", [np.int32, np.int64, np.uint32])
def test_gather_policies(hip_device, oob, idx):
    H.say(f"[case] gather bf16 {oob} idx={np.dtype(idx).name}")
    V, D, N = 1000, 64, 517
    table = synth.normal_bf16_bits(3, V * D, 0.02).reshape(V, D)
    r = rng(15)
    ids = r.integers(0, V, size=N).astype(np.int64)
    ids[::7] = V + r.integers(0, 50, size=ids[::7].size)  # past the end
    if idx != np.uint32:
        ids[3::11] = -1 - r.integers(0, 50, size=ids[3::11].size)  # before the start
    ids = ids.astype(idx)
    init = np.full((N, D), 0x7777, np.uint16)  # Skip must leave these
    got = H.gather_rows(table, ids, oob, out_init=init, elem_kind="Bf16")
    want = oracle.gather_rows(table, ids, oob, out_init=init)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("D", [1, 3, 8, 9, 4096])
def test_gather_row_widths(hip_device, D):
    H.say(f"[case] gather widths D={D}")
    V, N = 300, 1000
    t16 = synth.normal_bf16_bits(3, V * D, 0.02).reshape(V, D)
    ids = rng(16).integers(-5, V + 5, size=N).astype(np.int32)
    assert np.array_equal(H.gather_rows(t16, ids, "ZeroFill", elem_kind="Bf16"),
                          oracle.gather_rows(t16, ids, "ZeroFill"))
    t32 = rng(17).normal(size=(V, D)).astype(np.float32)
    assert np.array_equal(H.gather_rows(t32, ids, "Clamp"), oracle.gather_rows(t32, ids, "Clamp"))


@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
def test_gather_many_rows_whole_row_path(hip_device, oob):
    """More output rows than waves, 8 KiB rows (the predicate-free whole-row path): each wave
    loads its next row's id ahead, across in-range and out-of-range ids."""
    H.say(f"[case] gather many rows {oob}")
    V, D, N = 300, 4096, 5001  # odd: a wave's last step has one live row of two
    table = synth.normal_bf16_bits(9, V * D, 0.02).reshape(V, D)
    ids = rng(18).integers(-40, V + 40, size=N).astype(np.int32)
    init = np.full((N, D), 0x1234, np.uint16)
    got = H.gather_rows(table, ids, oob, out_init=init, elem_kind="Bf16")
    assert np.array_equal(got, oracle.gather_rows(table, ids, oob, out_init=init))


@pytest.mark.parametrize("shape,axis", [((4, 300, 16), 1), ((3, 5, 4096), 1), ((8, 100), 1), ((2, 3, 50, 7), 2),
                                        ((64, 1000), 0), ((5, 9, 2048), 1), ((3, 40, 1), 1)])
@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
@pytest.mark.parametrize("idx", [np.int32, np.int64, np.uint32])
def test_gather_along_any_axis(hip_device, shape, axis, oob, idx):
    """index_select along any axis (OpDef::gather with a 1-D index, ir.rs:3838-3876; the gather lift's
    cell, gather.rs:184-232): bit-exact against the oracle, out-of-range ids under each policy."""
    H.say(f"[case] gather axis {axis} of {shape} {oob} {np.dtype(idx).name}")
    r = rng(50)
    t = r.integers(0, 2**16, size=shape, dtype=np.uint16)
    V = shape[axis]
    ids = r.integers(-3 if idx != np.uint32 else 0, V + 3, 37).astype(idx)
    out_shape = shape[:axis] + (37,) + shape[axis + 1:]
    init = r.integers(0, 2**16, size=out_shape, dtype=np.uint16)
    got = H.gather_axis(t, ids, axis, oob, out_init=init, elem_kind="Bf16")
    assert np.array_equal(got, oracle.gather_axis(t, ids, axis, oob, out_init=init))
    tf = r.normal(size=shape).astype(np.float32)
    got = H.gather_axis(tf, ids, axis, oob, out_init=init.astype(np.float32))
    assert np.array_equal(got, oracle.gather_axis(tf, ids, axis, oob, out_init=init.astype(np.float32)))


def test_gather_empty_source_zero_fills(hip_device):
    H.say("[case] gather empty source")
    table = np.zeros((1, 8), np.uint16)
    ids = np.array([0, 1, -1], np.int32)
    got = H.gather_rows(table, ids, "ZeroFill", out_init=np.full((3, 8), 5, np.uint16), src_extent=0,
                        elem_kind="Bf16")
    assert np.array_equal(got, np.zeros((3, 8), np.uint16))


# ---------------------------------------------------------------------------------------
# Dequant
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols,group", [(8, 256, 128), (3, 96, 32), (5, 100, 10), (2, 30, 7), (7, 4096, 128), (6, 240, 24), (3, 1000, 8),
                                             (4, 320, 96), (1, 32, 32), (37, 1152, 64), (1101, 4224, 128)])
@pytest.mark.parametrize("q_kind,z_kind", [("U4", "U4"), ("I4", "U4"), ("U4", "I4"), ("I4", "I4")])
def test_dequant_bit_exact(hip_device, rows, cols, group, q_kind, z_kind):
    H.say(f"[case] dequant {q_kind}/{z_kind} {rows}x{cols} g{group}")
    ng = -(-cols // group)
    q = synth.nibbles(4, rows * cols)
    z = synth.nibbles(5, rows * ng)
    s = synth.uniform_f16_bits(6, rows * ng, 0.001, 0.02)
    got = H.dequant4(q, s, z, rows, cols, group, q_kind, z_kind)
    want = oracle.dequant4_bf16(q, s, z, rows, cols, group, q_kind == "I4", z_kind == "I4")
    assert np.array_equal(got, want)


def test_dequant_special_scales(hip_device):
    """Negative, subnormal, zero, huge, infinite and NaN scales: the chain's exact value, one RNE."""
    H.say("[case] dequant special scales")
    rows, cols, group = 4, 256, 32
    ng = cols // group
    specials = np.array([0xBC00, 0x0001, 0x03FF, 0x0000, 0x8000, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x3555,
                         0xC7FF, 0x1400, 0x2E66, 0x8001, 0xFE01, 0x3C00] * 2, np.uint16)
    s = specials[: rows * ng]
    q = synth.nibbles(7, rows * cols)
    z = synth.nibbles(8, rows * ng)
    got = H.dequant4(q, s, z, rows, cols, group)
    want = oracle.dequant4_bf16(q, s, z, rows, cols, group)
    nan_g, nan_w = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_g, nan_w)
    assert np.array_equal(got[~nan_g], want[~nan_w])


# ---------------------------------------------------------------------------------------
# The dequantizing GEMM (crates/unpopped/tests/support/dequant.rs:104-181;
# tests/kernel_dequant_gemm.rs): I32 arithmetic that wraps, so every case is bit-exact.
# ---------------------------------------------------------------------------------------

def _gemm_data(seed, R, K, C, G, x_dtype, full_range=True):
    r = np.random.default_rng(seed)
    ng = -(-K // G)
    w = synth.nibbles(seed, R * K)
    lo, hi = (-2 ** 31, 2 ** 31) if full_range else (-3, 4)
    zero = r.integers(lo, hi, size=R * ng, dtype=np.int64).astype(np.int32)
    scale = r.integers(lo, hi, size=R * ng, dtype=np.int64).astype(np.int32)
    info = np.iinfo(x_dtype)
    x = r.integers(int(info.min), int(info.max) + 1, size=K * C, dtype=np.int64).astype(x_dtype)
    return w, zero, scale, x


def _gemm_entry(w_kind, x_dtype, group):
    kind = "I32" if x_dtype == np.int32 else "I8"
    return H.executor(kind="dequant_gemm", q_kind=w_kind, dtype=kind, group=group).last_launch()["entry"]


def _gemm_last_launch(w_kind, x_dtype, group):
    kind = "I32" if x_dtype == np.int32 else "I8"
    return H.executor(kind="dequant_gemm", q_kind=w_kind, dtype=kind, group=group).last_launch()


def test_dequant_gemm_reference_fixture(hip_device):
    """kernel_dequant_gemm.rs:26-49 on the fixture of support/dequant.rs:145-181 (R=4, K=8, C=4,
    GROUP=4): the host loop's answer for I4 and U4 weights, and the two differ."""
    H.say("[case] dequant GEMM reference fixture")
    R, K, C, GROUP = 4, 8, 4, 4
    G = K // GROUP
    nib = [(r * 5 + k * 3 + 1) % 16 for r in range(R) for k in range(K)]
    packed = np.array([nib[i] | nib[i + 1] << 4 for i in range(0, len(nib), 2)], np.uint8)
    zero = np.array([(i % 3) - 1 for i in range(R * G)], np.int32)
    scale = np.array([1 + (i * 2 % 3) for i in range(R * G)], np.int32)
    x = np.array([(i * 7 % 9) - 4 for i in range(K * C)], np.int32)
    answers = []
    for w_kind, signed in (("I4", True), ("U4", False)):
        want = np.zeros((R, C), np.int64)
        for r in range(R):
            for c in range(C):
                for k in range(K):
                    n = nib[r * K + k]
                    n = n - 16 if signed and n >= 8 else n
                    g = r * G + k // GROUP
                    want[r, c] += (n - int(zero[g])) * int(scale[g]) * int(x[k * C + c])
        got = H.dequant_gemm(packed, zero, scale, x, R, K, C, GROUP, w_kind=w_kind)
        assert np.array_equal(got, want), w_kind
        answers.append(got)
    assert not np.array_equal(answers[0], answers[1])


GEMM_MFMA_CASES = [
    # (R, K, C, group, x dtype): whole groups.  A group of 64-multiples takes the streaming
    # entry (split-K with atomics when the tiles are few), another 32-multiple the LDS-transpose
    # MFMA entry.
    (64, 128, 64, 128, np.int32),
    (130, 384, 132, 128, np.int32),   # ragged row and column tiles
    (70, 96, 68, 32, np.int32),       # one 32-deep step per group
    (65, 512, 36, 256, np.int32),     # several chunks per group
    (1, 256, 4, 64, np.int32),
    (130, 384, 132, 128, np.int8),
    (33, 2048, 12, 1024, np.int8),    # eight 128-deep chunks per group
    (200, 1152, 260, 96, np.int8),    # a 96-deep group: three steps
    (300, 4096, 64, 128, np.int32),   # split-K
    (257, 8192, 70, 128, np.int8),    # split-K, ragged columns
    (129, 6144, 33, 64, np.int32),    # split-K, 64-deep groups
    (257, 8192, 200, 128, np.int8),   # C > 128: streaming split-K
    # C <= 128 with groups of 1..4 128-deep steps (1..2 for I32) take a decode entry.
    (64, 128, 16, 128, np.int8),      # one group: one split, plain stores
    (130, 384, 13, 128, np.int32),    # ragged rows, C not a multiple of 16
    (257, 8192, 32, 128, np.int8),    # split-K, two column tiles per block
    (300, 4096, 1, 256, np.int32),    # one column, two steps per group
    (129, 6144, 20, 512, np.int8),    # four steps per group
    (70, 1152, 17, 384, np.int8),     # three steps per group
    (1100, 2048, 16, 128, np.int8),   # row tiles not a multiple of the eight XCDs
    (200, 4096, 60, 128, np.int8),    # four column tiles per block
    (96, 2048, 100, 256, np.int32),   # I32 decode past 64 columns
    (200, 4096, 100, 128, np.int8),   # I8 past 64 columns: streaming, 2 x 2 tiles per wave
    (300, 8192, 300, 256, np.int8),   # three 128-column tiles, the last partly padding
    (130, 4096, 150, 64, np.int8),    # 64-value chunks: four waves of one tile over 128 x 32
    (257, 8192, 200, 128, np.int32),  # I32 streaming: 1 x 2 tiles per wave, split-K, ragged last tile
    (96, 2048, 128, 256, np.int8),
    # I8 with C <= 16: eight waves of 256 rows per block with x' staged in LDS (32 steps at most).
    (300, 24576, 9, 384, np.int8),    # three steps per group, ten groups per split at most
    (513, 16384, 16, 512, np.int8),   # four steps per group, ragged 256-row tiles
    (40, 256, 1, 256, np.int8),       # one column, one split of one group
]


def _expected_gemm_entry(xdt, C, group):
    """The entry the executor takes for aligned operands: decode for groups of 1..4 whole
    128-deep steps (1..2 for I32) and C <= 64 (I8: the one-tile entry that stages x' in LDS for
    C <= 16, else the entry with 2 or 4 column tiles that first covers C) or C <= 128 (I32: the
    one-tile entry), then streaming for 64-multiples, then the MFMA entry."""
    spg = group // 128 if group % 128 == 0 else 0
    if C <= (64 if xdt == np.int8 else 128) and 1 <= spg <= (4 if xdt == np.int8 else 2):
        if xdt != np.int8:
            return "_dec1"
        return "_dec1x" if C <= 16 else "_dec2" if C <= 32 else "_dec4"
    return "_stream" if group % 64 == 0 else "_mfma"


@pytest.mark.parametrize("R,K,C,group,xdt", GEMM_MFMA_CASES)
@pytest.mark.parametrize("w_kind", ["U4", "I4"])
def test_dequant_gemm_mfma_bit_exact(hip_device, R, K, C, group, xdt, w_kind):
    H.say(f"[case] dequant GEMM mfma {w_kind} x {np.dtype(xdt).name} {R}x{K}x{C} g{group}")
    w, zero, scale, x = _gemm_data(R * 7 + K + C, R, K, C, group, xdt)
    got = H.dequant_gemm(w, zero, scale, x, R, K, C, group, w_kind=w_kind)
    assert _gemm_entry(w_kind, xdt, group).endswith(_expected_gemm_entry(xdt, C, group))
    want = oracle.dequant_gemm_i32(w, zero, scale, x, R, K, C, group, w_signed=w_kind == "I4")
    assert np.array_equal(got, want)


def test_dequant_gemm_repeated_launches_reuse_the_workspace(hip_device):
    """Shapes in a row on one executor, switching between the decode and streaming entries (the
    workspace grows, the split-K output is zeroed afresh each launch), then the first shape again."""
    H.say("[case] dequant GEMM repeated launches")
    for R, K, C in ((96, 2048, 16), (160, 4096, 96), (96, 2048, 16), (300, 8192, 24)):
        w, zero, scale, x = _gemm_data(R + K + C, R, K, C, 128, np.int8)
        got = H.dequant_gemm(w, zero, scale, x, R, K, C, 128, w_kind="I4")
        assert np.array_equal(got, oracle.dequant_gemm_i32(w, zero, scale, x, R, K, C, 128, w_signed=True))


@pytest.mark.parametrize("R,K,C,group,xdt", [
    (9, 100, 8, 32, np.int32),   # a ragged last group
    (17, 128, 5, 32, np.int32),  # C % 4 != 0 with 32-deep groups (64-multiples stream)
    (6, 70, 3, 7, np.int8),      # a group of 7: no MFMA entry
    (3, 0, 8, 64, np.int32),     # K = 0: all zeros
])
def test_dequant_gemm_serial_entry_bit_exact(hip_device, R, K, C, group, xdt):
    H.say(f"[case] dequant GEMM serial {np.dtype(xdt).name} {R}x{K}x{C} g{group}")
    w, zero, scale, x = _gemm_data(R + K * 3 + C, R, max(K, 1), C, group, xdt)
    w, x = w[: (R * K + 1) // 2] if K else w, x[: K * C] if K else np.zeros(max(C, 1), xdt)
    if K == 0:
        zero, scale = np.zeros(1, np.int32), np.zeros(1, np.int32)
    got = H.dequant_gemm(w, zero, scale, x, R, K, C, group, w_kind="I4")
    if K:
        assert _gemm_entry("I4", xdt, group).endswith("_any")
    want = oracle.dequant_gemm_i32(w, zero, scale, x, R, K, C, group, w_signed=True) if K else np.zeros((R, C), np.int32)
    assert np.array_equal(got, want)


def test_dequant_gemm_entries_agree_by_alignment(hip_device):
    """One shape through each entry: aligned operands stream; w 8 bytes off a 16-byte boundary
    takes the LDS-transpose MFMA entry; x one element off its 16-byte boundary as well, the
    serial entry.  All equal the oracle."""
    H.say("[case] dequant GEMM entries by alignment")
    R, K, C, G = 64, 256, 64, 64
    w, zero, scale, x = _gemm_data(11, R, K, C, G, np.int32)
    want = oracle.dequant_gemm_i32(w, zero, scale, x, R, K, C, G)
    ex = H.executor(kind="dequant_gemm", q_kind="U4", dtype="I32", group=G)
    dz, ds = (u.DeviceBuffer.from_array(a) for a in (zero, scale))
    dw, dx = u.DeviceBuffer.from_array(w), u.DeviceBuffer.from_array(x)
    dw8 = u.DeviceBuffer.from_array(np.concatenate([np.zeros(8, np.uint8), w]))
    dx4 = u.DeviceBuffer.from_array(np.concatenate([np.zeros(1, np.int32), x]))
    for wb, xb, entry in ((dw, dx, "_stream"), (dw8.at(8), dx, "_mfma"), (dw8.at(8), dx4.at(4), "_any")):
        do = u.DeviceBuffer(R * C * 4)
        do.fill(0x5A)
        ex.launch(wb, dz, ds, xb, do, R, K, C)
        u.synchronize()
        assert ex.last_launch()["entry"].endswith(entry)
        assert np.array_equal(do.download(np.int32, R * C).reshape(R, C), want), entry


# ---------------------------------------------------------------------------------------
# Reductions over any axis set (ReductionShape::new, kernel_lift.rs:854-870): an outer axis
# (column sums), a middle run, several runs.  The oracle folds rows of the input with the
# reduced axes moved last, which keeps the serial lift's row-major order over the reduced
# coordinates.
# ---------------------------------------------------------------------------------------

def oracle_axes(x: np.ndarray, axes: tuple, op: str):
    kept = [d for d in range(x.ndim) if d not in axes]
    xt = np.ascontiguousarray(np.transpose(x, kept + list(axes)))
    rows = int(np.prod([x.shape[d] for d in kept], dtype=np.int64))
    cols = int(np.prod([x.shape[d] for d in axes], dtype=np.int64))
    x2d = xt.reshape(rows, cols)
    return x2d, oracle.reduce_rows(x2d, op)


AXES_CASES = [((64, 300), (0,)), ((4096, 1024), (0,)), ((1000, 37), (0,)), ((3, 257, 129), (1,)),
              ((8, 2048, 512), (1,)), ((5, 37, 64), (0, 1)), ((4, 33, 7), (0, 2)), ((2, 3, 4, 5), (1, 2)),
              ((3, 4, 5, 6), (0, 3)), ((2, 3, 4, 5, 6), (0, 2, 4)), ((7, 1, 9), (1,)), ((0, 5), (0,)), ((5, 0, 3), (1,))]


@pytest.mark.parametrize("shape,axes", AXES_CASES)
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.int64])
@pytest.mark.parametrize("op", ["Sum", "Max", "Min", "Mean", "Prod", "MaxNum", "MinNum", "And", "Or", "Xor"])
def test_reduce_any_axes(hip_device, shape, axes, dtype, op):
    is_int = dtype in (np.int32, np.int64)
    H.say(f"[case] reduce axes {axes} of {shape} {np.dtype(dtype).name} {op}")
    r = rng(40)
    if is_int:
        info = np.iinfo(dtype)
        x = r.integers(info.min, info.max, size=shape, dtype=dtype, endpoint=True)
    else:
        x = r.normal(size=shape).astype(dtype)
        if op in ("MaxNum", "MinNum") and x.size:
            x.ravel()[::7] = np.nan  # skipped by the NaN-ignoring folds
    if (op == "Mean" and is_int) or (op in ("And", "Or", "Xor") and not is_int):
        # No lift: an integer Mean, a bit fold of a float (check_accumulated_dtype, kernel_lift.rs:763-800).
        with pytest.raises(u.UnpError) as e:
            H.reduce_axes(x, axes, op)
        assert e.value.kind == "LiftDecline"
        assert ("an integer Mean" if op == "Mean" else "a bit reduction at a float dtype") in e.value.detail
        return
    got = H.reduce_axes(x, axes, op)
    x2d, want = oracle_axes(x, axes, op)
    want = want.reshape(got.shape)
    if op in ("Sum", "Mean") and dtype in (np.float32, np.float64) and x2d.shape[1] > 0:
        assert_sum_within_bound(x2d, got.ravel(), mean=(op == "Mean"))
    else:
        assert np.array_equal(got, want, equal_nan=True)


@pytest.mark.parametrize("shape,axes", [((4096, 1024), (0,)), ((8, 2048, 512), (1,)), ((4, 33, 7), (0, 2))])
def test_reduce_any_axes_dyadic_sum_is_bit_exact_and_repeats(hip_device, shape, axes):
    """Dyadic data: every f64 partial is exact, so any order gives RN32(exact sum); two
    launches in a row (the split schedule's ticket counters are left at zero) agree bit for bit."""
    H.say(f"[case] reduce axes dyadic {axes} of {shape}")
    x = dyadic(41, shape, np.float32)
    a = H.reduce_axes(x, axes, "Sum")
    b = H.reduce_axes(x, axes, "Sum")
    _, want = oracle_axes(x, axes, "Sum")
    assert np.array_equal(a.ravel(), want.ravel())
    assert np.array_equal(a, b)


def test_reduce_any_axes_keepdim_and_nan(hip_device):
    H.say("[case] reduce axes keepdim, NaN column")
    x = rng(42).normal(size=(300, 3, 70)).astype(np.float32)
    x[17, 1, 5] = np.nan
    x[4, 2, 9] = np.inf
    got = H.reduce_axes(x, (0,), "Max", keepdim=True)
    assert got.shape == (1, 3, 70)
    _, want = oracle_axes(x, (0,), "Max")
    assert np.array_equal(got.ravel(), want.ravel(), equal_nan=True)
    assert np.isnan(got[0, 1, 5]) and got[0, 2, 9] == np.inf


# ---------------------------------------------------------------------------------------
# Reductions with a pre-map body over several inputs and a fused post (the reduction lift's
# body and post: kernel_lift.rs:807-831, 919-941, 987-1003; block_reduce.rs:292-307).  The
# oracle is the serial lifted row reduction with that one stage and the post as its epilogue,
# over the inputs with the reduced axes moved last.
# ---------------------------------------------------------------------------------------

def oracle_expr(inputs, axes, op, body, post):
    x0 = inputs[0]
    kept = [d for d in range(x0.ndim) if d not in axes]
    rows = int(np.prod([x0.shape[d] for d in kept], dtype=np.int64))
    cols = int(np.prod([x0.shape[d] for d in axes], dtype=np.int64))
    xs = [np.ascontiguousarray(np.transpose(a, kept + list(axes))).reshape(rows, cols) for a in inputs]
    full = oracle.row_reduce(xs, [(body, op)], X.reduced(0) if post is None else post)
    return xs, full[:, 0]


def xr_cases():
    x0, x1, r0 = X.input(0), X.input(1), X.reduced(0)
    return [
        ("sumsq_rows", [(37, 1000)], (1,), "Sum", x0 * x0, None),
        ("l2norm_rows", [(64, 4096)], (1,), "Sum", x0 * x0, r0.sqrt()),
        ("rms_rows", [(5, 777)], (1,), "Mean", x0 * x0, (r0 + X.konst(0.5)).sqrt()),
        ("dot_rows_unaligned", [(9, 1001)] * 2, (1,), "Sum", x0 * x1, None),
        ("dot_all", [(100003,)] * 2, (0,), "Sum", x0 * x1, None),
        ("dot_all_rank2", [(64, 4096)] * 2, (0, 1), "Sum", x0 * x1, r0 / X.konst(4.0)),
        ("weighted_cols", [(300, 70)] * 2, (0,), "Sum", x0 * x1 + x0, None),
        ("absmean_mid", [(6, 50, 9)], (1,), "Mean", x0.abs(), None),
        ("max_scaled_generic", [(4, 33, 7)], (0, 2), "Max", x0 - X.konst(1.0), r0 * X.konst(2.0)),
        ("min_three_inputs", [(11, 513)] * 3, (1,), "Min", x0 * x1 - x0, -r0),
    ]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", range(10))
def test_reduce_body_and_post_dyadic_bit_exact(hip_device, dtype, case):
    """Dyadic inputs: every body value and partial sum is exact in f64, so the device's fold
    order cannot move a bit, and the post (+, -, *, /, sqrt: correctly rounded) matches too."""
    name, shapes, axes, op, body, post = xr_cases()[case]
    H.say(f"[case] reduce body/post {name} {np.dtype(dtype).name}")
    ins = [dyadic(50 + k, sh, dtype) for k, sh in enumerate(shapes)]
    got = H.reduce_expr(ins, axes, op, body, post)
    _, want = oracle_expr(ins, axes, op, body, post)
    assert np.array_equal(got.ravel(), want, equal_nan=True)


@pytest.mark.parametrize("case", [0, 3, 4, 6])
def test_reduce_body_normal_data_within_bound(hip_device, case):
    """Normal data, no post: every output within the declared bound of the body values' sum."""
    name, shapes, axes, op, body, post = xr_cases()[case]
    H.say(f"[case] reduce body normal {name}")
    ins = [rng(60 + k).normal(size=sh).astype(np.float32) for k, sh in enumerate(shapes)]
    got = H.reduce_expr(ins, axes, op, body, post)
    xs, _ = oracle_expr(ins, axes, op, body, post)
    # The body's value at each position, evaluated in f64 and rounded once: the oracle's row
    # reduction with the body as its full-width epilogue.
    vals = oracle.row_reduce(xs, [(X.input(0), "Max")], body)
    assert_sum_within_bound(vals, got.ravel())


def test_reduce_body_and_post_launched_kernel_and_keepdim(hip_device):
    """The launched lift lowers to the same kernel; keepdim keeps size-1 axes."""
    H.say("[case] reduce body/post keepdim")
    x0, r0 = X.input(0), X.reduced(0)
    x = dyadic(70, (3, 40, 5), np.float32)
    got = H.reduce_expr([x], (1,), "Sum", x0 * x0, r0.sqrt(), keepdim=True)
    assert got.shape == (3, 1, 5)
    _, want = oracle_expr([x], (1,), "Sum", x0 * x0, r0.sqrt())
    assert np.array_equal(got.ravel(), want)


# ---------------------------------------------------------------------------------------
# Fused row reductions: the launched Access::RowReduce lift (softmax, RMS norm, ...)
#
# Bars: Max/Min stages bit-exact (kernel_parallel_row_reduce_agrees.rs:255-268); identity Sum/Mean
# epilogues within the declared bound (:270-303); F32 epilogues within 2 ulps of the serial lift
# (kernel_row_reduce_agrees.rs:25, :180-194); transcendental F64 epilogues within 4 ulps
# (kernel_parallel_row_reduce_agrees.rs:368-388) plus the Sum stage's own order term; same NaN cells.
# ---------------------------------------------------------------------------------------

from unpopped_amd import expr as X  # noqa: E402


def ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in representable values (+0 and -0 are one value); NaN against NaN is 0, NaN
    against a number is infinite."""
    it = np.int32 if a.dtype == np.float32 else np.int64
    lo = np.int64(np.iinfo(it).min)

    def key(x):
        k = x.view(it).astype(np.int64)
        with np.errstate(over="ignore"):
            return np.where(k < 0, lo - k, k)  # monotone in the value

    ka, kb = key(a), key(b)
    same = (ka >= 0) == (kb >= 0)
    with np.errstate(over="ignore"):
        d = np.where(same, np.abs(ka - kb).astype(np.float64), np.abs(ka.astype(np.float64) - kb.astype(np.float64)))
    an, bn = np.isnan(a), np.isnan(b)
    return np.where(an | bn, np.where(an == bn, 0.0, np.inf), d)


def gentle(rows, cols, dtype):
    """Values in [-2, 4] (kernel_parallel_row_reduce_agrees.rs:58-63)."""
    i = np.arange(rows * cols)
    return (((i * 7 + 3) % 19) * 0.37 - 2.0).astype(dtype).reshape(rows, cols)


def dyadic(seed, shape, dtype):
    """Every partial sum exact in f64 (and the mean a single rounding), so any order agrees."""
    return (rng(seed).integers(-64, 65, size=shape) / 8.0).astype(dtype)


RR_SHAPES = [(1, 1), (3, 13), (5, 96), (4, 256), (7, 1000), (3, 4096), (2, 8192), (2, 8200), (3, 20000),
             (2, 100003), (300, 20), (0, 7), (4, 0)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", RR_SHAPES)
def test_row_reduce_identity_epilogues(hip_device, dtype, shape):
    H.say(f"[case] row_reduce identity {np.dtype(dtype).name} {shape}")
    x = rng(31).normal(size=shape).astype(dtype) * 100
    for op in ("Sum", "Mean", "Max", "Min"):
        got = H.row_reduce([x], [(X.input(0), op)], X.reduced(0))
        want = oracle.row_reduce([x], [(X.input(0), op)], X.reduced(0))
        if x.size == 0:
            assert got.shape == want.shape
        elif op in ("Max", "Min"):
            assert equal_extremum(got, want), op
        else:
            assert (got == got[:, :1]).all()  # the stage result broadcast along the row
            assert_sum_within_bound(x, got[:, 0], mean=(op == "Mean"))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("which", ["rms_norm", "centred_quotient"])
@pytest.mark.parametrize("shape", [(3, 13), (5, 96), (9, 1000), (4, 8192), (2, 30000)])
def test_row_reduce_dyadic_rows_are_bit_exact(hip_device, dtype, which, shape):
    """With every partial sum exact the order cannot matter.  Centred quotient is then exact
    arithmetic and equals the oracle bit for bit; rms norm also takes a square root in f64,
    within 1 ulp at F32 and the 4 ulps of the transcendental bar at F64."""
    H.say(f"[case] row_reduce dyadic {which} {np.dtype(dtype).name} {shape}")
    x = dyadic(32, shape, dtype)
    stages, epi = getattr(X, which)()
    got = H.row_reduce([x], stages, epi)
    want = oracle.row_reduce([x], stages, epi)
    if which == "centred_quotient":
        assert np.array_equal(got, want, equal_nan=True)
    else:
        assert ulps(got, want).max() <= (1 if dtype == np.float32 else 4)


def f64_order_tolerance(x, want, which):
    """The Sum stage of softmax and the Mean of rms norm fold only nonnegative terms, so each
    order lies within gamma_(n-1) relative of the exact value; two orders differ by twice that."""
    n = x.shape[1]
    u = 2.0 ** -53
    g = (n - 1) * u / (1 - (n - 1) * u)
    rel = 2 * g if which == "softmax" else g  # x / sqrt(m): half the relative error of m
    return np.abs(want) * 2 * rel + 4 * np.spacing(np.abs(want))


@pytest.mark.parametrize("which", ["softmax", "rms_norm"])
@pytest.mark.parametrize("shape", [(5, 96), (3, 13), (64, 4096), (4, 20000), (2, 100003)])
def test_row_reduce_transcendental_epilogues(hip_device, which, shape):
    H.say(f"[case] row_reduce {which} {shape}")
    stages, epi = getattr(X, which)()
    for dtype in (np.float32, np.float64):
        x = gentle(*shape, dtype) if shape == (5, 96) else rng(33).normal(size=shape).astype(dtype) * 3
        got = H.row_reduce([x], stages, epi)
        want = oracle.row_reduce([x], stages, epi)
        if dtype == np.float32:
            assert ulps(got, want).max() <= 2, which
        else:
            far = ulps(got, want) > 4
            assert (np.abs(got - want)[far] <= f64_order_tolerance(x, want, which)[far]).all(), which


def test_row_reduce_centred_quotient_f32(hip_device):
    """The two-stage form on the reference's gentle rows and on wide rows."""
    stages, epi = X.centred_quotient()
    for x in (gentle(5, 96, np.float32), rng(34).normal(size=(16, 5000)).astype(np.float32)):
        H.say(f"[case] row_reduce centred quotient f32 {x.shape}")
        got = H.row_reduce([x], stages, epi)
        want = oracle.row_reduce([x], stages, epi)
        assert ulps(got, want).max() <= 2


def test_row_reduce_nan_and_infinity_rows(hip_device):
    """kernel_row_reduce_agrees.rs:232-264: the same cells are NaN, the rest within 2 ulps."""
    H.say("[case] row_reduce nan/inf rows")
    x = np.array([[1.0, np.nan, 2.0, 3.0], [np.inf, 1.0, 2.0, -np.inf], [0.0, -0.0, 1.0, 2.0]], np.float32)
    for stages, epi in (X.softmax(), X.centred_quotient()):
        for arr in (x, np.repeat(x, 64, axis=1)):  # the second takes the vector entry
            got = H.row_reduce([arr], stages, epi)
            want = oracle.row_reduce([arr], stages, epi)
            assert np.array_equal(np.isnan(got), np.isnan(want))
            assert ulps(got, want).max() <= 2


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", [(4099, 1000), (3333, 4096), (2049, 2000), (2050, 6000)])
def test_row_reduce_many_rows_per_block(hip_device, dtype, shape):
    """More rows than blocks (the grid is at most 8 per CU): each block takes several rows, its next
    row loaded while this one runs, the odd counts ending on either half of the two-row loop, and
    rows whose length leaves lanes past the end.  The shapes reach the four-vector and eight-vector
    register entries at both widths and, with 6000 f64 columns, the entry that re-reads the row.
    Same bars as the short rows."""
    _, cus = u.device_info()
    assert shape[0] > 8 * cus  # every block holds more than one row
    # The centred quotient's f64 bar is its dyadic bit-exact test; here it runs at F32.
    for which in ("softmax", "rms_norm") + (("centred_quotient",) if dtype == np.float32 else ()):
        H.say(f"[case] row_reduce many rows {which} {np.dtype(dtype).name} {shape}")
        stages, epi = getattr(X, which)()
        x = rng(38).normal(size=shape).astype(dtype) * 3
        got = H.row_reduce([x], stages, epi)
        want = oracle.row_reduce([x], stages, epi)
        if dtype == np.float32:
            assert ulps(got, want).max() <= 2, which
        else:
            far = ulps(got, want) > 4
            assert (np.abs(got - want)[far] <= f64_order_tolerance(x, want, which)[far]).all(), which


def test_row_reduce_two_inputs_many_rows(hip_device):
    """Two inputs through the two-row loop: 4000 rows of 300 (dyadic, so every order agrees)."""
    H.say("[case] row_reduce two inputs 40x100x300")
    a, b = dyadic(39, (40, 100, 300), np.float32), dyadic(40, (40, 100, 300), np.float32)
    stages = [(X.input(0) * X.input(1), "Sum"), (X.input(0) - X.reduced(0), "Max")]
    epi = X.fma(X.input(0), X.reduced(1), X.input(1) - X.reduced(0))
    got = H.row_reduce([a, b], stages, epi)
    want = oracle.row_reduce([a, b], stages, epi)
    assert np.array_equal(got, want)


def test_row_reduce_two_inputs_rank_three(hip_device):
    """Two inputs, rank 3 (rows are the product of the leading extents)."""
    H.say("[case] row_reduce two inputs rank 3")
    a, b = dyadic(35, (2, 3, 700), np.float32), dyadic(36, (2, 3, 700), np.float32)
    stages = [(X.input(0) * X.input(1), "Sum"), (X.input(0) - X.reduced(0), "Max")]
    epi = X.fma(X.input(0), X.reduced(1), X.input(1) - X.reduced(0))
    got = H.row_reduce([a, b], stages, epi)
    want = oracle.row_reduce([a, b], stages, epi)
    assert np.array_equal(got, want)


def test_row_reduce_entries_and_reproducibility(hip_device):
    """Each entry runs where it should, and a launch repeats bit for bit."""
    stages, epi = X.softmax()
    for shape, suffix in (((8, 4096), "_c4"), ((8, 6000), "_c"), ((8, 8196), "_v"), ((8, 4099), "_s")):
        H.say(f"[case] row_reduce entry {suffix} {shape}")
        x = rng(37).normal(size=shape).astype(np.float32)
        ex = H.row_reduce_executor("F32", 2, stages, epi)
        din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(x.nbytes)
        outs = []
        for _ in range(2):
            ex.launch(din, dout, *shape)
            u.synchronize()
            outs.append(dout.download(np.float32, x.size).reshape(shape))
        assert ex.last_launch()["entry"].endswith(suffix)
        assert np.array_equal(outs[0], outs[1])
        assert ulps(outs[0], oracle.row_reduce([x], stages, epi)).max() <= 2


# ---------------------------------------------------------------------------------------
# The benchmark configurations at full size
# ---------------------------------------------------------------------------------------

def test_config2_rowreduce_full(hip_device):
    H.say("[case] config 2: f32 8192x4096 sum+max")
    x = synth.normal_f32(1, 8192 * 4096).reshape(8192, 4096)
    s, m = H.reduce_rows(x, "Sum", op1="Max")
    assert np.array_equal(m, oracle.reduce_rows(x, "Max"))
    want = oracle.reduce_rows(x, "Sum")
    # f64 accumulation: equal to the serial result except where the f64 sums straddle an f32
    # rounding boundary; every row within the declared bound.
    assert np.mean(s == want) > 0.999
    bad = np.nonzero(s != want)[0]
    assert_sum_within_bound(x[bad], s[bad])


def test_config3a_i32_scan_full(hip_device):
    H.say("[case] config 3a: i32 inclusive scan 2^28")
    n = 1 << 28
    x = synth.int16_i32(2, n)
    got = H.scan_rows(x, "Sum")
    want = oracle.scan_rows(x.reshape(1, n), "Sum").ravel()
    assert np.array_equal(got, want)


def test_config3b_f32_scan_full(hip_device):
    H.say("[case] config 3b: f32 inclusive scan 2^26")
    n = 1 << 26
    x = synth.uniform_01_f32(2, n)
    got = H.scan_rows(x, "Sum")
    want = oracle.scan_rows(x.reshape(1, n), "Sum").ravel()
    assert np.array_equal(got, want)  # dyadic: every prefix exact in f64 -> RN32(exact)


@pytest.mark.parametrize("dist", ["uniform", "zipf"])
def test_config4_gather_full(hip_device, dist):
    H.say(f"[case] config 4: bf16 262144x4096 gather of 65536 ({dist})")
    V, D, N = 262144, 4096, 65536
    table = synth.normal_bf16_bits(3, V * D, 0.02).reshape(V, D)
    ids = synth.uniform_ids_i32(3, N, V) if dist == "uniform" else synth.zipf_ids_i32(3, N, V, 1.1)
    got = H.gather_rows(table, ids, "ZeroFill", elem_kind="Bf16")
    assert np.array_equal(got, table[ids])


@pytest.mark.parametrize("C,xdt,entry", [(16, np.int8, "_dec1x"), (64, np.int8, "_dec4"), (1024, np.int8, "_stream"),
                                          (16, np.int32, "_dec1"), (32, np.int32, "_dec1")])
def test_dequant_gemm_full_size(hip_device, C, xdt, entry):
    """The dequantizing GEMM at the bench's LLM shape (U4 w 8192 x 28672, full-range I32 zero
    points and scales per 128 columns), with sampled rows against the oracle: rows are
    independent, so the oracle runs on the sampled rows alone.  The samples include both edges
    of every 128-row tile (256 rows for the entry that stages x' in LDS) and a spread inside."""
    R, K, G = 8192, 28672, 128
    ng = K // G
    H.say(f"[case] dequant GEMM full size U4 {R}x{K} g{G} times {np.dtype(xdt).name} {K}x{C}")
    r = np.random.default_rng(C * 7 + np.dtype(xdt).itemsize)
    w = synth.nibbles(6, R * K)
    zero = r.integers(-2 ** 31, 2 ** 31, size=R * ng, dtype=np.int64).astype(np.int32)
    scale = r.integers(-2 ** 31, 2 ** 31, size=R * ng, dtype=np.int64).astype(np.int32)
    info = np.iinfo(xdt)
    x = r.integers(int(info.min), int(info.max) + 1, size=K * C, dtype=np.int64).astype(xdt)
    got = H.dequant_gemm(w, zero, scale, x, R, K, C, G)
    assert _gemm_entry("U4", xdt, G).endswith(entry)
    rows = sorted({0, R - 1, *range(127, R, 1024), *range(128, R, 1024), *r.integers(0, R, size=24).tolist()})
    half = K // 2
    for row in rows:
        want = oracle.dequant_gemm_i32(w[row * half:(row + 1) * half], zero[row * ng:(row + 1) * ng],
                                       scale[row * ng:(row + 1) * ng], x, 1, K, C, G)
        assert np.array_equal(got[row], want[0]), row


def test_config5_dequant_full(hip_device):
    H.say("[case] config 5: dequant 8192x28672 g128")
    R, Cc, G = 8192, 28672, 128
    q = synth.nibbles(4, R * Cc)
    z = synth.nibbles(41, R * (Cc // G))
    s = synth.uniform_f16_bits(42, R * (Cc // G), 0.001, 0.02)
    got = H.dequant4(q, s, z, R, Cc, G)
    want = oracle.dequant4_bf16(q, s, z, R, Cc, G)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------------------
# Buffers as storage images (unp_hip_exec_launch_views; TypedBuffer, oracle/buffers.rs:16-42)
# ---------------------------------------------------------------------------------------

def test_views_dense_with_base_match_the_pointer_launch(hip_device):
    """Dense row-major views at a base offset launch the kernel on data + base.  The results equal the
    pointer launch bit for bit."""
    H.say("[case] views: dense, base offset")
    R, Cc = 37, 300
    x = synth.normal_f32(11, R * Cc + 5)
    ex = H.executor(kind="row_reduce2", dtype="F32", rank=2, op="Sum", op1="Max")
    din = u.DeviceBuffer.from_array(x)
    a0, a1, b0, b1 = (u.DeviceBuffer(R * 4) for _ in range(4))
    ex.launch(din.at(20), a0, a1, R, Cc)
    ex.launch_views([(din, (R, Cc), None, 5), (b0, (R,), None, 0), (b1, (R,), (1,), 0)], [R, Cc])
    u.synchronize()
    assert np.array_equal(a0.download(np.float32, R), b0.download(np.float32, R))
    assert np.array_equal(a1.download(np.float32, R), b1.download(np.float32, R))
    assert np.array_equal(b1.download(np.float32, R), oracle.reduce_rows(x[5:].reshape(R, Cc), "Max"))


def test_views_gather_index_broadcast(hip_device):
    """The reference's embedding passes the ids as a broadcast [n, d] view with strides [1, 0]
    (tests/kernel_parallel_gather_agrees.rs:80-84); the table and the output are dense."""
    H.say("[case] views: gather index broadcast")
    V, D, n = 50, 64, 33
    table = (np.arange(V * D, dtype=np.uint16) * 7).reshape(V, D)
    ids = synth.uniform_ids_i32(12, n, V)
    ex = H.executor(kind="gather", dtype="Bf16", rank=2, index_dtype="I32", oob="ZeroFill")
    dt, di, do = u.DeviceBuffer.from_array(table), u.DeviceBuffer.from_array(ids), u.DeviceBuffer(n * D * 2)
    ex.launch_views([(dt, (V, D), None, 0), (di, (n, D), (1, 0), 0), (do, (n, D), None, 0)], [n, D, V])
    u.synchronize()
    assert np.array_equal(do.download(np.uint16, n * D).reshape(n, D), table[ids])


def _logical(storage: np.ndarray, shape, strides, base: int = 0) -> np.ndarray:
    """The numpy view a storage image names: ``storage``'s elements from ``base`` on, at the given
    extents and signed element strides (oracle/buffers.rs:16-42)."""
    flat = storage.reshape(-1)
    it = flat.itemsize
    return np.lib.stride_tricks.as_strided(flat[base:], shape=tuple(shape), strides=tuple(st * it for st in strides))


def _run_images(ex, images, scalars):
    """Upload each image's storage, launch through unp_hip_exec_launch_views, download every
    storage array (the outputs with whatever the launch left outside their views)."""
    bufs = [u.DeviceBuffer.from_array(st) for st, _, _, _ in images]
    ex.launch_views([(b, shape, strides, base) for b, (_, shape, strides, base) in zip(bufs, images)], scalars)
    u.synchronize()
    return [b.download(st.dtype, st.size).reshape(st.shape) for b, (st, _, _, _) in zip(bufs, images)]


def _expect(storage: np.ndarray, shape, strides, base, values) -> np.ndarray:
    """``storage`` with ``values`` written through the view (every other element unchanged)."""
    want = storage.copy()
    _logical(want, shape, strides, base)[...] = values
    return want


def _fold_axes(x: np.ndarray, axes, op: str) -> np.ndarray:
    """The oracle's fold of ``x`` over ``axes`` (row-major over the reduced axes), kept shape."""
    kept = [d for d in range(x.ndim) if d not in axes]
    m = np.ascontiguousarray(np.transpose(x, kept + list(axes)))
    outs = int(np.prod([x.shape[d] for d in kept], dtype=np.int64))
    return oracle.reduce_rows(m.reshape(outs, -1), op).reshape([x.shape[d] for d in kept])


STRIDED_REDUCTIONS = [
    # (dtype, op, storage shape, view shape, view strides, base, reduced axes)
    ("F32", "Sum", (300, 40), (40, 300), (1, 40), 0, (1,)),           # transposed
    ("F32", "Max", (300, 40), (40, 300), (1, 40), 0, (0,)),
    ("I64", "Sum", (12, 10, 18), (12, 10, 9), (180, -18, 2), 162, (0, 2)),  # reversed axis 1, every 2nd of axis 2
    ("I32", "Min", (12, 10, 18), (10, 12), (1, 180), 0, (1,)),        # a transposed slice
    ("F64", "Mean", (64, 33), (33, 64), (1, 33), 0, (0,)),
    ("F32", "Prod", (50, 21), (21, 50), (-1, 21), 20, (1,)),          # the serial product, reversed rows
    ("F32", "MaxNum", (40, 64), (40, 32), (64, -2), 63, (1,)),
    ("I64", "Xor", (16, 30), (30, 16), (1, 16), 0, (1,)),
]


@pytest.mark.parametrize("case", STRIDED_REDUCTIONS, ids=lambda c: f"{c[0]}-{c[1]}-{c[3]}-{c[4]}")
def test_reductions_read_through_view_strides(hip_device, case):
    """A reduction over a transposed, reversed or strided storage image reads through its strides: the
    result equals the oracle's fold of the logical array (bit for bit for integers, Max/Min/MaxNum, the
    serial Prod and dyadic data; float Sum/Mean within the declared bound on normal data), and the
    output, itself a strided view, leaves every other element of its storage untouched."""
    dtype, op, sshape, vshape, vstrides, base, axes = case
    H.say(f"[case] strided reduction {dtype} {op} view {vshape} strides {vstrides} base {base} axes {axes}")
    nt = {"F32": np.float32, "F64": np.float64, "I32": np.int32, "I64": np.int64}[dtype]
    n = int(np.prod(sshape))
    if dtype.startswith("F"):
        data = (synth.uniform_pm1_f32(17, n).astype(nt) if op != "Prod" else
                (1 + synth.uniform_pm1_f32(17, n) / 64).astype(nt))
        if op == "MaxNum":
            data[::5] = np.nan
    else:
        info = np.iinfo(nt)
        data = RNG.integers(info.min // 2, info.max // 2, n, dtype=np.int64).astype(nt)
    storage = data.reshape(sshape)
    x = _logical(storage, vshape, vstrides, base).copy()
    kept = [vshape[d] for d in range(len(vshape)) if d not in axes]
    want_vals = _fold_axes(x, axes, op)
    # The output: every 3rd element of a larger buffer, from element 1, reversed.
    outs = int(np.prod(kept, dtype=np.int64))
    ostore = np.full(3 * outs + 2, 7, nt)
    ostrides = [0] * len(kept)
    acc = -3
    for d in range(len(kept) - 1, -1, -1):
        ostrides[d], acc = acc, acc * kept[d]
    obase = 1 + 3 * (outs - 1)
    ex = H.executor(kind="reduction", dtype=dtype, rank=len(vshape), op=op, axes=axes)
    _, got = _run_images(ex, [(storage, vshape, vstrides, base), (ostore, kept, ostrides, obase)], list(vshape))
    want = _expect(ostore, kept, ostrides, obase, want_vals)
    if dtype.startswith("F") and op in ("Sum", "Mean"):
        # Dyadic data: every order of the f64 fold is exact, so the bits match.
        assert got.tobytes() == want.tobytes()
        xn = synth.normal_f32(18, n).astype(nt).reshape(sshape)
        _, got = _run_images(ex, [(xn, vshape, vstrides, base), (ostore, kept, ostrides, obase)], list(vshape))
        xl = _logical(xn, vshape, vstrides, base)
        g = _logical(got, kept, ostrides, obase)
        rows = np.transpose(xl, [d for d in range(len(vshape)) if d not in axes] + list(axes)).reshape(outs, -1)
        for r, gv in zip(rows, g.reshape(-1)):
            assert abs(float(gv) - oracle.neumaier(r) / (len(r) if op == "Mean" else 1)) <= \
                oracle.sum_bound(r, float(gv), mean=op == "Mean", f32=dtype == "F32")
        mask = np.ones(ostore.size, bool)
        _logical(mask, kept, ostrides, obase)[...] = False
        assert np.array_equal(got[mask], ostore[mask])
    else:
        assert got.tobytes() == want.tobytes()


def test_keepdim_output_and_fused_row_fold_through_strides(hip_device):
    """The keepdim output shape is accepted; the fused row fold (Sum + Max) reads a transposed input
    and writes both outputs through their own strides."""
    H.say("[case] strided keepdim reduction and row fold")
    R, Cc = 48, 96
    st = synth.uniform_pm1_f32(19, R * Cc).reshape(Cc, R)   # the view (R, Cc) is its transpose
    x = st.T.copy()
    ex = H.executor(kind="reduction", dtype="F32", rank=2, op="Max", axes=(1,), keepdim=True)
    o = np.zeros(2 * R, np.float32)
    _, got = _run_images(ex, [(st, (R, Cc), (1, R), 0), (o, (R, 1), (2, 5), 0)], [R, Cc])
    assert got.tobytes() == _expect(o, (R, 1), (2, 5), 0, oracle.reduce_rows(x, "Max").reshape(R, 1)).tobytes()
    ex2 = H.executor(kind="row_reduce2", dtype="F32", rank=2, op="Sum", op1="Max")
    o0, o1 = np.full(R, 3, np.float32), np.full(2 * R, 3, np.float32)
    _, g0, g1 = _run_images(ex2, [(st, (R, Cc), (1, R), 0), (o0, (R,), (-1,), R - 1), (o1, (R,), (2,), 1)], [R, Cc])
    assert g0.tobytes() == oracle.reduce_rows(x, "Sum")[::-1].tobytes()  # dyadic: exact
    assert g1.tobytes() == _expect(o1, (R,), (2,), 1, oracle.reduce_rows(x, "Max")).tobytes()


STRIDED_SCANS = [
    # (dtype, op, exclusive, reverse, storage shape, view shape, strides, base, axis)
    ("I32", "Sum", False, False, (500, 24), (24, 500), (1, 24), 0, 1),      # transposed, scan the long axis
    ("I64", "Max", True, False, (30, 200), (30, 200), (200, -1), 199, 1),   # reversed rows
    ("F32", "Sum", True, True, (8, 6, 70), (8, 70, 6), (420, 1, 70), 0, 1),  # non-innermost, transposed
    ("F64", "Mean", False, False, (40, 90), (45, 40), (2, 90), 0, 0),       # every 2nd of axis 0, transposed
    ("F32", "Prod", False, True, (64, 32), (32, 64), (1, 32), 0, 1),
]


@pytest.mark.parametrize("case", STRIDED_SCANS, ids=lambda c: f"{c[0]}-{c[1]}-{c[5]}-{c[6]}-ax{c[8]}")
def test_scans_read_through_view_strides(hip_device, case):
    """A scan over a transposed, reversed or strided storage image walks the scanned axis in the serial
    lift's order through the strides: bit-exact against the oracle's serial scan of the logical array for
    every op (float Sum too), the output written through its own strides."""
    dtype, op, excl, rev, sshape, vshape, vstrides, base, axis = case
    H.say(f"[case] strided scan {dtype} {op} excl={excl} rev={rev} view {vshape} strides {vstrides} axis {axis}")
    nt = {"F32": np.float32, "F64": np.float64, "I32": np.int32, "I64": np.int64}[dtype]
    n = int(np.prod(sshape))
    if op == "Prod":
        data = (1 + synth.normal_f32(21, n) / 32).astype(nt)
    elif dtype.startswith("F"):
        data = synth.normal_f32(21, n).astype(nt)
    else:
        data = RNG.integers(-2**20, 2**20, n).astype(nt)
    storage = data.reshape(sshape)
    x = _logical(storage, vshape, vstrides, base).copy()
    moved = np.ascontiguousarray(np.moveaxis(x, axis, -1))
    want_vals = np.moveaxis(oracle.scan_rows(moved.reshape(-1, moved.shape[-1]), op, excl, rev).reshape(moved.shape),
                            -1, axis)
    # The output: the transpose of a dense buffer of the view's reversed shape.
    ostore = np.full(vshape[::-1], 5, nt)
    ostrides = [int(np.prod(vshape[:d], dtype=np.int64)) for d in range(len(vshape))]
    ex = H.executor(kind="scan", dtype=dtype, rank=len(vshape), op=op, exclusive=excl, reverse=rev, axis=axis)
    _, got = _run_images(ex, [(storage, vshape, vstrides, base), (ostore, vshape, ostrides, 0)], list(vshape))
    assert got.tobytes() == _expect(ostore, vshape, ostrides, 0, want_vals).tobytes()


@pytest.mark.parametrize("index_dtype", ["I32", "I64", "U32"])
@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
def test_gather_with_a_full_shape_index_view(hip_device, index_dtype, oob):
    """The gather lift reads its index at every output coordinate (kernel_lift/gather.rs:184-232): a
    full-shape index view with a different id in every cell gathers element by element, equal to the
    oracle's per-cell gather and to the C99 leg on the same storage images."""
    H.say(f"[case] strided gather, full-shape index {index_dtype} {oob}")
    V, D, N = 40, 24, 33
    nt = {"I32": np.int32, "I64": np.int64, "U32": np.uint32}[index_dtype]
    table = synth.normal_bf16_bits(23, V * D, 0.02).reshape(V, D)
    lo = 0 if index_dtype == "U32" else -5
    ids = RNG.integers(lo, V + 5, (N, D)).astype(nt)
    init = np.full((N, D), 0x3C00, np.uint16)
    ex = H.executor(kind="gather", dtype="Bf16", rank=2, index_dtype=index_dtype, oob=oob)
    _, _, got = _run_images(ex, [(table, (V, D), (D, 1), 0), (ids, (N, D), (D, 1), 0), (init, (N, D), (D, 1), 0)],
                            [N, D, V])
    want = oracle.gather_cells(table, ids, 0, oob, out_init=init)
    assert np.array_equal(got, want)
    c = init.copy()
    assert cpuc.run(H.kernel_for(kind="gather", dtype="Bf16", rank=2, index_dtype=index_dtype, oob=oob), table, ids,
                    c, N, D, V) == cpuc.OK
    assert np.array_equal(got, c)


def test_gather_through_transposed_table_and_reversed_output(hip_device):
    """A transposed table, the broadcast index and a reversed output: read through the strides."""
    H.say("[case] strided gather, transposed table")
    V, D, N = 64, 48, 50
    tstore = synth.normal_bf16_bits(24, V * D, 0.02).reshape(D, V)  # the (V, D) table is its transpose
    ids = RNG.integers(-3, V + 3, N).astype(np.int64)
    init = np.full((N, D), 0x1111, np.uint16)
    for oob in ("Skip", "ZeroFill", "Clamp"):
        ex = H.executor(kind="gather", dtype="Bf16", rank=2, index_dtype="I64", oob=oob)
        _, _, got = _run_images(ex, [(tstore, (V, D), (1, V), 0), (ids, (N, D), (1, 0), 0),
                                     (init, (N, D), (-D, 1), (N - 1) * D)], [N, D, V])
        want = oracle.gather_rows(tstore.T.copy(), ids, oob, out_init=init[::-1].copy())[::-1]
        assert np.array_equal(got, want), oob


def test_gather_along_an_axis_of_a_longer_table(hip_device):
    """index_select along axis 1 from a table holding more rows along that axis than src_extent: the
    dense kernels step src_extent rows per slice, so the launch reads through the table's strides."""
    H.say("[case] strided gather, axis 1, table longer than src_extent")
    A, Vt, B, N, src = 6, 20, 10, 9, 15
    table = RNG.integers(0, 2**31, (A, Vt, B)).astype(np.int32)
    ids = RNG.integers(-2, src + 3, N).astype(np.int32)
    init = np.full((A, N, B), -7, np.int32)
    ex = H.executor(kind="gather", dtype="I32", rank=3, index_dtype="I32", oob="ZeroFill", axis=1)
    _, _, got = _run_images(ex, [(table, (A, Vt, B), (Vt * B, B, 1), 0), (ids, (A, N, B), (0, 1, 0), 0),
                                 (init, (A, N, B), (N * B, B, 1), 0)], [A, N, B, src])
    full = np.broadcast_to(ids.reshape(1, N, 1), (A, N, B))
    assert np.array_equal(got, oracle.gather_cells(table, full, 1, "ZeroFill", out_init=init, src_extent=src))


REFUSED_VIEWS = ["output shorter than the extents", "input of another shape", "wrong rank", "below the storage",
                 "overlapping dequant output", "table shorter than src_extent", "view count",
                 "overlapping output of a pre-map scan"]


@pytest.mark.parametrize("what", REFUSED_VIEWS)
def test_views_that_do_not_fit_are_refused(hip_device, what):
    """A view whose shape differs from what the form's extents ask for, that reaches below its storage,
    or that names an output element twice (a staged output would be unpacked over itself), is refused
    with INVALID_ARGUMENT before anything launches, and the output storage is untouched."""
    H.say(f"[case] views refused: {what}")
    if what == "overlapping dequant output":
        R, Cc, G = 4, 256, 128
        ex = H.executor(kind="dequant4", q_kind="U4", z_kind="U4", group=G)
        q, s, z = u.DeviceBuffer(R * Cc), u.DeviceBuffer(R * 2 * 2), u.DeviceBuffer(R)
        out = u.DeviceBuffer(2 * R * Cc * 2)
        out.fill(0x5A)
        views = [(q, (R * Cc,), None, 1), (s, (R * 2,), None, 0), (z, (R * 2,), None, 0),
                 (out, (R * Cc,), (0,), 0)]
        scalars = [R, Cc]
        check, nbytes = out, 2 * R * Cc * 2
    elif what == "overlapping output of a pre-map scan":
        from unpopped_amd import expr as X

        R, Cc = 8, 32
        ex = H.scan_expr_executor("F32", 2, "Sum", 1, X.input(0) * X.input(1), None, 2)
        a, b = u.DeviceBuffer(R * Cc * 4), u.DeviceBuffer(R * Cc * 4)
        out = u.DeviceBuffer(R * Cc * 4)
        out.fill(0x5A)
        views = [(a, (R, Cc), (1, R), 0), (b, (R, Cc), None, 0), (out, (R, Cc), (1, 1), 0)]
        scalars = [R, Cc]
        check, nbytes = out, R * Cc * 4
    elif what == "table shorter than src_extent":
        V, D, n = 10, 16, 5
        ex = H.executor(kind="gather", dtype="Bf16", rank=2, index_dtype="I32", oob="Clamp")
        t, i = u.DeviceBuffer(V * D * 2), u.DeviceBuffer(n * 4)
        out = u.DeviceBuffer(n * D * 2)
        out.fill(0x5A)
        views = [(t, (V, D), None, 0), (i, (n, D), (1, 0), 0), (out, (n, D), None, 0)]
        scalars = [n, D, V + 1]
        check, nbytes = out, n * D * 2
    else:
        R, Cc = 16, 64
        ex = H.executor(kind="row_reduce2", dtype="F32", rank=2, op="Sum", op1="Max")
        din = u.DeviceBuffer.from_array(synth.normal_f32(13, R * Cc))
        o0, o1 = u.DeviceBuffer(R * 4), u.DeviceBuffer(R * 4)
        o0.fill(0x5A)
        o1.fill(0x5A)
        iv, v0 = (din, (R, Cc), None, 0), (o0, (R,), None, 0)
        if what == "output shorter than the extents":
            v0 = (o0, (R - 1,), None, 0)
        elif what == "input of another shape":
            iv = (din, (R, Cc - 1), None, 0)
        elif what == "wrong rank":
            v0 = (o0, (1, R), None, 0)
        elif what == "below the storage":
            iv = (din, (R, Cc), (-Cc, 1), 0)
        views = [iv, v0, (o1, (R,), None, 0)]
        if what == "view count":
            views = views[:2]
        scalars = [R, Cc]
        check, nbytes = o0, R * 4
    with pytest.raises(u.UnpError) as e:
        ex.launch_views(views, scalars)
    assert e.value.kind == "InvalidArgument", e.value
    u.synchronize()
    assert np.all(check.download(np.uint8, nbytes) == 0x5A)

# ---- staged storage images: the forms whose kernels read dense storage ------------------

def _nibbles(storage_bytes: np.ndarray) -> np.ndarray:
    """The 4-bit elements of packed bytes, element 2i in the low nibble of byte i."""
    b = np.asarray(storage_bytes, np.uint8)
    return np.stack([b & 15, b >> 4], axis=1).reshape(-1)


def _pack(nib: np.ndarray) -> np.ndarray:
    n = np.asarray(nib, np.uint8)
    if n.size % 2:
        n = np.concatenate([n, np.zeros(1, np.uint8)])
    return (n[0::2] | (n[1::2] << 4)).astype(np.uint8)


def test_staged_views_of_a_pre_map_reduction(hip_device):
    """A float reduction with a body and a post over a transposed and a row-reversed input, into a
    strided output; and an integer-body reduction over a strided input: each equals the oracle on the
    logical arrays (dyadic data: bit for bit), with the output's other elements untouched."""
    H.say("[case] staged views: pre-map reduction")
    R, Cc = 33, 517
    x0s = dyadic(301, (Cc, R), np.float32)           # storage of the transposed input
    x1s = dyadic(302, (R, Cc), np.float32)           # rows reversed through a negative stride
    outs = np.full(2 * R + 1, 9.0, np.float32)
    body, post = X.input(0) * X.input(1) + X.input(0), X.reduced(0) * X.konst(0.5)
    ex = H.reduce_expr_executor("F32", 2, "Sum", (1,), body, post, 2)
    images = [(x0s, (R, Cc), (1, R), 0), (x1s, (R, Cc), (-Cc, 1), (R - 1) * Cc), (outs, (R,), (2,), 1)]
    got = _run_images(ex, images, [R, Cc])
    logical = [np.ascontiguousarray(_logical(st, sh, strd, b)) for st, sh, strd, b in images[:2]]
    _, want = oracle_expr(logical, (1,), "Sum", body, post)
    assert got[2].tobytes() == _expect(outs, (R,), (2,), 1, want).tobytes()
    assert ex.last_launch()["entry"].startswith(ex.kernel.name)
    # integer body, a strided input (every other column) and a reversed output
    xi = rng(303).integers(-1000, 1000, (R, 2 * Cc)).astype(np.int64)
    yi = rng(304).integers(-5, 5, (R, Cc)).astype(np.int64)
    oi = np.full(R, 77, np.int64)
    ibody = {"Div": [{"Mul": [{"Input": 0}, {"Input": 1}]}, {"Input": 1}]}
    k = u.lift_reduction("r", "I64", 2, "Sum", axes=(1,), n_inputs=2, body=ibody, launch=(256, 4))
    exi = u.Executor(u.HipBackend().lower_kernel(k))
    images = [(xi, (R, Cc), (2 * Cc, 2), 1), (yi, (R, Cc), None, 0), (oi, (R,), (-1,), R - 1)]
    got = _run_images(exi, images, [R, Cc])
    logical = [np.ascontiguousarray(_logical(st, sh, strd if strd else (Cc, 1), b)) for st, sh, strd, b in images[:2]]
    want = oracle.int_reduce_expr(logical, (1,), "Sum", ibody, "I64")
    assert got[2].tobytes() == want[::-1].tobytes()


def test_staged_views_of_a_pre_map_scan(hip_device):
    """A scan with a pre and a post over a transposed input and a strided one, into an output whose
    columns run backwards: the oracle's scan of the logical arrays (dyadic: bit for bit), the rest of
    the output storage untouched."""
    H.say("[case] staged views: pre-map scan")
    R, Cc = 7, 3001
    x0s = _eighths(311, (Cc, R))
    x1s = _eighths(312, (R, 2 * Cc))
    outs = np.full((R, Cc + 3), -4.0, np.float32)
    pre, post = X.input(0) * X.input(1), X.reduced(0) - X.input(0)
    ex = H.scan_expr_executor("F32", 2, "Sum", 1, pre, post, 2)
    oview = ((R, Cc), (Cc + 3, -1), Cc + 1)
    images = [(x0s, (R, Cc), (1, R), 0), (x1s, (R, Cc), (2 * Cc, 2), 0), (outs, *oview)]
    got = _run_images(ex, images, [R, Cc])
    logical = [np.ascontiguousarray(_logical(st, sh, strd, b)) for st, sh, strd, b in images[:2]]
    want = oracle.scan_expr(logical, 1, "Sum", pre, post)
    assert got[2].tobytes() == _expect(outs, *oview, want).tobytes()


def test_staged_views_of_a_row_reduce(hip_device):
    """Softmax over a transposed input into a row-strided output: bit for bit the dense launch on the
    logical array (the same kernels on the staged copy), within the row-reduce bars of the oracle."""
    H.say("[case] staged views: row reduce")
    R, Cc = 19, 1000
    xs = rng(321).normal(size=(Cc, R)).astype(np.float32)
    x0, r0, r1 = X.input(0), X.reduced(0), X.reduced(1)
    stages = [(x0, "Max"), ((x0 - r0).exp(), "Sum")]
    epi = (x0 - r0).exp() / r1
    ex = H.row_reduce_executor("F32", 2, stages, epi)
    outs = np.full((R, Cc + 8), 3.0, np.float32)
    images = [(xs, (R, Cc), (1, R), 0), (outs, (R, Cc), (Cc + 8, 1), 4)]
    got = _run_images(ex, images, [R, Cc])
    logical = np.ascontiguousarray(xs.T)
    dense = H.row_reduce([logical], stages, epi)
    assert got[1].tobytes() == _expect(outs, (R, Cc), (Cc + 8, 1), 4, dense).tobytes()
    want = oracle.row_reduce([logical], stages, epi)
    assert np.allclose(dense, want, rtol=1e-6, atol=0)


def test_staged_views_of_the_dequant(hip_device):
    """The int4 dequant with its weights every other nibble from an odd base, its scales reversed, its
    zero points strided, into every other bf16 of the output: the oracle on the logical arrays, bit for
    bit, and the output's other elements untouched."""
    H.say("[case] staged views: dequant4")
    R, Cc, G = 12, 384, 128
    ng = Cc // G
    r = rng(331)
    qst = r.integers(0, 256, R * Cc, dtype=np.uint8)       # 2 R C nibbles; the view takes 1, 3, 5, ...
    sst = np.array([0x3C00 + int(v) for v in r.integers(-600, 600, R * ng)], np.uint16)
    zst = r.integers(0, 256, R * ng, dtype=np.uint8)       # 2 R ng nibbles; the view takes every other
    outs = np.full(2 * R * Cc, 0x5A5A, np.uint16)
    ex = H.executor(kind="dequant4", q_kind="U4", z_kind="U4", group=G)
    dq, ds, dz, do = (u.DeviceBuffer.from_array(a) for a in (qst, sst, zst, outs))
    ex.launch_views([(dq, (R * Cc,), (2,), 1), (ds, (R * ng,), (-1,), R * ng - 1), (dz, (R * ng,), (2,), 0),
                     (do, (R * Cc,), (2,), 1)], [R, Cc])
    u.synchronize()
    got = do.download(np.uint16, outs.size)
    q_log = _pack(_nibbles(qst)[1::2][: R * Cc])
    s_log = sst[::-1].copy()
    z_log = _pack(_nibbles(zst)[0::2][: R * ng])
    want = oracle.dequant4_bf16(q_log, s_log, z_log, R, Cc, G)
    assert got[1::2].tobytes() == want.tobytes()
    assert np.all(got[0::2] == 0x5A5A)


def test_staged_views_of_the_dequant_gemm(hip_device):
    """The dequant GEMM with reversed weights (a negative stride over the nibbles), strided activations
    and a strided output: the oracle on the logical arrays, bit for bit."""
    H.say("[case] staged views: dequant GEMM")
    R, K, C, G = 32, 256, 16, 64
    w, zero, scale, x = _gemm_data(341, R, K, C, G, np.int32)
    wn = _nibbles(w)[: R * K]
    wst = _pack(wn[::-1])                                   # storage holds the nibbles backwards
    xst = np.zeros(2 * K * C, np.int32)
    xst[0::2] = x
    outs = np.full(3 * R * C, 11, np.int32)
    ex = H.executor(kind="dequant_gemm", q_kind="U4", dtype="I32", group=G)
    dw, dz, ds, dx, do = (u.DeviceBuffer.from_array(a) for a in (wst, zero, scale, xst, outs))
    ex.launch_views([(dw, (R * K,), (-1,), R * K - 1), (dz, (R * (K // G),), None, 0),
                     (ds, (R * (K // G),), None, 0), (dx, (K * C,), (2,), 0), (do, (R * C,), (3,), 2)], [R, K, C])
    u.synchronize()
    got = do.download(np.int32, outs.size)
    want = oracle.dequant_gemm_i32(w, zero, scale, x, R, K, C, G)
    assert got[2::3].tobytes() == want.reshape(-1).tobytes()
    assert np.all(got[0::3] == 11) and np.all(got[1::3] == 11)


# ---------------------------------------------------------------------------------------
# Launch geometry: a device-class grid, never derived from an extent (PATENT-SWEEP.md:269)
# ---------------------------------------------------------------------------------------

def test_raw_launch_and_timed_launch(hip_device):
    """The consumer's launch layer: a kernel compiled, loaded and launched with a packed argument
    block through unp_hip_launch and unp_hip_launch_timed.  The timed launch's events bracket the
    kernel, and a geometry past 2^32 work-items is refused before anything is launched."""
    import ctypes as C

    from unpopped_amd import _lib

    L = _lib.lib()
    src = ('extern "C" __global__ void __launch_bounds__(256) fill(unsigned* o, unsigned n, unsigned v) {\n'
           '  const unsigned i = blockIdx.x * 256 + threadIdx.x;\n  if (i < n) o[i] = v + i;\n}\n')
    co = u.HipCompiler().compile(src, "fill")
    img = C.create_string_buffer(co, len(co))
    m, f, err = C.c_void_p(), C.c_void_p(), _lib.Error()
    _lib.check(L.unp_hip_module_load(img, len(co), C.byref(m), C.byref(err)), err)

    class Args(C.Structure):
        _fields_ = [("o", C.c_uint64), ("n", C.c_uint32), ("v", C.c_uint32)]

    try:
        _lib.check(L.unp_hip_get_function(m, b"fill", C.byref(f), C.byref(err)), err)
        n = 100_003
        out = u.DeviceBuffer(4 * n)
        grid, block = (C.c_uint32 * 3)((n + 255) // 256, 1, 1), (C.c_uint32 * 3)(256, 1, 1)
        H.say("[case] raw launch")
        a = Args(out.ptr, n, 7)
        _lib.check(L.unp_hip_launch(f, grid, block, 0, None, C.byref(a), C.sizeof(a), C.byref(err)), err)
        u.synchronize()
        assert (out.download(np.uint32, n) == 7 + np.arange(n, dtype=np.uint32)).all()
        H.say("[case] timed raw launch")
        e0, e1 = u.Event(), u.Event()
        b = Args(out.ptr, n, 1000)
        _lib.check(L.unp_hip_launch_timed(f, grid, block, 0, None, C.byref(b), C.sizeof(b), e0._h, e1._h,
                                          C.byref(err)), err)
        e1.synchronize()
        assert 0.0 < e0.elapsed_ms(e1) < 100.0
        assert (out.download(np.uint32, n) == 1000 + np.arange(n, dtype=np.uint32)).all()
        # 2^24 blocks of 256 work-items: more than hipExtModuleLaunchKernel's 32-bit work-item count.
        too_big = (C.c_uint32 * 3)(1 << 24, 1, 1)
        rc = L.unp_hip_launch_timed(f, too_big, block, 0, None, C.byref(b), C.sizeof(b), None, None, C.byref(err))
        assert rc == _lib.INVALID_ARGUMENT
    finally:
        L.unp_hip_module_unload(m)


def test_grids_do_not_follow_the_extents(hip_device):
    """Every reduction, scan, gather and row-reduce launch takes the same grid whatever its extents:
    a multiple of the CU count fixed by the entry (blocks past the work exit)."""
    _, cus = u.device_info()
    cases = [
        (dict(kind="reduction", dtype="F32", rank=2, op="Sum", reduced_from=1), [(3, 8), (5000, 4096)]),
        (dict(kind="reduction", dtype="F32", rank=2, op="Sum", axes=(0,)), [(40, 8), (8192, 4096)]),
        (dict(kind="reduction", dtype="I64", rank=3, op="Max", axes=(0, 2)), [(2, 3, 4), (64, 500, 64)]),
        (dict(kind="reduction", dtype="F32", rank=2, op="Prod", axes=(1,)), [(2, 5), (3000, 64)]),
        (dict(kind="scan", dtype="F64", rank=2, op="Sum", axis=0), [(4, 3), (2000, 3000)]),
        (dict(kind="row_reduce2", dtype="F32", rank=2, op="Sum", op1="Max"), [(2, 64), (4096, 1024)]),
    ]
    for form, shapes in cases:
        ex = H.executor(**form)
        grids = set()
        for shape in shapes:
            nt = np.int64 if form["dtype"] == "I64" else (np.float64 if form["dtype"] == "F64" else np.float32)
            x = np.ones(shape, nt)
            kept = [n for d, n in enumerate(shape) if d not in (form.get("axes") or (len(shape) - 1,))]
            outs = int(np.prod(kept)) if form["kind"] != "scan" else x.size
            din = u.DeviceBuffer.from_array(x)
            bufs = [u.DeviceBuffer(max(outs, 1) * x.itemsize) for _ in range(2 if form["kind"] == "row_reduce2" else 1)]
            H.say(f"[case] grid {form} {shape}")
            ex.launch(din, *bufs, *shape)
            u.synchronize()
            grids.add(ex.last_launch()["grid"][0])
        assert len(grids) == 1, (form, grids)
        assert next(iter(grids)) % cus == 0, (form, grids)


def test_dequant_gemm_decode_and_mfma_grids_do_not_follow_the_extents(hip_device):
    """The dequant GEMM's decode entries (one block per CU) and MFMA entry (four per CU) take the same
    grid at every shape, their blocks striding over the items; results stay bit-exact, including a
    shape with more items than blocks."""
    _, cus = u.device_info()
    for xdt, group, shapes in ((np.int8, 128, [(40, 256, 9), (5000, 2048, 16), (2048, 1024, 64)]),
                               (np.int32, 128, [(64, 256, 16), (3000, 2048, 100)]),
                               (np.int8, 96, [(70, 192, 8), (3000, 1152, 64)])):
        grids = set()
        for (R, K, C) in shapes:
            H.say(f"[case] gemm grid {np.dtype(xdt).name} g{group} {R}x{K}x{C}")
            w, zero, scale, x = _gemm_data(R + K + C, R, K, C, group, xdt)
            got = H.dequant_gemm(w, zero, scale, x, R, K, C, group)
            want = oracle.dequant_gemm_i32(w, zero, scale, x, R, K, C, group)
            assert np.array_equal(got, want), (R, K, C)
            grids.add(_gemm_last_launch("U4", xdt, group)["grid"][0])
        assert len(grids) == 1 and next(iter(grids)) % cus == 0, (np.dtype(xdt).name, group, grids)


# ---------------------------------------------------------------------------------------
# The serial schedule: the sequential fold's bits (the cell's default, Backend::lower)
# ---------------------------------------------------------------------------------------

_serial_execs: dict = {}


def _serial_executor(**form):
    key = tuple(sorted(form.items()))
    if key not in _serial_execs:
        _serial_execs[key] = u.Executor(u.HipBackend().lower_form(schedule="serial", **form))
    return _serial_execs[key]


@pytest.mark.parametrize("dtype,op", [("F32", "Sum"), ("F32", "Mean"), ("F32", "Max"), ("F32", "MinNum"),
                                      ("F64", "Sum"), ("F64", "Min"), ("I32", "Sum"), ("I64", "Prod"),
                                      ("I32", "And")])
@pytest.mark.parametrize("axes", [(1,), (0,), (0, 2)])
def test_serial_reduction_schedule_is_the_serial_lift_bit_for_bit(hip_device, dtype, op, axes):
    """The serial schedule folds in the serial lift's order and accumulator: equal, bit for bit, to the
    oracle's serial fold and to the C99 leg of the serial lift, NaN payloads and signed zeros included,
    on normal (non-dyadic) data where any other order would round differently."""
    rank = 3 if 2 in axes else 2
    shape = (6, 700, 5) if rank == 3 else (37, 900)
    H.say(f"[case] serial reduction {dtype} {op} axes {axes} {shape}")
    nt = {"F32": np.float32, "F64": np.float64, "I32": np.int32, "I64": np.int64}[dtype]
    r = rng(61)
    if dtype.startswith("F"):
        x = r.normal(size=shape).astype(nt)
        flat = x.reshape(-1)
        flat[::97] = np.nan
        flat[1::89] = -0.0
        flat[2::83] = 0.0
        if op == "Sum":
            flat[::97] = 1.0  # keep the sums finite and comparable
    else:
        info = np.iinfo(nt)
        x = r.integers(info.min, info.max, size=shape, dtype=np.int64, endpoint=True).astype(nt)
    kept = [n for d, n in enumerate(shape) if d not in axes]
    ex = _serial_executor(kind="reduction", dtype=dtype, rank=rank, op=op, axes=axes)
    din = u.DeviceBuffer.from_array(x)
    dout = u.DeviceBuffer(int(np.prod(kept)) * x.itemsize)
    ex.launch(din, dout, *shape)
    u.synchronize()
    got = dout.download(nt, int(np.prod(kept))).reshape(kept)
    assert got.tobytes() == _fold_axes(x, axes, op).tobytes()
    want = np.zeros(kept, nt)
    assert cpuc.run(u.lift_reduction("serial", dtype, rank, op, axes=axes), x, want, *shape) == cpuc.OK
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("dtype,op", [("F32", "Sum"), ("F32", "Max"), ("F64", "Mean"), ("I64", "Sum")])
def test_serial_scan_schedule_is_the_serial_lift_bit_for_bit(hip_device, dtype, op):
    """The innermost-axis scan on the serial schedule: bit-exact to the oracle's serial scan on normal
    data (the device look-back schedule is only within the bound there)."""
    H.say(f"[case] serial scan {dtype} {op}")
    nt = {"F32": np.float32, "F64": np.float64, "I64": np.int64}[dtype]
    x = (rng(62).normal(size=(9, 5000)) * 1000).astype(nt)
    ex = _serial_executor(kind="scan", dtype=dtype, rank=2, op=op, exclusive=True)
    din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(x.nbytes)
    ex.launch(din, dout, *x.shape)
    u.synchronize()
    got = dout.download(nt, x.size).reshape(x.shape)
    assert got.tobytes() == oracle.scan_rows(x, op, True, False).tobytes()


# ---------------------------------------------------------------------------------------
# The fixed schedule: the device launch with a float look-back's association fixed by the
# tiling (tiles in groups of 64 per row): the same bits on every launch
# ---------------------------------------------------------------------------------------

_fixed_execs: dict = {}
# Block tiles of an 8-byte carry (an f32 Sum folds in f64): the staged entry's 4 waves x 64 lanes x
# 4 x 18 elements, the register entry's 16 waves x 64 lanes x 16.
_TILE_V, _TILE_S = 4 * 64 * 4 * 18, 16 * 64 * 16


def _fixed_scan(x: np.ndarray, op: str, exclusive=False, reverse=False):
    rows, cols = x.shape
    form = dict(kind="scan", dtype=H.NP_KIND[x.dtype.type], rank=2, op=op, exclusive=exclusive, reverse=reverse)
    key = tuple(sorted(form.items()))
    if key not in _fixed_execs:
        _fixed_execs[key] = u.Executor(u.HipBackend().lower_form(schedule="fixed", **form))
    ex = _fixed_execs[key]
    din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(max(x.nbytes, 1))
    ex.launch(din, dout, rows, cols)
    ex.check()
    return dout.download(x.dtype, x.size).reshape(x.shape), ex.last_launch()["entry"]


@pytest.mark.parametrize("shape,entry", [
    ((1, 64 * _TILE_V), "_v"),            # exactly one group: the next tile would start group 1
    ((1, 130 * _TILE_V), "_v"),           # groups 0..2 of the staged entry
    ((3, 66 * _TILE_V), "_v"),            # several rows, each with its own groups
    ((1, 129 * _TILE_S + 3), "_s"),       # the register entry (rows not a multiple of 4)
    ((2, 70 * _TILE_S + 1), "_s"),
])
@pytest.mark.parametrize("exclusive,reverse", [(False, False), (True, True)])
def test_fixed_scan_schedule_dyadic_bit_exact(hip_device, shape, entry, exclusive, reverse):
    """On the fixed schedule, dyadic data (every f64 partial exact) give RN32 of the exact prefix: the
    oracle's bits, through the staged and the register entry, across group boundaries and rows."""
    H.say(f"[case] fixed scan f32 Sum dyadic {shape} excl={exclusive} rev={reverse}")
    x = synth.uniform_01_f32(31, shape[0] * shape[1]).reshape(shape)
    got, ran = _fixed_scan(x, "Sum", exclusive, reverse)
    assert ran.endswith(entry), ran
    assert got.tobytes() == oracle.scan_rows(x, "Sum", exclusive, reverse).tobytes()


@pytest.mark.parametrize("n", [1 << 24, (1 << 24) - 3])
def test_fixed_scan_schedule_repeats_bit_for_bit(hip_device, n):
    """Normal data, where every association rounds differently: eight launches (four on the register
    entry) give the same bits, each within the declared per-prefix bound of the serial lift's f64 scan
    (kernel_parallel_scan_agrees.rs:287-300)."""
    H.say(f"[case] fixed scan f32 Sum normal n={n}, repeated launches")
    x = rng(63).normal(size=(1, n)).astype(np.float32)
    want = oracle.scan_rows(x, "Sum").ravel().astype(np.float64)
    xs = x.ravel().astype(np.float64)
    u53 = 2.0 ** -53
    k = np.arange(n, dtype=np.float64)
    bound = 2 * (k * u53 / (1 - k * u53)) * np.cumsum(np.abs(xs))
    first, ran = _fixed_scan(x, "Sum")
    assert ran.endswith("_v" if n % 4 == 0 else "_s"), ran
    g = first.ravel()
    assert np.all(np.abs(g.astype(np.float64) - want) <= bound + np.spacing(np.abs(g)).astype(np.float64))
    for _ in range(7 if n % 4 == 0 else 3):
        assert _fixed_scan(x, "Sum")[0].tobytes() == first.tobytes()


@pytest.mark.parametrize("op", ["Max", "Min"])
def test_fixed_scan_schedule_extremum(hip_device, op):
    """Max/Min with NaN and infinities on the fixed schedule: the oracle's values (NaN wherever it has
    NaN), and the same bits on a second launch."""
    H.say(f"[case] fixed scan f32 {op} with NaN/inf")
    x = rng(64).normal(size=(2, 70 * _TILE_V)).astype(np.float32)
    x[0, 3 * _TILE_V + 17] = np.nan
    x[1, 10] = np.inf
    x[1, 65 * _TILE_V] = -np.inf
    got, _ = _fixed_scan(x, op)
    assert equal_extremum(got, oracle.scan_rows(x, op))
    assert _fixed_scan(x, op)[0].tobytes() == got.tobytes()


@pytest.mark.parametrize("shape", [(1, 70 * 4 * 64 * 2 * 18), (2, 66 * 4 * 64 * 2 * 18 + 1), (3, 5000)])
def test_fixed_scan_schedule_f64_and_mean_free_ops(hip_device, shape):
    """F64 data on the fixed schedule (the staged entry's 2-element vectors, and the register entry):
    a dyadic Sum bit-exact, Max/Min equal to the oracle's with NaN cells, a repeat identical."""
    H.say(f"[case] fixed scan f64 {shape}")
    x = (rng(65).integers(-2**20, 2**20, size=shape) / 1024.0).astype(np.float64)
    got, _ = _fixed_scan(x, "Sum", True, False)
    assert got.tobytes() == oracle.scan_rows(x, "Sum", True, False).tobytes()
    y = rng(66).normal(size=shape)
    y.ravel()[::5001] = np.nan
    for op in ("Max", "Min"):
        g1, _ = _fixed_scan(y, op, False, True)
        assert equal_extremum(g1, oracle.scan_rows(y, op, False, True)), op
        assert _fixed_scan(y, op, False, True)[0].tobytes() == g1.tobytes(), op


def test_fixed_scan_schedule_config3b_full(hip_device):
    H.say("[case] config 3b on the fixed schedule: f32 inclusive scan 2^26")
    n = 1 << 26
    x = synth.uniform_01_f32(2, n).reshape(1, n)
    got, _ = _fixed_scan(x, "Sum")
    assert got.tobytes() == oracle.scan_rows(x, "Sum").tobytes()


# ---------------------------------------------------------------------------------------
# The gather lift in general: n inputs, the index and the gathered one anywhere, a body
# (kernel_lift/gather.rs:35-101)
# ---------------------------------------------------------------------------------------

_gx_execs: dict = {}


def _gx_executor(key, make):
    if key not in _gx_execs:
        _gx_execs[key] = u.Executor(u.HipBackend().lower_kernel(make()))
    return _gx_execs[key]


@pytest.mark.parametrize("index_dtype", ["I32", "I64", "U32"])
@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
def test_gather_with_a_body_and_three_inputs(hip_device, index_dtype, oob):
    """out[n, d] = table[clamp(ids[n]), d] * scale[n, d] + 0.5 with the ids first and the table last:
    equal to the oracle's cell (f64, one rounding) and, on these dyadic values, to the C99 leg."""
    from unpopped_amd import expr as X

    H.say(f"[case] gather with a body, 3 inputs, {index_dtype} {oob}")
    V, D, N = 40, 48, 33
    nt = {"I32": np.int32, "I64": np.int64, "U32": np.uint32}[index_dtype]
    r = rng(81)
    table = (r.integers(-1000, 1000, (V, D)) / 64).astype(np.float32)
    scale = (r.integers(-64, 64, (N, D)) / 16).astype(np.float32)
    ids1 = r.integers(0 if index_dtype == "U32" else -4, V + 4, N).astype(nt)
    ids = np.broadcast_to(ids1.reshape(N, 1), (N, D)).copy()
    init = np.full((N, D), 7.0, np.float32)
    body = X.input(2) * X.input(1) + 0.5
    make = lambda: u.lift_gather("gx", "F32", 2, index_dtype, oob=oob, n_inputs=3, data=2, index=0,  # noqa: E731
                                 body=body, launch=(256, 64))
    ex = _gx_executor(("gx3", index_dtype, oob), make)
    bufs = [u.DeviceBuffer.from_array(a) for a in (ids1, scale, table, init)]
    ex.launch(*bufs, N, D, V)
    u.synchronize()
    got = bufs[3].download(np.float32, N * D).reshape(N, D)
    want = oracle.gather_expr([ids, scale, table], 0, 2, 0, oob, body.j, init, V)
    assert got.tobytes() == want.tobytes()
    c = init.copy()
    assert cpuc.run(make(), ids, scale, table, c, N, D, V) == cpuc.OK
    assert got.tobytes() == c.tobytes()


def test_gather_with_a_body_along_an_axis_reading_the_index(hip_device):
    """F64, rank 3, gathered along axis 1, the body reading the index value itself:
    out = table[a, clamp(i), b] + 0.25 * ids; every output cell equals the oracle's."""
    from unpopped_amd import expr as X

    H.say("[case] gather with a body along axis 1, F64")
    A, Vt, B, N = 3, 11, 6, 9
    r = rng(82)
    table = r.normal(size=(A, Vt, B))
    ids1 = r.integers(-2, Vt + 2, N).astype(np.int32)
    ids = np.broadcast_to(ids1.reshape(1, N, 1), (A, N, B)).copy()
    init = np.zeros((A, N, B))
    body = X.input(1) + X.input(0) * 0.25
    ex = _gx_executor(("gxa",), lambda: u.lift_gather("gx", "F64", 3, "I32", axis=1, oob="Clamp", n_inputs=2, data=1,
                                                      index=0, body=body))
    bufs = [u.DeviceBuffer.from_array(a) for a in (ids1, table, init)]
    ex.launch(*bufs, A, N, B, Vt)
    u.synchronize()
    got = bufs[2].download(np.float64, A * N * B).reshape(A, N, B)
    assert got.tobytes() == oracle.gather_expr([ids, table], 0, 1, 1, "Clamp", body.j, init, Vt).tobytes()


def test_gather_moving_one_input_of_three_through_views(hip_device):
    """A leaf body over three inputs moves bits (I64 here); through storage images: a full-shape index
    with a different id in every cell and a transposed table."""
    from unpopped_amd import expr as X

    H.say("[case] gather leaf body, 3 inputs, views")
    V, D, N = 20, 12, 15
    r = rng(83)
    tstore = r.integers(-2**62, 2**62, (D, V)).astype(np.int64)  # the (V, D) table is its transpose
    other = r.integers(0, 9, (N, D)).astype(np.int64)
    ids = r.integers(-3, V + 3, (N, D)).astype(np.int64)
    init = np.full((N, D), -1, np.int64)
    ex = _gx_executor(("gxv",), lambda: u.lift_gather("gx", "I64", 2, "I64", oob="ZeroFill", n_inputs=3, data=0,
                                                      index=2, body=X.input(0)))
    _, _, _, got = _run_images(ex, [(tstore, (V, D), (1, V), 0), (other, (N, D), (D, 1), 0), (ids, (N, D), (D, 1), 0),
                                    (init, (N, D), (D, 1), 0)], [N, D, V])
    want = oracle.gather_expr([tstore.T.copy(), other, ids], 2, 0, 0, "ZeroFill", {"Input": 0}, init, V)
    assert np.array_equal(got, want)
