"""GPU parity of reductions and scans with an integer pre-map body (I32, I64; the identity post,
kernel_lift.rs:755-800): the body evaluated by the total integer rule (docs/int-div-shift-semantics.md)
and folded at the element type, launched through the C ABI and compared bit for bit with the oracle
(the integer evaluator's values folded by the serial lift).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import unpopped_amd as u
from unpopped_amd import forms as H

pytestmark = pytest.mark.gpu

I = lambda k: {"Input": k}  # noqa: E741,E731
B = lambda op, a, b: {"Binary": [op, a, b]}  # noqa: E731


def body_for(dt):
    """(x0 * x1) / (x1 >> 2) + (x0 << 3): a wrapping product, a divisor that is often 0 or -1, shifts
    by counts past the width."""
    return {"Add": [{"Div": [{"Mul": [I(0), I(1)]}, B("Shr", I(1), {"ConstInt": [2, dt]})]},
                    B("Shl", I(0), I(1))]}


def ints(seed, shape, nt):
    """Full-range integers with zeros, -1 and the extremes mixed in."""
    r = np.random.default_rng(seed)
    info = np.iinfo(nt)
    a = r.integers(info.min, info.max, shape, dtype=nt, endpoint=True)
    flat = a.reshape(-1)
    flat[::7] = 0
    flat[3::11] = -1
    flat[5::13] = info.min
    flat[6::17] = r.integers(-4, 4, flat[6::17].size)
    return a


def launch_reduce(k, xs, out_shape, nt):
    ex = u.Executor(u.HipBackend().lower_kernel(k))
    dins = [u.DeviceBuffer.from_array(a) for a in xs]
    n = int(np.prod(out_shape, dtype=np.int64))
    dout = u.DeviceBuffer(max(n * np.dtype(nt).itemsize, 1))
    ex.launch(*dins, dout, *xs[0].shape)
    ex.check()
    return dout.download(nt, n).reshape(out_shape), ex.last_launch()["entry"]


@pytest.mark.parametrize("dt,nt", [("I32", np.int32), ("I64", np.int64)])
@pytest.mark.parametrize("op", ["Sum", "Prod", "Max", "Min"])
@pytest.mark.parametrize("axes,shape", [((1,), (37, 3001)), ((0, 1), (1, 1 << 20)), ((0,), (513, 29)),
                                        ((0, 2), (6, 7, 9))])
def test_launched_reduction_with_an_integer_body(hip_device, dt, nt, op, axes, shape):
    H.say(f"[case] integer-body reduction {dt} {op} axes {axes} {shape}")
    xs = [ints(100 + k, shape, nt) for k in range(2)]
    body = body_for(dt)
    k = u.lift_reduction("ir", dt, len(shape), op, axes=axes, n_inputs=2, body=body, launch=(256, 8))
    kept = [n for d, n in enumerate(shape) if d not in axes]
    got, _ = launch_reduce(k, xs, kept, nt)
    want = oracle.int_reduce_expr(xs, axes, op, body, dt)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("dt,nt", [("I32", np.int32), ("I64", np.int64)])
@pytest.mark.parametrize("op", ["And", "Or", "Xor"])
def test_serial_bit_reduction_with_an_integer_body(hip_device, dt, nt, op):
    H.say(f"[case] integer-body bit reduction {dt} {op}")
    shape = (41, 1037)
    xs = [ints(110 + k, shape, nt) for k in range(2)]
    body = B("BitXor", B("Shl", I(0), {"ConstInt": [5, dt]}), {"Div": [I(1), I(0)]})
    k = u.lift_reduction("ib", dt, 2, op, axes=(1,), n_inputs=2, body=body)
    got, _ = launch_reduce(k, xs, [shape[0]], nt)
    assert got.tobytes() == oracle.int_reduce_expr(xs, (1,), op, body, dt).tobytes()


@pytest.mark.parametrize("dt,nt", [("I32", np.int32), ("I64", np.int64)])
@pytest.mark.parametrize("op", ["Sum", "Prod", "Max", "Min"])
@pytest.mark.parametrize("excl,rev", [(False, False), (True, True)])
def test_launched_scan_with_an_integer_pre(hip_device, dt, nt, op, excl, rev):
    H.say(f"[case] integer-pre scan {dt} {op} excl={excl} rev={rev}")
    shape = (3, 70001)
    xs = [ints(120 + k, shape, nt) for k in range(2)]
    pre = body_for(dt)
    got = H.scan_expr(xs, 1, op, pre, exclusive=excl, reverse=rev)
    assert got.tobytes() == oracle.int_scan_expr(xs, 1, op, pre, dt, excl, rev).tobytes()


@pytest.mark.parametrize("dt,nt", [("I32", np.int32), ("I64", np.int64)])
def test_serial_scan_with_an_integer_pre_along_axis_0(hip_device, dt, nt):
    H.say(f"[case] integer-pre scan along axis 0 {dt}")
    shape = (300, 17)
    xs = [ints(130 + k, shape, nt) for k in range(2)]
    pre = {"Select": [B("CmpLt", I(0), I(1)), {"Sub": [I(1), I(0)]}, {"Div": [I(0), I(1)]}]}
    got = H.scan_expr(xs, 0, "Sum", pre, reverse=True)
    assert got.tobytes() == oracle.int_scan_expr(xs, 0, "Sum", pre, dt, False, True).tobytes()


def test_integer_scan_rows_of_2_26(hip_device):
    """Config 3a's size (2^26 int32) with a pre-map: bit-exact."""
    H.say("[case] integer-pre scan 2^26")
    n = 1 << 26
    r = np.random.default_rng(140)
    x = r.integers(-1000, 1000, (1, n), dtype=np.int32)
    y = r.integers(-3, 4, (1, n), dtype=np.int32)
    pre = {"Add": [{"Mul": [I(0), I(1)]}, {"Div": [I(0), I(1)]}]}
    got = H.scan_expr([x, y], 1, "Sum", pre)
    assert got.tobytes() == oracle.int_scan_expr([x, y], 1, "Sum", pre, "I32").tobytes()
