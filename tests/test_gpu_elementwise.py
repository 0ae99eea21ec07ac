"""GPU parity of the Access::Elementwise form (kernel_lift.rs:96-153) through the C ABI: the shared
launch_cases() corpus (launch_cases.rs:137-180), the integer rule's boundary vectors
(docs/int-div-shift-semantics.md) and every entry (`_v` 16-byte packs, `_s` any alignment, `_e`
strides and permuted reads), each against the CPU oracle on the same inputs.

Bars: bit-exact against the oracle for every case (a float body is evaluated in f64 and rounded once,
as the oracle does; integers by the total rule; single-input bodies move bits); against the C99 leg
within the corpus's stated ulps (launch_cases.rs:14-27).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import unpopped_amd as u
from oracle import cpuc
from tests.launch_corpus import corpus_args, elementwise_launched, launch_cases, over_inputs
from tests.test_elementwise import INT_DTYPES, B, I, body_of, grid
from unpopped_amd import forms as H

pytestmark = pytest.mark.gpu

_execs: dict = {}


def executor(kernel: dict) -> u.Executor:
    import json

    key = json.dumps(kernel, sort_keys=True)
    if key not in _execs:
        _execs[key] = u.Executor(u.HipBackend().lower_kernel(kernel))
    return _execs[key]


def run(kernel: dict, inputs, shape, out_dtype, offsets=None, static=False):
    """Launch with dense buffers (input k `offsets[k]` bytes into its allocation) and return the
    output and the entry that ran."""
    ex = executor(kernel)
    offsets = offsets or [0] * len(inputs)
    bufs = []
    for a, off in zip(inputs, offsets):
        a = np.ascontiguousarray(a)
        base = u.DeviceBuffer(a.nbytes + off + 16)
        v = base.at(off)
        v.upload(a)
        bufs.append(v)
    count = int(np.prod(shape))
    out = u.DeviceBuffer(max(count * np.dtype(out_dtype).itemsize, 1))
    out.fill(0)
    (ex.launch_static if static else ex.launch)(*bufs, out, *shape)
    u.synchronize()
    return out.download(out_dtype, count).reshape(shape), ex.last_launch()["entry"]


@pytest.mark.parametrize("case", launch_cases(), ids=lambda c: c[0])
def test_launch_cases_corpus_on_the_gpu(hip_device, case):
    """Every corpus kernel lowered by lower_kernel and run on its own inputs and on random ones: byte
    for byte the oracle's result, and within the case's ulps of the C99 leg."""
    name, dtype, shape, (block, grid_), ulps, body, _ = case
    H.say(f"[case] launch_cases {name} {dtype} {shape}")
    k = elementwise_launched(name, dtype, len(shape), body, block, grid_)
    b = over_inputs(body, len(shape))
    x, y, _ = corpus_args(dtype, shape)
    r = np.random.default_rng(11)
    if dtype == "F32":
        xr, yr = r.normal(size=shape).astype(np.float32), r.normal(size=shape).astype(np.float32)
        yr.ravel()[::4] = 0
    else:
        nt = np.int32 if dtype == "I32" else np.uint32
        info = np.iinfo(nt)
        xr = r.integers(info.min, info.max, shape, dtype=np.int64, endpoint=True).astype(nt)
        yr = r.integers(info.min, info.max, shape, dtype=np.int64, endpoint=True).astype(nt)
    for a, c in ((x, y), (xr, yr)):
        got, entry = run(k, [a, c], shape, a.dtype)
        assert entry.endswith("_v")
        want = oracle.elementwise([a, c], b, dtype)
        assert got.tobytes() == want.tobytes(), name
        leg = np.zeros(shape, a.dtype)
        assert cpuc.run(k, a, c, leg, *shape) == cpuc.OK
        if dtype == "F32":
            ia, ib = got.view(np.int32).astype(np.int64), leg.view(np.int32).astype(np.int64)
            same = (got == leg) | (np.isnan(got) & np.isnan(leg))
            assert (same | (np.abs(ia - ib) <= ulps)).all(), name
        else:
            assert got.tobytes() == leg.tobytes()


@pytest.mark.parametrize("dt", INT_DTYPES)
@pytest.mark.parametrize("op", ["Div", "Shl", "Shr", "Rem", "Add", "Sub", "Mul", "Min", "Max", "BitAnd", "BitOr",
                                "BitXor"])
def test_integer_rule_boundary_vectors_on_the_gpu(hip_device, dt, op):
    """Every pair of boundary values (dividends, divisors and counts of the rule's proof obligations)
    through the HIP spelling of Div, Shl, Shr, the remainder composition and the ring and bit ops:
    bit-exact against the oracle."""
    H.say(f"[case] integer boundary vectors {dt} {op}")
    x, y = grid(dt)
    body = {op: [I(0), I(1)]} if op in ("Add", "Sub", "Mul") else body_of(op, dt)
    k = u.lift_elementwise(f"bv_{op}", dt, 1, body, n_inputs=2, launch=(64, 2))
    got, _ = run(k, [x, y], (x.size,), x.dtype)
    assert got.tobytes() == oracle.elementwise([x, y], body, dt).tobytes()


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_integer_select_compare_and_constants_on_the_gpu(hip_device, dt):
    """Select over a comparison (the compute type's 0/1), constants wrapped to the kind, a wrap Cast."""
    H.say(f"[case] integer select/compare/constants {dt}")
    x, y = grid(dt)
    c = {"ConstInt": [-5, dt]}
    body = {"Select": [B("CmpLe", I(0), I(1)),
                       {"Add": [B("CmpNe", I(0), c), {"Cast": [I(1), {"to": dt, "round": "NearestEven", "sat": "Wrap"}]}]},
                       {"Mul": [I(0), c]}]}
    k = u.lift_elementwise("sel", dt, 2, body, n_inputs=2, launch=(128, 3))
    side = int(round(np.sqrt(x.size)))  # the grid is every pair of the kind's boundary values
    shape = (side, side)
    got, _ = run(k, [x.reshape(shape), y.reshape(shape)], shape, x.dtype)
    assert got.tobytes() == oracle.elementwise([x.reshape(shape), y.reshape(shape)], body, dt).tobytes()


def test_entries_by_alignment_and_permutation(hip_device):
    """2^20 + 3 elements: 16-byte-aligned buffers take `_v` (packs and a tail), an input 4 bytes off
    takes `_s`, a permuted input `_e`; each result the oracle's."""
    H.say("[case] elementwise entries: _v, _s, _e")
    n = (1 << 20) + 3
    r = np.random.default_rng(21)
    x, y = r.normal(size=n).astype(np.float32), r.normal(size=n).astype(np.float32)
    body = {"Fma": [I(0), I(1), {"Unary": ["Sqrt", {"Unary": ["Abs", I(0)]}]}]}
    k = u.lift_elementwise("fm", "F32", 1, body, n_inputs=2, launch=(256, 64))
    want = oracle.elementwise([x, y], body, "F32")
    got, entry = run(k, [x, y], (n,), np.float32)
    assert entry.endswith("_v") and got.tobytes() == want.tobytes()
    got, entry = run(k, [x, y], (n,), np.float32, offsets=[0, 4])
    assert entry.endswith("_s") and got.tobytes() == want.tobytes()
    a, bsrc = r.normal(size=(300, 517)), r.normal(size=(517, 300))
    kp = u.lift_elementwise("tp", "F64", 2, {"Sub": [I(0), {"Mul": [I(1), {"Const": 0.5}]}]}, n_inputs=2,
                            perms=[[0, 1], [1, 0]], launch=(256, 16))
    got, entry = run(kp, [a, bsrc], (300, 517), np.float64)
    assert entry.endswith("_e")
    assert got.tobytes() == oracle.elementwise([a, bsrc], {"Sub": [I(0), {"Mul": [I(1), {"Const": 0.5}]}]}, "F64",
                                               perms=[[0, 1], [1, 0]]).tobytes()


def test_storage_images_read_through_their_strides(hip_device):
    """Storage images that are not dense row-major (a transposed input, an output written into every
    other column of a wider buffer, a base offset) run the strided entry: the oracle's result lands at
    the view's elements and nothing else moves."""
    H.say("[case] elementwise storage images")
    r = np.random.default_rng(22)
    R, Cc = 37, 53
    a = r.normal(size=(R, Cc)).astype(np.float32)
    bt = r.normal(size=(Cc, R)).astype(np.float32)  # stored transposed
    body = {"Div": [I(0), {"Add": [I(1), {"Const": 3.0}]}]}
    k = u.lift_elementwise("sv", "F32", 2, body, n_inputs=2, launch=(256, 8))
    ex = executor(k)
    da, db = u.DeviceBuffer.from_array(a), u.DeviceBuffer.from_array(bt)
    wide = np.full((R, 2 * Cc + 1), 7.0, np.float32)
    dout = u.DeviceBuffer.from_array(wide)
    ex.launch_views([(da, (R, Cc), None, 0), (db, (R, Cc), (1, R), 0), (dout, (R, Cc), (2 * Cc + 1, 2), 1)], [R, Cc])
    u.synchronize()
    got = dout.download(np.float32, wide.size).reshape(wide.shape)
    assert ex.last_launch()["entry"].endswith("_e")
    want = oracle.elementwise([a, bt.T.copy()], body, "F32")
    assert got[:, 1::2][:, :Cc].tobytes() == want.tobytes()
    untouched = np.ones_like(wide, bool)
    untouched[:, 1:2 * Cc:2] = False
    assert (got[untouched] == 7.0).all()


@pytest.mark.parametrize("dt,nt", [("Bf16", np.uint16), ("U8", np.uint8), ("I64", np.int64)])
def test_single_input_bodies_move_bits(hip_device, dt, nt):
    """A body that is one input moves its bits at any whole-byte kind (NaN patterns of a Bf16 too)."""
    H.say(f"[case] elementwise bit move {dt}")
    r = np.random.default_rng(23)
    n = 4099
    x = r.integers(0, np.iinfo(nt).max, n, dtype=np.uint64).astype(nt)
    y = r.integers(0, np.iinfo(nt).max, n, dtype=np.uint64).astype(nt)
    k = u.lift_elementwise("mv", dt, 1, I(1), n_inputs=2, launch=(64, 4))
    got, _ = run(k, [x, y], (n,), nt)
    assert got.tobytes() == y.tobytes()


def test_static_launch_matches_the_allocating_one(hip_device):
    """The no-allocation entry point runs the same kernels (the elementwise form has no workspace)."""
    H.say("[case] elementwise static launch")
    x, y = grid("I32")
    k = u.lift_elementwise("st", "I32", 1, body_of("Rem", "I32"), n_inputs=2, launch=(64, 2))
    a, _ = run(k, [x, y], (x.size,), x.dtype)
    b, _ = run(k, [x, y], (x.size,), x.dtype, static=True)
    assert a.tobytes() == b.tobytes()


def test_full_size_f32_corpus_body_at_2_26(hip_device):
    """The corpus's fma_shape body over 2^26 elements (a full HBM-resident size): equal to numpy's
    float64 evaluation rounded once, the model the oracle is pinned to on the CPU."""
    H.say("[case] elementwise fma_shape at 2^26")
    n = 1 << 26
    r = np.random.default_rng(24)
    x, y = r.normal(size=n).astype(np.float32), r.normal(size=n).astype(np.float32)
    body = {"Add": [{"Mul": [{"Unary": ["Abs", I(0)]}, {"Unary": ["Abs", I(1)]}]}, {"Unary": ["Abs", I(0)]}]}
    k = u.lift_elementwise("big", "F32", 1, body, n_inputs=2, launch=(4, 2))
    got, entry = run(k, [x, y], (n,), np.float32)
    assert entry.endswith("_v")
    want = (np.abs(x.astype(np.float64)) * np.abs(y) + np.abs(x)).astype(np.float32)
    assert got.tobytes() == want.tobytes()
