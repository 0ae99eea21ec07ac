"""The cpu-c C99 leg on the CPU: the restated emitter (oracle/cpuc.cpp) lowers every kernel this
backend recognises to the reference's serial or serialized-thread-loop C
(crates/unpopped-cpu-c/src/{kernel,launch}.rs), the C compiles with the reference's flags
(tests/support/cc.rs:163-176), and its results equal the CPU oracle's:

* bit-exact for integer folds and scans, Max/Min, the gather, the dequant and the dequantizing GEMM;
* float Sum of a serial lift bit-exact to the oracle's ascending f64 fold, and float Sum of a launched
  lift bit-exact to the written-order reimplementation of that lift
  (kernel_parallel_reduction_float_sum_bound.rs:147-169; kernel_parallel_scan_agrees.rs:195-260);
* RowReduce epilogues within the reference's own C-leg tolerance (per-operation float rounding against
  the oracle's one rounding per statement, launch_cases.rs:12-27).

BASELINE config 1 (2^24 f32 from seed 0, uniform[-1,1)) runs here end to end: lift -> C99 -> equal to
the oracle and to RN32 of the exact sum."""
from __future__ import annotations

import copy

import numpy as np
import pytest

import oracle
import unpopped_amd as u
from oracle import cpuc
from oracle.cpuc import View
from unpopped_amd import synth
from unpopped_amd import expr as X

RNG = np.random.default_rng(20261202)

FLOAT_OPS = ("Sum", "Prod", "Max", "Min", "Mean")
INT_OPS = ("Sum", "Prod", "Max", "Min")


def data(dtype: str, shape, rng=RNG) -> np.ndarray:
    if dtype == "F32":
        return rng.standard_normal(shape).astype(np.float32)
    if dtype == "F64":
        return rng.standard_normal(shape)
    if dtype == "I32":
        return rng.integers(-2**31, 2**31, shape, dtype=np.int64).astype(np.int32)
    return rng.integers(-2**63, 2**63 - 1, shape, dtype=np.int64)


NP = {"F32": np.float32, "F64": np.float64, "I32": np.int32, "I64": np.int64}


# ---- reductions ----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["F32", "F64", "I32", "I64"])
def test_serial_row_reduction_equals_the_oracle(dtype):
    x = data(dtype, (7, 45))
    for op in (FLOAT_OPS if dtype[0] == "F" else INT_OPS):
        k = u.lift_reduction("rr", dtype, 2, op)
        out = np.full(7, 99, NP[dtype])
        assert cpuc.run(k, x, out, 7, 45) == cpuc.OK
        want = oracle.reduce_rows(x, op)
        assert out.tobytes() == want.tobytes(), (dtype, op)


@pytest.mark.parametrize("block,grid", [(1, 1), (4, 3), (64, 2), (256, 5)])
def test_launched_row_reduction_is_the_written_order(block, grid):
    x = data("F32", (9, 300))
    for op in ("Sum", "Mean", "Max", "Min"):
        k = u.lift_reduction("rl", "F32", 2, op, launch=(block, grid))
        out = np.zeros(9, np.float32)
        assert cpuc.run(k, x, out, 9, 300) == cpuc.OK
        if op in ("Max", "Min"):
            want = oracle.reduce_rows(x, op)
        else:
            want = np.array([oracle.sum_launched_order(x[r].astype(np.float64), block, op == "Mean")
                             for r in range(9)]).astype(np.float32)
        assert out.tobytes() == want.tobytes(), (op, block)
    xi = data("I64", (5, 77))
    for op in INT_OPS:
        k = u.lift_reduction("rl", "I64", 2, op, launch=(block, grid))
        out = np.zeros(5, np.int64)
        assert cpuc.run(k, xi, out, 5, 77) == cpuc.OK
        assert np.array_equal(out, oracle.reduce_rows(xi, op)), op


def test_launched_order_differs_from_the_serial_order():
    """The written-order check is not vacuous: at F64 the launched (block 64) fold equals the
    written-order restatement bit for bit and differs from the serial fold on some rows."""
    x = data("F64", (64, 1000))
    k = u.lift_reduction("rl", "F64", 2, "Sum", launch=(64, 4))
    out = np.zeros(64)
    assert cpuc.run(k, x, out, 64, 1000) == cpuc.OK
    want = np.array([oracle.sum_launched_order(x[r], 64) for r in range(64)])
    assert out.tobytes() == want.tobytes()
    assert not np.array_equal(out, oracle.reduce_rows(x, "Sum"))


@pytest.mark.parametrize("axes,keepdim", [((0,), False), ((1,), True), ((0, 2), False), ((0, 1, 2), False)])
def test_reductions_over_axis_sets(axes, keepdim):
    x = data("F64", (4, 5, 6))
    moved = np.moveaxis(x, axes, range(3 - len(axes), 3))
    kept = moved.shape[:3 - len(axes)]
    flat = moved.reshape(int(np.prod(kept)) if kept else 1, -1)
    for op in ("Sum", "Max"):
        want = oracle.reduce_rows(np.ascontiguousarray(flat), op)
        for launch in (None, (16, 3)):
            k = u.lift_reduction("ra", "F64", 3, op, axes=axes, keepdim=keepdim, launch=launch)
            oshape = tuple(1 if (d in axes) else x.shape[d] for d in range(3)) if keepdim else kept
            out = np.zeros(oshape if oshape else (), np.float64)
            assert cpuc.run(k, x, View(out.reshape(-1) if out.ndim else out.reshape(1), oshape, None), 4, 5, 6) == 0
            if launch is None or op == "Max":
                assert out.reshape(-1).tobytes() == want.tobytes(), (axes, op, launch)
            else:
                for i in range(want.size):
                    assert abs(out.reshape(-1)[i] - want[i]) <= 1e-12 * np.abs(flat[i]).sum()


def test_reduction_with_a_body_and_a_post():
    a, b = data("F32", (6, 40)), data("F32", (6, 40))
    k = u.lift_reduction("rx", "F32", 2, "Sum", n_inputs=2, body=X.input(0) * X.input(1),
                         post=X.reduced(0) * 0.5 + 1.0)
    out = np.zeros(6, np.float32)
    assert cpuc.run(k, a, b, out, 6, 40) == cpuc.OK
    for r in range(6):
        prods = (a[r].astype(np.float64) * b[r]).astype(np.float32).astype(np.float64)
        s = np.float32(oracle.reduce_rows(prods.reshape(1, -1), "Sum")[0])
        # the post is one F32 statement of two operations: C rounds each (two roundings), the oracle once
        want = np.float32(np.float32(s * np.float32(0.5)) + np.float32(1.0))
        assert abs(float(out[r]) - float(want)) <= 2 * np.spacing(np.float32(abs(want))), r


# ---- scans ---------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["F32", "F64", "I32", "I64"])
def test_serial_scans_equal_the_oracle(dtype):
    x = data(dtype, (3, 50))
    for op in (("Sum", "Max", "Min", "Prod") if dtype[0] == "I" else ("Sum", "Max", "Min")):
        for exclusive in (False, True):
            for reverse in (False, True):
                k = u.lift_scan("sc", dtype, 2, op, exclusive=exclusive, reverse=reverse)
                out = np.zeros_like(x)
                assert cpuc.run(k, x, out, 3, 50) == cpuc.OK
                want = oracle.scan_rows(x, op, exclusive, reverse)
                assert out.tobytes() == want.tobytes(), (dtype, op, exclusive, reverse)


@pytest.mark.parametrize("block", [1, 2, 8, 64])
def test_launched_scan_is_the_written_order(block):
    x = data("F32", (1, 333))
    for exclusive in (False, True):
        for reverse in (False, True):
            k = u.lift_scan("sl", "F32", 1, "Sum", exclusive=exclusive, reverse=reverse, launch=(block, 2))
            out = np.zeros(333, np.float32)
            assert cpuc.run(k, x.ravel(), out, 333) == cpuc.OK
            want = oracle.scan_launched_order_f32(x.ravel(), block, exclusive, reverse)
            assert out.tobytes() == want.tobytes(), (block, exclusive, reverse)
    xi = data("I32", (1, 333)).ravel()
    k = u.lift_scan("sl", "I32", 1, "Sum", launch=(block, 2))
    out = np.zeros(333, np.int32)
    assert cpuc.run(k, xi, out, 333) == cpuc.OK
    assert np.array_equal(out, oracle.scan_rows(xi.reshape(1, -1), "Sum").ravel())


@pytest.mark.parametrize("dtype", ["F32", "F64"])
@pytest.mark.parametrize("axis", [0, 1])
def test_scans_with_a_pre_and_a_post_equal_the_oracle(dtype, axis):
    """A scan of two inputs with the pre-map `x * y` and the post `Reduced(0) - Input(0)` (one
    operation each, so C's per-operation rounding and the kernel evaluator's per-statement rounding
    agree): the C leg of the serial lift equals orc_scan_x bit for bit on every op, direction and
    exclusivity; the launched lift's C leg (another association of the Sum) stays within the
    per-prefix bound and is exact for Max / Min."""
    a, b = data(dtype, (5, 37)), data(dtype, (5, 37))
    pre, post = X.input(0) * X.input(1), X.reduced(0) - X.input(0)
    for op in ("Sum", "Max", "Min", "Mean", "Prod"):
        for exclusive in (False, True):
            for reverse in (False, True):
                k = u.lift_scan("sx", dtype, 2, op, axis=axis, exclusive=exclusive, reverse=reverse, n_inputs=2,
                                pre=pre, post=post)
                out = np.zeros_like(a)
                assert cpuc.run(k, a, b, out, 5, 37) == cpuc.OK
                want = oracle.scan_expr([a, b], axis, op, pre, post, exclusive, reverse)
                assert out.tobytes() == want.tobytes(), (op, exclusive, reverse)
    if axis == 1:
        for op in ("Sum", "Max", "Min"):
            k = u.lift_scan("sx", dtype, 2, op, n_inputs=2, pre=pre, post=post, launch=(8, 2))
            out = np.zeros_like(a)
            assert cpuc.run(k, a, b, out, 5, 37) == cpuc.OK
            want = oracle.scan_expr([a, b], 1, op, pre, post)
            if op == "Sum":
                v = (a.astype(np.float64) * b).astype(a.dtype).astype(np.float64)
                bound = 37 * 2.0 ** -52 * np.cumsum(np.abs(v), axis=1) + 2 * np.spacing(np.abs(want).astype(a.dtype))
                assert np.all(np.abs(out.astype(np.float64) - want) <= bound)
            else:
                assert out.tobytes() == want.tobytes(), op


# ---- gather --------------------------------------------------------------------------------

@pytest.mark.parametrize("index_dtype", ["I32", "I64", "U32"])
@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
@pytest.mark.parametrize("launch", [None, (32, 3)])
def test_gather_equals_the_oracle(index_dtype, oob, launch):
    rows, d, n = 37, 24, 50
    table = RNG.integers(0, 2**16, (rows, d), dtype=np.uint16)
    ids = RNG.integers(-5, rows + 5, n).astype({"I32": np.int32, "I64": np.int64, "U32": np.int64}[index_dtype])
    if index_dtype == "U32":
        ids = np.where(ids < 0, 2**32 - 3, ids).astype(np.uint32)
    k = u.lift_gather("ga", "Bf16", 2, index_dtype, 0, oob, launch=launch)
    out = np.full((n, d), 0xABCD, np.uint16)
    rc = cpuc.run(k, table, View(ids, (n, d), (1, 0)), out, n, d, rows)
    assert rc == cpuc.OK
    want = oracle.gather_rows(table, ids, oob, out_init=np.full((n, d), 0xABCD, np.uint16))
    assert np.array_equal(out, want)


# ---- fused row sum + max, dequant, dequantizing GEMM -----------------------------------------

@pytest.mark.parametrize("launch", [None, (64, 3)])
def test_row_reduce2_equals_two_serial_folds(launch):
    x = data("F32", (11, 130))
    k = u.kernel_row_reduce2("r2", "F32", "Sum", "Max", launch=launch)
    s, m = np.zeros(11, np.float32), np.zeros(11, np.float32)
    assert cpuc.run(k, x, s, m, 11, 130) == cpuc.OK
    assert m.tobytes() == oracle.reduce_rows(x, "Max").tobytes()
    if launch is None:
        assert s.tobytes() == oracle.reduce_rows(x, "Sum").tobytes()
    else:
        want = np.array([oracle.sum_launched_order(x[r].astype(np.float64), 64) for r in range(11)], np.float32)
        assert s.tobytes() == want.tobytes()


@pytest.mark.parametrize("q_kind,z_kind", [("U4", "U4"), ("I4", "U4"), ("U4", "I4")])
@pytest.mark.parametrize("launch", [None, (64, 4)])
def test_dequant_is_bit_exact(q_kind, z_kind, launch):
    R, Cc, G = 6, 256, 64
    q = synth.nibbles(4, R * Cc)
    z = synth.nibbles(41, R * Cc // G)
    s = synth.uniform_f16_bits(42, R * Cc // G, 0.001, 0.02)
    k = u.kernel_dequant4("dq", q_kind, z_kind, G, launch=launch)
    out = np.zeros(R * Cc, np.uint16)
    rc = cpuc.run(k, View(q, (R * Cc,), (1,)), s, View(z, (R * Cc // G,), (1,)), out, R, Cc)
    assert rc == cpuc.OK
    want = oracle.dequant4_bf16(q, s, z, R, Cc, G, q_signed=q_kind == "I4", z_signed=z_kind == "I4")
    assert np.array_equal(out, want.ravel())


@pytest.mark.parametrize("w_kind,x_kind", [("U4", "I32"), ("I4", "I32"), ("U4", "I8")])
@pytest.mark.parametrize("launch", [None, (32, 3)])
def test_dequant_gemm_wraps_like_the_oracle(w_kind, x_kind, launch):
    R, K, Cc, G = 5, 24, 6, 8
    w = synth.nibbles(5, R * K)
    zero = RNG.integers(-2**31, 2**31, R * K // G, dtype=np.int64).astype(np.int32)
    scale = RNG.integers(-2**31, 2**31, R * K // G, dtype=np.int64).astype(np.int32)
    x = (RNG.integers(-2**31, 2**31, K * Cc, dtype=np.int64).astype(np.int32) if x_kind == "I32"
         else RNG.integers(-128, 128, K * Cc).astype(np.int8))
    k = u.kernel_dequant_gemm("dg", w_kind, x_kind, G, launch=launch)
    out = np.zeros(R * Cc, np.int32)
    assert cpuc.run(k, View(w, (R * K,), (1,)), zero, scale, x, out, R, K, Cc) == cpuc.OK
    want = oracle.dequant_gemm_i32(w, zero, scale, x, R, K, Cc, G, w_signed=w_kind == "I4")
    assert np.array_equal(out, want.ravel())


def test_dequant_gemm_known_answer():
    """The reference fixture's own known answer (crates/unpopped/tests/support/dequant.rs:145-181:
    R=4, K=8, C=4, GROUP=4), through the C99 of the serial kernel."""
    from tests.golden import corpora

    case = corpora.dequant_gemm_fixture()
    k = u.kernel_dequant_gemm("dg", "I4", "I32", case["group"])
    out = np.zeros(case["rows"] * case["cols"], np.int32)
    rc = cpuc.run(k, View(case["w_packed"], (case["rows"] * case["k"],), (1,)), case["zero"], case["scale"],
                  case["x"], out, case["rows"], case["k"], case["cols"])
    assert rc == cpuc.OK
    assert np.array_equal(out, case["expected"].ravel())


# ---- RowReduce -----------------------------------------------------------------------------

def ulps32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.astype(np.float32).view(np.int32).astype(np.int64)
    ib = b.astype(np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(2**31) - ia, ia)
    ib = np.where(ib < 0, -(2**31) - ib, ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("launch", [None, (128, 3)])
def test_row_reduce_softmax_within_the_c_leg_tolerance(launch):
    x = data("F32", (5, 200))
    stages, epi = X.softmax()
    k = u.lift_row_reduce("sm", "F32", 2, stages, epi, launch=launch)
    out = np.zeros_like(x)
    assert cpuc.run(k, x, out, 5, 200) == cpuc.OK
    want = oracle.row_reduce([x], stages, epi)
    # The C leg computes the F32 epilogue per operation in float where the oracle evaluates each
    # statement in f64 and rounds once (launch_cases.rs:12-27): the reference's C leg allows 3 ulps for
    # such an epilogue (kernel_emit_row_reduce_agrees.rs:6-7), and the float rounding of x - max before
    # expf is amplified by exp's condition number |x - max| (docs/ir-kernel-layer.md 7.1), which that
    # corpus keeps small and normal data does not.
    bound = 3 + np.ceil(np.abs(x - x.max(axis=1, keepdims=True)))
    assert (ulps32(out, want) <= bound).all()
    assert ulps32(out, want).max() >= 1  # the two roundings really differ on this corpus


# ---- BASELINE config 1 ---------------------------------------------------------------------

def test_config1_full_sum_through_the_c_leg():
    """2^24 f32 uniform[-1,1) from seed 0 (dyadic: k 2^-24), lifted, lowered to C99, run: equal to the
    oracle and to RN32 of the exact sum, for the serial lift and the launched lift (block 256)."""
    n = 1 << 24
    x = synth.uniform_pm1_f32(0, n)
    k_int = np.round(x.astype(np.float64) * 2.0**24).astype(np.int64)
    assert np.array_equal(k_int.astype(np.float64) * 2.0**-24, x.astype(np.float64))
    exact = np.float32(float(int(k_int.sum())) * 2.0**-24)
    want = oracle.reduce_rows(x.reshape(1, -1), "Sum")[0]
    assert want == exact
    for launch in (None, (256, 1)):
        k = u.lift_reduction("cfg1", "F32", 1, "Sum", launch=launch)
        out = np.zeros(1, np.float32)
        assert cpuc.run(k, x, View(out.reshape(()), (), ()), n) == cpuc.OK
        assert out[0] == exact, launch


# ---- codecs, status codes, refusals -----------------------------------------------------------

def _cast_kernel(src: str, dst: str) -> dict:
    """A serial kernel out[i] = Cast(in[i] -> dst) of a 1-D buffer (handwritten KernelFn)."""
    cast = {"Cast": [{"Local": 2}, {"to": dst, "round": "NearestEven", "sat": "Wrap"}]}
    body = [{"For": {"local": 1, "start": {"ConstInt": [0, "I32"]}, "end": {"Local": 0},
                     "step": {"ConstInt": [1, "I32"]}, "unroll": "None",
                     "body": [{"Load": {"local": 2, "place": {"Logical": {"buffer": 0, "coords": [{"Local": 1}]}}}},
                              {"Store": {"place": {"Logical": {"buffer": 1, "coords": [{"Local": 1}]}},
                                         "value": cast}}]}}]
    return {"name": f"cast_{src}_{dst}", "compute": "F32",
            "params": [{"name": "in0", "kind": {"Buffer": {"elem": src, "role": "Read", "rank": 1}}},
                       {"name": "out", "kind": {"Buffer": {"elem": dst, "role": "Write", "rank": 1}}},
                       {"name": "n", "kind": {"Scalar": {"ty": "I32", "local": 0}}}],
            "locals": [{"elem": "I32", "lanes": 1}, {"elem": "I32", "lanes": 1}, {"elem": src, "lanes": 1}],
            "body": body, "launch": None, "allocs": [], "result": None, "results": []}


def _f32_corpus() -> np.ndarray:
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2**16, 20000).astype(np.uint32) << 16) | 0x8000  # exact bf16 ties
    near = ties + rng.integers(-2, 3, 20000).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x00000001, 0x807FFFFF, 0x7F7F8000,
                        0x7F7FC000, 0x3F808000, 0x3F818000, 0x00008000, 0x00018000], np.uint32)
    f = np.concatenate([bits, ties, near, special]).view(np.float32)
    return f[~np.isnan(f)]


def test_bf16_codec_matches_the_oracle_codec():
    x = _f32_corpus()
    out = np.zeros(x.size, np.uint16)
    assert cpuc.run(_cast_kernel("F32", "Bf16"), x, out, x.size) == cpuc.OK
    assert np.array_equal(out, oracle.f32_to_bf16_bits(x))
    # F64 -> Bf16 rounds once from the double (narrow.rs exact encoder): equal to the oracle's
    # f32_to_bf16(f64_to_f32_odd(v)) (expr_eval.rs:503-527)
    d = np.random.default_rng(8).standard_normal(50000) * np.exp2(np.random.default_rng(9).integers(-140, 120, 50000))
    out = np.zeros(d.size, np.uint16)
    assert cpuc.run(_cast_kernel("F64", "Bf16"), d, out, d.size) == cpuc.OK
    lib = oracle.lib()
    want = np.array([lib.orc_store_bf16(float(v)) for v in d[:5000]], np.uint16)
    assert np.array_equal(out[:5000], want)
    # decode: every pattern
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = np.zeros(65536, np.float32)
    assert cpuc.run(_cast_kernel("Bf16", "F32"), pats, back, 65536) == cpuc.OK
    ref = (pats.astype(np.uint32) << 16).view(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(back[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(back[~ok]).all()


def test_f16_codec_matches_numpy():
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = np.zeros(65536, np.float32)
    assert cpuc.run(_cast_kernel("F16", "F32"), pats, back, 65536) == cpuc.OK
    ref = pats.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(back[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(back[~ok]).all()
    x = _f32_corpus()
    x = x[np.abs(x) < 1e6]
    out = np.zeros(x.size, np.uint16)
    assert cpuc.run(_cast_kernel("F32", "F16"), x, out, x.size) == cpuc.OK
    with np.errstate(over="ignore"):
        assert np.array_equal(out, x.astype(np.float16).view(np.uint16))


def test_out_of_bounds_access_returns_status_1():
    k = u.lift_reduction("oob", "F32", 2, "Sum")
    x = data("F32", (4, 8))
    out = np.zeros(4, np.float32)
    # the view says 4 x 7 while the extents say 4 x 8: the eighth column is outside the buffer
    assert cpuc.run(k, View(x, (4, 7), (8, 1)), out, 4, 8) == cpuc.OUT_OF_BOUNDS


def test_zero_loop_step_returns_status_2():
    k = _cast_kernel("F32", "F64")
    k["body"][0]["For"]["step"] = {"ConstInt": [0, "I32"]}
    assert cpuc.run(k, np.zeros(3, np.float32), np.zeros(3), 3) == cpuc.ZERO_STEP


def test_a_strided_view_is_read_through_its_strides():
    """The storage image carries signed strides and a base (oracle/buffers.rs:16-42): a transposed
    and a reversed view reduce like their dense copies."""
    x = data("F64", (6, 9))
    k = u.lift_reduction("sv", "F64", 2, "Sum")
    out = np.zeros(9)
    assert cpuc.run(k, View(x, (9, 6), (1, 9)), out, 9, 6) == cpuc.OK
    assert out.tobytes() == oracle.reduce_rows(np.ascontiguousarray(x.T), "Sum").tobytes()
    out = np.zeros(6)
    assert cpuc.run(k, View(x, (6, 9), (9, -1), 8), out, 6, 9) == cpuc.OK
    assert out.tobytes() == oracle.reduce_rows(np.ascontiguousarray(x[:, ::-1]), "Sum").tobytes()


def test_refusals_are_typed():
    k = u.lift_reduction("bad", "F32", 2, "Sum")
    bad = copy.deepcopy(k)
    bad["compute"] = "Fp8E4M3FN"
    with pytest.raises(cpuc.Declined) as e:
        cpuc.lower(bad)
    assert e.value.code == cpuc.UNSUPPORTED_KERNEL
    bad = copy.deepcopy(k)
    bad["body"].insert(0, {"Barrier": {"scope": "Block", "kind": "Full"}})
    with pytest.raises(cpuc.Declined) as e:
        cpuc.lower(bad)
    assert e.value.code == cpuc.UNSUPPORTED_KERNEL and "launch" in e.value.detail
    kl = u.lift_reduction("bad", "F32", 2, "Sum", launch=(2048, 1))
    with pytest.raises(cpuc.Declined) as e:
        cpuc.lower(kl)
    assert "threads" in e.value.detail
    with pytest.raises(cpuc.Declined) as e:
        cpuc.lower("{not json")
    assert e.value.code == cpuc.PARSE_ERROR


@pytest.mark.parametrize("dtype,op", [("F32", "MaxNum"), ("F64", "MinNum"), ("I32", "And"), ("I64", "Or"),
                                      ("I32", "Xor"), ("I64", "MaxNum")])
def test_sequential_only_folds_equal_the_oracle(dtype, op):
    x = data(dtype, (8, 29))
    if dtype[0] == "F":
        x[1, 0], x[2, :], x[3, 11] = np.nan, np.nan, np.nan
    k = u.lift_reduction("so", dtype, 2, op)
    out = np.zeros(8, NP[dtype])
    assert cpuc.run(k, x, out, 8, 29) == cpuc.OK
    assert np.array_equal(out, oracle.reduce_rows(x, op), equal_nan=dtype[0] == "F"), (dtype, op)


@pytest.mark.parametrize("dtype", ["F32", "F64", "I64"])
@pytest.mark.parametrize("axis", [0, 1, 2])
def test_scans_along_any_axis_equal_the_oracle(dtype, axis):
    """The serial scan lift along each axis of a rank-3 input (lift_scan_opdef, kernel_lift.rs:504-519):
    the oracle scans the same elements with that axis moved last."""
    x = data(dtype, (3, 4, 5))
    ops = ("Sum", "Max", "Min", "Prod") + (("Mean",) if dtype[0] == "F" else ())
    for op in ops:
        for exclusive, reverse in ((False, False), (True, True)):
            k = u.lift_scan("sa", dtype, 3, op, axis=axis, exclusive=exclusive, reverse=reverse)
            out = np.zeros_like(x)
            assert cpuc.run(k, x, out, 3, 4, 5) == cpuc.OK
            xm = np.ascontiguousarray(np.moveaxis(x, axis, -1))
            want = np.moveaxis(oracle.scan_rows(xm.reshape(-1, xm.shape[-1]), op, exclusive, reverse).reshape(xm.shape),
                               -1, axis)
            assert out.tobytes() == np.ascontiguousarray(want).tobytes(), (op, exclusive, reverse)


@pytest.mark.parametrize("axis", [0, 1, 2])
@pytest.mark.parametrize("oob", ["Skip", "ZeroFill", "Clamp"])
def test_gather_along_any_axis_equals_the_oracle(axis, oob):
    t = RNG.integers(0, 2**16, (3, 8, 5), dtype=np.uint16)
    V = t.shape[axis]
    ids = RNG.integers(-2, V + 2, 6).astype(np.int32)
    osh = t.shape[:axis] + (6,) + t.shape[axis + 1:]
    strides = tuple(1 if d == axis else 0 for d in range(3))
    init = RNG.integers(0, 2**16, osh, dtype=np.uint16)
    for launch in (None, (32, 2)):
        out = init.copy()
        k = u.lift_gather("ga", "Bf16", 3, "I32", axis, oob, launch=launch)
        assert cpuc.run(k, t, View(ids, osh, strides), out, *osh, V) == cpuc.OK
        assert np.array_equal(out, oracle.gather_axis(t, ids, axis, oob, out_init=init)), launch
