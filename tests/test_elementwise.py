"""The Access::Elementwise form on the CPU: the oracle's integer rule pinned by boundary vectors with a
planted mistake per guard (docs/int-div-shift-semantics.md, "Proof obligations"), the float statement
model against numpy's f64, the lift restatement (kernel_lift.rs:96-153), lower_kernel's recognition
and its typed refusals, and the C99 leg against the oracle.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import oracle
import unpopped_amd as u
from oracle import cpuc
from tests.launch_corpus import corpus_args, launch_cases, over_inputs
from unpopped_amd import _lib

I = lambda k: {"Input": k}  # noqa: E741,E731
B = lambda op, a, b: {"Binary": [op, a, b]}  # noqa: E731
INT_DTYPES = ["I32", "I64", "U32", "U64"]


def width(dt):
    return 64 if dt in ("I64", "U64") else 32


def boundary(dt):
    """The boundary vectors (docs/int-div-shift-semantics.md, "Proof obligations"): dividends 0, 1, -1,
    MIN, MAX; divisors 0, 1, -1, MIN; counts 0, 1, N-1, N, N+1, 255, -1, each wrapped to the kind, plus
    a few ordinary values."""
    nt = oracle.NP_KINDS[dt]
    info = np.iinfo(nt)
    n = width(dt)
    vals = [0, 1, -1, int(info.min), int(info.max), 7, -7, 2, -2, n - 1, n, n + 1, 255, 3]
    m = 1 << n
    wrapped = sorted({(v % m) if dt[0] == "U" else ((v + m // 2) % m - m // 2) for v in vals})
    return np.array(wrapped, dtype=object).astype(nt)


def grid(dt):
    v = boundary(dt)
    x, y = np.meshgrid(v, v, indexing="ij")
    return x.ravel().copy(), y.ravel().copy()


def rem_body():
    """Integer remainder as the reference composes it: Select(b == 0, 0, a - (a / b) * b) over the
    total Div (docs/int-div-shift-semantics.md)."""
    return lambda dt: {"Select": [B("CmpEq", I(1), {"ConstInt": [0, dt]}), {"ConstInt": [0, dt]},
                                  {"Sub": [I(0), {"Mul": [{"Div": [I(0), I(1)]}, I(1)]}]}]}


# ---- known answers, from the rule's text (rules 1-3) ---------------------------------------

MIN32, MAX32, MIN64 = -(1 << 31), (1 << 31) - 1, -(1 << 63)
KNOWN = {
    "I32": [("Div", 7, 0, 7), ("Div", MIN32, -1, MIN32), ("Div", -7, 2, -3), ("Div", 7, -2, -3), ("Div", -1, MIN32, 0),
            ("Div", MIN32, MIN32, 1), ("Shl", 1, 31, MIN32), ("Shl", 1, 32, 1), ("Shl", 1, 33, 2), ("Shl", 1, -1, MIN32),
            ("Shl", 3, 255, MIN32), ("Shr", MIN32, 31, -1), ("Shr", MIN32, 32, MIN32), ("Shr", -8, 1, -4),
            ("Shr", -1, 255, -1), ("Shr", MAX32, -1, 0), ("Rem", MIN32, -1, 0), ("Rem", 7, 0, 0), ("Rem", -7, 2, -1),
            ("Rem", 7, -2, 1)],
    "U32": [("Div", 7, 0, 7), ("Div", 0xFFFFFFFF, 2, 0x7FFFFFFF), ("Shr", 0x80000000, 31, 1),
            ("Shr", 0x80000000, 0xFFFFFFFF, 1), ("Shl", 1, 32, 1), ("Shl", 1, 0xFFFFFFFF, 0x80000000), ("Rem", 7, 0, 0)],
    "I64": [("Div", MIN64, -1, MIN64), ("Div", 5, 0, 5), ("Div", -9, 4, -2), ("Shl", 1, 63, MIN64), ("Shl", 1, 64, 1),
            ("Shr", MIN64, 63, -1), ("Shr", MIN64, 64, MIN64), ("Shr", MIN64, -1, -1), ("Rem", MIN64, -1, 0)],
    "U64": [("Shr", 1 << 63, 63, 1), ("Shl", 1, 64, 1), ("Div", (1 << 64) - 1, 0, (1 << 64) - 1),
            ("Shr", 1 << 63, (1 << 64) - 1, 1)],
}


def body_of(op, dt):
    if op == "Div":
        return {"Div": [I(0), I(1)]}
    if op == "Rem":
        return rem_body()(dt)
    return B(op, I(0), I(1))


def known_red(dt, mutant=0):
    """The known answers the oracle (with `mutant` planted) gets wrong."""
    nt = oracle.NP_KINDS[dt]
    bad = []
    for op, x, y, want in KNOWN[dt]:
        got = oracle.elementwise([np.array([x]).astype(nt), np.array([y]).astype(nt)], body_of(op, dt), dt,
                                 mutant=mutant)
        if int(got[0]) != int(np.array([want]).astype(nt)[0]):
            bad.append((op, x, y, int(got[0]), want))
    return bad


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_oracle_integer_rule_known_answers(dt):
    assert known_red(dt) == []


@pytest.mark.parametrize("mutant", [oracle.MUT_DIV0, oracle.MUT_MINNEG1, oracle.MUT_CLAMP, oracle.MUT_LOGICAL,
                                    oracle.MUT_FLOOR])
def test_every_planted_mistake_turns_a_known_answer_red(mutant):
    """A mutation check per guard: dropping the zero-divisor guard, the MIN / -1 guard or the count
    mask, a logical Shr on a signed kind, or a flooring Div each disagrees with a known answer."""
    assert any(known_red(dt, mutant) for dt in INT_DTYPES)
    assert any(known_red(dt, mutant) for dt in ("I32", "I64")) or mutant == oracle.MUT_DIV0


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_oracle_integer_div_is_the_truncating_quotient(dt):
    """Away from the two defined cases the quotient truncates toward zero: x = q * y + r with |r| < |y|
    and r zero or of x's sign (Python integers, no division rule restated)."""
    x, y = grid(dt)
    q = oracle.elementwise([x, y], {"Div": [I(0), I(1)]}, dt)
    lo = int(np.iinfo(oracle.NP_KINDS[dt]).min)
    for a, b, c in zip(x.tolist(), y.tolist(), q.tolist()):
        if b == 0:
            assert c == a
        elif lo < 0 and a == lo and b == -1:
            assert c == a
        else:
            r = a - c * b
            assert abs(r) < abs(b) and (r == 0 or (r < 0) == (a < 0)), (a, b, c)


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_oracle_integer_shifts_match_numpy_and_wrap_the_count(dt):
    """Shl/Shr by a count c equal the shift by c mod N (N = 64 for a 64-bit kind, else 32), and for an
    in-range count numpy's own shift of the same kind (arithmetic >> on a signed kind)."""
    nt = oracle.NP_KINDS[dt]
    ut = np.uint64 if width(dt) == 64 else np.uint32
    x, y = grid(dt)
    n = width(dt)
    k = (y.astype(ut) & ut(n - 1)).astype(nt)
    for op in ("Shl", "Shr"):
        got = oracle.elementwise([x, y], B(op, I(0), I(1)), dt)
        assert np.array_equal(got, oracle.elementwise([x, k], B(op, I(0), I(1)), dt)), op
        if op == "Shl":
            native = np.left_shift(x.astype(ut), k.astype(ut)).astype(nt)
        else:
            native = np.right_shift(x, k.astype(nt))
        assert np.array_equal(got, native), op


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_oracle_integer_ring_ops_match_numpy(dt):
    """Add, Sub and Mul wrap exactly as numpy's fixed-width arrays do; Min, Max and the bitwise ops
    act on the kind's values."""
    x, y = grid(dt)
    with np.errstate(over="ignore"):
        ref = {"Add": x + y, "Sub": x - y, "Mul": x * y}
    for op, want in ref.items():
        assert np.array_equal(oracle.elementwise([x, y], {op: [I(0), I(1)]}, dt), want), op
    for op, want in {"Min": np.minimum(x, y), "Max": np.maximum(x, y), "BitAnd": x & y, "BitOr": x | y,
                     "BitXor": x ^ y}.items():
        assert np.array_equal(oracle.elementwise([x, y], B(op, I(0), I(1)), dt), want), op


@pytest.mark.parametrize("dt", INT_DTYPES)
def test_oracle_integer_remainder_composition_is_checked_rem_or_zero(dt):
    """Select(b == 0, 0, a - (a / b) * b) is Rust's checked_rem(..).unwrap_or(0): 0 for a zero divisor
    and for MIN % -1, else the remainder with the dividend's sign."""
    x, y = grid(dt)
    got = oracle.elementwise([x, y], rem_body()(dt), dt)
    lo = int(np.iinfo(oracle.NP_KINDS[dt]).min)
    for a, b, c in zip(x.tolist(), y.tolist(), got.tolist()):
        want = 0 if b == 0 or (lo < 0 and a == lo and b == -1) else (abs(a) % abs(b)) * (1 if a >= 0 else -1)
        assert c == want, (a, b, c, want)


def test_oracle_select_evaluates_the_comparison_at_the_operands_type():
    """A comparison inside an I32 body yields the compute type's 1 or 0 (types.rs:735-737); a Select
    tests its condition != 0."""
    x = np.array([5, -3, 0, 9], np.int32)
    y = np.array([5, 2, 0, -9], np.int32)
    body = {"Select": [B("CmpLt", I(0), I(1)), {"ConstInt": [100, "I32"]}, B("CmpGe", I(0), I(1))]}
    assert oracle.elementwise([x, y], body, "I32").tolist() == [1, 100, 1, 1]


@pytest.mark.parametrize("case", launch_cases(), ids=lambda c: c[0])
def test_oracle_float_statement_model_matches_numpy_f64(case):
    """The oracle's float elementwise (the body in f64, one rounding at the store) equals numpy computing
    the same expression in float64 and casting once, on the corpus's inputs and on normal values with
    zero denominators."""
    name, dtype, shape, _, _, body, ref = case
    b = over_inputs(body, len(shape))
    x, y, _ = corpus_args(dtype, shape)
    samples = [(x, y)]
    if dtype == "F32":
        r = np.random.default_rng(3)
        xs, ys = r.normal(size=shape).astype(np.float32), r.normal(size=shape).astype(np.float32)
        ys.ravel()[::4] = 0
        samples.append((xs, ys))
    for a, c in samples:
        with np.errstate(all="ignore"):
            want = np.asarray(ref(a, c)).astype(a.dtype)
        got = oracle.elementwise([a, c], b, dtype)
        assert np.array_equal(got, want, equal_nan=True), name


def test_oracle_permuted_read_is_numpy_transpose():
    """View::Permute: iteration axis d reads the input's axis perm[d] (kernel_lift.rs:315-324)."""
    r = np.random.default_rng(5)
    a = r.normal(size=(3, 4, 5))
    bsrc = r.normal(size=(5, 3, 4))  # its axes (2, 0, 1) are the iteration axes
    got = oracle.elementwise([a, bsrc], {"Sub": [I(0), I(1)]}, "F64", perms=[[0, 1, 2], [1, 2, 0]])
    assert np.array_equal(got, a - np.transpose(bsrc, (1, 2, 0)))


# ---- the lift and lower_kernel ---------------------------------------------------------------

def test_lift_elementwise_serial_and_permuted_shapes():
    """The serial lift nests the axes outermost first, loads each input at the counters (a permuted one
    at its permuted coordinates) and stores the body at the counters (kernel_lift.rs:96-130)."""
    k = u.lift_elementwise("e", "F32", 2, {"Add": [I(0), I(1)]}, n_inputs=2, perms=[[0, 1], [1, 0]])
    assert k["launch"] is None
    inner = k["body"][0]["For"]["body"][0]["For"]["body"]
    assert inner[0]["Load"]["place"]["Logical"]["coords"] == [{"Local": 2}, {"Local": 3}]
    assert inner[1]["Load"]["place"]["Logical"]["coords"] == [{"Local": 3}, {"Local": 2}]
    assert inner[2]["Store"]["value"] == {"Add": [{"Local": 4}, {"Local": 5}]}
    assert [p["name"] for p in k["params"]] == ["in0", "in1", "out", "n0", "n1"]
    with pytest.raises(_lib.UnpError) as e:
        u.lift_elementwise("e", "F32", 2, {"Add": [I(0), I(1)]}, n_inputs=2, perms=[[0, 1], [1, 1]])
    assert "view" in str(e.value)
    with pytest.raises(_lib.UnpError):
        u.lift_elementwise("e", "F32", 2, {"Add": [I(0), I(2)]}, n_inputs=2)


def test_lower_kernel_takes_serial_permuted_and_renumbered_elementwise_kernels():
    b = u.HipBackend()
    body = {"Mul": [I(0), {"Add": [I(1), I(2)]}]}
    k = u.lift_elementwise("e3", "F64", 3, body, n_inputs=3, perms=[[0, 1, 2], [2, 1, 0], [1, 0, 2]], launch=(64, 3))
    g = b.lower_kernel(k)
    assert g.interface["views"][1] == {"Permute": {"perm": [2, 1, 0]}} and g.interface["inputs"] == 3
    assert json.loads(g.interface["body"]) == body
    s = b.lower_kernel(u.lift_elementwise("s", "I64", 1, {"Div": [I(0), {"ConstInt": [-3, "I64"]}]}))
    assert s.interface["lift"] == "lift_elementwise_opdef"
    # the loaded locals numbered the other way round: the same kernel
    k2 = u.lift_elementwise("e2", "F32", 1, {"Sub": [I(0), I(1)]}, n_inputs=2, launch=(32, 2))
    swap = json.loads(json.dumps(k2).replace('{"Local": 2}', '{"Local": 9}').replace('{"Local": 3}', '{"Local": 2}')
                      .replace('{"Local": 9}', '{"Local": 3}').replace('"local": 2', '"local": 9')
                      .replace('"local": 3', '"local": 2').replace('"local": 9', '"local": 3'))
    assert swap != k2
    g2 = b.lower_kernel(swap)
    assert json.loads(g2.interface["body"]) == {"Sub": [I(0), I(1)]}


@pytest.mark.parametrize("dtype,body,kind", [
    ("I32", {"Unary": ["Neg", I(0)]}, "UnsupportedOp"),          # no integer Unary in eval_int
    ("F16", {"Add": [I(0), I(1)]}, "UnsupportedDtype"),           # bodies at F32/F64 and the integer kinds
    ("I8", {"Add": [I(0), I(1)]}, "UnsupportedDtype"),            # 8-bit operands stay leaf-only
    ("I32", {"Add": [I(0), {"ConstInt": [1, "I64"]}]}, "UnsupportedOp"),  # an ill-typed sum
    ("F32", {"Add": [I(0), {"ConstInt": [1, "I32"]}]}, "UnsupportedOp"),  # a mixed float body
    ("U4", {"Input": 1}, "UnsupportedDtype"),                     # a sub-byte move
])
def test_lower_kernel_refuses_what_it_cannot_spell_with_a_typed_error(dtype, body, kind):
    k = u.lift_elementwise("r", dtype, 1, body, n_inputs=2, launch=(64, 1))
    with pytest.raises(_lib.UnpError) as e:
        u.HipBackend().lower_kernel(k)
    assert e.value.kind == kind


def test_raw_moves_and_integer_bodies_compile_for_gfx950():
    b, cc = u.HipBackend(), u.HipCompiler()
    for dt in ("Bf16", "U8", "I16", "F16", "Complex128"):
        g = b.lower_kernel(u.lift_elementwise("mv", dt, 2, I(1), n_inputs=2, launch=(64, 2)))
        cc.compile(g.source, g.name)
    for dt in INT_DTYPES:
        body = {"Select": [B("CmpLt", I(0), I(1)), rem_body()(dt),
                           B("BitXor", B("Shl", I(0), I(1)), B("Shr", I(1), {"ConstInt": [3, dt]}))]}
        g = b.lower_kernel(u.lift_elementwise("ix", dt, 2, body, n_inputs=2, launch=(256, 4)))
        assert "unp::xi::div<" in g.source and "unp::xi::shl<" in g.source
        cc.compile(g.source, g.name)


# ---- the C99 leg against the oracle (the compiled C against the interpreter) -------------------

@pytest.mark.parametrize("dt", INT_DTYPES)
@pytest.mark.parametrize("op", ["Div", "Shl", "Shr", "Rem", "Mul", "Sub"])
def test_c99_leg_meets_the_oracle_on_the_boundary_vectors(dt, op):
    x, y = grid(dt)
    body = body_of(op, dt) if op not in ("Mul", "Sub") else {op: [I(0), I(1)]}
    k = u.lift_elementwise("bv", dt, 1, body, n_inputs=2, launch=(32, 3))
    out = np.zeros_like(x)
    assert cpuc.run(k, x, y, out, x.size) == cpuc.OK
    assert out.tobytes() == oracle.elementwise([x, y], body, dt).tobytes()


# ---- integer pre-map bodies of reductions and scans (kernel_lift.rs:755-800) --------------------

@pytest.mark.parametrize("dt,nt", [("I32", np.int32), ("I64", np.int64)])
@pytest.mark.parametrize("op", ["Sum", "Prod", "Max", "Min", "Xor"])
def test_integer_body_reduction_oracle_meets_the_c99_leg(dt, nt, op):
    """The oracle's integer-body reduction (the integer evaluator's values folded by the serial lift)
    equals the C99 leg running the serial lifted kernel on boundary-heavy data."""
    x, y = grid(dt)
    side = int(round(np.sqrt(x.size)))
    xs = [x.reshape(side, side), y.reshape(side, side)]
    body = {"Add": [{"Div": [I(0), I(1)]}, B("Shl", I(1), I(0))]}
    k = u.lift_reduction("r", dt, 2, op, axes=(1,), n_inputs=2, body=body)
    out = np.zeros(side, nt)
    assert cpuc.run(k, *xs, out, side, side) == cpuc.OK
    assert out.tobytes() == oracle.int_reduce_expr(xs, (1,), op, body, dt).tobytes()


@pytest.mark.parametrize("dt,nt", [("I32", np.int32), ("I64", np.int64)])
@pytest.mark.parametrize("op", ["Sum", "Max"])
def test_integer_pre_scan_oracle_meets_the_c99_leg(dt, nt, op):
    x, y = grid(dt)
    side = int(round(np.sqrt(x.size)))
    xs = [x.reshape(side, side), y.reshape(side, side)]
    pre = {"Sub": [{"Mul": [I(0), I(1)]}, B("Shr", I(0), I(1))]}
    for excl, rev in ((False, False), (True, True)):
        k = u.lift_scan("s", dt, 2, op, exclusive=excl, reverse=rev, n_inputs=2, pre=pre)
        out = np.zeros((side, side), nt)
        assert cpuc.run(k, *xs, out, side, side) == cpuc.OK
        assert out.tobytes() == oracle.int_scan_expr(xs, 1, op, pre, dt, excl, rev).tobytes()


def test_integer_bodies_lower_with_the_integer_rule_and_refuse_a_post():
    b = u.HipBackend()
    body = {"Div": [I(0), I(1)]}
    g = b.lower_kernel(u.lift_reduction("r", "I64", 2, "Prod", axes=(1,), n_inputs=2, body=body, launch=(256, 4)))
    assert "unp::xi::div<long long>" in g.source and "integer rule" in g.interface["fidelity_notes"][0]
    s = b.lower_kernel(u.lift_scan("s", "I32", 1, "Sum", n_inputs=2, pre=body, launch=(256, 4)))
    assert s.interface["schedule"] == "device" and "integer rule" in s.interface["fidelity_notes"][0]
    with pytest.raises(_lib.UnpError) as e:
        u.lift_reduction("r", "I32", 1, "Sum", n_inputs=2, body=body,
                         post={"Add": [{"Reduced": 0}, {"ConstInt": [1, "I32"]}]})
    assert "post" in str(e.value)
    with pytest.raises(_lib.UnpError) as e:
        u.lift_scan("s", "I32", 1, "Sum", n_inputs=2, pre=body, post={"Add": [{"Reduced": 0}, I(0)]})
    assert "post" in str(e.value)
