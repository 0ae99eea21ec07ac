"""CPU oracle for the unpopped-hip hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this package, and only as the checker (or the timed CPU baseline); the product path never
calls it.  The C restatement is ``oracle.c`` (each function cites the reference file:line it
follows); this module binds it with ctypes and numpy.

Parity pinning: every function here is checked in ``tests/test_oracle.py`` against the
reference's own golden vectors where its tests hold them, and against closed forms, independent
library routines (numpy float16, torch bfloat16) or brute force otherwise.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

SUM, PROD, MAX, MIN, MEAN, AND, OR, XOR, MAXNUM, MINNUM = range(10)
OPS = {"Sum": SUM, "Prod": PROD, "Max": MAX, "Min": MIN, "Mean": MEAN, "And": AND, "Or": OR, "Xor": XOR,
       "MaxNum": MAXNUM, "MinNum": MINNUM}
SKIP, ZEROFILL, CLAMP = 0, 1, 2
POLICIES = {"Skip": SKIP, "ZeroFill": ZEROFILL, "Clamp": CLAMP}
IDX_KINDS = {"I32": 9, "I64": 10, "U32": 23}

_L = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _L
    if _L is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P, i64, i32, d, f = C.c_void_p, C.c_int64, C.c_int, C.c_double, C.c_float
        sig = {
            "orc_f32_to_bf16_bits": (C.c_uint16, [f]),
            "orc_bf16_to_f64": (d, [C.c_uint16]),
            "orc_f16_to_f64": (d, [C.c_uint16]),
            "orc_f32_to_f16_bits": (C.c_uint16, [f]),
            "orc_f64_to_f32_odd": (f, [d]),
            "orc_store_bf16": (C.c_uint16, [d]),
            "orc_f32_to_bf16_array": (None, [P, i64, P]),
            "orc_f16_to_f64_array": (None, [P, i64, P]),
            "orc_u4_load": (C.c_int32, [P, i64]),
            "orc_i4_load": (C.c_int32, [P, i64]),
            "orc_sub4_store": (None, [P, i64, C.c_int32]),
            "orc_reduce_rows_f32": (None, [P, i64, i64, i32, P]),
            "orc_reduce_rows_f64": (None, [P, i64, i64, i32, P]),
            "orc_reduce_rows_i32": (None, [P, i64, i64, i32, P]),
            "orc_reduce_rows_i64": (None, [P, i64, i64, i32, P]),
            "orc_sum_launched_order": (d, [P, i64, i64, i32]),
            "orc_rx_eval": (d, [P, C.c_int32, P, P, i32]),
            "orc_row_reduce": (None, [P, C.c_int32, i64, i64, i32, C.c_int32, P, P, P, P, C.c_int32, P]),
            "orc_scan_x": (None, [P, C.c_int32, i64, i64, i64, i32, i32, i32, i32, P, C.c_int32, P, C.c_int32, P]),
            "orc_sum_bound": (d, [P, i64, i32, i32, d]),
            "orc_neumaier": (d, [P, i64]),
            "orc_scan_rows_f32": (None, [P, i64, i64, i32, i32, i32, P]),
            "orc_scan_rows_f64": (None, [P, i64, i64, i32, i32, i32, P]),
            "orc_scan_rows_i32": (None, [P, i64, i64, i32, i32, i32, P]),
            "orc_scan_rows_i64": (None, [P, i64, i64, i32, i32, i32, P]),
            "orc_scan_launched_order_f32": (None, [P, i64, i64, i32, i32, P]),
            "orc_gather_rows": (None, [P, i64, i64, P, i32, i64, i32, P]),
            "orc_dequant4_bf16": (None, [P, i32, P, P, i32, i64, i64, i64, P]),
            "orc_dequant_gemm_i32": (None, [P, i32, P, P, P, i32, i64, i64, i64, i64, P]),
            "orc_elementwise_f": (None, [P, C.c_int32, i64, i32, P, C.c_int32, P]),
            "orc_elementwise_i": (None, [P, C.c_int32, i64, P, C.c_int32, C.c_int32, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _L = L
    return _L


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- codecs ---------------------------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_bf16_array(_p(x), x.size, _p(out))
    return out


def f16_to_f64(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float64)
    lib().orc_f16_to_f64_array(_p(h), h.size, _p(out))
    return out


# ---- reductions -----------------------------------------------------------------------

_RED = {np.float32: "orc_reduce_rows_f32", np.float64: "orc_reduce_rows_f64",
        np.int32: "orc_reduce_rows_i32", np.int64: "orc_reduce_rows_i64"}


def reduce_rows(x: np.ndarray, op: str) -> np.ndarray:
    """Fold each row of a 2-D array (the serial reduction lift's order and rounding)."""
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    out = np.empty(rows, x.dtype)
    getattr(lib(), _RED[x.dtype.type])(_p(x), rows, cols, OPS[op], _p(out))
    return out


def sum_launched_order(xs: np.ndarray, block: int, mean: bool = False) -> float:
    xs = np.ascontiguousarray(xs, dtype=np.float64)
    return lib().orc_sum_launched_order(_p(xs), xs.size, block, int(mean))


def sum_bound(xs: np.ndarray, got: float, mean: bool = False, f32: bool = True) -> float:
    xs = np.ascontiguousarray(xs, dtype=np.float64)
    return lib().orc_sum_bound(_p(xs), xs.size, int(mean), int(f32), float(got))


def neumaier(xs: np.ndarray) -> float:
    xs = np.ascontiguousarray(xs, dtype=np.float64)
    return lib().orc_neumaier(_p(xs), xs.size)


# ---- scans ----------------------------------------------------------------------------

_SCAN = {np.float32: "orc_scan_rows_f32", np.float64: "orc_scan_rows_f64",
         np.int32: "orc_scan_rows_i32", np.int64: "orc_scan_rows_i64"}


def scan_rows(x: np.ndarray, op: str, exclusive: bool = False, reverse: bool = False) -> np.ndarray:
    """Scan each row of a 2-D array along its last axis (the serial scan lift)."""
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    out = np.empty_like(x)
    getattr(lib(), _SCAN[x.dtype.type])(_p(x), rows, cols, OPS[op], int(exclusive), int(reverse), _p(out))
    return out


def scan_launched_order_f32(x: np.ndarray, block: int, exclusive=False, reverse=False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_scan_launched_order_f32(_p(x), x.size, block, int(exclusive), int(reverse), _p(out))
    return out


# ---- gather ---------------------------------------------------------------------------

def gather_rows(table: np.ndarray, ids: np.ndarray, policy: str, out_init: np.ndarray | None = None,
                src_extent: int | None = None) -> np.ndarray:
    """``out[r] = table[clamp(ids[r])]`` under the policy; rows are raw bytes."""
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids)
    ext = table.shape[0] if src_extent is None else src_extent
    row_bytes = table[0].nbytes if table.shape[0] else int(np.prod(table.shape[1:])) * table.itemsize
    n = ids.shape[0]
    out = (np.zeros((n,) + table.shape[1:], table.dtype) if out_init is None
           else np.ascontiguousarray(out_init).copy())
    kind = {np.int32: 9, np.int64: 10, np.uint32: 23}[ids.dtype.type]
    lib().orc_gather_rows(_p(table), ext, row_bytes, _p(ids), kind, n, POLICIES[policy], _p(out))
    return out


def gather_axis(table: np.ndarray, ids: np.ndarray, axis: int, policy: str,
                out_init: np.ndarray | None = None) -> np.ndarray:
    """index_select along ``axis`` with a 1-D index (the gather lift's cell, kernel_lift/gather.rs:184-232,
    at every coordinate of the other axes): the table seen as A x V x B, each of the A slices a row
    gather of B-element rows."""
    table = np.ascontiguousarray(table)
    V = table.shape[axis]
    A = int(np.prod(table.shape[:axis], dtype=np.int64))
    B = int(np.prod(table.shape[axis + 1:], dtype=np.int64))
    out_shape = table.shape[:axis] + (ids.shape[0],) + table.shape[axis + 1:]
    out = (np.zeros(out_shape, table.dtype) if out_init is None else np.array(out_init, copy=True)).reshape(
        A, ids.shape[0], B)
    t3 = table.reshape(A, V, B)
    for a in range(A):
        out[a] = gather_rows(t3[a], ids, policy, out_init=out[a], src_extent=V)
    return out.reshape(out_shape)


def gather_cells(table: np.ndarray, ids: np.ndarray, axis: int, policy: str, out_init: np.ndarray | None = None,
                 src_extent: int | None = None) -> np.ndarray:
    """The gather lift's cell at every output coordinate c (kernel_lift/gather.rs:184-232), with an
    index of the output's own shape (a storage image of any strides, not only the broadcast 1-D
    index): ``raw = ids[c]``; when ``0 <= raw < src_extent`` the cell stores ``table[c with axis :=
    raw]``; otherwise Skip leaves it, ZeroFill stores 0 and Clamp stores the row clamped into
    ``[0, src_extent - 1]``.  ``table`` has the output's extents except along ``axis``."""
    ids = np.asarray(ids)
    ext = table.shape[axis] if src_extent is None else int(src_extent)
    raw = ids.astype(np.int64)
    below = raw < 0
    oob = below | (raw >= ext)
    out = np.zeros(ids.shape, table.dtype) if out_init is None else np.array(out_init, copy=True)
    if policy == "Clamp":
        if ext < 1:
            raise ValueError("a Clamp gather needs a source extent of at least 1")
        take = np.ones(ids.shape, bool)
    else:
        take = ~oob
    cl = np.where(below, 0, np.where(oob, max(ext - 1, 0), raw))
    cl = np.where(take, cl, 0)
    if table.shape[axis] == 0:
        got = np.zeros(ids.shape, table.dtype)
    else:
        got = np.take_along_axis(table, cl, axis)
    out[take] = got[take]
    if policy == "ZeroFill":
        out[oob] = 0
    return out


def gather_expr(inputs, index: int, data: int, axis: int, policy: str, body, out_init: np.ndarray,
                src_extent: int) -> np.ndarray:
    """The gather lift's cell in general (kernel_lift/gather.rs:35-101, 184-232), one output cell at a
    time (small cases only): ``raw = inputs[index][c]``; out of ``[0, src_extent)`` Skip leaves the cell
    and ZeroFill stores 0; otherwise (and always under Clamp) every other input is read at ``c``, the
    gathered one with ``c[axis]`` replaced by the clamped index, and the body is evaluated on them
    (the index input as its value) at f64, rounded once to the output's dtype (rx_eval)."""
    out = np.array(out_init, copy=True)
    f32 = out.dtype == np.float32
    leaf = isinstance(body, dict) and list(body) == ["Input"]
    for c in np.ndindex(out.shape):
        raw = int(inputs[index][c])
        below = raw < 0
        oob = below or raw >= src_extent
        if oob and policy != "Clamp":
            if policy == "ZeroFill":
                out[c] = 0
            continue
        cl = 0 if below else (src_extent - 1 if oob else raw)
        vals = []
        for k, a in enumerate(inputs):
            if k == index:
                vals.append(raw)
            elif k == data:
                cc = list(c)
                cc[axis] = cl
                vals.append(a[tuple(cc)])
            else:
                vals.append(a[c])
        if leaf:
            out[c] = vals[int(body["Input"])]
        else:
            out[c] = rx_eval(body, np.array(vals, np.float64), f32=f32)
    return out


# ---- dequant --------------------------------------------------------------------------

def dequant4_bf16(q_packed: np.ndarray, scales_f16_bits: np.ndarray, zeros_packed: np.ndarray, rows: int,
                  cols: int, group: int, q_signed: bool = False, z_signed: bool = False) -> np.ndarray:
    q = np.ascontiguousarray(q_packed, dtype=np.uint8)
    s = np.ascontiguousarray(scales_f16_bits, dtype=np.uint16)
    z = np.ascontiguousarray(zeros_packed, dtype=np.uint8)
    out = np.empty(rows * cols, np.uint16)
    lib().orc_dequant4_bf16(_p(q), int(q_signed), _p(s), _p(z), int(z_signed), rows, cols, group, _p(out))
    return out.reshape(rows, cols)


def dequant_gemm_i32(w_packed: np.ndarray, zero: np.ndarray, scale: np.ndarray, x: np.ndarray, rows: int, k: int,
                     cols: int, group: int, w_signed: bool = False) -> np.ndarray:
    """The dequantizing GEMM (crates/unpopped/tests/support/dequant.rs:104-181), I32 arithmetic that
    wraps.  ``x`` is I32 (the reference's activations) or I8, by its numpy dtype."""
    w = np.ascontiguousarray(w_packed, dtype=np.uint8)
    z = np.ascontiguousarray(zero, dtype=np.int32)
    s = np.ascontiguousarray(scale, dtype=np.int32)
    x_i32 = np.asarray(x).dtype != np.int8
    xx = np.ascontiguousarray(x, dtype=np.int32 if x_i32 else np.int8)
    out = np.empty(rows * cols, np.int32)
    lib().orc_dequant_gemm_i32(_p(w), int(w_signed), _p(z), _p(s), _p(xx), int(x_i32), rows, k, cols, group, _p(out))
    return out.reshape(rows, cols)


# ---- row reduction -----------------------------------------------------------------------

ORC_UNARY_NAMES = ["Neg", "Abs", "Sqr", "Sqrt", "Rsqrt", "Recip", "Exp", "Log", "Tanh", "Sigmoid", "Relu", "Erf",
                   "Gelu", "Silu", "Sin", "Cos", "Floor", "Ceil", "Round", "Sign", "Step", "Erfc", "Trunc", "Exp2",
                   "Expm1", "Log2", "Log10", "Log1p", "Sinh", "Cosh", "Tan", "Asin", "Acos", "Atan", "Asinh", "Acosh",
                   "Atanh", "Cbrt"]
ORC_BINARY_NAMES = ["Max", "Min", "Pow", "Rem", "RemTrunc", "Atan2", "Copysign", "FmaxIeee", "FminIeee", "CmpEq",
                    "CmpNe", "CmpLt", "CmpLe", "CmpGt", "CmpGe"]


class RX(C.Structure):
    _fields_ = [("op", C.c_int32), ("arg", C.c_int32), ("c", C.c_double)]


def program(e) -> list[tuple[int, int, float]]:
    """A ScalarExpr (serde dict, or an ``unpopped_amd.expr.Expr``) as the C oracle's postfix
    program of (op, arg, const)."""
    if hasattr(e, "j"):
        e = e.j
    (tag, p), = e.items()
    if tag == "Input":
        return [(1, int(p), 0.0)]
    if tag == "Reduced":
        return [(2, int(p), 0.0)]
    if tag == "Const":
        v = {"NaN": float("nan"), "inf": float("inf"), "-inf": float("-inf")}.get(p, p) if isinstance(p, str) else p
        return [(3, 0, float(v))]
    arith = {"Add": 4, "Sub": 5, "Mul": 6, "Div": 7}
    if tag in arith:
        return program(p[0]) + program(p[1]) + [(arith[tag], 0, 0.0)]
    if tag in ("Fma", "Select"):
        return program(p[0]) + program(p[1]) + program(p[2]) + [(8 if tag == "Fma" else 9, 0, 0.0)]
    if tag == "Unary":
        return program(p[1]) + [(10, ORC_UNARY_NAMES.index(p[0]), 0.0)]
    if tag == "Binary":
        return program(p[1]) + program(p[2]) + [(11, ORC_BINARY_NAMES.index(p[0]), 0.0)]
    raise ValueError(f"the oracle has no {tag}")


def _rx_array(e):
    prog = program(e)
    depth = peak = 0
    for op, _, _ in prog:
        depth += 1 if op <= 3 else (0 if op == 10 else (-2 if op in (8, 9) else -1))
        peak = max(peak, depth)
    if peak > 64:
        raise ValueError("expression deeper than the oracle's stack")
    arr = (RX * len(prog))(*[RX(op, arg, c) for op, arg, c in prog])
    return arr, len(prog)


def rx_eval(e, x, red=(), f32: bool = True) -> float:
    arr, n = _rx_array(e)
    xs = np.ascontiguousarray(np.asarray(x, np.float64).reshape(-1))
    rs = np.ascontiguousarray(np.asarray(list(red) + [0.0], np.float64))
    return lib().orc_rx_eval(arr, n, _p(xs), _p(rs), int(f32))


def row_reduce(inputs, stages, epilogue) -> np.ndarray:
    """The serial lifted row reduction over the innermost axis of the inputs (all the same shape
    and dtype, float32 or float64); ``stages`` is [(pre, op)], ``epilogue`` the output expression."""
    xs = [np.ascontiguousarray(a) for a in inputs]
    dt = xs[0].dtype
    assert dt in (np.float32, np.float64) and all(a.dtype == dt and a.shape == xs[0].shape for a in xs)
    assert 1 <= len(xs) <= 16 and 1 <= len(stages) <= 16
    cols = xs[0].shape[-1] if xs[0].ndim else 1
    rows = xs[0].size // cols if cols else 0
    out = np.empty(xs[0].shape, dt)
    progs = [_rx_array(pre) for pre, _ in stages]
    ops = (C.c_int32 * len(stages))(*[OPS[op] for _, op in stages])
    pre_ptrs = (C.c_void_p * len(stages))(*[C.cast(a, C.c_void_p) for a, _ in progs])
    pre_lens = (C.c_int32 * len(stages))(*[n for _, n in progs])
    epi, epi_n = _rx_array(epilogue)
    ins = (C.c_void_p * len(xs))(*[_p(a) for a in xs])
    lib().orc_row_reduce(ins, len(xs), rows, cols, int(dt == np.float64), len(stages), ops, pre_ptrs, pre_lens, epi,
                         epi_n, _p(out))
    return out


def scan_expr(inputs, axis: int, op: str, pre, post=None, exclusive: bool = False, reverse: bool = False) -> np.ndarray:
    """The serial lifted scan of ``inputs`` (one shape, float32 or float64) along ``axis``: the
    pre-map evaluated in f64 and rounded once per position, the prefix rounded once, and the post
    (``None``: the identity) over that prefix and the position's inputs, rounded once at the store."""
    xs = [np.ascontiguousarray(a) for a in inputs]
    dt = xs[0].dtype
    assert dt in (np.float32, np.float64) and all(a.dtype == dt and a.shape == xs[0].shape for a in xs)
    assert 1 <= len(xs) <= 16
    shape = xs[0].shape
    a_ext = int(np.prod(shape[:axis], dtype=np.int64))
    b_ext = int(np.prod(shape[axis + 1:], dtype=np.int64))
    out = np.empty(shape, dt)
    pre_arr, pre_n = _rx_array(pre)
    post_arr, post_n = _rx_array(post) if post is not None else (None, 0)
    ins = (C.c_void_p * len(xs))(*[_p(a) for a in xs])
    lib().orc_scan_x(ins, len(xs), a_ext, shape[axis], b_ext, int(dt == np.float64), OPS[op], int(exclusive),
                     int(reverse), pre_arr, pre_n, post_arr, post_n, _p(out))
    return out


# ---- Access::Elementwise ---------------------------------------------------------------

NP_KINDS = {"F32": np.float32, "F64": np.float64, "I32": np.int32, "I64": np.int64, "U32": np.uint32,
            "U64": np.uint64, "I8": np.int8, "U8": np.uint8, "I16": np.int16, "U16": np.uint16,
            "F16": np.float16, "Bf16": np.uint16}
INT_KINDS = {"I32": 9, "I64": 10, "U32": 23, "U64": 24}
MUT_DIV0, MUT_MINNEG1, MUT_CLAMP, MUT_LOGICAL, MUT_FLOOR = 1, 2, 4, 8, 16
_IX = {"Input": 1, "ConstInt": 2, "Cast": 3, "Add": 4, "Sub": 5, "Mul": 6, "Div": 7, "Shl": 8, "Shr": 9,
       "Min": 10, "Max": 11, "BitAnd": 12, "BitOr": 13, "BitXor": 14, "Cmp": 15, "Select": 16}
_CMPS = ["CmpEq", "CmpNe", "CmpLt", "CmpLe", "CmpGt", "CmpGe"]


class IX(C.Structure):
    _fields_ = [("op", C.c_int32), ("arg", C.c_int32), ("kind", C.c_int32), ("pad", C.c_int32), ("v", C.c_int64)]


def int_type(e, compute: str) -> str:
    """The type of an integer expression node (crates/unpopped/src/types.rs:679-751 over the subset
    eval_int takes): an Input is the compute dtype, a ConstInt its kind, a Cast its target,
    arithmetic its operands' common type, a comparison the compute dtype, a Select its arms'."""
    if hasattr(e, "j"):
        e = e.j
    (tag, p), = e.items()
    if tag == "Input":
        return compute
    if tag == "ConstInt":
        return p[1]
    if tag == "Cast":
        return p[1]["to"]
    if tag in ("Add", "Sub", "Mul", "Div"):
        a, b = int_type(p[0], compute), int_type(p[1], compute)
    elif tag == "Binary":
        a, b = int_type(p[1], compute), int_type(p[2], compute)
        if a == b and p[0] in _CMPS:
            return compute
    elif tag == "Select":
        a, b = int_type(p[1], compute), int_type(p[2], compute)
    else:
        raise ValueError(f"the integer evaluator has no {tag}")
    if a != b:
        raise ValueError(f"{tag} of {a} and {b}")
    return a


def int_program(e, t: str, compute: str) -> list[tuple[int, int, int, int]]:
    """A ScalarExpr as the C oracle's typed postfix program (op, arg, kind, literal), each node at
    the kind eval_int (oracle/kernel_eval.rs:809-848) evaluates it at: `t` for an operand, its own
    type for a Cast's operand, a comparison's operands and a Select's condition."""
    if hasattr(e, "j"):
        e = e.j
    (tag, p), = e.items()
    k = INT_KINDS[t]
    own = lambda x: int_program(x, int_type(x, compute), compute)  # noqa: E731
    if tag == "Input":
        return [(1, int(p), k, 0)]
    if tag == "ConstInt":
        return [(2, 0, k, int(p[0]))]
    if tag == "Cast":
        if p[1].get("sat", "Wrap") != "Wrap" or p[1]["to"] != t:
            raise ValueError("only an integer wrap to the node's type")
        return own(p[0]) + [(3, 0, k, 0)]
    if tag in ("Add", "Sub", "Mul", "Div"):
        return int_program(p[0], t, compute) + int_program(p[1], t, compute) + [(_IX[tag], 0, k, 0)]
    if tag == "Binary":
        if p[0] in _CMPS:
            return own(p[1]) + own(p[2]) + [(15, _CMPS.index(p[0]), k, 0)]
        return int_program(p[1], t, compute) + int_program(p[2], t, compute) + [(_IX[p[0]], 0, k, 0)]
    if tag == "Select":
        return own(p[0]) + int_program(p[1], t, compute) + int_program(p[2], t, compute) + [(16, 0, k, 0)]
    raise ValueError(f"the integer evaluator has no {tag}")


def elementwise(inputs, body, dtype: str, perms=None, mutant: int = 0) -> np.ndarray:
    """The serial Access::Elementwise kernel (kernel_lift.rs:96-130) as the kernel evaluator runs it:
    input k is read through its View::Permute (iteration axis d reads its axis ``perms[k][d]``,
    counter_place :315-324), and the body is evaluated per output element -- in f64 and rounded once
    at the store for F32/F64 (orc_elementwise_f), by eval_int's total rule for I32/I64/U32/U64
    (orc_elementwise_i, ``mutant`` planting a mistake for the tests), or as a bit move of one input."""
    if hasattr(body, "j"):
        body = body.j
    xs = [np.asarray(a) if perms is None else np.transpose(np.asarray(a), perms[k]) for k, a in enumerate(inputs)]
    xs = [np.ascontiguousarray(a) for a in xs]
    shape = xs[0].shape
    if list(body) == ["Input"]:
        return xs[int(body["Input"])].copy()
    n = int(np.prod(shape, dtype=np.int64))
    if dtype in ("F32", "F64"):
        f64 = dtype == "F64"
        ys = [np.ascontiguousarray(a, np.float64 if f64 else np.float32) for a in xs]
        ptrs = (C.c_void_p * len(ys))(*[_p(a) for a in ys])
        arr, ln = _rx_array(body)
        out = np.empty(shape, np.float64 if f64 else np.float32)
        lib().orc_elementwise_f(ptrs, len(ys), n, int(f64), arr, ln, _p(out))
        return out
    if dtype not in INT_KINDS:
        raise ValueError(f"no elementwise body at {dtype}")
    prog = int_program(body, dtype, dtype)
    arr = (IX * len(prog))(*[IX(op, arg, kind, 0, v) for op, arg, kind, v in prog])
    ys = [np.ascontiguousarray(a.astype(NP_KINDS[dtype]).view(np.uint64) if dtype == "U64" else
                               a.astype(NP_KINDS[dtype]).astype(np.int64)).view(np.int64) for a in xs]
    ptrs = (C.c_void_p * len(ys))(*[_p(a) for a in ys])
    raw = np.empty(shape, np.int64)
    lib().orc_elementwise_i(ptrs, len(ys), n, arr, len(prog), int(mutant), _p(raw))
    if dtype == "U64":
        return raw.view(np.uint64)
    return raw.astype(NP_KINDS[dtype])


def int_reduce_expr(inputs, axes, op: str, body, dtype: str) -> np.ndarray:
    """The serial lifted reduction of an integer body (I32/I64; kernel_lift.rs:919-941 with
    `val = body`, no up-cast and no post): the body evaluated per position by eval_int's total rule
    (``elementwise``), then folded at the element type (``reduce_rows`` over the reduced axes moved
    last).  Integer folds wrap, so the fold's order does not change the bits."""
    v = elementwise(inputs, body, dtype)
    axes = tuple(sorted(axes))
    kept = [d for d in range(v.ndim) if d not in axes]
    t = np.ascontiguousarray(np.transpose(v, kept + list(axes)))
    rows = int(np.prod([v.shape[d] for d in kept], dtype=np.int64))
    cols = int(np.prod([v.shape[d] for d in axes], dtype=np.int64))
    return reduce_rows(t.reshape(rows, cols), op).reshape([v.shape[d] for d in kept])


def int_scan_expr(inputs, axis: int, op: str, pre, dtype: str, exclusive: bool = False,
                  reverse: bool = False) -> np.ndarray:
    """The serial lifted scan of an integer pre-map (I32/I64, identity post): the pre evaluated per
    position by the total rule, then scanned along ``axis`` at the element type (``scan_rows``)."""
    v = elementwise(inputs, pre, dtype)
    m = np.ascontiguousarray(np.moveaxis(v, axis, -1))
    out = scan_rows(m.reshape(-1, m.shape[-1]), op, exclusive, reverse).reshape(m.shape)
    return np.ascontiguousarray(np.moveaxis(out, -1, axis))
