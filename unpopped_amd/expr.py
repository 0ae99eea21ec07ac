"""ScalarExpr builders: the reference's expression vocabulary (crates/unpopped/src/ir.rs:235-420,
`input`, `konst`, `reduced` and the operator overloads of `Expr`) as the serde JSON the KernelFn
carries, for building row-reduction ops in Python."""
from __future__ import annotations

import math


class Expr:
    """A ScalarExpr as its serde dict, with the arithmetic operators and the unary/binary ops."""

    def __init__(self, j: dict):
        self.j = j

    def _bin(self, tag: str, other) -> "Expr":
        return Expr({tag: [self.j, as_json(other)]})

    def __add__(self, o): return self._bin("Add", o)
    def __sub__(self, o): return self._bin("Sub", o)
    def __mul__(self, o): return self._bin("Mul", o)
    def __truediv__(self, o): return self._bin("Div", o)
    def __radd__(self, o): return Expr({"Add": [as_json(o), self.j]})
    def __rsub__(self, o): return Expr({"Sub": [as_json(o), self.j]})
    def __rmul__(self, o): return Expr({"Mul": [as_json(o), self.j]})
    def __rtruediv__(self, o): return Expr({"Div": [as_json(o), self.j]})
    def __neg__(self): return self.unary("Neg")

    def unary(self, op: str) -> "Expr":
        return Expr({"Unary": [op, self.j]})

    def binary(self, op: str, other) -> "Expr":
        return Expr({"Binary": [op, self.j, as_json(other)]})

    def exp(self): return self.unary("Exp")
    def log(self): return self.unary("Log")
    def sqrt(self): return self.unary("Sqrt")
    def rsqrt(self): return self.unary("Rsqrt")
    def tanh(self): return self.unary("Tanh")
    def sigmoid(self): return self.unary("Sigmoid")
    def abs(self): return self.unary("Abs")
    def maximum(self, o): return self.binary("Max", o)
    def minimum(self, o): return self.binary("Min", o)


def konst(v: float) -> Expr:
    """Const(f64); a non-finite value is its string tag (crates/unpopped/src/text.rs:241-276)."""
    v = float(v)
    if math.isnan(v):
        return Expr({"Const": "NaN"})
    if math.isinf(v):
        return Expr({"Const": "inf" if v > 0 else "-inf"})
    return Expr({"Const": v})


def input(k: int) -> Expr:  # noqa: A001 - the reference's name
    return Expr({"Input": int(k)})


def reduced(t: int) -> Expr:
    return Expr({"Reduced": int(t)})


def fma(a, b, c) -> Expr:
    return Expr({"Fma": [as_json(a), as_json(b), as_json(c)]})


def select(c, a, b) -> Expr:
    return Expr({"Select": [as_json(c), as_json(a), as_json(b)]})


def as_json(e) -> dict:
    if isinstance(e, Expr):
        return e.j
    if isinstance(e, (int, float)):
        return konst(e).j
    if isinstance(e, dict):
        return e
    raise TypeError(f"not a ScalarExpr: {e!r}")


# The row reductions of the reference's tests (crates/unpopped/tests/kernel_row_reduce_agrees.rs:112-139).
def softmax():
    return [(input(0), "Max"), ((input(0) - reduced(0)).exp(), "Sum")], (input(0) - reduced(0)).exp() / reduced(1)


def centred_quotient():
    return [(input(0), "Mean"), (input(0) - reduced(0), "Max")], (input(0) - reduced(0)) / reduced(1)


def rms_norm(eps: float = 1.0e-3):
    return [(input(0) * input(0), "Mean")], input(0) / (reduced(0) + konst(eps)).sqrt()
