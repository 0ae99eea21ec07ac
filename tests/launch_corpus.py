"""The reference's shared cross-emitter corpus for Backend::lower_kernel (launch_cases.rs:137-180),
restated: four launched elementwise kernels over F32, I32 and U32, grid-strided so the launch is
smaller than the data, with the corpus's own deterministic inputs (launch_cases.rs:72-99).

The expected outputs come from the oracle (``oracle.elementwise``), which follows the kernel
evaluator's rounding model the corpus states (launch_cases.rs:14-27): a statement evaluated in f64
and rounded once.  ``ulps`` is the corpus's tolerance for an emitter that rounds per operation; an
emitter that evaluates in f64 (as the HIP backend does) meets every case at 0.
"""
from __future__ import annotations

import numpy as np


def elementwise_launched(name: str, dtype: str, rank: int, body: dict, block: int, grid: int) -> dict:
    """lift_elementwise_opdef_launched (kernel_lift.rs:145, grid_stride_outermost :256-285) for two
    inputs: loads of in0/in1 at the counters, the body stored to out, the outermost loop grid-strided."""
    r = rank
    i32 = lambda v: {"ConstInt": [v, "I32"]}  # noqa: E731
    coords = [{"Local": r + d} for d in range(r)]
    inner = [{"Load": {"local": 2 * r + k, "place": {"Logical": {"buffer": k, "coords": coords}}}} for k in range(2)]
    inner.append({"Store": {"place": {"Logical": {"buffer": 2, "coords": coords}}, "value": body}})
    blk = inner
    for d in reversed(range(r)):
        blk = [{"For": {"local": r + d, "start": i32(0), "end": {"Local": d}, "step": i32(1), "unroll": "None",
                        "body": blk}}]
    cast = lambda e: {"Cast": [e, {"to": "I32", "round": "NearestEven", "sat": "Wrap"}]}  # noqa: E731
    ex = lambda i: {"Exec": {i: 0}}  # noqa: E731
    blk[0]["For"]["start"] = cast({"Add": [{"Mul": [ex("BlockIdx"), ex("BlockDim")]}, ex("ThreadIdx")]})
    blk[0]["For"]["step"] = cast({"Mul": [ex("GridDim"), ex("BlockDim")]})
    params = [{"name": f"in{k}", "kind": {"Buffer": {"elem": dtype, "role": "Read", "rank": r}}} for k in range(2)]
    params.append({"name": "out", "kind": {"Buffer": {"elem": dtype, "role": "Write", "rank": r}}})
    params += [{"name": f"n{d}", "kind": {"Scalar": {"ty": "I32", "local": d}}} for d in range(r)]
    locals_ = [{"elem": "I32", "lanes": 1}] * (2 * r) + [{"elem": dtype, "lanes": 1}] * 2
    return {"name": name, "compute": dtype, "params": params, "locals": locals_, "body": blk,
            "launch": {"block": [block, 1, 1], "grid": [grid, 1, 1], "subgroup": None, "cluster": None,
                       "devices": 1, "grid_dims": None},
            "allocs": [], "result": None, "results": []}


def launch_cases():
    """The corpus's four cases: (name, dtype, shape, (block, grid), ulps, body over the loaded locals,
    numpy f64 model of the body)."""

    def case(name, dtype, shape, launch, ulps, body, ref):
        r = len(shape)
        la, lb = {"Local": 2 * r}, {"Local": 2 * r + 1}
        return name, dtype, shape, launch, ulps, body(la, lb), ref

    ab = lambda x: {"Unary": ["Abs", x]}  # noqa: E731
    return [
        case("fma_shape", "F32", (5, 7), (4, 2), 3, lambda x, y: {"Add": [{"Mul": [ab(x), ab(y)]}, ab(x)]},
             lambda x, y: np.abs(x.astype(np.float64)) * np.abs(y) + np.abs(x)),
        case("div", "F32", (6, 5), (8, 2), 0, lambda x, y: {"Div": [x, y]}, lambda x, y: x.astype(np.float64) / y),
        case("sub", "I32", (3, 11), (8, 1), 0, lambda x, y: {"Sub": [x, y]}, lambda x, y: x - y),
        case("add", "U32", (37,), (16, 3), 0, lambda x, y: {"Add": [x, y]}, lambda x, y: x + y),
    ]


def corpus_pattern(dtype: str, n: int, seed: int) -> np.ndarray:
    """pattern (launch_cases.rs:72-85): x_i = ((i * 7919 + seed * 104729) mod 2003) / 97 - 10, as F32
    (rounded to nearest) or as I32 truncated toward zero (the same bytes read as U32)."""
    i = np.arange(n, dtype=np.int64)
    x = ((i * 7919 + seed * 104729) % 2003).astype(np.float64) / 97.0 - 10.0
    if dtype == "F32":
        return x.astype(np.float32)
    v = np.trunc(x).astype(np.int32)
    return v if dtype == "I32" else v.view(np.uint32)


def corpus_args(dtype: str, shape) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The case's arguments (launch_cases.rs:88-99, 110-115): in0 from seed 1, in1 from seed 2, a
    zeroed output, all dense row-major."""
    n = int(np.prod(shape))
    x = corpus_pattern(dtype, n, 1).reshape(shape)
    y = corpus_pattern(dtype, n, 2).reshape(shape)
    return x, y, np.zeros(shape, x.dtype)


def over_inputs(body: dict, rank: int) -> dict:
    """A corpus body with its loaded locals (2r, 2r + 1) read back as Input(0), Input(1)."""
    if isinstance(body, dict):
        if list(body) == ["Local"] and body["Local"] >= 2 * rank:
            return {"Input": body["Local"] - 2 * rank}
        return {k: over_inputs(v, rank) for k, v in body.items()}
    if isinstance(body, list):
        return [over_inputs(v, rank) for v in body]
    return body
