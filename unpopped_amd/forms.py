"""Run one lowered form on the GPU through the C ABI: numpy in, numpy out.

Used by the GPU parity tests, the smoke check and the benchmark; every result comes
from a HIP kernel launched by ``unp_hip_exec_launch``.
"""
from __future__ import annotations

import numpy as np

import unpopped_amd as u

_backend = u.HipBackend()
_execs: dict = {}

# The KernelFn a caller hands the backend: the reference's launched lift at a caller-chosen
# geometry (the backend substitutes its own device-class launch and says so in the interface).
CALLER_LAUNCH = (256, 64)
SEQUENTIAL_ONLY = ("And", "Or", "Xor", "MaxNum", "MinNum")


def kernel_for(kind: str, dtype: str = "F32", rank: int = 1, op: str = "Sum", op1: str = "Max",
               reduced_from: int | None = None, exclusive: bool = False, reverse: bool = False,
               index_dtype: str = "I32", oob: str = "ZeroFill", q_kind: str = "U4", z_kind: str = "U4",
               group: int = 128, axes: tuple | None = None, keepdim: bool = False, axis: int | None = None,
               **_ignored) -> dict:
    """The KernelFn (as its serde JSON dict) of the lift or authored kernel for a form."""
    if kind == "reduction":
        k = rank - 1 if reduced_from is None else reduced_from
        ax = tuple(range(k, rank)) if axes is None else tuple(axes)
        # The bit and NaN-ignoring folds, and a float Prod, lift only sequentially
        # (kernel_lift/block_reduce.rs:97-133).
        serial = op in SEQUENTIAL_ONLY or (op == "Prod" and dtype in ("F32", "F64"))
        launch = None if serial else CALLER_LAUNCH
        return u.lift_reduction("reduce", dtype, rank, op, axes=ax, keepdim=keepdim, launch=launch)
    if kind == "row_reduce2":
        return u.kernel_row_reduce2("row_fold", dtype, op, op1, launch=CALLER_LAUNCH)
    if kind == "scan":
        # A scan along a non-innermost axis, a Mean scan and a float Prod scan lift only sequentially
        # (kernel_lift.rs:689-695, kernel_lift/scan_launched.rs:66-75).
        ax = rank - 1 if axis is None else axis
        serial = ax != rank - 1 or op == "Mean" or (op == "Prod" and dtype in ("F32", "F64"))
        return u.lift_scan("scan", dtype, rank, op, axis=ax, exclusive=exclusive, reverse=reverse,
                           launch=None if serial else CALLER_LAUNCH)
    if kind == "gather":
        return u.lift_gather("gather", dtype, rank, index_dtype, 0 if axis is None else axis, oob, launch=CALLER_LAUNCH)
    if kind == "dequant4":
        return u.kernel_dequant4("dequant", q_kind, z_kind, group, launch=CALLER_LAUNCH)
    if kind == "dequant_gemm":
        return u.kernel_dequant_gemm("dequant_gemm", q_kind, dtype, group, launch=CALLER_LAUNCH)
    raise ValueError(kind)

NP_KIND = {np.float32: "F32", np.float64: "F64", np.int32: "I32", np.int64: "I64", np.uint32: "U32",
           np.uint16: "Bf16", np.uint8: "U8", np.int8: "I8"}


def executor(**form) -> u.Executor:
    """Lift the form's KernelFn, lower it with Backend::lower_kernel, compile and load it."""
    key = tuple(sorted(form.items()))
    if key not in _execs:
        _execs[key] = u.Executor(_backend.lower_kernel(kernel_for(**form)))
    return _execs[key]


def say(msg: str) -> None:
    print(msg, flush=True)


def reduce_rows(x: np.ndarray, op: str, op1: str | None = None):
    """Fold each row of a 2-D array (op1: a second fold of the same read, ROW_REDUCE2)."""
    rows, cols = x.shape
    kind = NP_KIND[x.dtype.type]
    two = op1 is not None
    ex = executor(kind="row_reduce2" if two else "reduction", dtype=kind, rank=2, op=op,
                  op1=op1 or "Max", reduced_from=1)
    din = u.DeviceBuffer.from_array(x)
    o0 = u.DeviceBuffer(max(rows, 1) * x.itemsize)
    if two:
        o1 = u.DeviceBuffer(max(rows, 1) * x.itemsize)
        ex.launch(din, o0, o1, rows, cols)
    else:
        ex.launch(din, o0, rows, cols)
    u.synchronize()
    r0 = o0.download(x.dtype, rows)
    return (r0, o1.download(x.dtype, rows)) if two else r0


def reduce_axes(x: np.ndarray, axes: tuple, op: str, keepdim: bool = False) -> np.ndarray:
    """Fold `x` over the axes in `axes` (any set) with the reduction lift of that axis set."""
    kind = NP_KIND[x.dtype.type]
    axes = tuple(sorted(axes))
    ex = executor(kind="reduction", dtype=kind, rank=x.ndim, op=op, axes=axes, keepdim=keepdim)
    kept = tuple(n for d, n in enumerate(x.shape) if d not in axes)
    outs = int(np.prod(kept, dtype=np.int64))
    din = u.DeviceBuffer.from_array(x)
    dout = u.DeviceBuffer(max(outs * x.itemsize, 1))
    ex.launch(din, dout, *x.shape)
    ex.check()
    got = dout.download(x.dtype, outs)
    shape = tuple(1 if d in axes else n for d, n in enumerate(x.shape)) if keepdim else kept
    return got.reshape(shape)


def reduce_expr_executor(dtype: str, rank: int, op: str, axes: tuple, body, post=None, n_inputs: int = 1,
                         keepdim: bool = False) -> u.Executor:
    """The reduction lift with a pre-map body and a fused post, lowered, compiled and loaded."""
    import json

    from . import expr as X

    key = ("reduce_expr", dtype, rank, op, tuple(axes), keepdim, n_inputs, json.dumps(X.as_json(body)),
           json.dumps(X.as_json(post)) if post is not None else None)
    if key not in _execs:
        k = u.lift_reduction("reduce", dtype, rank, op, axes=tuple(axes), keepdim=keepdim, launch=CALLER_LAUNCH,
                             n_inputs=n_inputs, body=body, post=post)
        _execs[key] = u.Executor(_backend.lower_kernel(k))
    return _execs[key]


def reduce_expr(inputs, axes: tuple, op: str, body, post=None, keepdim: bool = False) -> np.ndarray:
    """Fold `body` over the inputs (one shape, float32/float64) along `axes`, then `post`."""
    xs = [np.ascontiguousarray(a) for a in inputs]
    x0 = xs[0]
    axes = tuple(sorted(axes))
    ex = reduce_expr_executor(NP_KIND[x0.dtype.type], x0.ndim, op, axes, body, post, len(xs), keepdim)
    kept = tuple(n for d, n in enumerate(x0.shape) if d not in axes)
    outs = int(np.prod(kept, dtype=np.int64))
    dins = [u.DeviceBuffer.from_array(a) for a in xs]
    dout = u.DeviceBuffer(max(outs * x0.itemsize, 1))
    ex.launch(*dins, dout, *x0.shape)
    ex.check()
    got = dout.download(x0.dtype, outs)
    return got.reshape(tuple(1 if d in axes else n for d, n in enumerate(x0.shape)) if keepdim else kept)


def reduce_all(x: np.ndarray, op: str):
    kind = NP_KIND[x.dtype.type]
    ex = executor(kind="reduction", dtype=kind, rank=1, op=op, reduced_from=0)
    din = u.DeviceBuffer.from_array(x)
    out = u.DeviceBuffer(16)
    ex.launch(din, out, x.size)
    ex.check()
    return out.download(x.dtype, 1)[0]


def scan_rows(x: np.ndarray, op: str, exclusive=False, reverse=False) -> np.ndarray:
    x2 = x.reshape(1, -1) if x.ndim == 1 else x
    rows, cols = x2.shape
    kind = NP_KIND[x.dtype.type]
    ex = executor(kind="scan", dtype=kind, rank=2, op=op, exclusive=exclusive, reverse=reverse)
    din = u.DeviceBuffer.from_array(x2)
    dout = u.DeviceBuffer(max(x2.nbytes, 1))
    ex.launch(din, dout, rows, cols)
    ex.check()
    return dout.download(x.dtype, rows * cols).reshape(x.shape)


def scan_axis(x: np.ndarray, axis: int, op: str, exclusive=False, reverse=False) -> np.ndarray:
    """Scan ``x`` (any rank) along ``axis`` with the lift of that axis."""
    ex = executor(kind="scan", dtype=NP_KIND[x.dtype.type], rank=x.ndim, op=op, exclusive=exclusive,
                  reverse=reverse, axis=axis)
    din = u.DeviceBuffer.from_array(np.ascontiguousarray(x))
    dout = u.DeviceBuffer(max(x.nbytes, 1))
    ex.launch(din, dout, *x.shape)
    ex.check()
    return dout.download(x.dtype, x.size).reshape(x.shape)


def gather_rows(table: np.ndarray, ids: np.ndarray, oob: str, out_init: np.ndarray | None = None,
                src_extent: int | None = None, elem_kind: str | None = None) -> np.ndarray:
    """out[r] = table[clamp(ids[r])] under the policy; ``table`` is (V, ...) of any dtype."""
    n = ids.shape[0]
    inner = table.shape[1:]
    kind = elem_kind or NP_KIND[table.dtype.type]
    rank = 1 + len(inner)
    ex = executor(kind="gather", dtype=kind, rank=rank, index_dtype=NP_KIND[ids.dtype.type], oob=oob)
    dt = u.DeviceBuffer.from_array(table)
    di = u.DeviceBuffer.from_array(ids)
    out_shape = (n,) + inner
    out0 = np.zeros(out_shape, table.dtype) if out_init is None else out_init
    do = u.DeviceBuffer.from_array(out0)
    ext = table.shape[0] if src_extent is None else src_extent
    ex.launch(dt, di, do, n, *inner, ext)
    u.synchronize()
    return do.download(table.dtype, int(np.prod(out_shape))).reshape(out_shape)


def gather_axis(table: np.ndarray, ids: np.ndarray, axis: int, oob: str, out_init: np.ndarray | None = None,
                elem_kind: str | None = None) -> np.ndarray:
    """index_select: ``out`` takes ``table``'s shape with ``axis`` replaced by ``len(ids)``, and
    ``out[.., i, ..] = table[.., clamp(ids[i]), ..]`` under the policy (1-D ``ids``)."""
    kind = elem_kind or NP_KIND[table.dtype.type]
    ex = executor(kind="gather", dtype=kind, rank=table.ndim, index_dtype=NP_KIND[ids.dtype.type], oob=oob, axis=axis)
    out_shape = table.shape[:axis] + (ids.shape[0],) + table.shape[axis + 1:]
    out0 = np.zeros(out_shape, table.dtype) if out_init is None else out_init
    dt, di, do = (u.DeviceBuffer.from_array(np.ascontiguousarray(a)) for a in (table, ids, out0))
    ex.launch(dt, di, do, *out_shape, table.shape[axis])
    u.synchronize()
    return do.download(table.dtype, int(np.prod(out_shape))).reshape(out_shape)


def dequant4(q_packed, scales, zeros_packed, rows, cols, group, q_kind="U4", z_kind="U4") -> np.ndarray:
    ex = executor(kind="dequant4", q_kind=q_kind, z_kind=z_kind, group=group, out_kind="Bf16")
    dq = u.DeviceBuffer.from_array(q_packed)
    ds = u.DeviceBuffer.from_array(scales)
    dz = u.DeviceBuffer.from_array(zeros_packed)
    do = u.DeviceBuffer(max(rows * cols * 2, 1))
    ex.launch(dq, ds, dz, do, rows, cols)
    u.synchronize()
    return do.download(np.uint16, rows * cols).reshape(rows, cols)


def dequant_gemm(w_packed, zero, scale, x, rows, k, cols, group, w_kind="U4") -> np.ndarray:
    """out = sum_k (w - zero) * scale * x over I32 that wraps; x is I32 or I8 by its dtype."""
    x = np.ascontiguousarray(x)
    ex = executor(kind="dequant_gemm", q_kind=w_kind, dtype=NP_KIND.get(x.dtype.type, "I8"), group=group)
    dw = u.DeviceBuffer.from_array(np.ascontiguousarray(w_packed, np.uint8))
    dz = u.DeviceBuffer.from_array(np.ascontiguousarray(zero, np.int32))
    ds = u.DeviceBuffer.from_array(np.ascontiguousarray(scale, np.int32))
    dx = u.DeviceBuffer.from_array(x)
    do = u.DeviceBuffer(max(rows * cols * 4, 1))
    ex.launch(dw, dz, ds, dx, do, rows, k, cols)
    u.synchronize()
    return do.download(np.int32, rows * cols).reshape(rows, cols)


def row_reduce_executor(dtype: str, rank: int, stages, epilogue, n_inputs: int = 1) -> u.Executor:
    """The launched Access::RowReduce lift of these expressions, lowered, compiled and loaded."""
    import json

    from . import expr as X

    key = ("row_reduce", dtype, rank, n_inputs, json.dumps([(X.as_json(p), op) for p, op in stages]),
           json.dumps(X.as_json(epilogue)))
    if key not in _execs:
        k = u.lift_row_reduce("row_reduce", dtype, rank, stages, epilogue, n_inputs=n_inputs, launch=CALLER_LAUNCH)
        _execs[key] = u.Executor(_backend.lower_kernel(k))
    return _execs[key]


def row_reduce(inputs, stages, epilogue) -> np.ndarray:
    """Run a row reduction over the innermost axis of the inputs (same shape, float32/float64)."""
    xs = [np.ascontiguousarray(a) for a in inputs]
    x0 = xs[0]
    rank = max(x0.ndim, 1)
    ex = row_reduce_executor(NP_KIND[x0.dtype.type], rank, stages, epilogue, n_inputs=len(xs))
    dins = [u.DeviceBuffer.from_array(a) for a in xs]
    dout = u.DeviceBuffer(max(x0.nbytes, 1))
    ex.launch(*dins, dout, *(x0.shape if x0.ndim else (1,)))
    u.synchronize()
    return dout.download(x0.dtype, x0.size).reshape(x0.shape)


def scan_expr_executor(dtype: str, rank: int, op: str, axis: int, pre, post=None, n_inputs: int = 1,
                       exclusive: bool = False, reverse: bool = False, launch=CALLER_LAUNCH) -> u.Executor:
    """The scan lift with a pre-map and a fused post (launched on the innermost axis unless a Mean, a
    float Prod or another axis makes it the serial lift), lowered, compiled and loaded."""
    import json

    from . import expr as X

    serial = axis != rank - 1 or op in ("Mean", "Prod") or launch is None
    key = ("scan_expr", dtype, rank, op, axis, n_inputs, exclusive, reverse, serial, json.dumps(X.as_json(pre)),
           json.dumps(X.as_json(post)) if post is not None else None)
    if key not in _execs:
        k = u.lift_scan("scan", dtype, rank, op, axis=axis, exclusive=exclusive, reverse=reverse,
                        launch=None if serial else launch, n_inputs=n_inputs, pre=pre, post=post)
        _execs[key] = u.Executor(_backend.lower_kernel(k))
    return _execs[key]


def scan_expr(inputs, axis: int, op: str, pre, post=None, exclusive: bool = False, reverse: bool = False,
              launch=CALLER_LAUNCH) -> np.ndarray:
    """Scan `pre` over the inputs (one shape, float32/float64) along `axis`, then `post` per position."""
    xs = [np.ascontiguousarray(a) for a in inputs]
    x0 = xs[0]
    ex = scan_expr_executor(NP_KIND[x0.dtype.type], x0.ndim, op, axis, pre, post, len(xs), exclusive, reverse, launch)
    dins = [u.DeviceBuffer.from_array(a) for a in xs]
    dout = u.DeviceBuffer(max(x0.nbytes, 1))
    ex.launch(*dins, dout, *x0.shape)
    ex.check()
    return dout.download(x0.dtype, x0.size).reshape(x0.shape)
