"""unpopped-hip: the MI355X (gfx950) backend for the Unpopped kernel generator.

The host side mirrors the reference's two seams over the C ABI (``include/unpopped_hip.h``):

* :class:`HipBackend` is ``trait Backend`` (crates/unpopped/src/backend.rs:668-807);
* :class:`HipCompiler` is ``trait Compiler`` (crates/unpopped/src/jit.rs:271-285);
* :class:`Executor` and :class:`DeviceBuffer` are the consumer's launch layer, which the
  reference leaves out by rule and this backend provides as a thin FFI over the HIP runtime.

Nothing here computes on the CPU: every result comes from a HIP kernel, and a missing
library raises.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import UnpError, check

ELEMENT_KINDS = {
    "F16": 0, "Bf16": 1, "F32": 2, "F32Strict": 3, "F64": 4, "I8": 5, "I16": 6, "U8": 7,
    "U16": 8, "I32": 9, "I64": 10, "Bool": 11, "Fp8E4M3FN": 12, "Fp8E4M3FNUZ": 13,
    "Fp8E5M2": 14, "F8E8M0": 15, "F8E6M2": 16, "Fp8E5M2FNUZ": 17, "I4": 18, "U4": 19, "B1": 20,
    "Complex64": 21, "Complex128": 22, "U32": 23, "U64": 24, "F4E2M1": 25, "F6E2M3": 26,
    "F6E3M2": 27,
}
REDUCE_OPS = {"Sum": 0, "Prod": 1, "Max": 2, "Min": 3, "Mean": 4, "And": 5, "Or": 6, "Xor": 7, "MaxNum": 8,
              "MinNum": 9}
OOB_POLICIES = {"Skip": 0, "ZeroFill": 1, "Clamp": 2}
SCHEDULES = {"device": 0, "serial": 1, "fixed": 2}
# VariantFidelity (backend.rs:204-309), in declaration order.
FIDELITIES = ["BitIdentical", "DeterministicallyDivergent", "Nondeterministic", "MorePrecise"]
FORMS = {"reduction": 0, "scan": 1, "gather": 2, "dequant4": 3, "row_reduce2": 4, "row_reduce": 5, "dequant_gemm": 6}
DTYPE_SUPPORT = {0: "Supported", 1: "Unsupported", 2: "NotExpressible"}
ARTIFACT_KINDS = {0: "Ptx", 1: "Cubin", 2: "HipCodeObject", 3: "SpirV", 4: "Stub"}


@dataclass
class GeneratedKernel:
    """``GeneratedKernel`` (backend.rs:105-193): name, source text and launch interface."""

    name: str
    source: str
    interface: dict
    _handle: C.c_void_p

    def revision_hash(self) -> int:
        """FNV-1a 64 over the source (crates/unpopped/src/revision.rs)."""
        return int(_lib.lib().unp_generated_revision_hash(self._handle))

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h:
            _lib.lib().unp_generated_free(h)
            self._handle = None


class HipBackend:
    """The ``Backend`` seam for ``rocm:gfx950``."""

    def name(self) -> str:
        return _lib.lib().unp_hip_name().decode()

    def provider(self) -> str:
        return _lib.lib().unp_hip_provider().decode()

    def total_integer_ops(self) -> bool:
        return bool(_lib.lib().unp_hip_total_integer_ops())

    def supports_dtype(self, dtype: str, target: str) -> str:
        return DTYPE_SUPPORT[_lib.lib().unp_hip_supports_dtype(ELEMENT_KINDS[dtype], target.encode())]

    def lower_form(self, kind: str, dtype: str = "F32", rank: int = 1, op: str = "Sum",
                   op1: str = "Max", reduced_from: int | None = None, exclusive: bool = False,
                   reverse: bool = False, index_dtype: str = "I32", oob: str = "ZeroFill",
                   data_slot: int = 0, q_kind: str = "U4", z_kind: str = "U4", group: int = 128,
                   out_kind: str = "Bf16", axes: tuple | None = None, schedule: str = "device") -> GeneratedKernel:
        """Lower one form (``unp_hip_lower_form``); ``schedule`` is ``"device"`` (this backend's
        device-class schedule), ``"serial"`` (the serial lift's own order) or ``"fixed"`` (the device
        schedule with every float association fixed by the tiling: the same bits on every launch)."""
        return self._wrap(lambda out, err: _lib.lib().unp_hip_lower_form(
            C.byref(self.form(kind, dtype, rank, op, op1, reduced_from, exclusive, reverse, index_dtype, oob,
                              data_slot, q_kind, z_kind, group, out_kind, axes, schedule)), out, err))

    @staticmethod
    def form(kind: str, dtype: str = "F32", rank: int = 1, op: str = "Sum", op1: str = "Max",
             reduced_from: int | None = None, exclusive: bool = False, reverse: bool = False,
             index_dtype: str = "I32", oob: str = "ZeroFill", data_slot: int = 0, q_kind: str = "U4",
             z_kind: str = "U4", group: int = 128, out_kind: str = "Bf16", axes: tuple | None = None,
             schedule: str = "device") -> "_lib.Form":
        """The C ABI's unp_form for these fields."""
        f = _lib.Form()
        f.kind = FORMS[kind]
        f.dtype = ELEMENT_KINDS[dtype]
        f.rank = rank
        f.op0 = REDUCE_OPS[op]
        f.op1 = REDUCE_OPS[op1]
        f.reduced_from = (rank - 1) if reduced_from is None else reduced_from
        f.exclusive = int(exclusive)
        f.reverse = int(reverse)
        f.index_dtype = ELEMENT_KINDS[index_dtype]
        f.oob = OOB_POLICIES[oob]
        f.data_slot = data_slot
        f.q_kind = ELEMENT_KINDS[q_kind]
        f.z_kind = ELEMENT_KINDS[z_kind]
        f.group = group
        f.out_kind = ELEMENT_KINDS[out_kind]
        f.axes_mask = sum(1 << d for d in axes) if axes else 0
        f.schedule = SCHEDULES[schedule]
        return f

    def form_variants(self, **form) -> list[dict]:
        """Backend::lower_variants for a form (``unp_hip_form_variants``): each schedule this backend
        has for the cell, the default first, with its fidelity and the GeneratedKernel it lowers to."""
        f = self.form(**form)
        cap = 8
        arr = (_lib.Variant * cap)()
        n = C.c_size_t()
        err = _lib.Error()
        check(_lib.lib().unp_hip_form_variants(C.byref(f), arr, cap, C.byref(n), C.byref(err)), err)
        out = []
        for v in arr[:min(n.value, cap)]:
            fv = _lib.Form.from_buffer_copy(v.form)
            g = self._wrap(lambda o, e, fv=fv: _lib.lib().unp_hip_lower_form(C.byref(fv), o, e))
            out.append({"tag": v.tag.decode(), "fidelity": FIDELITIES[v.fidelity],
                        "schedule": [k for k, s in SCHEDULES.items() if s == v.form.schedule][0],
                        "launch_note": v.launch_note.decode(), "kernel": g})
        return out

    def lower_kernel(self, kernel) -> GeneratedKernel:
        """``Backend::lower_kernel`` (backend.rs:726-737): ``kernel`` is a KernelFn as its serde
        JSON (a ``str``) or as the parsed ``dict``."""
        text = kernel if isinstance(kernel, str) else json.dumps(kernel)
        return self._wrap(lambda out, err: _lib.lib().unp_hip_lower_kernel(text.encode(), out, err))

    @staticmethod
    def _wrap(call) -> GeneratedKernel:
        L = _lib.lib()
        out = C.c_void_p()
        err = _lib.Error()
        check(call(C.byref(out), C.byref(err)), err)
        return GeneratedKernel(
            name=L.unp_generated_name(out).decode(),
            source=L.unp_generated_source(out).decode(),
            interface=json.loads(L.unp_generated_interface_json(out).decode()),
            _handle=out,
        )


def _lifted(call) -> dict:
    out = C.c_void_p()
    err = _lib.Error()
    check(call(C.byref(out), C.byref(err)), err)
    try:
        return json.loads(C.string_at(out).decode())
    finally:
        _lib.lib().unp_free_str(out)


def _geom(launch) -> tuple[int, int]:
    return (0, 0) if launch is None else (int(launch[0]), int(launch[1]))


def lift_reduction(name: str, dtype: str, rank: int, op: str, axes: tuple = (), keepdim: bool = False,
                   launch: tuple | None = None, n_inputs: int = 1, body=None, post=None) -> dict:
    """The reduction lift (serial, or launched on ``launch = (block, grid)``) as a KernelFn dict.
    ``body`` is the pre-map over ``Input(0..n_inputs)`` (default ``Input(0)``) and ``post`` a fused
    post over ``Reduced(0)`` (default the identity), each an ``expr.Expr`` or its serde dict."""
    mask = 0
    for d in axes:
        mask |= 1 << d
    b, g = _geom(launch)
    if body is None and post is None and n_inputs == 1:
        return _lifted(lambda o, e: _lib.lib().unp_lift_reduction(name.encode(), ELEMENT_KINDS[dtype], rank,
                                                                 REDUCE_OPS[op], mask, int(keepdim), b, g, o, e))
    from . import expr as X

    bj = json.dumps(X.as_json(X.input(0) if body is None else body)).encode()
    pj = None if post is None else json.dumps(X.as_json(post)).encode()
    return _lifted(lambda o, e: _lib.lib().unp_lift_reduction_x(name.encode(), ELEMENT_KINDS[dtype], rank,
                                                               REDUCE_OPS[op], mask, int(keepdim), n_inputs, bj, pj,
                                                               b, g, o, e))


def lift_scan(name: str, dtype: str, rank: int, op: str, axis: int | None = None, exclusive: bool = False,
              reverse: bool = False, launch: tuple | None = None, n_inputs: int = 1, pre=None, post=None) -> dict:
    """The scan lift (serial, or launched on ``launch = (block, grid)``) as a KernelFn dict.  ``pre``
    is the pre-map over ``Input(0..n_inputs)`` (default ``Input(0)``) and ``post`` a fused post over
    ``Reduced(0)`` (the prefix rounded once) and the position's ``Input(k)`` (default the identity),
    each an ``expr.Expr`` or its serde dict."""
    b, g = _geom(launch)
    ax = rank - 1 if axis is None else axis
    if pre is None and post is None and n_inputs == 1:
        return _lifted(lambda o, e: _lib.lib().unp_lift_scan(name.encode(), ELEMENT_KINDS[dtype], rank,
                                                            REDUCE_OPS[op], ax, int(exclusive), int(reverse), b, g,
                                                            o, e))
    from . import expr as X

    pj = json.dumps(X.as_json(X.input(0) if pre is None else pre)).encode()
    qj = None if post is None else json.dumps(X.as_json(post)).encode()
    return _lifted(lambda o, e: _lib.lib().unp_lift_scan_x(name.encode(), ELEMENT_KINDS[dtype], rank, REDUCE_OPS[op],
                                                          ax, int(exclusive), int(reverse), n_inputs, pj, qj, b, g,
                                                          o, e))


def lift_gather(name: str, dtype: str, rank: int, index_dtype: str = "I32", axis: int = 0, oob: str = "ZeroFill",
                launch: tuple | None = None, n_inputs: int = 2, data: int = 0, index: int = 1, body=None) -> dict:
    """The gather lift as a KernelFn dict: by default OpDef::gather (data Input(0), index Input(1), the
    identity body); in general ``n_inputs`` inputs with the ``data`` and ``index`` slots and ``body`` an
    elementwise expression over them (an ``expr.Expr`` or its serde dict)."""
    b, g = _geom(launch)
    if body is not None or n_inputs != 2 or data != 0 or index != 1:
        from . import expr as X

        bj = json.dumps(X.as_json(X.input(data) if body is None else body)).encode()
        return _lifted(lambda o, e: _lib.lib().unp_lift_gather_x(
            name.encode(), ELEMENT_KINDS[dtype], rank, ELEMENT_KINDS[index_dtype], axis, OOB_POLICIES[oob],
            n_inputs, data, index, bj, b, g, o, e))
    return _lifted(lambda o, e: _lib.lib().unp_lift_gather(name.encode(), ELEMENT_KINDS[dtype], rank,
                                                          ELEMENT_KINDS[index_dtype], axis, OOB_POLICIES[oob],
                                                          b, g, o, e))


def lift_elementwise(name: str, dtype: str, rank: int, body, n_inputs: int = 1, perms=None,
                     launch: tuple | None = None) -> dict:
    """The Access::Elementwise lift (kernel_lift.rs:96-153; serial, or launched on ``launch = (block,
    grid)``) as a KernelFn dict: ``body`` over ``Input(0..n_inputs)`` (an ``expr.Expr`` or its serde
    dict) stored at the output coordinate.  ``perms`` (one axis list per input, or None) reads input k
    through View::Permute: iteration axis d reads its axis ``perms[k][d]``."""
    from . import expr as X

    b, g = _geom(launch)
    bj = json.dumps(X.as_json(body)).encode()
    pp = None
    if perms is not None:
        flat = [int(a) for p in perms for a in p]
        pp = (C.c_int32 * max(1, len(flat)))(*flat)
    return _lifted(lambda o, e: _lib.lib().unp_lift_elementwise(name.encode(), ELEMENT_KINDS[dtype], rank, n_inputs,
                                                               bj, pp, b, g, o, e))


def kernel_row_reduce2(name: str, dtype: str, op0: str = "Sum", op1: str = "Max", launch: tuple | None = None) -> dict:
    b, g = _geom(launch)
    return _lifted(lambda o, e: _lib.lib().unp_kernel_row_reduce2(name.encode(), ELEMENT_KINDS[dtype],
                                                                 REDUCE_OPS[op0], REDUCE_OPS[op1], b, g, o, e))


def kernel_dequant4(name: str, q_kind: str = "U4", z_kind: str = "U4", group: int = 128,
                    launch: tuple | None = None) -> dict:
    b, g = _geom(launch)
    return _lifted(lambda o, e: _lib.lib().unp_kernel_dequant4(name.encode(), ELEMENT_KINDS[q_kind],
                                                              ELEMENT_KINDS[z_kind], group, b, g, o, e))


def kernel_dequant_gemm(name: str, w_kind: str = "U4", x_kind: str = "I32", group: int = 128,
                        launch: tuple | None = None) -> dict:
    """The dequantizing GEMM (crates/unpopped/tests/support/dequant.rs:104-181) as a KernelFn dict:
    buffers w (``w_kind``), zero, scale (I32), x (``x_kind``: I32 or I8), out (I32), scalars R, K, C."""
    b, g = _geom(launch)
    return _lifted(lambda o, e: _lib.lib().unp_kernel_dequant_gemm(name.encode(), ELEMENT_KINDS[w_kind],
                                                                  ELEMENT_KINDS[x_kind], group, b, g, o, e))


def lift_row_reduce(name: str, dtype: str, rank: int, stages, epilogue, n_inputs: int = 1,
                    launch: tuple | None = None) -> dict:
    """The Access::RowReduce lift (serial, or launched on ``launch = (block, grid)``) as a KernelFn
    dict.  ``stages`` is a list of ``(pre, op)`` with ``pre`` a ScalarExpr (an ``expr.Expr`` or its
    serde dict) over ``Input(k)`` and earlier ``Reduced(t)``; ``epilogue`` the full-width output."""
    from . import expr as X

    b, g = _geom(launch)
    st = json.dumps([{"pre": X.as_json(pre), "op": op} for pre, op in stages])
    ep = json.dumps(X.as_json(epilogue))
    return _lifted(lambda o, e: _lib.lib().unp_lift_row_reduce(name.encode(), ELEMENT_KINDS[dtype], rank, n_inputs,
                                                              st.encode(), ep.encode(), b, g, o, e))


class HipCompiler:
    """The ``Compiler`` seam: hipRTC for gfx950, artifacts are HIP code objects."""

    def compile(self, source: str, entry: str, max_compile_ms: int = 0) -> bytes:
        L = _lib.lib()
        data = C.POINTER(C.c_uint8)()
        n = C.c_size_t()
        diag = C.c_void_p()
        rc = L.unp_hip_compile(source.encode(), entry.encode(), max_compile_ms, C.byref(data),
                               C.byref(n), C.byref(diag))
        log = C.string_at(diag).decode(errors="replace") if diag.value else ""
        if diag.value:
            L.unp_free_str(diag)
        if rc != _lib.OK:
            raise UnpError(rc, log)
        try:
            return C.string_at(data, n.value)
        finally:
            L.unp_free_bytes(data)

    def artifact_kind(self) -> str:
        return ARTIFACT_KINDS[_lib.lib().unp_hip_artifact_kind()]


def device_count() -> int:
    n = C.c_int32()
    _lib.lib().unp_hip_device_count(C.byref(n))
    return int(n.value)


def device_info() -> tuple[str, int]:
    arch = C.create_string_buffer(128)
    cus = C.c_int32()
    check(_lib.lib().unp_hip_device_info(arch, 128, C.byref(cus)), what="unp_hip_device_info")
    return arch.value.decode(), int(cus.value)


def synchronize() -> None:
    check(_lib.lib().unp_hip_synchronize(), what="hipDeviceSynchronize")


class DeviceBuffer:
    """Device memory from ``hipMalloc``, with host copies through numpy arrays."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(_lib.lib().unp_hip_malloc(C.byref(p), self.nbytes), what=f"hipMalloc({nbytes})")
        self.ptr = int(p.value)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 1))
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        if a.nbytes:
            check(_lib.lib().unp_hip_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), what="hipMemcpy H2D")

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(_lib.lib().unp_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), what="hipMemcpy D2H")
        return out

    def fill(self, byte: int) -> None:
        check(_lib.lib().unp_hip_memset(self.ptr, byte, self.nbytes), what="hipMemset")

    def at(self, offset: int) -> "DeviceBuffer":
        """A view ``offset`` bytes into this buffer; it does not own the memory and keeps this
        buffer alive."""
        assert 0 <= offset <= self.nbytes
        v = DeviceBuffer.__new__(DeviceBuffer)
        v.nbytes, v.ptr, v._owner = self.nbytes - offset, self.ptr + offset, self
        return v

    def free(self) -> None:
        if getattr(self, "_owner", None) is not None:
            self.ptr, self._owner = 0, None
            return
        if self.ptr:
            _lib.lib().unp_hip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Executor:
    """A lowered kernel compiled, loaded and ready to launch on the current device."""

    def __init__(self, kernel: GeneratedKernel):
        self.kernel = kernel
        h = C.c_void_p()
        err = _lib.Error()
        check(_lib.lib().unp_hip_exec_create(kernel._handle, C.byref(h), C.byref(err)), err)
        self._h = h

    @staticmethod
    def _args(args):
        arr = (_lib.Arg * len(args))()
        for i, a in enumerate(args):
            if isinstance(a, DeviceBuffer):
                arr[i].is_buffer, arr[i].value = 1, a.ptr
            else:
                arr[i].is_buffer, arr[i].value = 0, int(a) & 0xFFFFFFFFFFFFFFFF
        return arr

    def launch(self, *args, stream: int = 0) -> None:
        """Arguments in the KernelFn's parameter order: buffers, then integer scalars."""
        err = _lib.Error()
        check(_lib.lib().unp_hip_exec_launch(self._h, self._args(args), len(args), stream, C.byref(err)), err)

    def launch_static(self, *args, stream: int = 0) -> None:
        """``launch`` with every workspace in the library's static device scratch
        (``unp_hip_exec_launch_static``): no allocation; a launch whose workspace does not fit is an
        INVALID_ARGUMENT error.  Calls that overlap on one GPU share the scratch and race."""
        err = _lib.Error()
        check(_lib.lib().unp_hip_exec_launch_static(self._h, self._args(args), len(args), stream, C.byref(err)),
              err)

    def launch_views(self, views, scalars, stream: int = 0) -> None:
        """The buffers as storage images: ``views`` is a list of ``(buffer, shape, strides, base)``
        in the KernelFn's buffer order (strides None: dense row-major; strides and base in
        elements), ``scalars`` the integer parameters after them."""
        arr = (_lib.View * len(views))()
        for i, (buf, shape, strides, base) in enumerate(views):
            shape = list(shape)
            if strides is None:
                strides, acc = [0] * len(shape), 1
                for d in range(len(shape) - 1, -1, -1):
                    strides[d], acc = acc, acc * shape[d]
            arr[i].data, arr[i].rank, arr[i].base = buf.ptr, len(shape), int(base)
            for d, (n, st) in enumerate(zip(shape, strides)):
                arr[i].shape[d], arr[i].stride[d] = int(n), int(st)
        sc = (C.c_int64 * max(len(scalars), 1))(*[int(v) for v in scalars])
        err = _lib.Error()
        check(_lib.lib().unp_hip_exec_launch_views(self._h, arr, len(views), sc, len(scalars), stream, C.byref(err)),
              err)

    def set_timing(self, start: "Event | None", end: "Event | None") -> None:
        """Record ``start``/``end`` from the first and last kernel's own dispatch timestamps on every
        later launch (``None, None`` stops)."""
        check(_lib.lib().unp_hip_exec_set_timing(self._h, start._h if start else None, end._h if end else None),
              what="set_timing")

    def set_wait_limit(self, wait_us: int) -> None:
        """Bound every wait of a kernel for another block of its launch to ``wait_us`` microseconds
        (default 1 s; 0 gives up at the first unanswered probe): a wait that runs out goes on with the
        fold's identity and is counted for ``check``."""
        check(_lib.lib().unp_hip_exec_set_wait_limit(self._h, int(wait_us)), what="set_wait_limit")

    def check(self) -> None:
        """Wait for the device; raise ``UnpError`` ("Stalled") when a launch since the last check
        gave up a wait, so its outputs are not valid (the count is then cleared)."""
        err = _lib.Error()
        check(_lib.lib().unp_hip_exec_check(self._h, C.byref(err)), err)

    def last_launch(self) -> dict:
        g = (C.c_uint32 * 3)()
        b = (C.c_uint32 * 3)()
        name = C.create_string_buffer(256)
        _lib.lib().unp_hip_exec_last_launch(self._h, g, b, name, 256)
        return {"grid": list(g), "block": list(b), "entry": name.value.decode()}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.lib().unp_hip_exec_destroy(h)
            self._h = None


class Event:
    def __init__(self):
        h = C.c_void_p()
        check(_lib.lib().unp_hip_event_create(C.byref(h)), what="hipEventCreate")
        self._h = h

    def record(self, stream: int = 0) -> None:
        check(_lib.lib().unp_hip_event_record(self._h, stream), what="hipEventRecord")

    def synchronize(self) -> None:
        check(_lib.lib().unp_hip_event_synchronize(self._h), what="hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(_lib.lib().unp_hip_event_elapsed_ms(self._h, end._h, C.byref(ms)), what="hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.lib().unp_hip_event_destroy(h)
            self._h = None
