"""ctypes binding of ``libunpopped_hip.so`` (declarations in ``include/unpopped_hip.h``).

The library is built in-tree by ``unpopped_amd/build.py``.  Loading fails loudly when it is
missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libunpopped_hip.so"

# enum unp_status
OK = 0
UNSUPPORTED_DTYPE = 1
UNSUPPORTED_SCHEDULE = 2
UNSUPPORTED_OP = 3
UNSUPPORTED_PLAN_SHAPE = 4
INADMISSIBLE_PLAN = 5
UNSUPPORTED_KERNEL = 6
LIFT_DECLINE = 10
COMPILE_ERROR = 20
HIP_ERROR = 30
STALLED = 31
INVALID_ARGUMENT = 40
PARSE_ERROR = 50

STATUS_NAMES = {
    OK: "Ok", UNSUPPORTED_DTYPE: "UnsupportedDtype", UNSUPPORTED_SCHEDULE: "UnsupportedSchedule",
    UNSUPPORTED_OP: "UnsupportedOp", UNSUPPORTED_PLAN_SHAPE: "UnsupportedPlanShape",
    INADMISSIBLE_PLAN: "InadmissiblePlan", UNSUPPORTED_KERNEL: "UnsupportedKernel",
    LIFT_DECLINE: "LiftDecline", COMPILE_ERROR: "CompileError", HIP_ERROR: "HipError", STALLED: "Stalled",
    INVALID_ARGUMENT: "InvalidArgument", PARSE_ERROR: "ParseError",
}


class Error(C.Structure):
    _fields_ = [("code", C.c_int32), ("detail", C.c_char * 512)]


class Form(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "kind", "dtype", "rank", "op0", "op1", "reduced_from", "exclusive", "reverse",
        "index_dtype", "oob", "data_slot", "q_kind", "z_kind", "group", "out_kind")] + [
        ("axes_mask", C.c_uint32), ("schedule", C.c_int32)]


class Variant(C.Structure):
    """unp_variant: Variant (backend.rs:313-353) as the backend describes it: a tag, a fidelity
    (VariantFidelity order), the form to lower and a launch note."""
    _fields_ = [("tag", C.c_char * 32), ("fidelity", C.c_int32), ("form", Form), ("launch_note", C.c_char * 256)]


class Arg(C.Structure):
    _fields_ = [("is_buffer", C.c_int32), ("pad", C.c_int32), ("value", C.c_uint64)]


MAX_RANK = 8


class View(C.Structure):
    """unp_view: a buffer as the reference's storage image (device address, rank, shape, signed
    element strides, base offset in elements)."""
    _fields_ = [("data", C.c_uint64), ("rank", C.c_int32), ("pad", C.c_int32), ("shape", C.c_int64 * MAX_RANK),
                ("stride", C.c_int64 * MAX_RANK), ("base", C.c_int64)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `python unpopped_amd/build.py`) first")
    L = C.CDLL(str(LIB_PATH))
    P = C.c_void_p
    i32, u32, u64, sz = C.c_int32, C.c_uint32, C.c_uint64, C.c_size_t
    E = C.POINTER(Error)
    sig = {
        "unp_hip_name": (C.c_char_p, []),
        "unp_hip_provider": (C.c_char_p, []),
        "unp_hip_total_integer_ops": (i32, []),
        "unp_hip_supports_dtype": (i32, [i32, C.c_char_p]),
        "unp_generated_name": (C.c_char_p, [P]),
        "unp_generated_source": (C.c_char_p, [P]),
        "unp_generated_interface_json": (C.c_char_p, [P]),
        "unp_generated_revision_hash": (u64, [P]),
        "unp_generated_free": (None, [P]),
        "unp_hip_lower_form": (i32, [C.POINTER(Form), C.POINTER(P), E]),
        "unp_hip_form_variants": (i32, [C.POINTER(Form), C.POINTER(Variant), sz, C.POINTER(sz), E]),
        "unp_hip_lower_kernel": (i32, [C.c_char_p, C.POINTER(P), E]),
        "unp_lift_reduction": (i32, [C.c_char_p, i32, i32, i32, u32, i32, u32, u32, C.POINTER(C.c_void_p), E]),
        "unp_lift_reduction_x": (i32, [C.c_char_p, i32, i32, i32, u32, i32, i32, C.c_char_p, C.c_char_p, u32, u32,
                                       C.POINTER(C.c_void_p), E]),
        "unp_lift_scan": (i32, [C.c_char_p, i32, i32, i32, i32, i32, i32, u32, u32, C.POINTER(C.c_void_p), E]),
        "unp_lift_scan_x": (i32, [C.c_char_p, i32, i32, i32, i32, i32, i32, i32, C.c_char_p, C.c_char_p, u32, u32,
                                  C.POINTER(C.c_void_p), E]),
        "unp_lift_gather": (i32, [C.c_char_p, i32, i32, i32, i32, i32, u32, u32, C.POINTER(C.c_void_p), E]),
        "unp_lift_elementwise": (i32, [C.c_char_p, i32, i32, i32, C.c_char_p, C.POINTER(i32), u32, u32,
                                       C.POINTER(C.c_void_p), E]),
        "unp_lift_gather_x": (i32, [C.c_char_p, i32, i32, i32, i32, i32, i32, i32, i32, C.c_char_p, u32, u32,
                                    C.POINTER(C.c_void_p), E]),
        "unp_kernel_row_reduce2": (i32, [C.c_char_p, i32, i32, i32, u32, u32, C.POINTER(C.c_void_p), E]),
        "unp_kernel_dequant4": (i32, [C.c_char_p, i32, i32, i32, u32, u32, C.POINTER(C.c_void_p), E]),
        "unp_kernel_dequant_gemm": (i32, [C.c_char_p, i32, i32, i32, u32, u32, C.POINTER(C.c_void_p), E]),
        "unp_lift_row_reduce": (i32, [C.c_char_p, i32, i32, i32, C.c_char_p, C.c_char_p, u32, u32,
                                      C.POINTER(C.c_void_p), E]),
        "unp_hip_compile": (i32, [C.c_char_p, C.c_char_p, u32, C.POINTER(C.POINTER(C.c_uint8)),
                                  C.POINTER(sz), C.POINTER(C.c_void_p)]),
        "unp_hip_artifact_kind": (i32, []),
        "unp_free_bytes": (None, [P]),
        "unp_free_str": (None, [P]),
        "unp_hip_device_count": (i32, [C.POINTER(i32)]),
        "unp_hip_set_device": (i32, [i32]),
        "unp_hip_device_info": (i32, [C.c_char_p, sz, C.POINTER(i32)]),
        "unp_hip_module_load": (i32, [P, sz, C.POINTER(P), E]),
        "unp_hip_module_unload": (i32, [P]),
        "unp_hip_get_function": (i32, [P, C.c_char_p, C.POINTER(P), E]),
        "unp_hip_launch": (i32, [P, C.POINTER(u32), C.POINTER(u32), u32, P, P, sz, E]),
        "unp_hip_launch_timed": (i32, [P, C.POINTER(u32), C.POINTER(u32), u32, P, P, sz, P, P, E]),
        "unp_hip_malloc": (i32, [C.POINTER(P), sz]),
        "unp_hip_free": (i32, [P]),
        "unp_hip_memcpy_h2d": (i32, [P, P, sz]),
        "unp_hip_memcpy_d2h": (i32, [P, P, sz]),
        "unp_hip_memset": (i32, [P, i32, sz]),
        "unp_hip_synchronize": (i32, []),
        "unp_hip_event_create": (i32, [C.POINTER(P)]),
        "unp_hip_event_destroy": (i32, [P]),
        "unp_hip_event_record": (i32, [P, P]),
        "unp_hip_event_synchronize": (i32, [P]),
        "unp_hip_event_elapsed_ms": (i32, [P, P, C.POINTER(C.c_float)]),
        "unp_hip_exec_create": (i32, [P, C.POINTER(P), E]),
        "unp_hip_exec_launch": (i32, [P, C.POINTER(Arg), sz, P, E]),
        "unp_hip_exec_launch_views": (i32, [P, C.POINTER(View), sz, C.POINTER(C.c_int64), sz, P, E]),
        "unp_hip_exec_launch_static": (i32, [P, C.POINTER(Arg), sz, P, E]),
        "unp_hip_exec_set_timing": (i32, [P, P, P]),
        "unp_hip_exec_set_wait_limit": (i32, [P, u32]),
        "unp_hip_exec_check": (i32, [P, E]),
        "unp_hip_exec_last_launch": (i32, [P, C.POINTER(u32), C.POINTER(u32), C.c_char_p, sz]),
        "unp_hip_exec_destroy": (None, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class UnpError(RuntimeError):
    """A typed refusal or failure from the library: ``kind`` names the status."""

    def __init__(self, code: int, detail: str):
        self.code = code
        self.kind = STATUS_NAMES.get(code, str(code))
        self.detail = detail
        super().__init__(f"{self.kind}: {detail}")


def check(rc: int, err: Error | None = None, what: str = "") -> None:
    if rc != OK:
        detail = err.detail.decode(errors="replace") if err is not None else what
        raise UnpError(rc, detail or what)
