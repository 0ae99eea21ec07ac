"""The reference's portable-C99 CPU leg (``unpopped-cpu-c``), restated -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may use this module,
as the second parity reference and as the timed CPU baseline; the product path never calls it.

``cpuc.cpp`` lowers a kernel-layer ``KernelFn`` (its serde JSON) to C99 in the scheme of
``crates/unpopped-cpu-c/src/{kernel,launch,base,typed,narrow}.rs``.  This module compiles that C with
the reference's own flags, ``cc -O2 -ffp-contract=off ... -lm``
(``crates/unpopped-cpu-c/tests/support/cc.rs:163-176``), into a shared object per distinct source
(cached by content hash, nothing persistent is shipped), and calls the entry point with the reference's
buffer ABI: four arguments per buffer, the storage, the per-axis extents, the signed element strides and
the base offset (``base.rs:65-103``), then one argument per scalar.  The entry returns 0 when the kernel
finished, 1 when an access fell outside its buffer and 2 for a zero loop step (``kernel.rs:9-11``).
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os
import shutil
import subprocess
import tempfile
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libcpuc.so"
CC = os.environ.get("CC", "cc")
# The reference's flags for the emitted C (cc.rs:163-176), plus what a shared object needs.
CFLAGS = ["-O2", "-ffp-contract=off"]
SO_FLAGS = ["-fPIC", "-shared"]

OK, OUT_OF_BOUNDS, ZERO_STEP = 0, 1, 2
UNSUPPORTED_KERNEL, PARSE_ERROR = 6, 50

_SCALAR_CTYPES = {"I32": C.c_int32, "I64": C.c_int64, "U32": C.c_uint32, "U64": C.c_uint64,
                  "F32": C.c_float, "F64": C.c_double, "I8": C.c_int8, "I16": C.c_int16,
                  "U8": C.c_uint8, "U16": C.c_uint16}
# Storage bytes per element of a buffer; sub-byte kinds pack two to a byte.
_ELEM_BYTES = {"F32": 4, "F32Strict": 4, "F64": 8, "F16": 2, "Bf16": 2, "I8": 1, "I16": 2, "I32": 4, "I64": 8,
               "U8": 1, "U16": 2, "U32": 4, "U64": 8, "U4": 0.5, "I4": 0.5}

_L = None


class Declined(Exception):
    """A typed refusal of the emitter: ``code`` 6 is LowerError::UnsupportedKernel."""

    def __init__(self, code: int, detail: str):
        super().__init__(f"[{code}] {detail}")
        self.code = code
        self.detail = detail


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "libcpuc.so"], check=True)
    return LIB


def _lib() -> C.CDLL:
    global _L
    if _L is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        pp = C.POINTER(C.c_char_p)
        L.cpuc_lower_kernel.restype = C.c_int
        L.cpuc_lower_kernel.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]
        L.cpuc_free.restype = None
        L.cpuc_free.argtypes = [C.c_void_p]
        del pp
        _L = L
    return _L


def lower(kernel) -> tuple[str, str]:
    """The C99 for ``kernel`` (a KernelFn dict or its JSON text): ``(entry, source)``; raises
    :class:`Declined` for a kernel the emitter refuses."""
    text = kernel if isinstance(kernel, str) else json.dumps(kernel)
    L = _lib()
    src, entry, detail = C.c_void_p(), C.c_void_p(), C.c_void_p()
    rc = L.cpuc_lower_kernel(text.encode(), C.byref(src), C.byref(entry), C.byref(detail))
    try:
        if rc != 0:
            raise Declined(rc, C.string_at(detail).decode() if detail.value else "")
        return C.string_at(entry).decode(), C.string_at(src).decode()
    finally:
        for p in (src, entry, detail):
            if p.value:
                L.cpuc_free(p)


def _cache_dir() -> Path:
    d = os.environ.get("UNPOPPED_CPUC_CACHE") or os.path.join(tempfile.gettempdir(), f"unpopped_cpuc_{os.getuid()}")
    Path(d).mkdir(parents=True, exist_ok=True)
    return Path(d)


def compile_source(source: str) -> Path:
    """Compile emitted C into a shared object (cached by the hash of source, compiler and flags)."""
    key = hashlib.sha1("\0".join([source, CC, *CFLAGS]).encode()).hexdigest()[:20]
    so = _cache_dir() / f"k_{key}.so"
    if so.exists():
        return so
    d = Path(tempfile.mkdtemp(dir=_cache_dir()))
    try:
        c = d / "kernel.c"
        c.write_text(source)
        out = d / "kernel.so"
        r = subprocess.run([CC, str(c), "-o", str(out), *CFLAGS, *SO_FLAGS, "-lm"], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"the emitted C does not compile:\n{r.stderr}\n{source}")
        os.replace(out, so)
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return so


@dataclass
class View:
    """A buffer argument as the reference's storage image (oracle/buffers.rs:16-42): the storage array,
    and the view's extents, signed element strides and base offset (elements; two to a byte for U4/I4).
    ``shape``/``strides`` default to the storage array's own dense layout."""

    data: np.ndarray
    shape: tuple | None = None
    strides: tuple | None = None
    base: int = 0


@dataclass
class CpuKernel:
    """One lowered and compiled kernel."""

    kernel: dict
    entry: str
    source: str
    _fn: object = None

    @classmethod
    def of(cls, kernel: dict) -> "CpuKernel":
        entry, source = lower(kernel)
        k = cls(kernel, entry, source)
        lib = C.CDLL(str(compile_source(source)))
        fn = getattr(lib, entry)
        fn.restype = C.c_int
        argt = []
        for p in kernel["params"]:
            (kind, body), = p["kind"].items()
            if kind == "Buffer":
                argt += [C.c_void_p, C.POINTER(C.c_longlong), C.POINTER(C.c_longlong), C.c_longlong]
            else:
                argt.append(_SCALAR_CTYPES[body["ty"]])
        fn.argtypes = argt
        k._fn = fn
        k._lib = lib
        return k

    def args(self, *args):
        """Pack one argument per parameter (a buffer: a View or an ndarray; a scalar: a number)."""
        params = self.kernel["params"]
        if len(args) != len(params):
            raise ValueError(f"{self.kernel['name']}: {len(params)} arguments expected, {len(args)} given")
        packed, keep = [], []
        for p, a in zip(params, args):
            (kind, body), = p["kind"].items()
            if kind != "Buffer":
                packed.append(a)
                continue
            v = a if isinstance(a, View) else View(a)
            data = v.data
            if not data.flags.c_contiguous:
                raise ValueError("a View's storage array must be contiguous; the view itself carries the strides")
            elem = body["elem"]
            if v.shape is None:
                if _ELEM_BYTES[elem] < 1:
                    raise ValueError(f"a {elem} buffer needs its shape in elements")
                shape = data.shape
                strides = tuple(s // data.itemsize for s in data.strides)
            else:
                shape = tuple(int(s) for s in v.shape)
                strides = tuple(int(s) for s in v.strides) if v.strides is not None else tuple(
                    int(np.prod(shape[i + 1:])) for i in range(len(shape)))
            sh = (C.c_longlong * max(1, len(shape)))(*shape)
            st = (C.c_longlong * max(1, len(strides)))(*strides)
            keep += [sh, st, data]
            packed += [data.ctypes.data, sh, st, int(v.base)]
        return packed, keep

    def __call__(self, *args) -> int:
        packed, keep = self.args(*args)
        rc = self._fn(*packed)
        del keep
        return rc

    def time(self, *args, reps: int = 5, warmup: int = 1) -> tuple[list[float], int]:
        """Seconds per call for ``reps`` calls after ``warmup``; and the last status."""
        packed, keep = self.args(*args)
        rc = 0
        for _ in range(warmup):
            rc = self._fn(*packed)
        out = []
        for _ in range(reps):
            t0 = time.perf_counter()
            rc = self._fn(*packed)
            out.append(time.perf_counter() - t0)
        del keep
        return out, rc


_CACHE: dict[str, CpuKernel] = {}


def kernel(k: dict) -> CpuKernel:
    """The compiled C99 of ``k``, compiled once per process."""
    key = json.dumps(k, sort_keys=True)
    if key not in _CACHE:
        _CACHE[key] = CpuKernel.of(k)
    return _CACHE[key]


def run(k: dict, *args) -> int:
    """Lower, compile and run ``k`` on ``args``; the status the C returns."""
    return kernel(k)(*args)
