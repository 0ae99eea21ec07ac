"""Benchmark: achieved HBM GB/s of the unpopped-hip reduce / scan / gather / dequant kernels on
one MI355X, against the 8 TB/s peak.

One step is one pass of the suite over the seeded synthetic inputs, each kernel launched once:
  cfg2   row Sum + Max of an f32 8192 x 4096 matrix, read once (normal(0,1), seed 1)
  cfg3a  inclusive i32 Sum scan of 2^28 elements in [0, 16) (seed 2)
  cfg3b  inclusive f32 Sum scan of 2^26 dyadic uniforms in [0, 1) (seed 2)
  cfg4u  bf16 262144 x 4096 row gather of 65536 uniform ids (seed 3)
  cfg4z  the same gather with Zipf(1.1) ids (seed 3)
  cfg5   U4 8192 x 28672 dequant, f16 scales and U4 zeros per 128 columns, bf16 out (seed 4)
Inputs are resident in HBM before the timed region.  Each kernel's time is the average over the
timed steps of the interval between two HIP events that take its own dispatch start and end
timestamps on the launch stream (hipExtModuleLaunchKernel); `value` is the algorithmic bytes of
the cases whose algorithmic bytes are HBM bytes (all but cfg4z, whose repeated rows come from L2
and the MALL; it runs in the same steps and is reported beside the aggregate) over their kernel
time.  The CPU baseline is the reference's
cpu-c C99 leg (restated in oracle/cpuc.*) for the same lifted kernels, one pinned core, on bounded
samples; it also runs config 1 (the CPU-only configuration) in full.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBPS = 8000.0
METRIC = "achieved HBM GB/s (% of ~8 TB/s peak) for reduce/scan/gather/dequant, 1 MI355X"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Case:
    def __init__(self, name, what, nbytes, elements, setup, ops=0, in_value=True):
        self.name, self.what, self.nbytes, self.elements, self.setup = name, what, nbytes, elements, setup
        self.ops = ops  # integer operations per launch, for the lines that run on MFMA
        # Whether the case's algorithmic bytes are HBM bytes and so count in `value`: the Zipf
        # gather's repeated rows come from L2 and the MALL, so it is reported beside the aggregate.
        self.in_value = in_value
        self.launch = None


def build_cases(u, synth):
    from unpopped_amd import forms as H

    cases = []

    def cfg2():
        R, Cc = 8192, 4096
        x = synth.normal_f32(1, R * Cc)
        ex = H.executor(kind="row_reduce2", dtype="F32", rank=2, op="Sum", op1="Max", reduced_from=1)
        din = u.DeviceBuffer.from_array(x)
        o0, o1 = u.DeviceBuffer(R * 4), u.DeviceBuffer(R * 4)
        return lambda: ex.launch(din, o0, o1, R, Cc), ex
    cases.append(Case("cfg2", "f32 8192x4096 row sum+max (fused, read once)", 8192 * 4096 * 4 + 2 * 8192 * 4,
                      8192 * 4096, cfg2))

    def cfg3a():
        n = 1 << 28
        x = synth.int16_i32(2, n)
        ex = H.executor(kind="scan", dtype="I32", rank=1, op="Sum")
        din = u.DeviceBuffer.from_array(x)
        dout = u.DeviceBuffer(n * 4)
        return lambda: ex.launch(din, dout, n), ex
    cases.append(Case("cfg3a", "i32 inclusive sum scan 2^28", 2 * (1 << 28) * 4, 1 << 28, cfg3a))

    def cfg3b():
        n = 1 << 26
        x = synth.uniform_01_f32(2, n)
        ex = H.executor(kind="scan", dtype="F32", rank=1, op="Sum")
        din = u.DeviceBuffer.from_array(x)
        dout = u.DeviceBuffer(n * 4)
        return lambda: ex.launch(din, dout, n), ex
    cases.append(Case("cfg3b", "f32 inclusive sum scan 2^26 (f64 carry, fixed schedule: reproducible bits)",
                      2 * (1 << 26) * 4, 1 << 26, cfg3b))

    table_holder = {}

    def gather(dist):
        def setup():
            V, D, N = 262144, 4096, 65536
            if "table" not in table_holder:
                log("[bench] generating the 2 GiB bf16 table")
                t = synth.normal_bf16_bits(3, V * D, 0.02)
                table_holder["table"] = u.DeviceBuffer.from_array(t)
                del t
            ids = synth.uniform_ids_i32(3, N, V) if dist == "uniform" else synth.zipf_ids_i32(3, N, V, 1.1)
            ex = H.executor(kind="gather", dtype="Bf16", rank=2, index_dtype="I32", oob="ZeroFill")
            dids = u.DeviceBuffer.from_array(ids)
            dout = u.DeviceBuffer(N * D * 2)
            dt = table_holder["table"]
            return lambda: ex.launch(dt, dids, dout, N, D, V), ex
        return setup
    gbytes = 65536 * 4096 * 2 * 2 + 65536 * 4
    cases.append(Case("cfg4u", "bf16 262144x4096 gather, 65536 uniform ids", gbytes, 65536 * 4096, gather("uniform")))
    cases.append(Case("cfg4z", "bf16 262144x4096 gather, 65536 Zipf(1.1) ids", gbytes, 65536 * 4096, gather("zipf"),
                      in_value=False))

    def cfg5():
        R, Cc, G = 8192, 28672, 128
        q = synth.nibbles(4, R * Cc)
        z = synth.nibbles(41, R * (Cc // G))
        s = synth.uniform_f16_bits(42, R * (Cc // G), 0.001, 0.02)
        ex = H.executor(kind="dequant4", q_kind="U4", z_kind="U4", group=G, out_kind="Bf16")
        dq, ds, dz = u.DeviceBuffer.from_array(q), u.DeviceBuffer.from_array(s), u.DeviceBuffer.from_array(z)
        do = u.DeviceBuffer(R * Cc * 2)
        return lambda: ex.launch(dq, ds, dz, do, R, Cc), ex
    dq_bytes = 8192 * 28672 // 2 + 8192 * 224 * 2 + 8192 * 224 // 2 + 8192 * 28672 * 2
    cases.append(Case("cfg5", "U4 8192x28672 -> bf16 dequant, g128", dq_bytes, 8192 * 28672, cfg5))
    return cases


def build_extras(u, synth):
    """The next rows of the hot path on the cfg2 input (an f32 8192 x 4096 matrix): the reduction
    over an outer axis (column sums; ReductionShape::new, kernel_lift.rs:854-870), and
    Access::RowReduce (kernel_lift/row_reduce_launched.rs:47-86) softmax and RMS norm, the row
    read once and the full-width epilogue written once.  Timed apart from the suite, each launch
    after a MALL flush (the lines that write 128-256 MB would otherwise leave their dirty lines to
    be written back during the next line's reads): not part of `value`."""
    from unpopped_amd import expr as X
    from unpopped_amd import forms as H

    extras = []

    def row_reduce(which):
        def setup():
            R, Cc = 8192, 4096
            x = synth.normal_f32(1, R * Cc)
            stages, epi = getattr(X, which)()
            ex = H.row_reduce_executor("F32", 2, stages, epi)
            din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(R * Cc * 4)
            return lambda: ex.launch(din, dout, R, Cc), ex
        return setup
    def colsum():
        R, Cc = 8192, 4096
        x = synth.normal_f32(1, R * Cc)
        ex = H.executor(kind="reduction", dtype="F32", rank=2, op="Sum", axes=(0,))
        din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(Cc * 4)
        return lambda: ex.launch(din, dout, R, Cc), ex
    extras.append(Case("rd_colsum", "f32 8192x4096 Sum over axis 0 (column sums, the outer-axis reduction)",
                       8192 * 4096 * 4 + 4096 * 4, 8192 * 4096, colsum))

    def full_sum():
        n = 1 << 24
        x = synth.uniform_pm1_f32(0, n)
        ex = H.executor(kind="reduction", dtype="F32", rank=1, op="Sum", reduced_from=0)
        din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(4)
        return lambda: ex.launch(din, dout, n), ex
    extras.append(Case("rd_all", "f32 2^24 full Sum (cfg1's data on the GPU; cfg1 itself is the CPU case)",
                       (1 << 24) * 4 + 4, 1 << 24, full_sum))
    def scan_device():
        # cfg3b on the device schedule, the Nondeterministic variant: the decoupled look-back folds
        # however far each look-back walked, so the f32 bits can change from launch to launch.  The
        # cfg3b line above runs what lower_kernel lowers, the fixed schedule (reproducible bits).
        n = 1 << 26
        x = synth.uniform_01_f32(2, n)
        ex = u.Executor(u.HipBackend().lower_form("scan", "F32", 1, "Sum", schedule="device"))
        din, dout = u.DeviceBuffer.from_array(x), u.DeviceBuffer(n * 4)
        return lambda: ex.launch(din, dout, n), ex
    extras.append(Case("cfg3b_device", "f32 inclusive sum scan 2^26 on the device schedule (bits vary run to run)",
                       2 * (1 << 26) * 4, 1 << 26, scan_device))
    rr_bytes = 2 * 8192 * 4096 * 4
    extras.append(Case("rr_softmax", "f32 8192x4096 RowReduce softmax (Max, Sum of exp, divide)", rr_bytes,
                       8192 * 4096, row_reduce("softmax")))
    extras.append(Case("rr_rmsnorm", "f32 8192x4096 RowReduce RMS norm (Mean of squares, scale)", rr_bytes,
                       8192 * 4096, row_reduce("rms_norm")))

    # The dequantizing GEMM (tests/support/dequant.rs:104-181) at a weight of LLM size, for a
    # decode width and a prefill width: U4 w 8192 x 28672, I32 zero point and scale per 128
    # columns, I8 activations.  Each launch is the x repack plus the main kernel.
    R, K, G = 8192, 28672, 128
    ng = K // G

    def gemm(C):
        def setup():
            w = synth.nibbles(6, R * K)
            zero = synth.int16_i32(61, R * ng)
            scale = (synth.int16_i32(62, R * ng) - 8) * 97
            x = (synth.int16_i32(63, K * C) * 13 - 100).astype(np.int8)
            # An executor of its own, so that its last launch names this case's entry.
            ex = u.Executor(u.HipBackend().lower_kernel(H.kernel_for(kind="dequant_gemm", q_kind="U4", dtype="I8",
                                                                     group=G)))
            dw, dz, ds, dx = (u.DeviceBuffer.from_array(a) for a in (w, zero, scale, x))
            do = u.DeviceBuffer(R * C * 4)
            return lambda: ex.launch(dw, dz, ds, dx, do, R, K, C), ex
        return setup
    for C, tag in ((16, "decode"), (1024, "prefill")):
        nbytes = R * K // 2 + R * ng * 8 + K * C + R * C * 4
        extras.append(Case(f"gemm_{tag}", f"dequant GEMM U4 {R}x{K} g{G} times I8 {K}x{C} (I32 out)", nbytes, R * C,
                           gemm(C), ops=2 * R * K * C))
    return extras


def time_cases(u, cases, steps, flush=None):
    """Average kernel time of each case's launch over `steps` rounds (one launch per case per round,
    on the launch stream).  Each launch carries a pair of HIP events that take the first and the last
    kernel's own dispatch timestamps (unp_hip_exec_set_timing, hipExtModuleLaunchKernel), so the time
    is the kernels' and not the queueing gap around them, as in a rocprofv3 kernel trace.  With
    `flush` (a MallFlush) every launch follows a MALL-evicting read: it starts from clean caches,
    its inputs in HBM and no earlier kernel's dirty lines left to write back while it runs."""
    events = [[(u.Event(), u.Event()) for _ in cases] for _ in range(steps)]
    u.synchronize()
    for s in range(steps):
        for i, c in enumerate(cases):
            if flush is not None:
                flush.run()
            c.exec.set_timing(*events[s][i])
            c.launch()
    u.synchronize()
    for c in cases:
        c.exec.set_timing(None, None)
        # A wait that ran out leaves the launch's outputs invalid (unp_hip_exec_check); a timing of
        # such a launch is no measurement, so the run stops here.
        try:
            c.exec.check()
        except u.UnpError as e:
            raise SystemExit(f"[bench] {c.name}: a timed launch reported {e.kind}: {e}; no line is printed")
    per = []
    for i, c in enumerate(cases):
        ms = sum(events[s][i][0].elapsed_ms(events[s][i][1]) for s in range(steps)) / steps
        gbps = c.nbytes / (ms * 1e-3) / 1e9
        per.append({
            "name": c.name, "what": c.what, "entry": c.exec.last_launch()["entry"],
            "grid": c.exec.last_launch()["grid"][0], "bytes": c.nbytes, "us": round(ms * 1e3, 2),
            "GBps": round(gbps, 1), "frac_of_peak": round(gbps / PEAK_GBPS, 4),
            "elements_per_s": round(c.elements / (ms * 1e-3), 1),
        })
        if c.ops:
            per[-1]["TOPs"] = round(c.ops / (ms * 1e-3) / 1e12, 1)
            per[-1]["frac_of_int8_mfma_peak"] = round(c.ops / (ms * 1e-3) / 1e12 / 5000, 4)
        log(f"[bench] {c.name}: {ms * 1e3:.1f} us, {gbps:.0f} GB/s ({100 * gbps / PEAK_GBPS:.1f}% of peak)")
    return per


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline(synth, budget_s: float = 30.0) -> dict:
    """The unpopped-cpu-c C99 leg, restated (oracle/cpuc.*: the reference emitter's serialized thread
    loop, bounds-checked, compiled with its flags -O2 -ffp-contract=off), run on the same launched
    KernelFns the GPU lowers (the caller's (256, 64) lifts), pinned to one host core: the median of
    up to 5 runs after a warm-up.  cfg2 runs in full; the scans, the gather and the dequant on bounded
    samples.  cfg1, the CPU-only configuration, runs in full through the serial and the launched lift
    and is checked against RN32 of its exact sum; it is reported apart from the aggregate."""
    import unpopped_amd as u
    from oracle import cpuc
    from oracle.cpuc import View
    from unpopped_amd import forms as H

    legs = []

    def timed(name, k, args, nbytes, what):
        ck = cpuc.kernel(k)
        ck.time(*args, reps=0, warmup=1)
        runs, t0 = [], time.perf_counter()
        while len(runs) < 5 and time.perf_counter() - t0 < budget_s / 6:
            ts, rc = ck.time(*args, reps=1, warmup=0)
            if rc != cpuc.OK:
                raise RuntimeError(f"the C99 of {name} returned status {rc}")
            runs.append(ts[0])
        s = float(np.median(runs))
        legs.append({"name": name, "sample": what, "bytes": nbytes, "s": s, "runs": len(runs),
                     "GBps": round(nbytes / s / 1e9, 4)})
        log(f"[bench] cpu-c {name}: {what}: {s * 1e3:.1f} ms, {nbytes / s / 1e9:.3f} GB/s")

    saved = os.sched_getaffinity(0)
    core = min(saved)
    os.sched_setaffinity(0, {core})
    try:
        R, Cc = 8192, 4096
        x2 = synth.normal_f32(1, R * Cc).reshape(R, Cc)
        timed("cfg2", H.kernel_for(kind="row_reduce2", dtype="F32", rank=2),
              (x2, np.zeros(R, np.float32), np.zeros(R, np.float32), R, Cc), x2.nbytes + 2 * R * 4, "full 8192x4096")
        del x2
        n = 1 << 24
        x3 = synth.int16_i32(2, n)
        timed("cfg3a", H.kernel_for(kind="scan", dtype="I32"), (x3, np.empty(n, np.int32), n), 8 * n, "2^24 of 2^28")
        x3b = synth.uniform_01_f32(2, n)
        timed("cfg3b", H.kernel_for(kind="scan", dtype="F32"), (x3b, np.empty(n, np.float32), n), 8 * n,
              "2^24 of 2^26")
        del x3, x3b
        V, D, N = 16384, 4096, 4096
        t = synth.normal_bf16_bits(3, V * D, 0.02).reshape(V, D)
        ids = synth.uniform_ids_i32(3, N, V)
        timed("cfg4", H.kernel_for(kind="gather", dtype="Bf16", rank=2),
              (t, View(ids, (N, D), (1, 0)), np.empty((N, D), np.uint16), N, D, V), 2 * N * D * 2 + N * 4,
              "4096 uniform ids into a 16384-row table")
        del t
        R, Cc, G = 256, 28672, 128
        q, z = synth.nibbles(4, R * Cc), synth.nibbles(41, R * (Cc // G))
        sc = synth.uniform_f16_bits(42, R * (Cc // G), 0.001, 0.02)
        timed("cfg5", H.kernel_for(kind="dequant4"),
              (View(q, (R * Cc,), (1,)), sc, View(z, (R * Cc // G,), (1,)), np.empty(R * Cc, np.uint16), R, Cc),
              R * Cc // 2 + R * (Cc // G) * 3 + R * Cc * 2, "256 of 8192 rows")
        # cfg1: the CPU configuration in full, lift -> C99 -> checked against RN32(exact sum).
        n1 = 1 << 24
        x1 = synth.uniform_pm1_f32(0, n1)
        exact = np.float32(float(int(np.round(x1.astype(np.float64) * 2.0**24).astype(np.int64).sum())) * 2.0**-24)
        cfg1 = {}
        for tag, launch in (("serial", None), ("launched_256x64", (256, 64))):
            k = u.lift_reduction("cfg1", "F32", 1, "Sum", launch=launch)
            out = np.zeros(1, np.float32)
            ck = cpuc.kernel(k)
            ts, rc = ck.time(x1, View(out.reshape(()), (), ()), n1, reps=5, warmup=1)
            s = float(np.median(ts))
            cfg1[tag] = {"s": round(s, 6), "GBps": round(4 * n1 / s / 1e9, 4), "status": rc,
                         "equals_rn32_exact": bool(out[0] == exact)}
            log(f"[bench] cpu-c cfg1 {tag}: {s * 1e3:.1f} ms, sum {out[0]!r} (exact {exact!r})")
    finally:
        os.sched_setaffinity(0, saved)
    total_b = sum(l["bytes"] for l in legs)
    total_s = sum(l["s"] for l in legs)
    return {
        "value": round(total_b / total_s / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "emitter": "unpopped-cpu-c C99 (restated: oracle/cpuc.cpp), cc -O2 -ffp-contract=off",
        "host": f"core {core} of {os.cpu_count()} ({cpu_model()})",
        "sample": "; ".join(f"{l['name']} {l['sample']}: {l['GBps']:.3f} GB/s" for l in legs)
                  + "; median of up to 5 runs after a warm-up, the (256, 64) launched lifts",
        "legs": legs,
        "cfg1": cfg1,
    }


COPY_PROBE_SRC = r"""
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
extern "C" __global__ void __launch_bounds__(256) unp_copy_probe(const u32x4* __restrict__ s, u32x4* __restrict__ d,
                                                                  long long n) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) d[i] = s[i];
}
"""


def copy_probe(u, nbytes: int = 256 << 20) -> None:
    """A plain copy of `nbytes` (read nbytes, write nbytes): the reference point that converts
    the FETCH_SIZE / WRITE_SIZE counters of a profiled run into bytes."""
    import ctypes as C

    from unpopped_amd import _lib

    L = _lib.lib()
    co = u.HipCompiler().compile(COPY_PROBE_SRC, "unp_copy_probe")
    img = C.create_string_buffer(co, len(co))
    m, f, err = C.c_void_p(), C.c_void_p(), _lib.Error()
    _lib.check(L.unp_hip_module_load(img, len(co), C.byref(m), C.byref(err)), err)
    _lib.check(L.unp_hip_get_function(m, b"unp_copy_probe", C.byref(f), C.byref(err)), err)
    a, b = u.DeviceBuffer(nbytes), u.DeviceBuffer(nbytes)
    a.fill(1)
    args = (C.c_uint64 * 3)(a.ptr, b.ptr, nbytes // 16)
    g, blk = (C.c_uint32 * 3)(1024, 1, 1), (C.c_uint32 * 3)(256, 1, 1)
    for _ in range(3):
        _lib.check(L.unp_hip_launch(f, g, blk, 0, None, args, C.sizeof(args), C.byref(err)), err)
    u.synchronize()
    log(f"[bench] copy probe: 3 launches of a {nbytes} B copy")


CEILING_SRC = r"""
typedef unsigned int u32;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
// Plain streaming kernels, 16 bytes per lane, 4 in flight, nontemporal: what this device moves
// for a pure read, a pure write and a 1:1 copy, with no algorithm in the way.
extern "C" __global__ void __launch_bounds__(256) unp_ceiling_read(const u32x4* __restrict__ s, u32* __restrict__ sink,
                                                                    long long n) {
  const long long st = (long long)gridDim.x * 256;
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  u32 acc = 0;
  for (; i + 3 * st < n; i += 4 * st) {
    const u32x4 a = __builtin_nontemporal_load(s + i), b = __builtin_nontemporal_load(s + i + st);
    const u32x4 c = __builtin_nontemporal_load(s + i + 2 * st), d = __builtin_nontemporal_load(s + i + 3 * st);
    acc ^= a.x ^ b.y ^ c.z ^ d.w;
  }
  for (; i < n; i += st) acc ^= s[i].x;
  if (acc == 0x9E3779B9u) sink[0] = acc;
}
extern "C" __global__ void __launch_bounds__(256) unp_ceiling_write(u32x4* __restrict__ d, long long n) {
  const long long st = (long long)gridDim.x * 256;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += st) {
    const u32x4 v = {(u32)i, 1u, 2u, 3u};
    __builtin_nontemporal_store(v, d + i);
  }
}
extern "C" __global__ void __launch_bounds__(256) unp_ceiling_copy(const u32x4* __restrict__ s, u32x4* __restrict__ d,
                                                                    long long n) {
  const long long st = (long long)gridDim.x * 256;
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * st < n; i += 4 * st) {
    const u32x4 a = __builtin_nontemporal_load(s + i), b = __builtin_nontemporal_load(s + i + st);
    const u32x4 c = __builtin_nontemporal_load(s + i + 2 * st), e = __builtin_nontemporal_load(s + i + 3 * st);
    __builtin_nontemporal_store(a, d + i);
    __builtin_nontemporal_store(b, d + i + st);
    __builtin_nontemporal_store(c, d + i + 2 * st);
    __builtin_nontemporal_store(e, d + i + 3 * st);
  }
  for (; i < n; i += st) __builtin_nontemporal_store(__builtin_nontemporal_load(s + i), d + i);
}
"""


# Each suite kernel's own byte pattern and size: the ceiling it is read against.  The scans and the
# gather read and write the same bytes (copy); the row reduce only reads; the dequant mostly writes.
CEILING_SIZES = [
    ("read", 1 << 30, "1 GiB"),
    ("read", 128 << 20, "cfg2: 8192 x 4096 f32"),
    ("read", 64 << 20, "the full sum: 2^24 f32"),
    ("write", 1 << 30, "1 GiB"),
    ("write", 448 << 20, "cfg5's output: 8192 x 28672 bf16"),
    ("copy", 1 << 30, "1 GiB, cfg3a: 2^28 i32"),
    ("copy", 512 << 20, "cfg4: 65536 rows of 8 KiB"),
    ("copy", 256 << 20, "cfg3b: 2^26 f32"),
    ("copy", 128 << 20, "RowReduce: 8192 x 4096 f32 in and out"),
]


def ceilings(u, cus: int, reps: int = 10) -> None:
    """Streaming read / write / copy rates of this device (median of `reps` launches, the best of 1, 2
    and 4 blocks of 256 threads per CU), on 1 GiB and at each suite kernel's own size: the practical
    ceilings that the suite's kernels are read against, beside the 8 TB/s peak.  A copy of `size`
    reads `size` bytes and writes `size` bytes.  Launches are timed by their own dispatch timestamps,
    as the suite's kernels are."""
    import ctypes as C

    from unpopped_amd import _lib

    L = _lib.lib()
    co = u.HipCompiler().compile(CEILING_SRC, "unp_ceiling_copy")
    img = C.create_string_buffer(co, len(co))
    m, err = C.c_void_p(), _lib.Error()
    _lib.check(L.unp_hip_module_load(img, len(co), C.byref(m), C.byref(err)), err)
    fns = {}
    for name in ("unp_ceiling_read", "unp_ceiling_write", "unp_ceiling_copy"):
        f = C.c_void_p()
        _lib.check(L.unp_hip_get_function(m, name.encode(), C.byref(f), C.byref(err)), err)
        fns[name] = f
    def timed(f, g, blk, args, e0, e1):
        # Each launch is timed by its own dispatch timestamps, as the suite's kernels are: events
        # recorded on the stream around it would add their own latency (2-3 us on this device).
        _lib.check(L.unp_hip_launch_timed(f, g, blk, 0, None, args, C.sizeof(args), e0._h, e1._h, C.byref(err)), err)

    big = max(size for _, size, _ in CEILING_SIZES)
    flush = MallFlush(u, cus)
    a, b, sink = u.DeviceBuffer(big), u.DeviceBuffer(big), u.DeviceBuffer(64)
    a.fill(1)
    for label, size, what in CEILING_SIZES:
        n = size // 16
        name, vals, moved = {
            "read": ("unp_ceiling_read", (a.ptr, sink.ptr, n), size),
            "write": ("unp_ceiling_write", (b.ptr, n), size),
            "copy": ("unp_ceiling_copy", (a.ptr, b.ptr, n), 2 * size),
        }[label]
        args = (C.c_uint64 * len(vals))(*vals)
        best = None
        for bpc in (1, 2, 4):
            g, blk = (C.c_uint32 * 3)(cus * bpc, 1, 1), (C.c_uint32 * 3)(256, 1, 1)
            ts = []
            for i in range(reps + 2):
                e0, e1 = u.Event(), u.Event()
                timed(fns[name], g, blk, args, e0, e1)
                e1.synchronize()
                if i >= 2:
                    ts.append(e0.elapsed_ms(e1))
            ms = float(np.median(ts))
            gbps = moved / (ms * 1e-3) / 1e9
            log(f"[bench] ceiling {label} {size} B: {cus * bpc} blocks, {ms * 1e3:.1f} us, {gbps:.0f} GB/s")
            if best is None or gbps > best[0]:
                best = (gbps, cus * bpc, ms)
        # The same launch with the MALL evicted before each one: a buffer under 256 MB read back to
        # back is partly served from the MALL, which a kernel that follows other work does not see.
        g = (C.c_uint32 * 3)(best[1], 1, 1)
        blk = (C.c_uint32 * 3)(256, 1, 1)
        ts = []
        for i in range(reps):
            flush.run()
            e0, e1 = u.Event(), u.Event()
            timed(fns[name], g, blk, args, e0, e1)
            e1.synchronize()
            ts.append(e0.elapsed_ms(e1))
        cold = float(np.median(ts))
        log(f"[bench] ceiling {label} {size} B cold: {cold * 1e3:.1f} us")
        print(json.dumps({"ceiling": label, "size": size, "what": what, "bytes": moved, "blocks": best[1],
                          "us": round(best[2] * 1e3, 1), "GBps": round(best[0], 1),
                          "frac_of_peak": round(best[0] / PEAK_GBPS, 4), "cold_us": round(cold * 1e3, 1),
                          "cold_GBps": round(moved / (cold * 1e-3) / 1e9, 1)}), flush=True)


FLUSH_SRC = r"""
typedef unsigned int u32;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
// Plain (cached) loads over a buffer larger than the MALL: evicts what earlier launches left
// there with clean lines, so the next timed launch reads its inputs from HBM.
extern "C" __global__ void __launch_bounds__(256) unp_mall_flush(const u32x4* __restrict__ s, u32* __restrict__ sink,
                                                                  long long n) {
  const long long st = (long long)gridDim.x * 256;
  u32 acc = 0;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += st) acc ^= s[i].x ^ s[i].w;
  if (acc == 0x9E3779B9u) sink[0] = acc;
}
"""


class MallFlush:
    """Reads 512 MiB with plain loads; launched between timed launches of one kernel."""

    def __init__(self, u, cus: int):
        import ctypes as C

        from unpopped_amd import _lib

        self.C, self._lib, self.L = C, _lib, _lib.lib()
        co = u.HipCompiler().compile(FLUSH_SRC, "unp_mall_flush")
        self.img = C.create_string_buffer(co, len(co))
        self.m, self.f, err = C.c_void_p(), C.c_void_p(), _lib.Error()
        _lib.check(self.L.unp_hip_module_load(self.img, len(co), C.byref(self.m), C.byref(err)), err)
        _lib.check(self.L.unp_hip_get_function(self.m, b"unp_mall_flush", C.byref(self.f), C.byref(err)), err)
        self.buf, self.sink = u.DeviceBuffer(512 << 20), u.DeviceBuffer(64)
        self.buf.fill(1)
        self.args = (C.c_uint64 * 3)(self.buf.ptr, self.sink.ptr, (512 << 20) // 16)
        self.grid, self.block = (C.c_uint32 * 3)(cus * 4, 1, 1), (C.c_uint32 * 3)(256, 1, 1)

    def run(self) -> None:
        err = self._lib.Error()
        self._lib.check(self.L.unp_hip_launch(self.f, self.grid, self.block, 0, None, self.args,
                                              self.C.sizeof(self.args), self.C.byref(err)), err)


def gemm_lines(u, synth, steps: int, warmup: int, shapes: str = "") -> None:
    """The dequantizing GEMM (tests/support/dequant.rs:104-181) at a weight of LLM size: U4 w
    8192 x 28672 with an I32 zero point and scale per 128 columns, times x of C columns (I8 and I32),
    one JSON line per shape: the median of `steps` launches, each timed alone by its kernels' own
    dispatch timestamps after a 512 MiB read with plain loads has evicted the weight from the MALL.  Bytes are w + zero + scale + x + out;
    operations 2 R K C.  ``shapes`` ("I8:16,I32:1024") keeps only those (activation, C) pairs."""
    from unpopped_amd import forms as H

    keep = {tuple(s.split(":")) for s in shapes.split(",") if s}
    R, K, G = 8192, 28672, 128
    ng = K // G
    # Streamed between timed launches so that no launch finds the weight in the 256 MB MALL
    # from the one before, as consecutive layers of a model would not.
    flush = MallFlush(u, u.device_info()[1])
    w = synth.nibbles(6, R * K)
    zero = synth.int16_i32(61, R * ng)
    scale = (synth.int16_i32(62, R * ng) - 8) * 97
    dw, dz, ds = (u.DeviceBuffer.from_array(a) for a in (w, zero, scale))
    for xk, xdt in (("I8", np.int8), ("I32", np.int32)):
        ex = H.executor(kind="dequant_gemm", q_kind="U4", dtype=xk, group=G)
        for C in (16, 32, 64, 128, 256, 1024):
            if keep and (xk, str(C)) not in keep:
                continue
            x = (synth.int16_i32(63, K * C) * 13 - 100).astype(xdt)
            dx, do = u.DeviceBuffer.from_array(x), u.DeviceBuffer(R * C * 4)
            for _ in range(warmup):
                ex.launch(dw, dz, ds, dx, do, R, K, C)
            u.synchronize()
            ts = []
            for i in range(steps):
                flush.run()
                e0, e1 = u.Event(), u.Event()
                # From the prep kernel's start to the main kernel's end, by their own dispatch
                # timestamps (the gap between the two launches included).
                ex.set_timing(e0, e1)
                ex.launch(dw, dz, ds, dx, do, R, K, C)
                ex.set_timing(None, None)
                e1.synchronize()
                ts.append(e0.elapsed_ms(e1) * 1e3)
            us = float(np.median(ts))
            nbytes = R * K // 2 + R * ng * 8 + K * C * x.itemsize + R * C * 4
            ops = 2 * R * K * C
            log(f"[bench] gemm x {xk} C {C}: {us:.1f} us")
            print(json.dumps({"gemm": f"U4 {R}x{K} g{G} times {xk} {K}x{C}", "entry": ex.last_launch()["entry"],
                              "us": round(us, 1), "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
                              "frac_of_hbm_peak": round(nbytes / us / 1e3 / PEAK_GBPS, 4),
                              "TOPs": round(ops / us / 1e6, 1), "frac_of_int8_mfma_peak": round(ops / us / 1e6 / 5000, 4)}),
                  flush=True)
            del dx, do


def attach_traffic(per, cases) -> None:
    """HBM bytes per launch from the committed FETCH_SIZE / WRITE_SIZE profile (each counter scaled by
    what it reads for a plain copy of known size), attached only to a case whose running kernel has
    the source revision (FNV-1a of the generated source) that was profiled, and labelled with the
    file it comes from; a kernel changed since its profile gets no figure."""
    tf = ROOT / "profiles" / "traffic.json"
    known = json.loads(tf.read_text()).get("cases", {}) if tf.exists() else {}
    for p, c in zip(per, cases):
        t = known.get(p["name"])
        rev = f"{c.exec.kernel.revision_hash():016x}"
        p["revision"] = rev
        if t and t.get("kernel") == p["entry"] and t.get("revision") == rev:
            p["traffic"] = t["traffic_bytes"]
            p["traffic_source"] = f"profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; revision {rev})"


def _pmc_dispatches(d: Path, counter: str) -> list:
    """(kernel name, value) of every dispatch in one rocprofv3 --pmc pass under `d`, in dispatch order."""
    import csv

    files = sorted(d.rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] == counter:
                    name = r["Kernel_Name"].strip()
                    name = name[:-3] if name.endswith(".kd") else name
                    rows.append((int(r["Dispatch_Id"]), name, float(r["Counter_Value"])))
    rows.sort()
    return [(k, v) for _, k, v in rows]


def _bench_line(path: Path) -> dict:
    for line in reversed(path.read_text().splitlines()):
        if line.startswith('{"metric"'):
            return json.loads(line)
    raise SystemExit(f"no bench JSON line in {path}")


def _per_case(dispatches: list, line: dict) -> dict:
    """Mean counter value per case.  The suite launches each case `warmup` times in order, then one
    launch per case per step; the extra lines follow the same pattern.  A kernel that several cases
    share (the gather: cfg4u, cfg4z) is split by that order."""
    W, S = line["warmup"], line["steps"]
    order: dict = {}
    for group in (line["config"]["kernels"], line.get("extra_kernels") or []):
        names = {}
        for k in group:
            names.setdefault(k["entry"], []).append(k["name"])
        for entry, cs in names.items():
            order.setdefault(entry, []).extend([c for c in cs for _ in range(W)] + cs * S)
    seen: dict = {}
    for name, v in dispatches:
        seen.setdefault(name, []).append(v)
    out: dict = {}
    for entry, cs in order.items():
        vals = seen.get(entry, [])
        if len(vals) != len(cs):
            log(f"[traffic] {entry}: {len(vals)} dispatches, expected {len(cs)}: skipped")
            continue
        for c, v in zip(cs, vals):
            out.setdefault(c, []).append(v)
    return {c: float(np.mean(v)) for c, v in out.items()}


def assemble_traffic(d: Path) -> None:
    """Writes profiles/traffic.json from four rocprofv3 --pmc passes under `d` (fetch/, write/: the
    bench; cfetch/, cwrite/: the plain 256 MiB copy of --copy-probe) and the bench's JSON lines
    (fetch.json, write.json: the stdout of the two bench passes).  FETCH_SIZE and WRITE_SIZE are KiB
    per dispatch; each is scaled by what it reads for the copy of known size.  Every case carries the
    source revision of the kernel that ran, so bench.py attaches the figure only to that kernel."""
    fl, wl = _bench_line(d / "fetch.json"), _bench_line(d / "write.json")
    kernels = {k["name"]: k for k in fl["config"]["kernels"] + (fl.get("extra_kernels") or [])}
    wrev = {k["name"]: k.get("revision") for k in wl["config"]["kernels"] + (wl.get("extra_kernels") or [])}
    probe_kib = (256 << 20) / 1024
    cf = [v for k, v in _pmc_dispatches(d / "cfetch", "FETCH_SIZE") if k == "unp_copy_probe"]
    cw = [v for k, v in _pmc_dispatches(d / "cwrite", "WRITE_SIZE") if k == "unp_copy_probe"]
    fscale, wscale = probe_kib / float(np.mean(cf)), probe_kib / float(np.mean(cw))
    fetch = _per_case(_pmc_dispatches(d / "fetch", "FETCH_SIZE"), fl)
    write = _per_case(_pmc_dispatches(d / "write", "WRITE_SIZE"), wl)
    cases = {}
    for name, k in kernels.items():
        if name not in fetch or name not in write or wrev.get(name) != k.get("revision"):
            continue
        fb, wb = fetch[name] * 1024 * fscale, write[name] * 1024 * wscale
        cases[name] = {"kernel": k["entry"], "revision": k.get("revision"), "fetch_bytes": round(fb),
                       "write_bytes": round(wb), "traffic_bytes": round(fb + wb), "algorithmic_bytes": k["bytes"],
                       "ratio": round((fb + wb) / k["bytes"], 4)}
        log(f"[traffic] {name}: fetch {fb / 1e6:.1f} MB, write {wb / 1e6:.1f} MB, ratio {(fb + wb) / k['bytes']:.4f}")
    out = {"fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4), "cases": cases}
    (ROOT / "profiles" / "traffic.json").write_text(json.dumps(out, indent=1) + "\n")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default="", help="comma-separated case names (default: the whole suite)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the column-sum and RowReduce lines timed after the suite (not part of `value`)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only launch a plain 256 MiB copy (calibrates the HBM byte counters)")
    ap.add_argument("--ceilings", action="store_true",
                    help="only measure this device's streaming read / write / copy rates, on 1 GiB and at each suite kernel's size")
    ap.add_argument("--gemm", action="store_true",
                    help="only time the dequantizing GEMM at LLM shapes (one JSON line per shape)")
    ap.add_argument("--gemm-shapes", default="", help='with --gemm: only these "I8:16,I32:1024" (activation:C) pairs')
    ap.add_argument("--traffic-from", default="",
                    help="write profiles/traffic.json from the rocprofv3 --pmc passes under this folder (no GPU)")
    args = ap.parse_args()
    if args.traffic_from:
        assemble_traffic(Path(args.traffic_from))
        return 0
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import unpopped_amd as u
    from unpopped_amd import synth

    if u.device_count() < 1:
        print("no HIP device", file=sys.stderr)
        return 1
    arch, cus = u.device_info()
    log(f"[bench] device {arch}, {cus} CUs")
    if args.copy_probe:
        copy_probe(u)
        return 0
    if args.ceilings:
        ceilings(u, cus)
        return 0
    if args.gemm:
        gemm_lines(u, synth, args.steps, args.warmup, args.gemm_shapes)
        return 0
    cases = build_cases(u, synth)
    if args.only:
        keep = set(args.only.split(","))
        cases = [c for c in cases if c.name in keep]
    for c in cases:
        log(f"[bench] setup {c.name}: {c.what}")
        c.launch, c.exec = c.setup()
    for c in cases:
        log(f"[bench] warmup {c.name}")
        for _ in range(args.warmup):
            c.launch()
    u.synchronize()

    log(f"[bench] timing {args.steps} steps")
    u.synchronize()
    t0 = time.perf_counter()
    per = time_cases(u, cases, args.steps)
    wall = time.perf_counter() - t0
    for p, c in zip(per, cases):
        p["in_value"] = c.in_value
    hbm = [(p, c) for p, c in zip(per, cases) if c.in_value]
    total_bytes = sum(c.nbytes for _, c in hbm)
    ms_step = sum(p["us"] for p in per) / 1e3
    value = total_bytes / (sum(p["us"] for p, _ in hbm) * 1e-6) / 1e9 if hbm else 0.0
    dom = max(per, key=lambda p: p["us"])

    # HBM bytes per launch from the committed FETCH_SIZE/WRITE_SIZE passes, for kernels whose source
    # is the profiled one; null otherwise.
    attach_traffic(per, cases)
    traffic = dom.get("traffic")

    extra = None
    if not args.no_extras and not args.only:
        xs = build_extras(u, synth)
        for c in xs:
            log(f"[bench] setup {c.name}: {c.what}")
            c.launch, c.exec = c.setup()
            for _ in range(args.warmup):
                c.launch()
        log(f"[bench] timing {args.steps} steps of the extra lines, each launch after a MALL flush")
        extra = time_cases(u, xs, args.steps, flush=MallFlush(u, cus))
        attach_traffic(extra, xs)

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline (the cpu-c C99 leg, 1 thread)")
        cpu = cpu_baseline(synth)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (f64 accumulate), i32, bf16 (raw move), u4 -> bf16",
        "data": "synthetic: seeded LCG streams (dyadic uniforms, Box-Muller normals, Zipf ids)",
        "config": {
            "workload": "suite: " + ", ".join(c.name for c in cases),
            "value_counts": ", ".join(c.name for _, c in hbm) + " (algorithmic bytes = HBM bytes); "
                            + ", ".join(c.name for c in cases if not c.in_value)
                            + " timed in the same steps and reported beside it (cache-served rows)",
            "timing": "per-kernel dispatch timestamps (HIP events via hipExtModuleLaunchKernel) on the launch stream",
            "device": arch,
            "cu_count": cus,
            "wall_s_timed_region": round(wall, 4),
            "kernels": per,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom["name"],
            "achieved": dom["GBps"],
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dom["GBps"] / PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": dom.get("traffic_source"),
        },
        "cpu_baseline": cpu,
        "extra_kernels": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
