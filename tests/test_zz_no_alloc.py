"""The no-allocation launch (unp_hip_exec_launch_static) against the allocating one
(unp_hip_exec_launch), both called through the C ABI on the same executor and inputs: two calls in a
row, the second smaller, for every form whose kernels use a workspace -- the scans (tile status and
ticket counter), the full reduction (partials and counter), the column reduction (partials and strip
counters) and the dequantizing GEMM (repacked activations and column sums).  Results are compared bit
for bit: the integer forms and the fixed-order float reductions are deterministic, the f32 scan
runs on dyadic data, where every association is exact, and on normal data on the fixed schedule.  A launch whose workspace exceeds the static
scratch is refused before anything runs."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import unpopped_amd as u
from unpopped_amd import _lib
from unpopped_amd import forms as H
from unpopped_amd import synth

pytestmark = pytest.mark.gpu

STATIC_BYTES = 4 << 20  # UNP_STATIC_SCRATCH_BYTES


def c_args(args):
    arr = (_lib.Arg * len(args))()
    for i, a in enumerate(args):
        if isinstance(a, u.DeviceBuffer):
            arr[i].is_buffer, arr[i].value = 1, a.ptr
        else:
            arr[i].is_buffer, arr[i].value = 0, int(a) & 0xFFFFFFFFFFFFFFFF
    return arr


def launch_allocating(ex, *args):
    err = _lib.Error()
    rc = _lib.lib().unp_hip_exec_launch(ex._h, c_args(args), len(args), None, C.byref(err))
    assert rc == 0, err.detail
    u.synchronize()


def launch_static(ex, *args) -> tuple[int, str]:
    err = _lib.Error()
    rc = _lib.lib().unp_hip_exec_launch_static(ex._h, c_args(args), len(args), None, C.byref(err))
    u.synchronize()
    return rc, err.detail.decode()


def both(ex, make_args, download):
    """The outputs of the allocating and the static launch of the same arguments."""
    args = make_args()
    launch_allocating(ex, *args)
    want = download(args)
    args = make_args()
    rc, why = launch_static(ex, *args)
    assert rc == 0, why
    return download(args), want


def test_scans_match_the_allocating_launch(hip_device):
    ex = H.executor(kind="scan", dtype="I32", rank=2, op="Sum")
    for n in (1 << 28, (1 << 20) + 37):  # the first near the scratch's limit (3.7 MB of status)
        print(f"[no_alloc] i32 scan n={n}", flush=True)
        x = synth.int16_i32(2, n)
        din = u.DeviceBuffer.from_array(x)

        def make():
            out = u.DeviceBuffer(n * 4)
            out.fill(0xAB)
            return din, out, 1, n
        got, want = both(ex, make, lambda a: a[1].download(np.int32, n))
        assert np.array_equal(got, want)
        del din
    exf = H.executor(kind="scan", dtype="F32", rank=2, op="Sum")
    for n in (1 << 24, 100003):
        print(f"[no_alloc] f32 scan n={n}", flush=True)
        x = synth.uniform_01_f32(2, n)  # dyadic: every association is exact
        din = u.DeviceBuffer.from_array(x)

        def make():
            return din, u.DeviceBuffer(n * 4), 1, n
        got, want = both(exf, make, lambda a: a[1].download(np.float32, n))
        assert got.tobytes() == want.tobytes()
    # The fixed schedule on normal data: only an association fixed by the tiling makes the two
    # launches agree bit for bit here.
    exx = u.Executor(u.HipBackend().lower_form("scan", "F32", 2, "Sum", schedule="fixed"))
    for n in (1 << 24, 100003):
        print(f"[no_alloc] f32 scan, fixed schedule, normal data n={n}", flush=True)
        din = u.DeviceBuffer.from_array(synth.normal_f32(5, n))

        def make():
            return din, u.DeviceBuffer(n * 4), 1, n
        got, want = both(exx, make, lambda a: a[1].download(np.float32, n))
        assert got.tobytes() == want.tobytes()


def test_full_reduction_matches_the_allocating_launch(hip_device):
    ex = H.executor(kind="reduction", dtype="F32", rank=1, op="Sum", reduced_from=0)
    for n in (1 << 24, (1 << 20) + 5):
        print(f"[no_alloc] full sum n={n}", flush=True)
        din = u.DeviceBuffer.from_array(synth.normal_f32(1, n))

        def make():
            return din, u.DeviceBuffer(16), n
        got, want = both(ex, make, lambda a: a[1].download(np.float32, 1))
        assert got.tobytes() == want.tobytes()


def test_column_reduction_matches_the_allocating_launch(hip_device):
    ex = H.executor(kind="reduction", dtype="F32", rank=2, op="Sum", axes=(0,))
    for r, c in ((2048, 1024), (1000, 512)):
        print(f"[no_alloc] column sums {r}x{c}", flush=True)
        din = u.DeviceBuffer.from_array(synth.normal_f32(1, r * c))

        def make():
            return din, u.DeviceBuffer(c * 4), r, c
        got, want = both(ex, make, lambda a: a[1].download(np.float32, c))
        assert got.tobytes() == want.tobytes()
        # a device-class grid; with c / 256 column strips the schedule splits R into chunks whose
        # partials live in the workspace
        assert ex.last_launch()["grid"][0] == u.device_info()[1]


def test_dequant_gemm_matches_the_allocating_launch(hip_device):
    ex = H.executor(kind="dequant_gemm", q_kind="U4", dtype="I8", group=128)
    for R, K, Cc in ((256, 1024, 16), (128, 512, 8)):
        print(f"[no_alloc] dequant gemm {R}x{K}x{Cc}", flush=True)
        w = synth.nibbles(5, R * K)
        zero, scale = synth.int16_i32(51, R * K // 128), synth.int16_i32(52, R * K // 128)
        x = (synth.int16_i32(53, K * Cc) * 13 - 100).astype(np.int8)
        bufs = [u.DeviceBuffer.from_array(a) for a in (w, zero, scale, x)]

        def make():
            return (*bufs, u.DeviceBuffer(R * Cc * 4), R, K, Cc)
        got, want = both(ex, make, lambda a: a[4].download(np.int32, R * Cc))
        assert np.array_equal(got, want)


def test_interleaved_calls_keep_the_allocating_state(hip_device):
    """Static launches between allocating ones leave the executor's own scan state intact."""
    ex = H.executor(kind="scan", dtype="I32", rank=2, op="Sum")
    n = 1 << 22
    x = synth.int16_i32(9, n)
    din = u.DeviceBuffer.from_array(x)
    outs = []
    for static in (False, True, False, True):
        out = u.DeviceBuffer(n * 4)
        if static:
            rc, why = launch_static(ex, din, out, 1, n)
            assert rc == 0, why
        else:
            launch_allocating(ex, din, out, 1, n)
        outs.append(out.download(np.int32, n))
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def test_a_workspace_beyond_the_scratch_is_refused(hip_device):
    """The dequant GEMM at C = 1024 repacks 29 MB of activations: more than the static scratch, so
    the call is refused before any kernel runs and the output keeps its contents."""
    R, K, Cc = 64, 28672, 1024
    ex = H.executor(kind="dequant_gemm", q_kind="U4", dtype="I8", group=128)
    bufs = [u.DeviceBuffer.from_array(a) for a in (synth.nibbles(5, R * K), synth.int16_i32(51, R * K // 128),
                                                   synth.int16_i32(52, R * K // 128),
                                                   np.zeros(K * Cc, np.int8))]
    out = u.DeviceBuffer(R * Cc * 4)
    out.fill(0x5A)
    rc, why = launch_static(ex, *bufs, out, R, K, Cc)
    assert rc == _lib.INVALID_ARGUMENT, (rc, why)
    assert "static scratch" in why and str(STATIC_BYTES) in why
    assert (out.download(np.uint8, R * Cc * 4) == 0x5A).all()
