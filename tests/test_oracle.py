"""Pins for the CPU oracle (oracle/oracle.c).  CPU only.

Every oracle function is checked here against something that is not itself:
  * golden vectors the reference's own tests hold (sub-byte packing, bf16 bit patterns, the
    dequant-GEMM known answer);
  * independent library routines (numpy float16 conversions, torch bfloat16 rounding, numpy's
    int32 wrapping sums, Python's exact rationals);
  * closed forms (dyadic sums are exact in f64, so every order rounds to RN32(exact)) and brute
    force on tiny inputs;
and planted mistakes (an f32 accumulator, a dropped element, a swapped nibble order) are shown
to fail the same checks.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from tests.golden import corpora
from unpopped_amd import synth

rng = np.random.default_rng


def bits32(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------------------
# bf16 / f16 codecs (crates/unpopped/src/oracle/float_codec.rs)
# ---------------------------------------------------------------------------------------

def test_bf16_codec_matches_torch_round_to_nearest_even():
    r = rng(0)
    x = np.concatenate([
        r.normal(size=200000).astype(np.float32),
        (r.normal(size=50000) * 1e30).astype(np.float32),
        (r.normal(size=50000) * 1e-38).astype(np.float32),  # f32 subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, -3.3895314e38, 1.0, 257.0, 6.0], np.float32),
    ])
    # every tie: the low 16 bits exactly 0x8000, both parities of the kept half
    ties = (r.integers(0, 1 << 15, size=20000, dtype=np.uint32) << 16 | 0x8000).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    assert np.array_equal(oracle.f32_to_bf16_bits(x), torch_bf16_bits(x))


def test_bf16_codec_reference_vectors():
    # crates/unpopped/tests/kernel_atomic_half.rs:76-94: 1.0 = 0x3F80, 256 = 0x4380,
    # 256 + 1 rounds (tie, even) to 0x4380, 12 * 0.5 = 6.0 = 0x40C0
    got = oracle.f32_to_bf16_bits(np.array([1.0, 256.0, 257.0, 6.0], np.float32))
    assert list(got) == [0x3F80, 0x4380, 0x4380, 0x40C0]
    # a NaN keeps its top half and is quieted (float_codec.rs:259-266)
    nans = np.array([0x7FC50000, 0x7F800001, 0xFFA00000, 0x7FFFFFFF], np.uint32).view(np.float32)
    assert list(oracle.f32_to_bf16_bits(nans)) == [0x7FC5, 0x7FC0, 0xFFE0, 0x7FFF]


def test_f16_decode_all_patterns_match_numpy():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f64(h)
    want = h.view(np.float16).astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(np.signbit(got), np.signbit(want))  # a NaN keeps its sign too


def test_f16_encode_matches_numpy():
    L = oracle.lib()
    r = rng(1)
    x = np.concatenate([r.normal(size=20000) * 1e3, r.normal(size=5000) * 1e-5, r.normal(size=1000) * 7e4,
                        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6e-8, 2.98e-8, np.inf, -np.inf])]).astype(np.float32)
    got = np.array([L.orc_f32_to_f16_bits(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert L.orc_f32_to_f16_bits(float("nan")) == 0x7E00


def test_round_to_odd_then_bf16_is_correctly_rounded():
    """expr_eval.rs:503-527: bf16(odd(v)) must equal the correctly rounded bf16 of the f64 value
    (checked with exact rationals), where a plain f64 -> f32 -> bf16 double-rounds."""
    L = oracle.lib()
    r = rng(2)
    # values just off a bf16 tie, where double rounding bites
    base = r.integers(0x3F800000, 0x4F000000, size=3000, dtype=np.uint64).astype(np.uint32)
    base = (base & 0xFFFF0000) | 0x8000
    vals = base.view(np.float32).astype(np.float64) * (1 + r.choice([-1, 1], size=base.size) * 2.0 ** -40)
    double_rounding_seen = 0
    for v in vals:
        got = L.orc_store_bf16(float(v))
        # exact: the two neighbouring bf16 values of v, pick nearest, ties to even
        f = Fraction(float(v))
        lo_bits = int(np.float32(v).view(np.uint32)) >> 16
        cands = [lo_bits - 1, lo_bits, lo_bits + 1]
        vals_c = [Fraction(float(np.uint32(c << 16).view(np.float32))) for c in cands]
        best = min(range(3), key=lambda i: (abs(vals_c[i] - f), cands[i] & 1))
        assert got == cands[best], (v, hex(got), hex(cands[best]))
        if oracle.f32_to_bf16_bits(np.float32(v))[0] != got:
            double_rounding_seen += 1
    assert double_rounding_seen > 0  # the naive path really is wrong on these inputs


# ---------------------------------------------------------------------------------------
# Sub-byte elements (crates/unpopped/tests/kernel_subbyte_load.rs, sub_byte_packing.rs)
# ---------------------------------------------------------------------------------------

def test_nibble_golden_vectors():
    L = oracle.lib()
    nib = np.array([0x8, 0xF, 0x0, 0x1, 0x7, 0x3, 0xC, 0x5], np.int32)
    packed = np.zeros(4, np.uint8)
    for i, v in enumerate(nib):
        L.orc_sub4_store(packed.ctypes.data, i, int(v))
    assert list(packed) == [0xF8, 0x10, 0x37, 0x5C]  # low nibble first (kernel_subbyte_load.rs:129)
    assert [L.orc_u4_load(packed.ctypes.data, i) for i in range(8)] == [8, 15, 0, 1, 7, 3, 12, 5]
    assert [L.orc_i4_load(packed.ctypes.data, i) for i in range(8)] == [-8, -1, 0, 1, 7, 3, -4, 5]
    two = np.zeros(2, np.uint8)
    for i, v in enumerate([1, 2, 3, 4]):
        L.orc_sub4_store(two.ctypes.data, i, v)
    assert list(two) == [0x21, 0x43]  # sub_byte_packing.rs:31-38, :128
    L.orc_sub4_store(two.ctypes.data, 1, 9)  # a store keeps its byte neighbour
    assert list(two) == [0x91, 0x43]


def test_synth_nibbles_are_low_nibble_first():
    s = synth.nibbles(4, 1001)
    vals = np.array([oracle.lib().orc_u4_load(s.ctypes.data, i) for i in range(1001)])
    # the same stream, drawn by the LCG directly
    st, want = 4, []
    for _ in range(1001):
        st = (st * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
        want.append(st >> 60)
    assert np.array_equal(vals, want)


# ---------------------------------------------------------------------------------------
# Dequant
# ---------------------------------------------------------------------------------------

def _dequant_numpy(q, s, z, rows, cols, group, q_signed, z_signed):
    qv = np.stack([q & 15, q >> 4], axis=1).ravel()[: rows * cols].astype(np.int64)
    ng = -(-cols // group)
    zv = np.stack([z & 15, z >> 4], axis=1).ravel()[: rows * ng].astype(np.int64)
    if q_signed:
        qv = np.where(qv >= 8, qv - 16, qv)
    if z_signed:
        zv = np.where(zv >= 8, zv - 16, zv)
    sv = s.view(np.float16).astype(np.float64)
    g = (np.arange(rows)[:, None] * ng + np.arange(cols)[None, :] // group).ravel()
    v = (qv - zv[g]).astype(np.float64) * sv[g]
    return torch_bf16_bits(v.astype(np.float32)).reshape(rows, cols)  # exact products: one rounding


@pytest.mark.parametrize("qs,zs", [(False, False), (True, False), (False, True), (True, True)])
def test_dequant_matches_numpy_and_torch_rounding(qs, zs):
    rows, cols, group = 9, 200, 24
    ng = -(-cols // group)
    q, z = synth.nibbles(4, rows * cols), synth.nibbles(5, rows * ng)
    s = synth.uniform_f16_bits(6, rows * ng, 0.001, 0.02)
    got = oracle.dequant4_bf16(q, s, z, rows, cols, group, qs, zs)
    assert np.array_equal(got, _dequant_numpy(q, s, z, rows, cols, group, qs, zs))
    # a swapped nibble order is caught
    swapped = ((q >> 4) | (q << 4)).astype(np.uint8)
    assert not np.array_equal(oracle.dequant4_bf16(swapped, s, z, rows, cols, group, qs, zs), got)


def test_dequant_gemm_known_answer():
    """crates/unpopped/tests/support/dequant.rs:145-181 (R=4, K=8, C=4, GROUP=4): the int4 GEMM's
    host answer, reproduced from the oracle's dequantized weights (exact in bf16) times x."""
    R, K, C, GROUP = 4, 8, 4, 4
    G = K // GROUP
    nib = [(r * 5 + k * 3 + 1) % 16 for r in range(R) for k in range(K)]
    packed = np.array([nib[i] | nib[i + 1] << 4 for i in range(0, len(nib), 2)], np.uint8)
    zero = [(i % 3) - 1 for i in range(R * G)]
    scale = [1 + (i * 2 % 3) for i in range(R * G)]
    x = np.array([(i * 7 % 9) - 4 for i in range(K * C)], np.int64).reshape(K, C)
    zp = np.array([(zero[i] & 15) | ((zero[i + 1] & 15) << 4) for i in range(0, R * G, 2)], np.uint8)
    sc = np.array(scale, np.float16).view(np.uint16)
    for signed in (False, True):
        w = oracle.dequant4_bf16(packed, sc, zp, R, K, GROUP, q_signed=signed, z_signed=True)
        wv = (w.astype(np.uint32) << 16).view(np.float32).astype(np.int64)
        got = wv @ x
        want = np.zeros((R, C), np.int64)  # the fixture's own host formula
        for r in range(R):
            for c in range(C):
                for k in range(K):
                    n = nib[r * K + k]
                    n = n - 16 if signed and n >= 8 else n
                    g = r * G + k // GROUP
                    want[r, c] += (n - zero[g]) * scale[g] * x[k, c]
        assert np.array_equal(got, want)


def _gemm_fixture():
    """crates/unpopped/tests/support/dequant.rs:145-163 (R=4, K=8, C=4, GROUP=4)."""
    R, K, C, GROUP = 4, 8, 4, 4
    G = K // GROUP
    nib = [(r * 5 + k * 3 + 1) % 16 for r in range(R) for k in range(K)]
    packed = np.array([nib[i] | nib[i + 1] << 4 for i in range(0, len(nib), 2)], np.uint8)
    zero = np.array([(i % 3) - 1 for i in range(R * G)], np.int32)
    scale = np.array([1 + (i * 2 % 3) for i in range(R * G)], np.int32)
    x = np.array([(i * 7 % 9) - 4 for i in range(K * C)], np.int32)
    return R, K, C, GROUP, nib, packed, zero, scale, x


def test_dequant_gemm_i32_fixture_known_answer():
    """The oracle's integer dequant GEMM on the reference's fixture equals the fixture's host
    answer (support/dequant.rs:166-181), computed here from the nibble formula, for I4 and U4."""
    R, K, C, GROUP, nib, packed, zero, scale, x = _gemm_fixture()
    G = K // GROUP
    xs = x.astype(np.int64).reshape(K, C)
    answers = []
    for signed in (False, True):
        want = np.zeros((R, C), np.int64)
        for r in range(R):
            for c in range(C):
                for k in range(K):
                    n = nib[r * K + k]
                    n = n - 16 if signed and n >= 8 else n
                    g = r * G + k // GROUP
                    want[r, c] += (n - int(zero[g])) * int(scale[g]) * int(xs[k, c])
        got = oracle.dequant_gemm_i32(packed, zero, scale, x, R, K, C, GROUP, w_signed=signed)
        assert np.array_equal(got, want)
        # the fixture's activations fit I8: the int8-activation form gives the same answer
        assert np.array_equal(oracle.dequant_gemm_i32(packed, zero, scale, x.astype(np.int8), R, K, C, GROUP,
                                                      w_signed=signed), want)
        answers.append(got)
    # the two weight types give different results, so the check can tell them apart
    # (kernel_dequant_gemm.rs:52-54)
    assert not np.array_equal(answers[0], answers[1])


def test_dequant_gemm_i32_seeded_mutations_change_the_answer():
    """docs/options-u9b-subbyte-dequant.md:28-30: nibble order swapped, sign extension dropped,
    scale group off by one and zero point ignored each move the fixture's answer."""
    R, K, C, GROUP, nib, packed, zero, scale, x = _gemm_fixture()
    base = oracle.dequant_gemm_i32(packed, zero, scale, x, R, K, C, GROUP, w_signed=True)
    swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
    assert not np.array_equal(oracle.dequant_gemm_i32(swapped, zero, scale, x, R, K, C, GROUP, w_signed=True), base)
    assert not np.array_equal(oracle.dequant_gemm_i32(packed, zero, scale, x, R, K, C, GROUP, w_signed=False), base)
    shifted = np.roll(scale, 1)
    assert not np.array_equal(oracle.dequant_gemm_i32(packed, zero, shifted, x, R, K, C, GROUP, w_signed=True), base)
    assert not np.array_equal(
        oracle.dequant_gemm_i32(packed, np.zeros_like(zero), scale, x, R, K, C, GROUP, w_signed=True), base)


@pytest.mark.parametrize("xdt", [np.int8, np.int32])
@pytest.mark.parametrize("R,K,C,GROUP", [(7, 96, 5, 32), (3, 100, 9, 7), (16, 256, 33, 128)])
def test_dequant_gemm_i32_matches_wrapping_int64_einsum(R, K, C, GROUP, xdt):
    """Random data with full-range I32 scales and zero points: int64 einsum reduced mod 2^32
    (the ring the kernel's wrapping I32 arithmetic lives in), ragged last group included."""
    r = np.random.default_rng(R * 1000 + K)
    G = -(-K // GROUP)
    nib = r.integers(0, 16, size=R * K)
    packed = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8) if K % 2 == 0 or R % 2 == 0 else None
    if packed is None:
        nib = np.concatenate([nib, [0]])
        packed = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        nib = nib[:-1]
    zero = r.integers(-2 ** 31, 2 ** 31, size=R * G, dtype=np.int64).astype(np.int32)
    scale = r.integers(-2 ** 31, 2 ** 31, size=R * G, dtype=np.int64).astype(np.int32)
    info = np.iinfo(xdt)
    x = r.integers(int(info.min), int(info.max) + 1, size=K * C, dtype=np.int64).astype(xdt)
    for signed in (False, True):
        w = nib.reshape(R, K).astype(np.int64)
        if signed:
            w = np.where(w >= 8, w - 16, w)
        gi = np.arange(K) // GROUP
        zz = zero.reshape(R, G).astype(np.int64)[:, gi]
        ss = scale.reshape(R, G).astype(np.int64)[:, gi]
        d = (((w - zz) % 2 ** 32) * (ss % 2 ** 32)) % 2 ** 32  # (w - z) * s in the ring
        want = (d @ (x.reshape(K, C).astype(np.int64) % 2 ** 32)) % 2 ** 32
        want = want.astype(np.uint32).view(np.int32)
        got = oracle.dequant_gemm_i32(packed, zero, scale, x, R, K, C, GROUP, w_signed=signed)
        assert np.array_equal(got, want)


def test_dequant_special_scales_follow_the_codec():
    rows, cols, group = 2, 64, 8
    ng = cols // group
    s = np.array([0xBC00, 0x0001, 0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x7BFF] * 2, np.uint16)
    q, z = synth.nibbles(7, rows * cols), synth.nibbles(8, rows * ng)
    got = oracle.dequant4_bf16(q, s, z, rows, cols, group)
    qv = np.stack([q & 15, q >> 4], 1).ravel().astype(np.int64)
    zv = np.stack([z & 15, z >> 4], 1).ravel().astype(np.int64)
    g = np.arange(rows * cols) // group
    with np.errstate(invalid="ignore"):
        v = ((qv - zv[g]).astype(np.float32) * s.view(np.float16).astype(np.float32)[g]).ravel()
    nan = np.isnan(v)
    assert np.array_equal((got.ravel() & 0x7FFF) > 0x7F80, nan)
    assert np.array_equal(got.ravel()[~nan], torch_bf16_bits(v[~nan]))
    assert np.array_equal(got.ravel()[~nan] >> 15, np.signbit(v[~nan]).astype(np.uint16))  # signed zeros


# ---------------------------------------------------------------------------------------
# Reductions
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_int_reductions_wrap_and_match_numpy(dtype):
    info = np.iinfo(dtype)
    x = rng(3).integers(info.min, info.max, size=(7, 1001), dtype=dtype, endpoint=True)
    assert np.array_equal(oracle.reduce_rows(x, "Sum"), np.sum(x, axis=1, dtype=dtype))
    assert np.array_equal(oracle.reduce_rows(x, "Prod"), np.prod(x, axis=1, dtype=dtype))
    assert np.array_equal(oracle.reduce_rows(x, "Max"), x.max(axis=1))
    assert np.array_equal(oracle.reduce_rows(x, "Min"), x.min(axis=1))


def test_float_extrema_keep_nan_and_empty_rows_store_zero():
    x = rng(4).normal(size=(5, 300)).astype(np.float32)
    x[1, 7] = np.nan
    x[2, :] = -np.inf
    assert np.array_equal(oracle.reduce_rows(x, "Max"), x.max(axis=1), equal_nan=True)
    assert np.array_equal(oracle.reduce_rows(x, "Min"), x.min(axis=1), equal_nan=True)
    empty = np.zeros((3, 0), np.float32)
    assert list(oracle.reduce_rows(empty, "Max")) == [0.0] * 3  # the fold's starting value
    assert np.isnan(oracle.reduce_rows(empty, "Mean")).all()  # 0 / 0


def test_dyadic_sums_round_the_exact_sum_and_an_f32_accumulator_fails():
    x = synth.uniform_pm1_f32(0, 1 << 20).reshape(4, -1)
    exact = [sum(Fraction(float(v)) for v in row[:4096]) for row in x[:, :4096]]
    got = oracle.reduce_rows(np.ascontiguousarray(x[:, :4096]), "Sum")
    assert all(float(np.float32(float(e))) == g for e, g in zip(exact, got))
    full = oracle.reduce_rows(x, "Sum")
    assert np.array_equal(full, x.astype(np.float64).sum(axis=1).astype(np.float32))
    f32_acc = np.array([np.add.reduce(r, dtype=np.float32) for r in x])  # a planted mistake
    assert not np.array_equal(f32_acc, full)


def test_neumaier_is_near_exact():
    r = rng(5)
    for _ in range(20):
        xs = r.normal(size=500) * 10.0 ** r.integers(-8, 8, size=500)
        exact = float(sum(Fraction(v) for v in xs))
        assert abs(oracle.neumaier(xs) - exact) <= 4 * 2.0 ** -53 * abs(exact) + 1e-300


def test_launched_order_and_bound_on_the_reference_corpus():
    """tests/kernel_parallel_reduction_float_sum_bound.rs: the declared bound holds for the
    launched order at every geometry, block 1 is the serial order, and the corpus makes the
    bound bite (a visible difference between orders)."""
    corpus = corpora.float_sum_bound_corpus()
    orders_differ = False
    for row in corpus:
        serial = oracle.reduce_rows(row.reshape(1, -1), "Sum")[0]
        for block in (1, 2, 8, 32, 128):
            for mean in (False, True):
                tot = oracle.sum_launched_order(row, block, mean)
                exact = float(sum(Fraction(float(v)) for v in row)) / (row.size if mean else 1)
                b = oracle.sum_bound(row, tot, mean=mean, f32=False)
                assert abs(tot - exact) <= b
            orders_differ |= oracle.sum_launched_order(row, block) != serial
        # block 1 folds in the serial order
        assert oracle.sum_launched_order(row, 1) == serial
    assert orders_differ
    # the corpus rows generated from the reference's LCG (values drawn, not retyped)
    assert corpus[1, 1] == -1.0e8 and corpus[3, 5] == 0.1


def test_sum_bound_rejects_a_dropped_element():
    x = rng(6).normal(size=(1, 4000)).astype(np.float64)
    got = oracle.reduce_rows(x, "Sum")[0]
    assert abs(got - oracle.neumaier(x[0])) <= oracle.sum_bound(x[0], got, f32=False)
    wrong = got - x[0, 17]  # a dropped term
    assert abs(wrong - oracle.neumaier(x[0])) > oracle.sum_bound(x[0], wrong, f32=False)


# ---------------------------------------------------------------------------------------
# Scans
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_int_scans_match_numpy(dtype):
    info = np.iinfo(dtype)
    x = rng(7).integers(info.min, info.max, size=(3, 777), dtype=dtype, endpoint=True)
    inc = np.cumsum(x, axis=1, dtype=dtype)
    assert np.array_equal(oracle.scan_rows(x, "Sum"), inc)
    exc = np.concatenate([np.zeros((3, 1), dtype), inc[:, :-1]], axis=1)
    assert np.array_equal(oracle.scan_rows(x, "Sum", exclusive=True), exc)
    rev = np.flip(np.cumsum(np.flip(x, 1), axis=1, dtype=dtype), 1)
    assert np.array_equal(oracle.scan_rows(x, "Sum", reverse=True), rev)
    assert np.array_equal(oracle.scan_rows(x, "Max"), np.maximum.accumulate(x, axis=1))
    ex_max = oracle.scan_rows(x, "Max", exclusive=True)
    assert (ex_max[:, 0] == info.min).all()  # the integer Max identity (scan_identity)
    assert np.array_equal(oracle.scan_rows(x, "Min"), np.minimum.accumulate(x, axis=1))
    assert np.array_equal(oracle.scan_rows(x, "Prod"), np.cumprod(x, axis=1, dtype=dtype))


def test_float_scans():
    x = synth.uniform_01_f32(2, 3 * 5000).reshape(3, 5000)
    assert np.array_equal(oracle.scan_rows(x, "Sum"), np.cumsum(x.astype(np.float64), axis=1).astype(np.float32))
    y = rng(8).normal(size=(2, 3000)).astype(np.float32)
    y[0, 1500] = np.nan
    assert np.array_equal(oracle.scan_rows(y, "Max"), np.maximum.accumulate(y, axis=1), equal_nan=True)
    ex = oracle.scan_rows(y, "Max", exclusive=True)
    assert ex[0, 0] == -np.inf and np.isnan(ex[0, 1501]) and not np.isnan(ex[0, 1500])
    m = oracle.scan_rows(y[1:].astype(np.float64), "Mean")
    assert np.allclose(m[0], np.cumsum(y[1].astype(np.float64)) / np.arange(1, 3001), rtol=1e-12)
    assert np.isnan(oracle.scan_rows(y[1:].astype(np.float64), "Mean", exclusive=True)[0, 0])  # 0 / 0


def test_launched_scan_order():
    x = synth.uniform_01_f32(2, 10007)
    serial = oracle.scan_rows(x.reshape(1, -1), "Sum").ravel()
    for block in (1, 4, 64, 256):
        for ex in (False, True):
            for rev in (False, True):
                got = oracle.scan_launched_order_f32(x, block, ex, rev)
                assert np.array_equal(got, oracle.scan_rows(x.reshape(1, -1), "Sum", ex, rev).ravel())
    y = rng(9).normal(size=5000).astype(np.float32)
    assert np.array_equal(oracle.scan_launched_order_f32(y, 1), oracle.scan_rows(y.reshape(1, -1), "Sum").ravel())
    assert not np.array_equal(serial[1:], serial[:-1])


# ---------------------------------------------------------------------------------------
# Gather
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("idx", [np.int32, np.int64, np.uint32])
@pytest.mark.parametrize("policy", ["Skip", "ZeroFill", "Clamp"])
def test_gather_policies_match_numpy(idx, policy):
    V, D, N = 50, 7, 300
    table = rng(10).normal(size=(V, D)).astype(np.float32)
    ids = rng(11).integers(-20 if idx != np.uint32 else 0, V + 20, size=N).astype(idx)
    init = np.full((N, D), 123.0, np.float32)
    got = oracle.gather_rows(table, ids, policy, out_init=init)
    raw = ids.astype(np.int64)
    oob = (raw < 0) | (raw >= V)
    want = table[np.clip(raw, 0, V - 1)].copy()
    if policy == "Skip":
        want[oob] = 123.0
    elif policy == "ZeroFill":
        want[oob] = 0.0
    assert np.array_equal(got, want)


def test_gather_empty_source():
    ids = np.array([0, -1, 3], np.int32)
    got = oracle.gather_rows(np.zeros((1, 4), np.uint16), ids, "ZeroFill", out_init=np.full((3, 4), 9, np.uint16),
                             src_extent=0)
    assert not got.any()


# ---------------------------------------------------------------------------------------
# The synthetic generator (inputs of the parity tests and the benchmark)
# ---------------------------------------------------------------------------------------

def test_synth_parallel_chunks_equal_the_sequential_stream():
    n = (1 << 20) + 5  # crosses the generator's chunk boundary
    got = synth.uniform_pm1_f32(0, n)
    s, M = 0, (1 << 64) - 1
    idx = [0, 1, 2, (1 << 20) - 1, 1 << 20, (1 << 20) + 4]
    want = {}
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & M
        if i in idx:
            want[i] = ((s >> 39) - (1 << 24)) / float(1 << 24)
    assert all(got[i] == want[i] for i in idx)
    assert got.min() >= -1.0 and got.max() < 1.0
    z = synth.zipf_ids_i32(3, 65536, 262144, 1.1)
    assert z.min() >= 0 and z.max() < 262144
    assert np.bincount(z).max() > 1000  # heavy-tailed: the top row repeats


# ---------------------------------------------------------------------------------------
# Row reductions (crates/unpopped/src/kernel_lift/row_reduce.rs; tests/kernel_row_reduce_agrees.rs)
# ---------------------------------------------------------------------------------------

import math  # noqa: E402
from functools import reduce as _fold  # noqa: E402

from unpopped_amd import expr as X  # noqa: E402

# the corpus of kernel_row_reduce_agrees.rs:33-35 and :141-145
RR_VALUES = [1.0e8, 1.0, -1.0e8, 0.5, 3.25, -2.0, 7.0, 0.1, -0.75, 12.0, -5.5, 0.3, 2.0]


def rr_data(rows, k, dtype):
    return np.array([RR_VALUES[i % 13] * (1.0 + (i // 13) * 0.37) for i in range(rows * k)]).astype(dtype).reshape(rows, k)


def rnd(v, dtype):
    return float(np.asarray(v, dtype=dtype)) if dtype == np.float32 else v


def test_row_reduce_identity_epilogues_equal_the_reduction_oracle():
    """kernel_row_reduce_agrees.rs:148-160: an identity epilogue is the lifted reduction."""
    x = rr_data(3, 13, np.float32)
    for op in ("Sum", "Mean", "Max", "Min"):
        got = oracle.row_reduce([x], [(X.input(0), op)], X.reduced(0))
        want = oracle.reduce_rows(x, op)
        assert np.array_equal(got, np.repeat(want[:, None], 13, axis=1)), op


def test_row_reduce_wide_accumulator_known_answer():
    """kernel_row_reduce_agrees.rs:213-229: 1e8 + 1 - 1e8 in a row needs an f64 accumulator."""
    x = np.array([[1.0e8, 1.0, -1.0e8, 0.5, 2.0]], np.float32)
    got = oracle.row_reduce([x], [(X.input(0), "Sum")], X.reduced(0))
    assert got[0, 0] == 3.5


def closed_form(x, dtype, which):
    """The serial lifted kernel restated with Python floats (f64) and math (the host libm, as
    Rust's f64 methods call it): ascending folds, one rounding per statement."""
    out = np.empty_like(x)
    for r, row in enumerate(x.astype(np.float64)):
        if which == "softmax":
            m = rnd(_fold(lambda a, v: v if (v != v or v > a) else a, row), dtype)
            s = rnd(_fold(lambda a, v: a + rnd(math.exp(v - m), dtype), row, 0.0), dtype)
            out[r] = [math.exp(v - m) / s for v in row]
        elif which == "rms_norm":
            mean = rnd(_fold(lambda a, v: a + rnd(v * v, dtype), row, 0.0) / len(row), dtype)
            out[r] = [v / math.sqrt(mean + 1.0e-3) for v in row]
        else:  # centred quotient
            mean = rnd(_fold(lambda a, v: a + v, row, 0.0) / len(row), dtype)
            mx = rnd(_fold(lambda a, v: v if (v != v or v > a) else a, [rnd(v - mean, dtype) for v in row]), dtype)
            out[r] = [(v - mean) / mx for v in row]
    return out


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("which", ["softmax", "rms_norm", "centred_quotient"])
def test_row_reduce_matches_the_closed_form(dtype, which):
    x = rr_data(5, 13, dtype)
    stages, epi = getattr(X, which)()
    got = oracle.row_reduce([x], stages, epi)
    assert np.array_equal(got, closed_form(x, dtype, which))
    # a planted mistake: the stage value left unrounded at f32 moves some softmax output
    if dtype == np.float32 and which == "softmax":
        moved = False
        for rows in range(1, 40):
            src = np.array([((i * 7 + 3) % 19) * 0.37 - 2.0 for i in range(rows * 11)], np.float32).reshape(rows, 11)
            exact = closed_form(src.astype(np.float64), np.float64, "softmax").astype(np.float32)
            moved |= not np.array_equal(oracle.row_reduce([src], stages, epi), exact)
        assert moved  # kernel_row_reduce_agrees.rs:186-204: the rounding is not vacuous


def test_row_reduce_nan_and_infinity_rows():
    """kernel_row_reduce_agrees.rs:232-260: NaN and infinite rows."""
    x = np.array([[1.0, np.nan, 2.0, 3.0], [np.inf, 1.0, 2.0, -np.inf], [0.0, -0.0, 1.0, 2.0]], np.float32)
    sm = oracle.row_reduce([x], *X.softmax())
    assert np.isnan(sm[0]).all()            # a NaN max poisons its row
    assert np.isnan(sm[1]).all()            # max is inf, exp(inf - inf) is NaN, so the sum is NaN
    assert np.allclose(sm[2].sum(), 1.0, rtol=1e-6)
    cq = oracle.row_reduce([x], *X.centred_quotient())
    assert np.isnan(cq[0]).all()


def test_rx_program_ops_follow_the_host_libm():
    """Every op the programs carry, against Python's math (the same libm)."""
    for v in (-2.5, -0.3, 0.0, 0.7, 1.9):
        for name, f in [("Neg", lambda a: -a), ("Abs", abs), ("Sqr", lambda a: a * a), ("Exp", math.exp),
                        ("Tanh", math.tanh), ("Sigmoid", lambda a: 1.0 / (1.0 + math.exp(-a))),
                        ("Relu", lambda a: 0.0 if a < 0.0 else a), ("Erf", math.erf), ("Sin", math.sin),
                        ("Cos", math.cos), ("Floor", math.floor), ("Ceil", math.ceil), ("Trunc", math.trunc),
                        ("Expm1", math.expm1), ("Atan", math.atan), ("Asinh", math.asinh), ("Sinh", math.sinh),
                        ("Silu", lambda a: a * (1.0 / (1.0 + math.exp(-a)))),
                        ("Gelu", lambda a: 0.5 * a * (1.0 + math.erf(a * 0.70710678118654752440)))]:
            assert oracle.rx_eval(X.input(0).unary(name), [v]) == float(f(v)), (name, v)
        if v > 0:
            for name, f in [("Sqrt", math.sqrt), ("Log", math.log), ("Log2", math.log2), ("Log10", math.log10),
                            ("Rsqrt", lambda a: 1.0 / math.sqrt(a)), ("Recip", lambda a: 1.0 / a)]:
                assert oracle.rx_eval(X.input(0).unary(name), [v]) == f(v), (name, v)
    # Max/Min: NaN-propagating, the left operand on ties (scalar_ops.rs:90-112)
    mx = X.input(0).maximum(X.input(1))
    assert oracle.rx_eval(mx, [-0.0, 0.0]) == 0.0 and math.copysign(1, oracle.rx_eval(mx, [-0.0, 0.0])) < 0
    assert math.isnan(oracle.rx_eval(mx, [1.0, float("nan")]))
    # Sign decides on the argument rounded to the compute dtype first (expr_eval.rs:130-137)
    tiny = 1e-50
    assert oracle.rx_eval(X.input(0).unary("Sign"), [tiny], f32=True) == 0.0
    assert oracle.rx_eval(X.input(0).unary("Sign"), [tiny], f32=False) == 1.0
    # Fma rounds once: 0.1 * 10 - 1 is exactly 2^-54 (0.1 is 0x1.999999999999ap-4), the two-step form gives 0
    assert oracle.rx_eval(X.fma(X.input(0), X.input(1), X.input(2)), [0.1, 10.0, -1.0]) == 2.0 ** -54
    assert oracle.rx_eval(X.input(0) * X.input(1) + X.input(2), [0.1, 10.0, -1.0]) == 0.0


def test_nan_ignoring_folds_against_numpy():
    """MaxNum/MinNum (kernel_lift.rs nan_arm: a NaN accumulator is replaced, a NaN element is
    skipped) equal numpy's fmax/fmin reductions, which ignore NaN unless every element is NaN; an
    empty row stores 0.  The NaN-keeping Max differs on every row holding a NaN."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((8, 33)).astype(np.float32)
    x[1, 0] = np.nan
    x[2, :] = np.nan
    x[3, 17] = np.nan
    x[4, -1] = np.nan
    x[5, ::2] = np.nan
    for op, f in (("MaxNum", np.fmax), ("MinNum", np.fmin)):
        got = oracle.reduce_rows(x, op)
        assert np.array_equal(got, f.reduce(x, axis=1), equal_nan=True), op
        assert np.array_equal(oracle.reduce_rows(x.astype(np.float64), op), f.reduce(x.astype(np.float64), axis=1),
                              equal_nan=True)
        keep = oracle.reduce_rows(x, op[:3])
        for r in (1, 3, 4, 5):
            assert np.isnan(keep[r]) and not np.isnan(got[r]), (op, r)
    assert np.array_equal(oracle.reduce_rows(np.zeros((3, 0), np.float32), "MaxNum"), np.zeros(3, np.float32))


def test_bit_folds_against_numpy():
    """And/Or/Xor (kernel_lift.rs bit_step, seeded by the first element) equal numpy's bitwise
    reductions over full-range integers; an empty row stores 0 (not And's all-ones identity); at an
    integer MaxNum/MinNum are Max/Min."""
    rng = np.random.default_rng(12)
    for nt in (np.int32, np.int64):
        info = np.iinfo(nt)
        x = rng.integers(info.min, info.max, (9, 21), dtype=np.int64).astype(nt)
        x[0] = -1
        for op, f in (("And", np.bitwise_and), ("Or", np.bitwise_or), ("Xor", np.bitwise_xor)):
            assert np.array_equal(oracle.reduce_rows(x, op), f.reduce(x, axis=1)), (nt, op)
            assert np.array_equal(oracle.reduce_rows(np.zeros((2, 0), nt), op), np.zeros(2, nt))
        assert np.array_equal(oracle.reduce_rows(x, "MaxNum"), x.max(axis=1))
        assert np.array_equal(oracle.reduce_rows(x, "MinNum"), x.min(axis=1))


def test_gather_along_any_axis_against_numpy():
    """index_select along each axis: numpy's take of the clamped index, with the policy applied to the
    stored cells (Skip leaves them, ZeroFill zeroes them, Clamp keeps the clamped read)."""
    rng = np.random.default_rng(13)
    t = rng.integers(0, 2**16, (4, 6, 5), dtype=np.uint16)
    for axis in range(3):
        V = t.shape[axis]
        ids = rng.integers(-3, V + 3, 7).astype(np.int64)
        init = rng.integers(0, 2**16, t.shape[:axis] + (7,) + t.shape[axis + 1:], dtype=np.uint16)
        taken = np.take(t, np.clip(ids, 0, V - 1), axis=axis)
        oob = (ids < 0) | (ids >= V)
        shape = [1, 1, 1]
        shape[axis] = 7
        mask = np.broadcast_to(oob.reshape(shape), taken.shape)
        for policy, want in (("Clamp", taken), ("ZeroFill", np.where(mask, 0, taken)),
                             ("Skip", np.where(mask, init, taken))):
            got = oracle.gather_axis(t, ids, axis, policy, out_init=init)
            assert np.array_equal(got, want), (axis, policy)


def test_gather_cells_pins():
    """The per-cell gather (an index of the output's own shape) against: the index_select oracle when
    the index is the same along every other axis; the C99 leg running the gather lift on the same
    storage images; the identity index reproducing the table."""
    from unpopped_amd import forms as H
    from oracle import cpuc
    from oracle.cpuc import View

    rng_ = np.random.default_rng(23)
    t = rng_.integers(0, 2**16, (5, 6, 4), dtype=np.uint16)
    for axis in range(3):
        V = t.shape[axis]
        n = 7
        out_shape = t.shape[:axis] + (n,) + t.shape[axis + 1:]
        ids1 = rng_.integers(-3, V + 3, n).astype(np.int64)
        shape = [1, 1, 1]
        shape[axis] = n
        full = np.broadcast_to(ids1.reshape(shape), out_shape)
        init = rng_.integers(0, 2**16, out_shape, dtype=np.uint16)
        for policy in ("Skip", "ZeroFill", "Clamp"):
            want = oracle.gather_axis(t, ids1, axis, policy, out_init=init)
            assert np.array_equal(oracle.gather_cells(t, full, axis, policy, out_init=init), want), (axis, policy)
        # A different index in every cell: the C99 leg of the lift reads it through the view.
        ids = rng_.integers(-2, V + 2, out_shape).astype(np.int32)
        k = H.kernel_for(kind="gather", dtype="Bf16", rank=3, index_dtype="I32", oob="ZeroFill", axis=axis)
        got = init.copy()
        assert cpuc.run(k, t, View(ids), got, *out_shape, V) == cpuc.OK
        assert np.array_equal(oracle.gather_cells(t, ids, axis, "ZeroFill", out_init=init), got), axis
    ident = np.broadcast_to(np.arange(5).reshape(5, 1, 1), t.shape)
    assert np.array_equal(oracle.gather_cells(t, ident, 0, "Skip"), t)
    # A planted mistake (the index read at the transposed cell) fails the C99 comparison.
    ids = rng_.integers(0, 5, (5, 5)).astype(np.int32)
    t2 = rng_.integers(0, 2**16, (5, 5), dtype=np.uint16)
    good = oracle.gather_cells(t2, ids, 0, "Skip")
    assert not np.array_equal(oracle.gather_cells(t2, ids.T.copy(), 0, "Skip"), good)


def test_general_gather_cell_pins():
    """The general gather cell (any input order, a body over the gathered element and the other inputs):
    with the identity body and two inputs it is the per-cell gather; with a body it equals the C99 leg
    of the same lift on the same inputs within the C leg's per-operation rounding (one rounding at f64
    here, one per float operation there), and exactly on dyadic data where both are exact."""
    from unpopped_amd import expr as X
    from unpopped_amd import forms as H  # noqa: F401  (loads the library)
    import unpopped_amd as u
    from oracle import cpuc

    r = np.random.default_rng(71)
    t = r.integers(-100, 100, (7, 5)).astype(np.float32) / 8  # 7 rows, src_extent 6
    ids = np.broadcast_to(r.integers(-2, 9, 7).reshape(7, 1), (7, 5)).astype(np.int32).copy()
    init = np.full((7, 5), 3.0, np.float32)
    for policy in ("Skip", "ZeroFill", "Clamp"):
        want = oracle.gather_cells(t, ids, 0, policy, out_init=init, src_extent=6)
        got = oracle.gather_expr([t, ids], 1, 0, 0, policy, {"Input": 0}, init, 6)
        assert np.array_equal(got, want), policy
    # three inputs: ids first, a scale at the output coordinate, the table last; body table * scale + 0.5
    scale = r.integers(-16, 16, (7, 5)).astype(np.float32) / 4
    body = X.input(2) * X.input(1) + 0.5
    for policy in ("Skip", "ZeroFill", "Clamp"):
        got = oracle.gather_expr([ids, scale, t], 0, 2, 0, policy, body.j, init, 6)
        k = u.lift_gather("g", "F32", 2, "I32", axis=0, oob=policy, n_inputs=3, data=2, index=0, body=body)
        c = init.copy()
        assert cpuc.run(k, ids, scale, t, c, 7, 5, 6) == cpuc.OK
        assert np.array_equal(got, c), policy  # dyadic: both exact
    # a planted mistake (the clamped index applied to the wrong input) fails the C99 comparison
    bad = oracle.gather_expr([ids, scale, t], 0, 1, 0, "Clamp", body.j, init, 6)
    k = u.lift_gather("g", "F32", 2, "I32", axis=0, oob="Clamp", n_inputs=3, data=2, index=0, body=body)
    c = init.copy()
    assert cpuc.run(k, ids, scale, t, c, 7, 5, 6) == cpuc.OK
    assert not np.array_equal(bad, c)


# ---- scans with a pre-map and a fused post (orc_scan_x) ---------------------------------

SCAN_OPS = ["Sum", "Max", "Min", "Prod", "Mean"]


@pytest.mark.parametrize("op", SCAN_OPS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_scan_x_identity_pre_equals_the_scan_oracle(op, dt):
    """With the identity pre-map and no post the lifted scan is the plain one: orc_scan_x agrees
    bit for bit with orc_scan_rows (pinned above) on every op, direction and exclusivity, NaN and
    infinity included."""
    x = np.random.default_rng(51).normal(size=(3, 37)).astype(dt)
    x[0, 5] = np.nan
    x[1, 9] = np.inf
    x[2, 30] = -np.inf
    for excl in (False, True):
        for rev in (False, True):
            got = oracle.scan_expr([x], 1, op, X.input(0), exclusive=excl, reverse=rev)
            assert np.array_equal(got, oracle.scan_rows(x, op, excl, rev), equal_nan=True), (op, excl, rev)


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_scan_x_along_any_axis_equals_the_moved_axis_scan(axis):
    """The A x S x B indexing: a scan along `axis` equals the innermost-axis scan of the array with
    that axis moved last."""
    x = np.random.default_rng(52).normal(size=(4, 5, 6)).astype(np.float32)
    for op in ("Sum", "Max", "Mean"):
        got = oracle.scan_expr([x], axis, op, X.input(0), reverse=True)
        moved = np.moveaxis(x, axis, -1)
        want = oracle.scan_rows(moved.reshape(-1, moved.shape[-1]), op, False, True).reshape(moved.shape)
        assert np.array_equal(got, np.moveaxis(want, -1, axis)), (axis, op)


def test_scan_x_pre_rounds_once_before_the_fold():
    """`val = up(pre)`: the pre-map is rounded once to the dtype before the f64 fold.  For f32 inputs
    x * y rounded to f32 is numpy's f32 product, so the Sum scan is numpy's sequential f64 cumsum of
    that product, rounded once per prefix.  The same data scanned without the rounding differs, so
    the check sees a dropped rounding."""
    r = np.random.default_rng(53)
    x = r.normal(size=(2, 300)).astype(np.float32)
    y = r.normal(size=(2, 300)).astype(np.float32)
    got = oracle.scan_expr([x, y], 1, "Sum", X.input(0) * X.input(1))
    prod = x * y
    want = np.cumsum(prod.astype(np.float64), axis=1).astype(np.float32)
    assert np.array_equal(got, want)
    unrounded = np.cumsum(x.astype(np.float64) * y.astype(np.float64), axis=1).astype(np.float32)
    assert not np.array_equal(unrounded, want)


def test_scan_x_post_reads_the_rounded_prefix_and_the_position():
    """scan_write: the post reads Reduced(0) as the prefix rounded once and Input(k) as the element at
    the position.  On data whose every prefix is exact in f32 (multiples of 1/8 below 2^7)
    `Reduced(0) - Input(0)` after an inclusive Sum is the exclusive prefix, and
    `Reduced(0) * 2 + Input(1)` is that closed form too."""
    r = np.random.default_rng(54)
    x = (r.integers(-100, 100, size=(4, 257)) / 8).astype(np.float32)
    y = (r.integers(-100, 100, size=(4, 257)) / 8).astype(np.float32)
    incl = np.cumsum(x.astype(np.float64), axis=1)
    got = oracle.scan_expr([x], 1, "Sum", X.input(0), post=X.reduced(0) - X.input(0))
    assert np.array_equal(got, (incl - x).astype(np.float32))
    assert np.array_equal(got, oracle.scan_rows(x, "Sum", True, False))
    got2 = oracle.scan_expr([x, y], 1, "Sum", X.input(0), post=X.reduced(0) * 2.0 + X.input(1))
    assert np.array_equal(got2, (incl.astype(np.float32).astype(np.float64) * 2 + y).astype(np.float32))


def test_scan_x_post_rounds_the_prefix_before_it():
    """The post sees the prefix rounded to f32, not the f64 fold: for `sqrt(Reduced(0))` the result
    is sqrt of the f32 prefix rounded once; a post fed the unrounded f64 fold differs on this data."""
    x = np.random.default_rng(56).random(size=(1, 2000)).astype(np.float32)
    got = oracle.scan_expr([x], 1, "Sum", X.input(0), post=X.reduced(0).sqrt())
    pref = np.cumsum(x.astype(np.float64), axis=1)
    want = np.sqrt(pref.astype(np.float32).astype(np.float64)).astype(np.float32)
    assert np.array_equal(got, want)
    assert not np.array_equal(np.sqrt(pref).astype(np.float32), want)


def test_scan_x_running_mean_and_nan_rules():
    """A Mean scan divides the f64 sum by the count so far (an exclusive first prefix is 0 / 0, NaN);
    a Max scan of a pre-map that makes NaN keeps it from there on (numpy's maximum.accumulate)."""
    x = synth.uniform_pm1_f32(57, 3 * 64).reshape(3, 64)
    y = synth.uniform_pm1_f32(58, 3 * 64).reshape(3, 64)
    got = oracle.scan_expr([x, y], 1, "Mean", X.input(0) + X.input(1))
    s = (x + y).astype(np.float64)
    want = (np.cumsum(s, axis=1) / np.arange(1, 65)).astype(np.float32)
    assert np.array_equal(got, want)
    ex = oracle.scan_expr([x, y], 1, "Mean", X.input(0) + X.input(1), exclusive=True)
    assert np.all(np.isnan(ex[:, 0])) and np.array_equal(ex[:, 1:], want[:, :-1])
    d = y.copy()
    d[1, 20] = 0.0
    x2 = x.copy()
    x2[1, 20] = 0.0  # 0 / 0: NaN from column 20 on
    v = (x2.astype(np.float64) / d.astype(np.float64)).astype(np.float32)
    got = oracle.scan_expr([x2, d], 1, "Max", X.input(0) / X.input(1))
    assert np.array_equal(got, np.maximum.accumulate(v, axis=1), equal_nan=True)
    assert np.isnan(got[1, 20:]).all() and not np.isnan(got[1, :20]).any()
