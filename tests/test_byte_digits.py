"""The signed byte digits the dequant GEMM's stream kernel uses for its zero-point pass
(unp_device.hip, dqg_stream): the bytes of (v + 0x80808080) ^ 0x80808080, read as int8, are
digits d_i in [-128, 127] with sum d_i 256^i = v modulo 2^32, and products of two such
expansions, summed by digit class i + j < 4 and shifted by 8 (i + j) bits, equal the 32-bit
wrapping product."""
import numpy as np

EDGES = np.array([0, 1, 127, 128, 255, 256, 0x7F7F7F7F, 0x80808080, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF,
                  0x00808080, 0x80000080, 0xFF00FF00], dtype=np.uint64)


def _digits(v):
    t = ((v.astype(np.uint64) + 0x80808080) & 0xFFFFFFFF) ^ 0x80808080
    return [((t >> (8 * i)) & 0xFF).astype(np.uint8).view(np.int8).astype(np.int64) for i in range(4)]


def _values(seed, n):
    r = np.random.default_rng(seed)
    return np.concatenate([EDGES, r.integers(0, 2 ** 32, size=n, dtype=np.uint64)])


def test_digits_recompose_modulo_2_32():
    v = _values(1, 1 << 20)
    d = _digits(v)
    assert all(int(x.min()) >= -128 and int(x.max()) <= 127 for x in d)
    back = sum(d[i] * (256 ** i) for i in range(4)) % (1 << 32)
    assert np.array_equal(back.astype(np.uint64), v)


def test_digit_class_products_give_the_wrapping_product():
    a, b = _values(2, 1 << 18), _values(3, 1 << 18)[::-1]
    da, db = _digits(a), _digits(b)
    total = np.zeros(a.shape, dtype=np.uint64)
    for sh in range(4):
        acc = sum(da[i] * db[sh - i] for i in range(sh + 1))  # at most 4 x 2^14 per class
        assert int(np.abs(acc).max()) <= 4 * 128 * 128
        total = (total + ((acc.astype(np.int64) << (8 * sh)) & 0xFFFFFFFF).astype(np.uint64)) & 0xFFFFFFFF
    want = (a * b) & 0xFFFFFFFF
    assert np.array_equal(total, want)
