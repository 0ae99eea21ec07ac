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


# ---------------------------------------------------------------------------------------
# The zero-point pass lane by lane.  A CPU restatement of dqg_stream's pass after the loop: the
# LDS staging of scale * zero under the step's group mask, each lane's packing of signed byte
# digits into the four i32x4 operand planes (lane (l32, q) holds groups 16 q .. 16 q + 15 of its
# row for A, of its column for B, the column sums masked past the step's last group), the
# v_mfma_i32_32x32x32_i8 lane layout (A row l32 / B column l32, k = 16 q + byte index; D row
# 8 (v >> 2) + 4 q + (v & 3) in accumulator v of lane (l32, q)), and the digit-class sums
# shifted into the wrapping total.  Checked against the wrapping int64 product of the same
# scale * zero and column sums.
# ---------------------------------------------------------------------------------------

def _pack_planes(vals16):
    """Four i32x4 operands (one per digit plane) from one lane's 16 u32 values, as the kernel
    packs them: word wd of plane pl holds byte pl of vb[4 wd + e] at byte e."""
    vb = ((vals16.astype(np.uint64) + 0x80808080) & 0xFFFFFFFF) ^ 0x80808080
    planes = np.zeros((4, 4), dtype=np.uint64)
    for wd in range(4):
        for pl in range(4):
            w = 0
            for e in range(4):
                w |= ((int(vb[4 * wd + e]) >> (8 * pl)) & 0xFF) << (8 * e)
            planes[pl, wd] = w
    return planes


def _operand_bytes(planes_pl):
    """The 16 int8 of one i32x4 operand, byte b = 4 wd + e."""
    return np.array([((int(planes_pl[b // 4]) >> (8 * (b % 4))) & 0xFF) for b in range(16)],
                    dtype=np.uint8).view(np.int8).astype(np.int64)


def _mfma_32x32x32_i8(a_lanes, b_lanes):
    """D[32 x 32] = A B over k = 32 from the lanes' 16-byte operands: lane (l32, q) = l32 + 32 q
    holds A[l32, 16 q + b] and B[16 q + b, l32]."""
    A = np.zeros((32, 32), dtype=np.int64)
    B = np.zeros((32, 32), dtype=np.int64)
    for lane in range(64):
        l32, q = lane % 32, lane // 32
        A[l32, 16 * q:16 * q + 16] = a_lanes[lane]
        B[16 * q:16 * q + 16, l32] = b_lanes[lane]
    return A @ B


def _zero_point_pass(sz, xsum, g0, g1, swap_q=False, masks=True, d_rows=None):
    """The pass for one 32 x 32 output tile: sz[32, ng] (scale * zero, u32), xsum[ng, 32] (column
    sums, u32), groups [g0, g1).  Returns the u32 amount the kernel subtracts from the tile, laid
    out by (row, column).  swap_q / masks / d_rows plant mistakes for the check below."""
    ng = sz.shape[1]
    total = np.zeros((64, 16), dtype=np.uint64)  # total[lane][v], as the kernel holds it
    for gc in range(g0, g1, 32):
        gl = min(32, g1 - gc)
        # LDS row of each tile row: 32 groups, those past gl zeroed (gmask); past ng reads 0.
        szs = np.zeros((32, 32), dtype=np.uint64)
        for row in range(32):
            for sg in range(32):
                g = gc + sg
                v = int(sz[row, g]) if g < ng else 0
                szs[row, sg] = v if (sg < gl or not masks) else 0
        a_pl = [[None] * 64 for _ in range(4)]
        b_pl = [[None] * 64 for _ in range(4)]
        for lane in range(64):
            l32, q = lane % 32, lane // 32
            qa = 1 - q if swap_q else q
            pa = _pack_planes(szs[l32, 16 * qa:16 * qa + 16])
            xv = np.array([int(xsum[gc + 16 * q + k, l32]) if gc + 16 * q + k < ng else 0 for k in range(16)],
                          dtype=np.uint64)
            if masks:
                xv = np.where(16 * q + np.arange(16) < gl, xv, 0).astype(np.uint64)
            pb = _pack_planes(xv)
            for pl in range(4):
                a_pl[pl][lane] = _operand_bytes(pa[pl])
                b_pl[pl][lane] = _operand_bytes(pb[pl])
        for sh in range(4):
            acc = sum(_mfma_32x32x32_i8(a_pl[i], b_pl[sh - i]) for i in range(sh + 1))
            assert int(np.abs(acc).max()) < 2 ** 31
            for lane in range(64):
                l32, q = lane % 32, lane // 32
                for v in range(16):
                    row = 8 * (v >> 2) + 4 * q + (v & 3)
                    total[lane, v] = (int(total[lane, v]) + ((int(acc[row, l32]) << (8 * sh)) & 0xFFFFFFFF)) & 0xFFFFFFFF
    rows = d_rows or (lambda v, q: 8 * (v >> 2) + 4 * q + (v & 3))
    out = np.zeros((32, 32), dtype=np.uint64)
    for lane in range(64):
        l32, q = lane % 32, lane // 32
        for v in range(16):
            out[rows(v, q), l32] = total[lane, v]
    return out


def _wrapping(sz, xsum, g0, g1):
    a = sz[:, g0:g1].astype(np.int64)
    b = xsum[g0:g1].astype(np.int64)
    # int64 products wrap harmlessly modulo 2^64; reduce modulo 2^32 at the end
    return (a @ b).astype(np.uint64) & 0xFFFFFFFF


def _zero_point_inputs(seed, ng):
    r = np.random.default_rng(seed)
    sz = r.integers(0, 2 ** 32, size=(32, ng), dtype=np.uint64)
    xsum = r.integers(0, 2 ** 32, size=(ng, 32), dtype=np.uint64)
    edges = EDGES[r.integers(0, EDGES.size, size=64)]
    sz[0, :min(ng, 64)] = edges[:min(ng, 64)]
    xsum[:min(ng, 64), 1] = edges[:min(ng, 64)]
    return sz, xsum


def test_zero_point_pass_lanes_give_the_wrapping_product():
    """Whole steps, a ragged last step (gl < 32, past the groups of the data: reads 0), a block
    whose range starts mid-array, and a single step of 5 groups."""
    for seed, ng, g0, g1 in ((4, 64, 0, 64), (5, 45, 0, 45), (6, 100, 32, 77), (7, 37, 30, 35)):
        sz, xsum = _zero_point_inputs(seed, ng)
        assert np.array_equal(_zero_point_pass(sz, xsum, g0, g1), _wrapping(sz, xsum, g0, g1)), (seed, ng, g0, g1)


def test_zero_point_pass_check_sees_planted_mistakes():
    """The restatement is sensitive to the lane layout and to the step masks: swapping the
    half-wave's group range, dropping both masks (so the groups after the block's last one, here
    nonzero, enter the ragged step; either mask alone zeroes their products, and the kernel keeps
    both), or a wrong accumulator-to-row map each changes the result."""
    sz, xsum = _zero_point_inputs(8, 70)
    want = _wrapping(sz, xsum, 0, 45)
    assert np.array_equal(_zero_point_pass(sz, xsum, 0, 45), want)
    assert not np.array_equal(_zero_point_pass(sz, xsum, 0, 45, swap_q=True), want)
    assert not np.array_equal(_zero_point_pass(sz, xsum, 0, 45, masks=False), want)
    assert not np.array_equal(_zero_point_pass(sz, xsum, 0, 45, d_rows=lambda v, q: 8 * (v & 3) + 4 * q + (v >> 2)),
                              want)
