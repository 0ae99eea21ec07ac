"""The signed byte digits the dequant GEMM's stream kernel uses for its zero-point pass
(unp_device.hip, dqg_stream): the bytes of (v + 0x80808080) ^ 0x80808080, read as int8, are
digits d_i in [-128, 127] with sum d_i 256^i = v modulo 2^32, and products of two such
expansions, summed by digit class i + j < 4 and shifted by 8 (i + j) bits, equal the 32-bit
wrapping product."""
import numpy as np
import pytest

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


# ---------------------------------------------------------------------------------------
# The zero-point pass's buffer addresses, lane by lane.  Its loads are raw buffer loads: the
# resource holds num_records (R ng 4 bytes for scales and zero points, ng Cp 4 for the column
# sums) and the whole byte offset is the 32-bit vector offset, so a load past num_records reads 0
# and touches no memory.  What must hold: every offset the kernel forms (an int sum of ints)
# stays in [0, 2^31), and every load whose value enters an output reads its own element inside
# num_records.  A CPU restatement of the launcher's geometry (runtime.cpp run_dequant_gemm,
# streaming branch) and of the pass's offsets (unp_device.hip dqg_stream: sofs, load_step, cofs),
# for every thread of the blocks of the last row tile and of the last split.
# ---------------------------------------------------------------------------------------

LIMIT = 0x7FFFFFFF


def _stream_geometry(x_bytes, group):
    """The emitter's stream entry shape (emit_hip.cpp lower_dequant_gemm): waves WR x WC, tiles
    TM x TN of 32 x 32 per wave."""
    skc = 0 if group % 64 else (128 if x_bytes == 1 and group % 128 == 0 else 64)
    big = x_bytes == 1 and skc == 128
    two = big or x_bytes == 4
    wr, wc = (2, 2) if big else (4, 1)
    tm, tn = (2 if big else 1), (2 if two else 1)
    return skc, wr, wc, tm, tn


def _zero_point_offsets(R, K, C, group, x_bytes, cu=256):
    """Yield, per examined block, the pass's loads: (kind, offsets, rows/cols, groups, used) arrays."""
    skc, WR, WC, TM, TN = _stream_geometry(x_bytes, group)
    assert skc, "a group of whole 64-value chunks"
    BM, BN, NW = 32 * WR * TM, 32 * WC * TN, 4
    ng = K // group
    cw = max(BN, 64)
    Cp = (C + cw - 1) // cw * cw
    admitted = (R + 256) * ng * 4 < LIMIT and (ng + 32) * Cp * 4 < LIMIT
    tiles_r, tiles_c = (R + BM - 1) // BM, (C + BN - 1) // BN
    S = max(1, min((2 * cu + tiles_r * tiles_c - 1) // (tiles_r * tiles_c), ng // 4))
    units = tiles_r * S
    blocks = (units + 7) // 8 * 8 * tiles_c
    tid = np.arange(256, dtype=np.int64)
    lane, wave = tid & 63, tid >> 6
    wc, q, l32 = wave % WC, lane >> 5, lane & 31
    srow, sg = tid // 32, tid % 32
    SZN = BM * 32 // (64 * NW)
    # the units of the first and last row tiles (every split) and the last split of the last two
    # row tiles, each at its first and last column tile; their block ids by inverting the
    # XCD-aware mapping b -> (u, ct): slot = b / 8, u = (slot / tiles_c) 8 + b % 8, ct = slot % tiles_c
    wanted = {(tiles_r - 1, sp) for sp in range(S)} | {(0, sp) for sp in range(S)}
    wanted |= {(r, S - 1) for r in range(max(0, tiles_r - 2), tiles_r)}
    picks = []
    for rt, split in sorted(wanted):
        u = rt * S + split
        for ct in sorted({0, tiles_c - 1}):
            b = ((u // 8) * tiles_c + ct) * 8 + u % 8
            assert b < blocks
            xcd, slot = b % 8, b // 8
            assert ((slot // tiles_c) * 8 + xcd, slot % tiles_c) == (u, ct)
            picks.append((u, ct))
    out = []
    for u, ct in picks:
        rt, split = u // S, u % S
        tile_r, tile_c = rt * BM, ct * BN
        g0, g1 = ng * split // S, ng * (split + 1) // S
        sofs = ((tile_r + srow) * ng + sg) * 4
        steps = list(range(g0, g1, 32))
        for gc in steps:
            gl = min(g1 - gc, 32)
            for m in range(SZN):
                so = (gc + m * (64 * NW // 32) * ng) * 4
                row = tile_r + srow + 8 * m
                grp = sg + gc
                out.append(("sz", sofs, so, row, grp, sg < gl))
            for t in range(TN):
                col = tile_c + 32 * (wc * TN + t) + l32
                cofs = (16 * q * Cp + col) * 4
                for k in range(16):
                    grp = gc + 16 * q + k
                    out.append(("cs", cofs, (gc + k) * Cp * 4, col, grp, (16 * q + k) < gl))
    return admitted, ng, Cp, out


SHAPES = [
    # (R, K, C, group, activation bytes): ragged rows and columns, a few splits and the last one
    (4096 + 17, 4096, 200, 128, 1),
    (300, 8192, 96, 64, 4),
    (129, 1024, 65, 128, 1),
    (1000, 2048, 130, 256, 4),
    (33, 512, 31, 64, 1),
]


@pytest.mark.parametrize("R,K,C,group,xb", SHAPES)
def test_zero_point_pass_reads_its_own_elements_inside_num_records(R, K, C, group, xb):
    admitted, ng, Cp, loads = _zero_point_offsets(R, K, C, group, xb)
    assert admitted and loads
    for kind, base, step, idx, grp, used in loads:
        total = base + step  # the kernel adds the two ints
        assert (base >= 0).all() and (base < LIMIT).all() and 0 <= step < LIMIT
        assert (total >= 0).all() and (total < LIMIT).all(), kind
        if kind == "sz":
            rows = np.broadcast_to(idx, base.shape)
            live = np.broadcast_to(used, base.shape) & (rows < R)
            want = (rows * ng + grp) * 4
            assert np.array_equal(total[live], want[live])
            assert (total[live] < R * ng * 4).all()
            # a row past R reads nothing: its offset lies past num_records
            assert (total[rows >= R] >= R * ng * 4).all()
        else:
            cols = np.broadcast_to(idx, base.shape)
            live = np.broadcast_to(used, base.shape) & (grp < ng)
            want = (grp * Cp + cols) * 4
            assert np.array_equal(total[live], want[live])
            assert (cols < Cp).all() and (total[live] < ng * Cp * 4).all()


@pytest.mark.parametrize("which", ["rows", "columns"])
def test_zero_point_pass_offsets_fit_at_the_launchers_bound(which):
    """Shapes just inside the launcher's admission bound ((R + 256) ng 4 and (ng + 32) Cp 4 under
    2^31): the largest offset any lane forms still fits, and one step more is refused."""
    K, group, xb = 8192, 128, 1
    ng = K // group
    if which == "rows":
        R = LIMIT // (4 * ng) - 257
        C = 64
    else:
        R = 128
        C = LIMIT // (4 * (ng + 32)) // 128 * 128 - 128
    admitted, ng2, Cp, loads = _zero_point_offsets(R, K, C, group, xb)
    assert admitted
    for _, base, step, *_ in loads:
        assert ((base + step) < LIMIT).all() and ((base + step) >= 0).all()
    R2, C2 = (R + 300, C) if which == "rows" else (R, C + 8 * 128)
    assert not _zero_point_offsets(R2, K, C2, group, xb)[0]
