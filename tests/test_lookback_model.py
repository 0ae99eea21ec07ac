"""A CPU model of the fixed-schedule scan's look-back protocol (``lookback_grouped`` in
unpopped_amd/csrc/kernels/unp_device.hip), run over random interleavings.

The protocol gives a float scan reproducible bits (the reference's launched scan promises results
"reproducible and independent of grid", crates/unpopped/src/kernel_lift/scan_launched.rs:22-27): a
row's tiles form groups of 64; G(k) = fold(G(k-1), tree(aggregates of group k)); the carry into tile
j = 64k + q is fold(G(k-1), scan_tree(aggregates of tiles 64k .. j-1)).  Whoever computes a G(k) --
the group's last tile, or any later tile refolding groups it walked over -- must produce the same
bits, and every wait must end.

The model:
  * fold values are expression trees (nested tuples), so two results are equal only if they are the
    same association of the same aggregates -- a stricter test than equal floats;
  * the wave trees are the device's DPP shapes: a Hillis-Steele scan inside each 16-lane row over
    row_shr 1, 2, 4, 8, then the row totals folded in (wave_inclusive_scan), and wave_reduce as
    ((r15 . r31) . r47) . r63 of the row-scanned values;
  * a status slot holds W tagged words (tag = launch epoch, flag 1 for an inclusive total); every
    word read and written is its own scheduler step, so reads tear across writes, and the slots start
    out holding words of an earlier launch;
  * B persistent blocks draw tickets in order (each block its next ticket as its current tile starts)
    and run their tile to completion, the tile's loads taking a few steps before its aggregate is
    published; the scheduler picks
    a block for each step at random, weighted by speeds spread over three decades and redrawn every
    few thousand steps, so a block can stall anywhere (before publishing its aggregate, say).
Checks: every tile finishes within a step bound (the waits end), every word a look-back waits on
belongs to a lower ticket, every carry and every published group total equals its definition.
Each planted mistake must fail at least one of the seeded schedules.
"""
from __future__ import annotations

import random

import pytest

D = 2  # groups probed behind the tile's own (the device's default)
LOAD_STEPS = 3  # scheduler steps between drawing a ticket and publishing the tile's aggregate
EPOCH, OLD = 7, 6


def fold(a, b):
    """The fold of the model: the identity is None; otherwise the ordered pair (an association)."""
    if a is None:
        return b
    if b is None:
        return a
    return (a, b)


def row_scan(x):
    x = list(x)
    for s in (1, 2, 4, 8):
        x = [fold(x[lane - s] if lane % 16 >= s else None, x[lane]) for lane in range(64)]
    return x


def wave_inclusive_scan(x):
    x = row_scan(x)
    r0 = x[15]
    r01 = fold(r0, x[31])
    r012 = fold(r01, x[47])
    pre = [None, r0, r01, r012]
    return [x[lane] if lane < 16 else fold(pre[lane >> 4], x[lane]) for lane in range(64)]


def wave_reduce(x, mutant=None):
    x = row_scan(x)
    if mutant == "reduce_tree":
        return fold(fold(x[15], fold(x[31], x[47])), x[63])
    return fold(fold(fold(x[15], x[31]), x[47]), x[63])


class Status:
    """The tile-status words: slot t holds W words (tag, flag, value part)."""

    def __init__(self, n, w, rng):
        self.w = w
        # words of an earlier launch: any flag, any value
        self.words = [[(OLD, rng.randint(0, 1), ("stale", t, i)) for i in range(w)] for t in range(n)]
        self.reads = []  # (reader tile, slot read)

    def publish(self, t, flag, v):
        for i in range(self.w):
            self.words[t][i] = (EPOCH, flag, (v, i))
            yield

    def fetch(self, reader, t, out):
        self.reads.append((reader, t))
        for i in range(self.w):
            out.append(self.words[t][i])
            yield


def decode(words, mutant=None):
    """2: an inclusive total, 1: an aggregate, 0: nothing of this launch (tile_status::decode)."""
    tags = {w[0] for w in words}
    flags = {w[1] for w in words}
    if mutant != "no_epoch" and tags != {EPOCH}:
        return 0, None
    if len(flags) != 1:
        return 0, None
    parts = {w[2][0] if isinstance(w[2], tuple) and len(w[2]) == 2 and w[2][1] in range(8) else w[2] for w in words}
    v = parts.pop() if len(parts) == 1 else ("torn",)
    return (2 if flags.pop() else 1), v


def tile_process(j, agg, st, out, mutant=None):
    """One tile's publication and look-back (lookback_grouped); records its carry in out['carry']."""
    k, q = j >> 6, j & 63
    for _ in range(LOAD_STEPS):  # the tile's loads and wave-local scan before its aggregate is out
        yield
    if j == 0:
        yield from st.publish(0, 1, agg[0])
        out["carry"][0] = None
        return
    yield from st.publish(j, 0, agg[j])
    while True:
        wa = [[] for _ in range(64)]
        wd = [[[] for _ in range(64)] for _ in range(D)]
        for lane in range(64):
            yield from st.fetch(j, 64 * k + lane if lane < q else j, wa[lane])
        for d in range(1, D + 1):
            for lane in range(64):
                yield from st.fetch(j, 64 * (k - d) + lane if k >= d else j, wd[d - 1][lane])
        va = [None] * 64
        sa = [1] * 64
        for lane in range(64):
            if lane < q:
                sa[lane], va[lane] = decode(wa[lane], mutant)
            else:
                va[lane] = agg[j] if lane == 63 else None
        ok = all(s != 0 for s in sa)
        vd = [None] * D
        depth, base = 0, None
        if ok:
            for d in range(1, D + 1):
                if k < d:
                    depth = d
                    break
                dec = [decode(w, mutant) for w in wd[d - 1]]
                sd = [s for s, _ in dec]
                vals = [v if s != 0 else None for s, v in dec]
                if sd[63] == 2 or (mutant == "total_from_aggregate" and sd[63] == 1):
                    base, depth = vals[63], d
                    break
                if any(s == 0 for s in sd) and mutant != "missing_as_identity":
                    break
                vd[d - 1] = vals
        if ok and depth:
            gprev = base
            for d in range(D, 0, -1):
                if d < depth:
                    gprev = fold(gprev, wave_reduce(vd[d - 1], mutant))
                    yield from st.publish(64 * (k - d) + 63, 1, gprev)
                    out["totals"].append((k - d, gprev))
            sc = wave_inclusive_scan(va)
            inner = sc[q - 1] if q > 0 else None
            if q == 63:
                total = fold(sc[63], gprev) if mutant == "total_flipped" else fold(gprev, sc[63])
                yield from st.publish(j, 1, total)
                out["totals"].append((k, total))
            out["carry"][j] = fold(gprev, inner) if q > 0 else gprev
            return
        yield  # sleep, then probe again


def canonical(n, agg):
    """The definitions: G(k) and every tile's carry."""
    groups = (n + 63) // 64
    g, carry = [], [None] * n
    prev = None
    for k in range(groups):
        vals = [agg[64 * k + lane] if 64 * k + lane < n else None for lane in range(64)]
        sc = wave_inclusive_scan(vals)
        for q in range(64):
            j = 64 * k + q
            if j < n:
                carry[j] = fold(prev, sc[q - 1]) if q > 0 else prev
        prev = fold(prev, wave_reduce(vals))
        g.append(prev)
    return g, carry


def simulate(n, blocks, seed, w, mutant=None, max_steps=2_000_000):
    rng = random.Random(seed)
    agg = [("a", j) for j in range(n)]
    st = Status(n, w, rng)
    out = {"carry": [("unset",)] * n, "totals": []}
    ticket = [0]
    running = [None] * blocks

    def draw():
        j = ticket[0]
        ticket[0] += 1
        return j

    def block(b):
        # as the device's persistent blocks: the next ticket is drawn as the current tile starts
        cur = draw()
        while cur < n:
            nxt = draw()
            yield from tile_process(cur, agg, st, out, mutant)
            cur = nxt

    gens = [block(b) for b in range(blocks)]
    live = list(range(blocks))
    steps = 0
    speed = []
    while live:
        if steps % 4000 == 0:
            # block speeds spread over three decades and redrawn now and then: a block can sit
            # between two of its steps (say, before publishing its aggregate) for a long while
            speed = [10 ** rng.uniform(-3, 0) for _ in range(blocks)]
        steps += 1
        if steps > max_steps:
            return None, st, agg, out
        b = rng.choices(live, [speed[i] for i in live])[0]
        try:
            next(gens[b])
        except StopIteration:
            live.remove(b)
    del running
    return steps, st, agg, out


def verdict(n, st, agg, out):
    """The list of violations of one finished run."""
    g, carry = canonical(n, agg)
    bad = []
    for j in range(n):
        if out["carry"][j] != carry[j]:
            bad.append(("carry", j))
    for k, total in out["totals"]:
        if total != g[k]:
            bad.append(("total", k))
    for reader, slot in st.reads:
        if slot > reader:
            bad.append(("waited on a later ticket", reader, slot))
    return bad


N_TILES = 64 * 3 + 23  # four groups, the last ragged


@pytest.mark.parametrize("w", [1, 2])
@pytest.mark.parametrize("seed", range(6))
def test_every_schedule_ends_with_the_defined_carries(w, seed):
    """Random interleavings (per-word reads tearing across writes, stale words of an earlier launch,
    12 persistent blocks): every tile finishes, every carry and group total is its definition, and no
    look-back reads a later ticket's slot (its own slot stands in for lanes with nothing to read)."""
    steps, st, agg, out = simulate(N_TILES, 12, seed, w)
    assert steps is not None, "a wait did not end"
    assert verdict(N_TILES, st, agg, out) == []


def test_one_block_runs_the_tiles_in_order():
    """One block: each tile's look-back finds every lower tile finished (no wait at all)."""
    steps, st, agg, out = simulate(N_TILES, 1, 0, 1)
    assert steps is not None and verdict(N_TILES, st, agg, out) == []


@pytest.mark.parametrize("mutant", ["total_flipped", "missing_as_identity", "total_from_aggregate", "reduce_tree",
                                    "no_epoch"])
def test_each_planted_mistake_is_caught(mutant):
    """A group total folded in the other order, a missing aggregate taken as the identity, an aggregate
    taken for a group total, a reduction tree unlike the scan's, or stale words of an earlier launch
    accepted: some schedule gives a carry or a total that is not its definition."""
    for seed in range(40):
        steps, st, agg, out = simulate(N_TILES, 12, 1000 + seed, 1, mutant)
        if steps is None or verdict(N_TILES, st, agg, out):
            return
    pytest.fail(f"no schedule caught {mutant}")
