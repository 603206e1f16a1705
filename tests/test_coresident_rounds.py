"""Co-resident GEMM+bias+LayerNorm in rounds, checked on the CPU.

Python mirrors of the launcher's round plan (`icpp_abi.hip`, ICPP_LN_CORESIDENT: the
8-way split of a round's row blocks x tile columns with the fewest A + B panels per
XCD, ties going to the most row splits) and of the kernel's workgroup -> tile map (`icpp_kernels.hpp`, `cr_item`), and a
discrete-event model of the dispatch they rely on: workgroup b runs on XCD b % 8, each
XCD starts its workgroups in order when one of its CUs is free, and a workgroup holds
its CU until every tile of its row block has arrived.  The model checks that every row
block completes -- no wait depends on a workgroup that cannot start -- whatever order
the resident workgroups finish their GEMMs in.
"""

import random

import pytest


def round_plan(tiles_m, tiles_n, cap):
    """(R, xa, xb) as the launcher picks them, or None when it falls back to chunks."""
    R = cap // tiles_n
    if tiles_m <= R:
        return None
    best, best_cost = None, 1 << 30
    xa = 1
    while xa <= 8:
        xb = 8 // xa
        if R % xa == 0 and tiles_n % xb == 0 and (R // xa) * (tiles_n // xb) <= cap // 8:
            cost = R // xa + tiles_n // xb
            if cost <= best_cost:
                best, best_cost = (R, xa, xb), cost
        xa *= 2
    return best


def cr_item(b, R, xa, xb, tiles_n):
    """The kernel's (row block, tile column) of workgroup b."""
    x, k = b & 7, b >> 3
    rx, cx = R // xa, tiles_n // xb
    r, pp = divmod(k, rx * cx)
    return r * R + (x // xb) * rx + pp % rx, (x % xb) * cx + pp // rx


def simulate(tiles_m, tiles_n, cus, R, xa, xb, seed):
    """In-order per-XCD dispatch with one workgroup per CU; returns the completed row blocks."""
    rng = random.Random(seed)
    rounds = -(-tiles_m // R)
    grid = rounds * R * tiles_n
    items = [cr_item(b, R, xa, xb, tiles_n) for b in range(grid)]
    queues = [[b for b in range(grid) if b % 8 == x] for x in range(8)]   # each XCD's workgroups, in order
    free = [cus // 8] * 8
    arrived = {}          # row block -> tiles whose GEMM is done (waiting or gone)
    running = []          # (finish time, b) of workgroups still in their GEMM
    waiting = {}          # row block -> workgroups holding a CU until the block is complete
    done_blocks, t = set(), 0.0
    while True:
        for x in range(8):  # start what fits, in order
            while queues[x] and free[x] > 0:
                b = queues[x].pop(0)
                rb, _ = items[b]
                if rb >= tiles_m:           # a spare workgroup of the last round exits at once
                    continue
                free[x] -= 1
                running.append((t + rng.uniform(0.9, 1.1), b))
        if not running:
            break
        running.sort()
        t, b = running.pop(0)
        rb, _ = items[b]
        arrived[rb] = arrived.get(rb, 0) + 1
        waiting.setdefault(rb, []).append(b)
        if arrived[rb] == tiles_n:          # the row block is complete: its workgroups leave
            done_blocks.add(rb)
            for w in waiting.pop(rb):
                free[w % 8] += 1
    assert all(not q for q in queues), "workgroups never started: a wait blocked the dispatch"
    return done_blocks


@pytest.mark.parametrize("tiles_m,tiles_n,cap", [(32, 16, 256), (20, 16, 256), (64, 4, 128), (40, 8, 256),
                                                 (33, 16, 256), (12, 2, 16)])
def test_round_map_covers_every_tile_once(tiles_m, tiles_n, cap):
    plan = round_plan(tiles_m, tiles_n, cap)
    assert plan is not None
    R, xa, xb = plan
    assert xa * xb == 8 and (R // xa) * (tiles_n // xb) * 8 == R * tiles_n <= cap
    rounds = -(-tiles_m // R)
    seen = {}
    for b in range(rounds * R * tiles_n):
        rb, tc = cr_item(b, R, xa, xb, tiles_n)
        assert 0 <= tc < tiles_n
        # workgroup b belongs to round (b >> 3) // share and its row block to that round
        share = R * tiles_n // 8
        assert rb // R == (b >> 3) // share
        if rb < tiles_m:
            assert (rb, tc) not in seen, (b, rb, tc)
            seen[(rb, tc)] = b
    assert len(seen) == tiles_m * tiles_n


def test_c3_n4096_plan_is_four_by_eight_per_xcd():
    """256 x 256 tiles at M = 8192, N = 4096 on 256 CUs: 2 rounds of 16 row blocks, each XCD
    holding 4 row blocks x 8 tile columns -- 12 A + B panels, the L2 footprint of the usual
    order's 8 x 4, with each row block on 2 XCDs instead of 4."""
    R, xa, xb = round_plan(32, 16, 256)
    assert (R, R // xa, 16 // xb) == (16, 4, 8)


def test_plans_that_do_not_split_fall_back_to_chunks():
    assert round_plan(43, 6, 256) is None       # 6 tile columns: no 8-way split
    assert round_plan(16, 16, 256) is None      # one round: a single launch without rounds


@pytest.mark.parametrize("tiles_m,tiles_n,cus", [(32, 16, 256), (20, 16, 256), (40, 8, 256), (64, 4, 128)])
def test_in_order_dispatch_completes_every_row_block(tiles_m, tiles_n, cus):
    R, xa, xb = round_plan(tiles_m, tiles_n, cus)
    for seed in range(5):
        assert simulate(tiles_m, tiles_n, cus, R, xa, xb, seed) == set(range(tiles_m))


def test_the_model_catches_a_map_that_splits_row_blocks_across_rounds():
    """Planted mistake: map workgroups in the usual order (row blocks striped over every XCD
    without regard to rounds) -- the model then finds workgroups that never start."""
    global cr_item
    keep = cr_item
    try:
        def striped(b, R, xa, xb, tiles_n):
            # consecutive workgroups walk down a tile column: a row block's tiles are
            # tiles_m workgroups apart, far beyond what the device holds at once
            return b % 32, b // 32
        cr_item = striped
        with pytest.raises(AssertionError):
            simulate(32, 16, 256, 16, 2, 4, 0)
    finally:
        cr_item = keep


def test_statistics_split_stays_inside_two_stage_arrays():
    """For every f16 GEMM tile and row width the co-resident strategy accepts
    (kernels/gemm_bias_layernorm.py coresident_fits, the launcher's own check), the
    kernel's split of a row block's [rows][tiles_n] (mean, M2) pairs -- an even r0 =
    min(rows, per & ~1) rows in the first stage array, the rest in the second, per =
    stage bytes / (8 tiles_n) -- keeps both parts inside one stage array each for every
    row count of a (possibly ragged) row block, and the first part ends on a 16-byte
    boundary (no 16-byte load straddles the arrays)."""
    from icpp_tuning_amd.kernels import gemm_bias_layernorm as ln
    from icpp_tuning_amd.kernels._base import family_instances

    checked = 0
    for inst in family_instances("gemm"):
        if inst.dtype != "f16":
            continue
        stage = (inst.bm + inst.bn) * inst.bk * 2
        for N in (8, 128, 776, 1024, 2304, 2312, 4096, 8192, 11008, 16384, 32768):
            if not ln.coresident_fits(inst, N):
                continue
            tiles_n = -(-N // inst.bn)
            rowb = 8 * tiles_n
            per = stage // rowb
            for rows in range(1, inst.bm + 1):
                r0 = min(rows, per & ~1)
                assert r0 % 2 == 0 or r0 == rows, (inst.name, N, rows)
                assert r0 * rowb <= stage and (rows - r0) * rowb <= stage, (inst.name, N, rows)
                assert (r0 * tiles_n) % 2 == 0 or r0 == rows   # nvec0 = r0 * tiles_n / 2 exact
            checked += 1
    assert checked > 100
