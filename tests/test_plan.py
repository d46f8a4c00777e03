"""The host tile planner (the ReadLayout replacement) on the CPU: every query
is covered once, the visited key tiles cover every visible key, skipped tiles
hold none, and unmasked tiles are fully visible -- checked key by key against
the oracle's visibility rule."""
import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from dan_amd import workloads as W
from dan_amd.attention import Batch, Segment, segment
from dan_amd.plan import KEY_TILE, build_tables, device_inputs, schedule, unit_records, validate_segments
from oracle import tree_attention as O


def check_plan(segments, num_tokens, tile_q):
    segs, work, key_lo, cost, past_dicts, col_seg = build_tables(segments, num_tokens, tile_q)
    # V^T columns: each segment owns a 64-aligned range of roundup(P + n) columns, in order
    col = 0
    for i, s in enumerate(segments):
        p = s.past_len if s.past else 0
        assert segs[i, 5] == col and col % KEY_TILE == 0
        span = _ceil(p + s.end - s.start, KEY_TILE)
        assert (col_seg[col // KEY_TILE: col // KEY_TILE + span] == i).all()
        col += span * KEY_TILE
    assert len(col_seg) * KEY_TILE == col
    assert (np.diff(cost) <= 0).all(), "work list must be sorted longest first"
    covered = np.zeros(num_tokens, int)
    for item in work:
        si, t0, tq, ja1, jb0, jb1, jfull, _ = (int(x) for x in item)
        s = segments[si]
        p = s.past_len if s.past else 0
        assert 1 <= tq <= tile_q and t0 % tile_q == 0
        assert jb0 >= ja1 and jb1 >= jb0
        covered[s.start + t0:s.start + t0 + tq] += 1
        vis = O.visible(s.trunk, list(s.branch_ids), p)[t0:t0 + tq]  # [tq, P + n]
        tiles = set(range(ja1)) | set(range(jb0, jb1))
        nkeys = vis.shape[1]
        for j in range(_ceil(nkeys, KEY_TILE)):
            block = vis[:, j * KEY_TILE:(j + 1) * KEY_TILE]
            if j not in tiles:
                assert not block.any(), f"skipped tile {j} holds visible keys"
            if j < jfull:
                assert block.shape[1] == KEY_TILE and block.all(), f"tile {j} below jfull is not fully visible"
        assert max(tiles, default=-1) < _ceil(nkeys, KEY_TILE)
        # outside [P + trunk, lo_max) the causal rule alone is the mask
        pt = p + s.trunk
        lo_max = int(item[7])
        for j in tiles:
            if j >= jfull and not (j * KEY_TILE + KEY_TILE > pt and j * KEY_TILE < lo_max):
                keys = np.arange(j * KEY_TILE, min((j + 1) * KEY_TILE, nkeys))
                causal = keys[None, :] <= (p + t0 + np.arange(tq))[:, None]
                assert (causal == vis[:, keys]).all(), f"tile {j} needs the branch test but lo_max={lo_max}"
        # the kernel's per-element rule reproduces the mask inside visited tiles
        for i in range(tq):
            qk = p + t0 + i
            lo = key_lo[s.start + t0 + i]
            keys = np.arange(nkeys)
            rule = (keys <= qk) & ((keys < pt) | (keys >= lo))
            assert (rule == vis[i]).all()
    for s in segments:
        assert (covered[s.start:s.end] == 1).all()
    return segs, work, key_lo, cost


def _ceil(a, b):
    return -(-a // b)


@pytest.mark.parametrize("tile_q", [64, 128, 256])
def test_plan_runner_shapes(tile_q):
    w = W.runner_shapes(0, dtype=torch.float32)
    check_plan(w.segments, w.num_tokens, tile_q)


def test_plan_config1_and_config2():
    for w in (W.config1(0), W.config2(0)):
        check_plan(w.segments, w.num_tokens, 64)


def test_plan_config3_tables():
    w = W.config3(0)
    segs, work, key_lo, cost = check_plan(w.segments, w.num_tokens, 64)
    assert len(segs) == 5 and (segs[:, 3] == 1024).all() and (segs[:, 4] == 0).all()
    # the trunk of the first tile sees only the past in full: 16 unmasked tiles
    first = [r for r in work if r[0] == 0 and r[1] == 0][0]
    assert first[6] == 1024 // KEY_TILE


@settings(max_examples=60, deadline=None)
@given(st.integers(0, 2 ** 31 - 1), st.sampled_from([64, 128]))
def test_plan_random_trees(seed, tile_q):
    rng = np.random.default_rng(seed)
    structure, pasts = [], []
    for _ in range(int(rng.integers(1, 4))):
        trunk = int(rng.integers(0, 150))
        lens = [int(x) for x in rng.integers(1, 100, int(rng.integers(0, 5)))]
        if trunk + sum(lens) == 0:
            trunk = 1
        structure.append((trunk, lens))
        pasts.append(int(rng.integers(1, 200)) if rng.random() < 0.5 else 0)
    w = W.build("random", structure, 2, 1, 64, torch.float32, "cpu", rng, per_segment_past=pasts)
    check_plan(w.segments, w.num_tokens, tile_q)


def test_shared_past_entries_are_deduplicated():
    w = W.config3(0)
    segs, _, _, _, past_dicts, _ = build_tables(w.segments, w.num_tokens, 64)
    assert len(past_dicts) == 1 and past_dicts[0] is w.segments[0].past


@pytest.mark.parametrize("bad", [
    lambda: Segment(0, 10, 11, []),                       # trunk longer than the segment
    lambda: Segment(0, 10, 4, [(4, 6), (7, 10)]),         # gap between branches
    lambda: Segment(0, 10, 4, [(4, 8)]),                  # branches end early
    lambda: Segment(5, 3, 0, []),                         # empty / reversed rows
    lambda: Segment(0, 40, 40, []),                       # beyond the packed batch
    lambda: Segment(0, 10, 10, [], past={0: None}, past_len=0),
])
def test_malformed_segments_raise(bad):
    with pytest.raises(ValueError):
        validate_segments(Batch([bad()]), 32)


def test_segment_mirrors_reference_construction():
    """segment() keeps dan/attention.py:114-126's fields."""
    s = segment(7, [0, 0, 0, 1, 1, 2], past={0: "kv"}, save=2, past_len=4, device="cpu")
    assert (s.start, s.end, s.trunk, s.branches, s.past_len, s.save) == (7, 13, 3, [(10, 12), (12, 13)], 4, 2)
    assert segment(0, [0, 1], past=None, past_len=9).past_len == 0
    assert s.mask.shape == (3, 4 + 6) and s.mask[:, :4].all()


def check_schedule(cost, groups, num_cus):
    sched, off = schedule(cost, groups, num_cus)
    slots = len(off) - 1
    units = len(cost) * groups
    assert off[0] == 0 and off[-1] == units and (np.diff(off) >= 0).all()
    assert sorted(sched.tolist()) == list(range(units)), "every unit exactly once"
    assert 1 <= slots <= max(num_cus, groups) and slots % groups == 0
    # slot s serves head group s % groups only (one kv head per XCD)
    for s in range(slots):
        assert all(u % groups == s % groups for u in sched[off[s]:off[s + 1]])
    loads = np.array([sum(int(cost[u // groups]) + 1 for u in sched[off[s]:off[s + 1]]) for s in range(slots)])
    per_class = slots // groups
    ideal = (int(cost.sum()) + len(cost)) / per_class
    # a balanced assignment: within one item of the mean (or the largest item)
    assert loads.max() <= max(ideal + int(cost.max()) + 1, int(cost.max()) + 1)
    return sched, off, loads, ideal


def test_unit_records_resolve_items_and_segments():
    w = W.config3(0)
    segs, work, _, cost, _, _ = build_tables(w.segments, w.num_tokens, 64)
    sched, off = schedule(cost, 8, 256)
    rec = unit_records(segs, work, sched, 8)
    assert rec.shape == (len(work) * 8, 16) and rec.dtype == np.int32
    for r, u in zip(rec, sched):
        item = work[u // 8]
        assert (r[:8] == item).all()
        assert (r[8:14] == segs[item[0], :6]).all()  # start, n, trunk, past_len, past_idx, vt_col
        assert r[14] == u % 8 and r[15] == 0
    assert unit_records(segs, work, np.zeros(0, np.int32), 8).shape == (0, 16)


def test_schedule_balances_config3():
    w = W.config3(0)
    _, _, _, cost, _, _ = build_tables(w.segments, w.num_tokens, 64)
    sched, off, loads, ideal = check_schedule(cost, 8, 256)
    assert len(off) - 1 == 256
    # hardware round-robin dispatch of 1040 work groups ends at 147 tile-steps on
    # the busiest CU; the planned schedule is within 1 % of the mean
    assert loads.max() <= 1.01 * ideal, (loads.max(), ideal)


@settings(max_examples=40, deadline=None)
@given(st.lists(st.integers(1, 200), min_size=1, max_size=300), st.sampled_from([1, 2, 4, 8, 16]),
       st.sampled_from([8, 64, 256]))
def test_schedule_random_costs(costs, groups, cus):
    check_schedule(np.array(sorted(costs, reverse=True), np.int64), groups, cus)


def test_schedule_fewer_items_than_cus():
    cost = np.array([5, 3, 1], np.int64)
    sched, off, loads, _ = check_schedule(cost, 8, 256)
    assert len(off) - 1 == 24 and (np.diff(off) == 1).all()  # one unit per work group
    assert len(schedule(np.zeros(0, np.int64), 8, 256)[0]) == 0


@settings(max_examples=40, deadline=None)
@given(st.integers(0, 2 ** 31 - 1), st.sampled_from([64, 128, 256]))
def test_device_planner_inputs(seed, tile_q):
    """The host part of the device planner: the segment table equals the host
    planner's, reserved[0] / reserved[1] are each segment's first work item
    and first branch, and the counts are the host planner's list lengths."""
    rng = np.random.default_rng(seed)
    structure, pasts = [], []
    for _ in range(int(rng.integers(1, 6))):
        trunk = int(rng.integers(0, 300))
        lens = [int(x) for x in rng.integers(1, 100, int(rng.integers(0, 6)))]
        if trunk + sum(lens) == 0:
            trunk = 1
        structure.append((trunk, lens))
        pasts.append(int(rng.integers(1, 200)) if rng.random() < 0.5 else 0)
    w = W.build("random", structure, 2, 1, 64, torch.float32, "cpu", rng, per_segment_past=pasts)
    segs, starts, nw, nc, past_dicts = device_inputs(w.segments, w.num_tokens, tile_q)
    hsegs, work, key_lo, cost, hpast, col_seg = build_tables(w.segments, w.num_tokens, tile_q)
    assert (segs[:, :6] == hsegs[:, :6]).all()
    assert nw == len(work) and nc == len(col_seg) and len(past_dicts) == len(hpast)
    item_of = np.bincount(work[:, 0], minlength=len(segs))  # items per segment
    assert (segs[:, 6] == np.concatenate([[0], np.cumsum(item_of)[:-1]])).all()
    at = 0
    for i, s in enumerate(w.segments):
        assert segs[i, 7] == at
        for a, b in s.branches:
            assert starts[at] == a
            assert (key_lo[a:b] == (s.past_len if s.past else 0) + a - s.start).all()
            at += 1
    assert at == len(starts)
