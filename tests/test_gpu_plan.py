"""The device-side tile planner (include/dan_tree_plan.h) on the GPU against
the host planner (dan_amd/plan.py), whose tables the CPU tests pin key by key
against the oracle's visibility rule (tests/test_plan.py).

Bars: key_lo, col_seg, the work list and its costs are identical to the host
planner's; the schedule is valid (every (item, head group) unit exactly once,
slot s only head group s % G, each slot's units longest first) and no worse
balanced than plain longest-processing-time dealing; attention through the
device plan equals attention through the host plan bit for bit (the output
does not depend on the schedule)."""
import heapq
import sys

import numpy as np
import pytest
import torch

from dan_amd import _native
from dan_amd import plan as P
from dan_amd import workloads as W
from dan_amd.attention import Batch, attend, get_plan, segment

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def random_batch(rng, device, max_segments=6):
    structure, pasts = [], []
    for _ in range(int(rng.integers(1, max_segments + 1))):
        trunk = int(rng.integers(0, 700))
        lens = [int(x) for x in rng.integers(1, 100, int(rng.integers(0, 7)))]
        if trunk + sum(lens) == 0:
            trunk = 1
        structure.append((trunk, lens))
        pasts.append(int(rng.integers(1, 300)) if rng.random() < 0.4 else 0)
    return W.build("random", structure, 8, 2, 64, torch.bfloat16, device, rng, per_segment_past=pasts)


def lpt_makespan(cost, k, overhead=1):
    heap = [(0, j) for j in range(k)]
    for c in sorted(cost, reverse=True):
        load, j = heapq.heappop(heap)
        heapq.heappush(heap, (load + int(c) + overhead, j))
    return max(x[0] for x in heap)


def check_device_plan(segments, n, tile_q, groups, num_cus, device):
    host = P.TilePlan.build(segments, n, tile_q, device)
    dev = P.TilePlan.build_device(segments, n, tile_q, device, groups, num_cus)
    torch.cuda.synchronize()
    w = host.num_work
    assert dev.num_work == w and dev.num_cols == host.num_cols
    assert np.array_equal(dev.key_lo_d.cpu().numpy(), host.key_lo)
    assert np.array_equal(dev.col_seg_d.cpu().numpy()[:dev.num_cols], host.col_seg)
    assert np.array_equal(dev.work_d.cpu().numpy()[:w], host.work)
    cost = dev.cost_d.cpu().numpy()[:w]
    assert np.array_equal(cost, host.cost)
    units, off, slots = dev.schedules[(groups, num_cus)]
    units, off = units.cpu().numpy()[:w * groups], off.cpu().numpy()
    k = slots // groups
    assert slots == _native.plan_slots(w, groups, num_cus) and off[0] == 0 and off[-1] == w * groups
    seen = np.zeros((w, groups), int)
    loads = []
    for s in range(slots):
        rec = units[off[s]:off[s + 1]]
        assert (rec[:, 14] == s % groups).all(), "slot s runs head group s % G"
        ranks = [int(np.flatnonzero((host.work == r[:8]).all(1))[0]) for r in rec]
        assert ranks == sorted(ranks), "each slot's units longest first"
        for r, rank in zip(rec, ranks):
            seen[rank, r[14]] += 1
            sg = host.segs[r[0]]
            assert list(r[8:14]) == list(sg[:6])
        loads.append(int((cost[ranks] + 1).sum()))
    assert (seen == 1).all(), "every unit exactly once"
    makespan = max(loads)
    lpt = lpt_makespan(cost, k)
    _, hoff = P.schedule(host.cost, groups, num_cus)
    sched, _ = P.schedule(host.cost, groups, num_cus)
    hl = [int((host.cost[sched[hoff[s]:hoff[s + 1]] // groups] + 1).sum()) for s in range(len(hoff) - 1)]
    say(f"  {w} items, {k} slots per head group: makespan {makespan} (host {max(hl)}, "
        f"longest-first dealing alone {lpt}, mean {(cost + 1).sum() / k:.1f})")
    assert makespan <= lpt
    return dev, host


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4", "c5"])
def test_device_tables_equal_host(gpu, cfg):
    w = W.CONFIGS[cfg](0, device=gpu)
    h, hkv = w.q.shape[0], w.k.shape[0]
    say(f"device planner: {cfg}")
    check_device_plan(w.segments, w.num_tokens, _native.tile_q(h, hkv), _native.head_groups(h, hkv), 256, gpu)


@pytest.mark.parametrize("seed", range(6))
def test_device_tables_random_trees(gpu, seed):
    rng = np.random.default_rng(100 + seed)
    w = random_batch(rng, gpu)
    tile_q, groups = _native.tile_q(8, 2), _native.head_groups(8, 2)
    say(f"device planner: random tree seed {seed}")
    for cus in (256, 40, 3):
        check_device_plan(w.segments, w.num_tokens, tile_q, groups, cus, gpu)
    check_device_plan(w.segments, w.num_tokens, 256, 1, 256, gpu)  # one head group, 256-token tiles


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_attend_device_plan_equals_host_plan(gpu, cfg):
    w = W.CONFIGS[cfg](0, device=gpu)
    h, hkv = w.q.shape[0], w.k.shape[0]
    say(f"attend, device vs host plan: {cfg}")
    w.segments.tile_plan = P.TilePlan.build(w.segments, w.num_tokens, _native.tile_q(h, hkv), gpu)
    ref = attend(w.q, w.k, w.v, w.segments, 0).clone()
    w.segments.tile_plan = None
    out = attend(w.q, w.k, w.v, w.segments, 0)
    torch.cuda.synchronize()
    assert w.segments.tile_plan.cost is None, "the default planner is the device planner"
    assert torch.equal(out, ref)


def test_beyond_limits_uses_host_planner(gpu):
    """A batch of 4097 one-token segments (4097 work items) exceeds the device
    planner: the host planner builds it."""
    segs = [segment(i, [0], device=str(gpu)) for i in range(_native.PLAN_MAX_WORK + 1)]
    batch = Batch(segs)
    plan = get_plan(batch, len(segs), 64, gpu, groups=8, num_cus=256)
    assert plan.cost is not None and plan.num_work == len(segs)


def test_planner_runs_on_the_current_stream(gpu):
    w = W.config3(0, device=gpu)
    h, hkv = w.q.shape[0], w.k.shape[0]
    ref = attend(w.q, w.k, w.v, w.segments, 0).clone()
    w.segments.tile_plan = None
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = attend(w.q, w.k, w.v, w.segments, 0)
    s.synchronize()
    assert torch.equal(out, ref)
