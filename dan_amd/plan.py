"""Host tile planner: segment tree -> the kernel's work list.

This replaces ``ReadLayout`` (dan/attention.py:138-172), which turned a
``Batch`` into packed row lists and cumulative lengths for three varlen flash
calls. Here the same segment metadata becomes:

- a segment table: start, new-token count, trunk, past length, past index;
- ``key_lo`` [N]: per packed token, the first key of its own branch in
  segment key coordinates (past keys are 0..P-1, new token i is key P+i), 0
  for trunk tokens. Key kc is visible to query qc iff
  ``kc <= qc and (kc < P + trunk or kc >= key_lo[query])``, which is the tree
  mask of dan/attention.py:54-59 with the past prepended as all-visible
  columns (dan/attention.py:86-95, :259-264);
- the V^T column plan: each segment owns a 64-aligned range of
  ``roundup(P + n, 64)`` columns (``vt_col``) of the fp16 V^T copy the kernel's
  pre-pass writes, holding its [past; new] keys in segment key coordinates;
  ``col_seg`` maps every 64-column block to its segment;
- a work list of query tiles (``tile_q`` queries of one segment). Each item
  lists the key tiles (64 keys) any of its queries can see -- the trunk (and
  past) range, then the branch range starting at the earliest branch start in
  the tile -- and how many leading tiles every query sees in full (no mask).
  Items are sorted by key-tile count, longest first, so the hardware's
  in-order dispatch approximates longest-processing-time scheduling.

It is built once per forward and cached on the ``Batch`` (as
dan/attention.py:211-215 caches ``layout``); only the per-layer table of
prefix-cache pointers is rebuilt per layer.

Two builders make the same tables. ``TilePlan.build`` runs here on the host
(numpy). ``TilePlan.build_device`` keeps O(segments) work on the host
(``device_inputs``: each segment's first V^T column, first work item and
first branch) and makes one upload and one launch of the device planner
(include/dan_tree_plan.h), which builds key_lo, col_seg, the work list and the
schedule on the GPU, on the current stream.
"""
from dataclasses import dataclass, field

import numpy as np

KEY_TILE = 64


def _ceil_div(a, b):
    return -(-a // b)


def validate_segments(segments, num_tokens):
    """Raise ValueError unless every segment is well formed: rows inside the
    packed batch, trunk first, branches contiguous and in order after it
    (the shape ``segment()`` builds, dan/attention.py:114-126)."""
    for i, s in enumerate(segments):
        if not (0 <= s.start < s.end <= num_tokens):
            raise ValueError(f"segment {i}: rows [{s.start}, {s.end}) outside the packed batch of {num_tokens}")
        n = s.end - s.start
        if not 0 <= s.trunk <= n:
            raise ValueError(f"segment {i}: trunk {s.trunk} outside [0, {n}]")
        at = s.start + s.trunk
        for a, b in s.branches:
            if a != at or b <= a:
                raise ValueError(f"segment {i}: branch span ({a}, {b}) is not contiguous after row {at}")
            at = b
        if at != s.end:
            raise ValueError(f"segment {i}: branches end at row {at}, segment at {s.end}")
        if s.past:
            if s.past_len <= 0:
                raise ValueError(f"segment {i}: past given with past_len {s.past_len}")
        elif s.past_len:
            raise ValueError(f"segment {i}: past_len {s.past_len} without past entries")


def build_tables(segments, num_tokens, tile_q, key_tile=KEY_TILE):
    """Host tables for the kernel. Returns (segs [S,8] int32, work [W,8] int32,
    key_lo [N] int32, cost [W] int64, past_dicts, col_seg [C] int32) with
    C * key_tile the V^T column count.

    ``past_dicts`` lists the distinct prefix-cache entries (by identity) in
    the order the segment table's past index refers to them."""
    if tile_q <= 0:
        raise ValueError(f"tile_q {tile_q}: unsupported head layout")
    validate_segments(segments, num_tokens)
    segs = np.zeros((len(segments), 8), np.int32)
    key_lo = np.zeros(num_tokens, np.int32)
    past_dicts, past_index = [], {}
    items, col_seg = [], []
    for i, s in enumerate(segments):
        n, t = s.end - s.start, s.trunk
        p = s.past_len if s.past else 0
        pidx = -1
        if s.past:
            pidx = past_index.setdefault(id(s.past), len(past_dicts))
            if pidx == len(past_dicts):
                past_dicts.append(s.past)
        segs[i, :6] = (s.start, n, t, p, pidx, len(col_seg) * key_tile)
        col_seg += [i] * _ceil_div(p + n, key_tile)
        for a, b in s.branches:
            key_lo[a:b] = p + (a - s.start)
        pt = p + t
        for t0 in range(0, n, tile_q):
            tq = min(tile_q, n - t0)
            top = p + t0 + tq  # one past the last query's own key
            kfull = min(p + t0 + 1, pt)
            ja1 = _ceil_div(min(pt, top), key_tile)
            lo_max = 0
            if t0 + tq > t:  # the tile holds branch queries
                first = s.start + max(t0, t)
                jb0 = max(int(key_lo[first]) // key_tile, ja1)
                jb1 = max(_ceil_div(top, key_tile), jb0)
                lo_max = int(key_lo[s.start + t0 + tq - 1])  # key_lo grows along the branch region
            else:
                jb0 = jb1 = ja1
            items.append((i, t0, tq, ja1, jb0, jb1, kfull // key_tile, lo_max))
    work = np.array(items, np.int32).reshape(-1, 8)
    cost = (work[:, 3].astype(np.int64) + work[:, 5] - work[:, 4]) if len(work) else np.zeros(0, np.int64)
    order = np.argsort(-cost, kind="stable")
    return segs, work[order], key_lo, cost[order], past_dicts, np.array(col_seg, np.int32)


def device_inputs(segments, num_tokens, tile_q, key_tile=KEY_TILE):
    """The host part of the device planner: (segs int32 [S, 8], branch_starts
    int32 [B], num_work, num_cols, past_dicts). segs rows are DanSegmentDesc
    with reserved[0] = the segment's first work item and reserved[1] its
    first branch; the counts are sums of ceil(n / tile_q) and
    ceil((P + n) / key_tile)."""
    if tile_q <= 0:
        raise ValueError(f"tile_q {tile_q}: unsupported head layout")
    validate_segments(segments, num_tokens)
    segs = np.zeros((len(segments), 8), np.int32)
    past_dicts, past_index, starts = [], {}, []
    w = c = 0
    for i, s in enumerate(segments):
        n = s.end - s.start
        p = s.past_len if s.past else 0
        pidx = -1
        if s.past:
            pidx = past_index.setdefault(id(s.past), len(past_dicts))
            if pidx == len(past_dicts):
                past_dicts.append(s.past)
        segs[i] = (s.start, n, s.trunk, p, pidx, c * key_tile, w, len(starts))
        starts += [a for a, _ in s.branches]
        w += _ceil_div(n, tile_q)
        c += _ceil_div(p + n, key_tile)
    return segs, np.array(starts, np.int32), w, c, past_dicts


def schedule(cost, groups, num_cus, overhead=1):
    """Persistent schedule of the attention launch: (sched int32[U], sched_off
    int32[S + 1]) for U = len(cost) * groups units, unit u = work item
    u // groups for head group u % groups.

    There are S = groups * k slots (work groups), k = min(num_cus // groups,
    items) (at least 1), about one per CU. Slot s takes only units of head
    group s % groups: the hardware deals work groups to the 8 XCDs round
    robin, so with 8 kv heads each XCD's L2 serves one kv head. Inside a
    class, items are dealt longest first to the least loaded slot (LPT),
    each costing its key tiles plus ``overhead`` for its prologue and
    epilogue. Every class sees the same item costs, so one assignment serves
    all of them. dan's varlen path has no counterpart: there the flash
    kernels' own grids decide (dan/attention.py:229-241)."""
    import heapq

    cost = np.asarray(cost, np.int64)
    n = len(cost)
    if n == 0 or groups <= 0:
        return np.zeros(0, np.int32), np.zeros(1, np.int32)
    k = max(1, min(num_cus // groups, n))
    heap = [(0, j) for j in range(k)]
    per = [[] for _ in range(k)]
    for i in np.argsort(-cost, kind="stable"):
        load, j = heapq.heappop(heap)
        per[j].append(int(i))
        heapq.heappush(heap, (load + int(cost[i]) + overhead, j))
    _rebalance(per, cost + overhead)
    for x in per:
        x.sort(key=lambda i: (-cost[i], i))
    lists = [[i * groups + s % groups for i in per[s // groups]] for s in range(k * groups)]
    off = np.zeros(len(lists) + 1, np.int32)
    off[1:] = np.cumsum([len(x) for x in lists])
    sched = np.array([u for x in lists for u in x], np.int32)
    return sched, off


def _rebalance(per, w, rounds=10000):
    """Lower the largest load of the lists ``per`` (item weights ``w``) by
    moving one item, or swapping two, between the most loaded list and
    another, while that strictly lowers the pair's larger load."""
    w = np.asarray(w, np.int64)
    loads = np.array([int(w[x].sum()) for x in per], np.int64)
    for _ in range(rounds):
        a = int(np.argmax(loads))
        top = loads[a]
        m = max(len(x) for x in per)
        # other[b, 0] = 0 (a move), other[b, 1 + t] = weight of list b's t-th item (a swap)
        other = np.full((len(per), m + 1), np.iinfo(np.int64).max // 4, np.int64)
        other[:, 0] = 0
        for b, x in enumerate(per):
            other[b, 1:1 + len(x)] = w[x]
        d = w[per[a]][:, None, None] - other[None]          # [items of a, b, option]: load moved a -> b
        new = np.maximum(top - d, loads[None, :, None] + d)
        new[(d <= 0) | (new >= top)] = np.iinfo(np.int64).max
        new[:, a, :] = np.iinfo(np.int64).max
        flat = int(np.argmin(new))
        if new.flat[flat] == np.iinfo(np.int64).max:
            return
        ia, b, t = np.unravel_index(flat, new.shape)
        i = per[a].pop(int(ia))
        if t > 0:
            j = per[b].pop(int(t) - 1)
            per[a].append(j)
        per[b].append(i)
        moved = int(d[ia, b, t])
        loads[a] -= moved
        loads[b] += moved


def unit_records(segs, work, sched, groups):
    """The attention launch's unit table in schedule order: int32 [U, 16]
    rows laid out as DanUnit -- the work item (8 fields), its segment's start,
    n, trunk, past_len, past_idx, vt_col, the head group, and 0."""
    sched = np.asarray(sched, np.int64)
    rec = np.zeros((len(sched), 16), np.int32)
    if len(sched):
        items = work[sched // groups]
        rec[:, :8] = items
        rec[:, 8:14] = segs[items[:, 0], :6]
        rec[:, 14] = sched % groups
    return rec


@dataclass
class TilePlan:
    """Device-resident tables of one packed forward (see module docstring)."""

    tile_q: int
    num_tokens: int
    device: object
    segs: np.ndarray
    work: np.ndarray  # host-built only (None from the device planner)
    key_lo: np.ndarray  # host-built only
    cost: np.ndarray  # host-built only
    past_dicts: list
    col_seg: np.ndarray = None  # host-built only
    num_work: int = 0
    num_cols: int = 0
    cost_d: object = None  # device planner: key tiles per item, longest first
    segs_d: object = None
    work_d: object = None
    key_lo_d: object = None
    col_seg_d: object = None
    past_tables: dict = field(default_factory=dict)  # layer -> (device bytes, keep-alive refs)
    schedules: dict = field(default_factory=dict)  # (groups, CUs) -> (units_d, sched_off_d, slots)

    @classmethod
    def build(cls, segments, num_tokens, tile_q, device):
        import torch

        segs, work, key_lo, cost, past_dicts, col_seg = build_tables(segments, num_tokens, tile_q)
        plan = cls(tile_q, num_tokens, torch.device(device), segs, work, key_lo, cost, past_dicts, col_seg,
                   num_work=len(work), num_cols=len(col_seg))
        plan.segs_d = _upload(segs, device)
        plan.work_d = _upload(work, device)
        plan.key_lo_d = _upload(key_lo, device)
        plan.col_seg_d = _upload(col_seg, device)
        return plan

    @classmethod
    def build_device(cls, segments, num_tokens, tile_q, device, groups, num_cus, overhead=1):
        """The same tables from the device planner (one upload, one launch on
        the current stream); the schedule is made for ``groups`` head groups
        on ``num_cus`` compute units. Raises ValueError when the batch exceeds
        the planner's limits (see ``device_fits``)."""
        import torch

        from . import _native

        segs, starts, w, c, past_dicts = device_inputs(segments, num_tokens, tile_q)
        lib = _native.load()
        slots = _native.plan_slots(w, groups, num_cus, lib) if w else 0
        if (w > _native.PLAN_MAX_WORK or (w and slots // groups > _native.PLAN_MAX_SLOTS)
                or len(segs) > _native.PLAN_MAX_SEGMENTS or len(starts) > _native.PLAN_MAX_BRANCHES):
            raise ValueError(f"{w} work items, {slots} slots, {len(segs)} segments or {len(starts)} branches "
                             "exceed the device planner's limits")
        dev = torch.device(device)
        plan = cls(tile_q, num_tokens, dev, segs, None, None, None, past_dicts, None, num_work=w, num_cols=c)
        blob = _upload(np.concatenate([segs.ravel(), starts]).astype(np.int32), dev)  # the one upload
        plan.segs_d = blob[:segs.size]
        plan.key_lo_d = torch.empty(num_tokens, dtype=torch.int32, device=dev)
        plan.col_seg_d = torch.empty(max(c, 1), dtype=torch.int32, device=dev)
        plan.work_d = torch.empty((max(w, 1), 8), dtype=torch.int32, device=dev)
        plan.cost_d = torch.empty(max(w, 1), dtype=torch.int32, device=dev)
        units = torch.empty((max(w * groups, 1), 16), dtype=torch.int32, device=dev)
        off = torch.empty(slots + 1, dtype=torch.int32, device=dev)
        if w:
            a = _native.DanTreePlanArgs()
            a.abi_version = _native.PLAN_ABI_VERSION
            a.num_tokens, a.num_segments, a.num_branches = num_tokens, len(segs), len(starts)
            a.num_work, a.num_cols, a.tile_q, a.groups, a.num_cus, a.overhead = w, c, tile_q, groups, num_cus, overhead
            a.segments = blob.data_ptr()
            a.branch_starts = blob.data_ptr() + 4 * segs.size
            a.key_lo, a.col_seg, a.work, a.cost = (plan.key_lo_d.data_ptr(), plan.col_seg_d.data_ptr(),
                                                   plan.work_d.data_ptr(), plan.cost_d.data_ptr())
            a.units, a.sched_off = units.data_ptr(), off.data_ptr()
            _native.plan(a, torch.cuda.current_stream(dev).cuda_stream, lib)
        plan.schedules[(groups, num_cus)] = (units, off, slots)
        return plan

    @property
    def vt_cols(self):
        return int(self.num_cols * KEY_TILE)

    def matches(self, num_tokens, tile_q, device):
        import torch

        return self.num_tokens == num_tokens and self.tile_q == tile_q and self.device == torch.device(device)

    def schedule(self, groups, num_cus):
        """Device copies of the unit records of ``schedule(self.cost, groups,
        num_cus)`` and of its slot offsets, and the slot count (cached; a plan
        from the device planner carries the schedule it was built for)."""
        key = (groups, num_cus)
        if key not in self.schedules:
            if self.cost is None:
                raise ValueError(f"this plan was scheduled on the device for {list(self.schedules)}, not {key}")
            sched, off = schedule(self.cost, groups, num_cus)
            units = unit_records(self.segs, self.work, sched, groups)
            self.schedules[key] = (_upload(units, self.device), _upload(off, self.device), len(off) - 1)
        return self.schedules[key]

    def key_tiles(self):
        """Total key tiles the work list visits (per kv head and head chunk)."""
        return int(self.cost.sum() if self.cost is not None else self.cost_d[:self.num_work].sum().item())


def _upload(arr, device):
    """Host array -> device tensor; pinned, non-blocking on the GPU (as
    dan/attention.py:106-111 uploads its index lists)."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(arr))
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)
