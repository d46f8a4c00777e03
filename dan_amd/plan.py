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


@dataclass
class TilePlan:
    """Device-resident tables of one packed forward (see module docstring)."""

    tile_q: int
    num_tokens: int
    device: object
    segs: np.ndarray
    work: np.ndarray
    key_lo: np.ndarray
    cost: np.ndarray
    past_dicts: list
    col_seg: np.ndarray = None
    segs_d: object = None
    work_d: object = None
    key_lo_d: object = None
    col_seg_d: object = None
    past_tables: dict = field(default_factory=dict)  # layer -> (device bytes, keep-alive refs)
    workspace: dict = field(default_factory=dict)  # bytes -> device scratch (reused by every layer)

    @classmethod
    def build(cls, segments, num_tokens, tile_q, device):
        import torch

        segs, work, key_lo, cost, past_dicts, col_seg = build_tables(segments, num_tokens, tile_q)
        plan = cls(tile_q, num_tokens, torch.device(device), segs, work, key_lo, cost, past_dicts, col_seg)
        plan.segs_d = _upload(segs, device)
        plan.work_d = _upload(work, device)
        plan.key_lo_d = _upload(key_lo, device)
        plan.col_seg_d = _upload(col_seg, device)
        return plan

    @property
    def vt_cols(self):
        return int(len(self.col_seg) * KEY_TILE)

    def matches(self, num_tokens, tile_q, device):
        import torch

        return self.num_tokens == num_tokens and self.tile_q == tile_q and self.device == torch.device(device)

    def key_tiles(self):
        """Total key tiles the work list visits (per kv head and head chunk)."""
        return int(self.cost.sum())


def _upload(arr, device):
    """Host array -> device tensor; pinned, non-blocking on the GPU (as
    dan/attention.py:106-111 uploads its index lists)."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(arr))
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)
