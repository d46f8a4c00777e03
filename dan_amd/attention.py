"""Tree attention for packed, prefill-only reads -- the gfx950 drop-in for
dan/attention.py.

Many requests are packed into one flat token sequence; attention runs per
request (a "segment"). Within a segment, tokens are a trunk (the prompt)
followed by one contiguous branch per question. A query may see a key when

    key comes first  and  (key is trunk or same branch)

and a segment may start from cached keys and values of its prompt's leading
tokens (``past``), which every query sees (dan/attention.py:1-13).

Public names and meanings follow dan/attention.py: ``tree_mask`` (:54),
``branch_rows_mask`` (:62), ``Segment`` (:72), ``Batch`` (:98),
``to_device`` (:106), ``segment`` (:114), ``attend`` (:200),
``repeat_heads`` (:273).

``attend`` has one backend: the fused gfx950 kernel of ``dan_amd/csrc``
(one launch, one online-softmax pass over exactly the visible key tiles). It
replaces the reference's three varlen flash calls plus log-sum-exp merge
(dan/attention.py:210-241) and its environment switch (:51, :175-176).
There is no CPU or fallback path: CPU tensors, a missing library or an
unsupported shape raise.
"""
import ctypes
import functools
import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from . import _native
from .plan import TilePlan


def tree_mask(branch):
    """[N, N] boolean mask (True = attend) from per-token branch ids (0 = trunk)
    (dan/attention.py:54-59)."""
    n = branch.shape[0]
    idx = torch.arange(n, device=branch.device)
    causal = idx[None, :] <= idx[:, None]
    return causal & ((branch[None, :] == 0) | (branch[None, :] == branch[:, None]))


def branch_rows_mask(branch, trunk):
    """The tree mask's rows for branch tokens, [N - trunk, N]: each sees the
    whole trunk and its own branch up to itself (dan/attention.py:62-69)."""
    n = branch.shape[0]
    cols = torch.arange(n, device=branch.device)
    rows = cols[trunk:]
    own = (branch[None, :] == branch[trunk:, None]) & (cols[None, :] <= rows[:, None])
    return (cols[None, :] < trunk) | own


@dataclass
class Segment:
    """One request of the packed batch (dan/attention.py:72-84)."""

    start: int  # this request's new tokens are packed[start:end]
    end: int
    trunk: int = 0  # new trunk tokens: packed[start:start + trunk]
    branches: list = field(default_factory=list)  # (start, end) of each branch in the packed sequence
    past: dict | None = None  # layer -> (k, v) each [Hkv, past, D]
    save: int = 0  # keep the cache entry after the first ``save`` new tokens
    saved: dict = field(default_factory=dict)
    past_len: int = 0
    branch_ids: list = field(default_factory=list, repr=False)
    device: str = "cpu"
    _mask: torch.Tensor | None = field(default=None, repr=False)

    @property
    def mask(self):
        """Branch rows of the tree mask with the past prepended as visible
        columns, [n - trunk, past + n] (dan/attention.py:86-95). Metadata for
        callers and tests; the kernel never materializes a mask."""
        if self._mask is None:
            m = branch_rows_mask(torch.tensor(self.branch_ids, device=self.device), self.trunk)
            if self.past:
                m = torch.cat([m.new_ones(m.shape[0], self.past_len), m], dim=1)
            self._mask = m
        return self._mask


class Batch(list):
    """The segments of one packed forward. Caches the tile plan every attention
    layer shares (as dan/attention.py:98-103 caches ``layout``)."""

    layout = None
    recurrent = None
    tile_plan = None


def to_device(xs, device):
    """A host list of indices as a long tensor on ``device`` (pinned,
    non-blocking upload on the GPU; dan/attention.py:106-111)."""
    t = torch.tensor(xs, dtype=torch.long)
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)


def segment(start, branch, past=None, save=0, past_len=0, device="cpu"):
    """A segment over new tokens with ``branch`` ids (trunk first, then each
    branch contiguous), after ``past_len`` cached tokens
    (dan/attention.py:114-126)."""
    trunk = next((i for i, b in enumerate(branch) if b), len(branch))
    spans, i = [], trunk
    while i < len(branch):
        j = i
        while j < len(branch) and branch[j] == branch[i]:
            j += 1
        spans.append((start + i, start + j))
        i = j
    return Segment(start, start + len(branch), trunk, spans, past, save, past_len=past_len if past else 0,
                   branch_ids=branch, device=device)


def repeat_heads(x, rep):
    """[N, H, D] -> [N, H * rep, D], each head repeated ``rep`` times in place
    (dan/attention.py:273-279). The kernel maps query head h to kv head
    h // rep by index arithmetic instead."""
    if rep == 1:
        return x
    n, h, d = x.shape
    return x[:, :, None].expand(n, h, rep, d).reshape(n, h * rep, d)


E4M3 = torch.float8_e4m3fn
_DTYPES = {torch.bfloat16: _native.DTYPE_BF16, torch.float16: _native.DTYPE_F16, torch.float32: _native.DTYPE_F32,
           E4M3: _native.DTYPE_E4M3}


def attend(q, k, v, segments, layer, scale=None, *, q_scale=None, k_scale=None, v_scale=None, save=True):
    """q: [H, N, D]; k, v: [Hkv, N, D] (rotary applied). Returns [H, N, D]
    (dan/attention.py:200-207).

    Side effect, as in the reference: a segment with ``save > 0`` keeps
    ``saved[layer] = (k[:, start:start+save].clone(), v[...].clone())``.
    The result is a [H, N, D] view of token-major [N, H, D] storage, so the
    caller's ``o.transpose(0, 1).reshape(n, H * D)`` needs no copy. Rows not
    covered by any segment are left uninitialized, as in the reference.

    FP8: q, k, v of dtype ``torch.float8_e4m3fn`` quantized per tensor as in
    dan/fused.py:85-91 and dan/quant.py:28-31 (x ~ xq * scale), with their
    fp32 scales in ``q_scale``, ``k_scale``, ``v_scale`` (one-element device
    tensors). The output is bf16. An e4m3 prefix-cache entry is
    ``past[layer] = (k, v, k_scale, v_scale)``; a saving segment keeps the
    same four-tuple.

    ``save=False`` skips the clones, for a caller whose front end already
    filled ``saved[layer]`` (``dan_amd.front.qkv_front``)."""
    fp8 = q.dtype == E4M3
    for s in segments if save else ():
        if s.save:
            kv = (k[:, s.start:s.start + s.save].clone(), v[:, s.start:s.start + s.save].clone())
            s.saved[layer] = kv + (k_scale.clone(), v_scale.clone()) if fp8 and k_scale is not None else kv
    return _attend_fused(q, k, v, segments, layer, scale, (q_scale, k_scale, v_scale) if fp8 else None)


def _check_inputs(q, k, v):
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q must be [H, N, D] and k, v [Hkv, N, D]")
    h, n, d = q.shape
    hkv = k.shape[0]
    if k.shape != (hkv, n, d) or v.shape != (hkv, n, d):
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must be [Hkv, {n}, {d}]")
    if hkv == 0 or h % hkv:
        raise ValueError(f"{h} query heads is not a multiple of {hkv} kv heads")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must share one of {list(_DTYPES)}; got {q.dtype}, {k.dtype}, {v.dtype}")
    if d not in (64, 128, 256):
        raise ValueError(f"head_dim {d}: the gfx950 kernel is built for 64, 128 and 256")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on one device")


def _check_scale(t, name, device):
    if not (isinstance(t, torch.Tensor) and t.numel() == 1 and t.dtype == torch.float32 and t.device == device):
        raise ValueError(f"e4m3 inputs need {name}: a one-element fp32 tensor on {device}")
    return t.reshape(1).contiguous()


def _aligned(t):
    """16-byte vector loads need 16-byte aligned rows with a unit-stride head_dim."""
    es = t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all((st * es) % 16 == 0 for st in t.stride()[:-1]))


def _kernel_view(t):
    """The tensor itself when the kernel can read it in place, else a fresh
    contiguous copy (unaligned rows, or token strides too large for the
    kernel's 32-bit in-tile offsets). The copy is a new allocation, so its
    base is aligned; ``contiguous()`` would return a contiguous but
    misaligned view unchanged."""
    small = abs(t.stride(-2)) * 64 < 2 ** 31
    if _aligned(t) and small:
        return t
    return torch.empty_like(t, memory_format=torch.contiguous_format).copy_(t)


# Which tile planner builds a batch's tables: "device" (one upload and one
# planner launch per forward; batches beyond its limits go to the host
# planner) or "host" (numpy). Both make the same tables.
PLANNER = "device"


def get_plan(segments, num_tokens, tile_q, device, groups=None, num_cus=None, planner=None):
    """The cached tile plan of this batch (built on first use). With
    ``groups`` and ``num_cus`` the device planner also makes the schedule."""
    planner = planner or PLANNER
    if planner not in ("device", "host"):
        raise ValueError(f"planner {planner!r}: 'device' or 'host'")
    plan = getattr(segments, "tile_plan", None)
    want_device = planner == "device" and groups is not None and torch.device(device).type == "cuda"
    stale = plan is None or not plan.matches(num_tokens, tile_q, device)
    if not stale and want_device and plan.cost is None and (groups, num_cus) not in plan.schedules:
        stale = True  # device-built for another head layout
    if stale:
        plan = None
        if want_device:
            try:
                plan = TilePlan.build_device(segments, num_tokens, tile_q, device, groups, num_cus)
            except ValueError as e:
                if "limits" not in str(e):
                    raise
        if plan is None:
            plan = TilePlan.build(segments, num_tokens, tile_q, device)
        if isinstance(segments, Batch):
            segments.tile_plan = plan
    return plan


def _qk_dtype(dtype):
    """Matrix-core type of q and k: fp32 callers' are staged as fp16 (``_stage_f16``)."""
    return torch.float16 if dtype == torch.float32 else dtype


def _stage_f16(x):
    """fp32 [d0, d1, d2] -> (fp16 copy, scale) with x = copy * scale, scale a
    power of 2 that keeps the copy within fp16's range
    (``dan_tree_attn_stage_f16``, two launches on the current stream)."""
    x = _kernel_view(x)
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    scratch = torch.empty(1 + _native.STAGE_PARTIALS, dtype=torch.float32, device=x.device)  # scale, then the partials
    scale, partial = scratch[:1], scratch[1:]
    a = _native.DanStageF16Args()
    a.abi_version = _native.ABI_VERSION
    a.d0, a.d1, a.d2 = x.shape
    a.x, a.stride0, a.stride1 = x.data_ptr(), x.stride(0), x.stride(1)
    a.out, a.scale, a.partial = out.data_ptr(), scale.data_ptr(), partial.data_ptr()
    _native.stage_f16(a, torch.cuda.current_stream(x.device).cuda_stream)
    return out, scale


def _past_table(plan, layer, hkv, d, dtype, device):
    """Device table of DanPastDesc for ``layer`` (cached on the plan). An
    e4m3 entry is (k, v, k_scale, v_scale)."""
    hit = plan.past_tables.get(layer)
    if hit is not None:
        return hit
    raw, refs = _past_descs(plan.past_dicts, plan.segs, layer, hkv, d, dtype, device)
    table = raw.pin_memory().to(device, non_blocking=True) if device.type == "cuda" else raw
    plan.past_tables[layer] = (table, refs)
    return plan.past_tables[layer]


def _past_descs(past_dicts, segs, layer, hkv, d, dtype, device, capacity=None):
    """The DanPastDesc bytes of ``layer``'s prefix-cache entries (host uint8
    tensor, ``capacity`` entries if given) and the device tensors they point
    at (kept alive by the caller); ``segs`` is the segment table, whose
    past lengths are checked against the entries."""
    n = len(past_dicts)
    descs = (_native.DanPastDesc * max(capacity or n, 1))()
    refs = []
    for i, past in enumerate(past_dicts):
        entry = past[layer]
        if dtype == E4M3:
            if len(entry) != 4:
                raise ValueError(f"past entry {i}, layer {layer}: e4m3 entries are (k, v, k_scale, v_scale)")
            pk, pv = entry[:2]
            pks, pvs = _check_scale(entry[2], "the past k_scale", device), _check_scale(entry[3], "the past v_scale", device)
            refs += [pks, pvs]
            descs[i].k_scale, descs[i].v_scale = pks.data_ptr(), pvs.data_ptr()
        else:
            pk, pv = entry[:2]
        plen = pk.shape[1] if pk.dim() == 3 else -1
        want = (hkv, plen, d)
        if pk.dim() != 3 or tuple(pk.shape) != want or tuple(pv.shape) != want:
            raise ValueError(f"past entry {i}, layer {layer}: k {tuple(pk.shape)}, v {tuple(pv.shape)}; want [Hkv, P, D]")
        if pk.dtype != dtype or pv.dtype != dtype or pk.device != device or pv.device != device:
            raise ValueError(f"past entry {i}, layer {layer}: dtype/device must match q")
        if dtype == torch.float32:
            pk, pks = _stage_f16(pk)
            refs.append(pks)
            descs[i].k_scale = pks.data_ptr()
        pk, pv = _kernel_view(pk), _kernel_view(pv)
        refs += [pk, pv]
        descs[i].k, descs[i].v = pk.data_ptr(), pv.data_ptr()
        descs[i].k_stride_head, descs[i].k_stride_tok = pk.stride(0), pk.stride(1)
        descs[i].v_stride_head, descs[i].v_stride_tok = pv.stride(0), pv.stride(1)
        descs[i].len = plen
    for row in segs:
        if row[4] >= 0 and row[3] != descs[row[4]].len:
            raise ValueError(f"segment past_len {row[3]} differs from its past entry's {descs[row[4]].len} keys")
    return torch.frombuffer(bytearray(bytes(descs)), dtype=torch.uint8), refs


@functools.lru_cache(maxsize=None)
def _num_cus(device):
    """Compute units of the device (the persistent grid's size)."""
    return torch.cuda.get_device_properties(device).multi_processor_count


def _attend_fused(q, k, v, segments, layer, scale, fp8_scales=None, phases=_native.PHASES_ALL, noalloc=False,
                  workspace=None):
    """The kernel call behind ``attend`` (no save side effect). ``phases``
    selects the launches (the C ABI's ``phases``); a split call passes its own
    ``workspace`` (``workspace_bytes`` bytes of uint8 on the device) so that
    the attention-only launch reads the V^T copy an earlier PHASE_PACK or full
    call wrote there -- bench.py times the attention launch alone that way.
    ``noalloc`` launches through ``dan_tree_attn_fwd_noalloc`` (the V^T copy in
    the library's own per-GPU scratch instead of a workspace)."""
    if phases != _native.PHASES_ALL and noalloc:
        # the operator declares no mutation of the library's scratch, so a
        # split pack / attend pair through it could be reordered or dropped
        raise ValueError("noalloc calls run both phases (PHASES_ALL); a split call needs a workspace")
    if phases != _native.PHASES_ALL and workspace is None:
        raise ValueError("a split call (PHASE_PACK / PHASE_ATTEND) needs the workspace the two phases share")
    return _call_op(*_op_args(q, k, v, segments, layer, scale, fp8_scales, phases, noalloc), workspace)


def _call_op(*args):
    """``torch.ops.dan_amd.tree_attn`` under ``torch.compile``; in eager mode
    the launch itself, without the operator dispatch (the autograd and
    in-place wrappers cost about as much host time per call as the launch:
    the call is forward-only and its workspace is the call's own)."""
    if torch.compiler.is_compiling():
        return torch.ops.dan_amd.tree_attn(*args)
    return _launch_tree_attn(*args)


def workspace_bytes(q, k, segments):
    """Bytes of the V^T workspace of a split ``_attend_fused`` call on this
    batch (the plan is built or found as for the call itself)."""
    h, n, d = q.shape
    hkv = k.shape[0]
    lib = _native.load()
    tile_q = _native.tile_q(h, hkv, d, lib=lib)
    groups = _native.head_groups(h, hkv, lib)
    plan = get_plan(segments, n, tile_q, q.device, groups=groups, num_cus=_num_cus(q.device))
    return _native.workspace_size(hkv, d, plan.vt_cols, lib)


def _op_args(q, k, v, segments, layer, scale, fp8_scales=None, phases=_native.PHASES_ALL, noalloc=False):
    """Checks the inputs, builds (or finds) the batch's plan and the layer's
    prefix-cache table, and returns the arguments of ``tree_attn``."""
    if not q.is_cuda:
        raise RuntimeError("dan_amd.attend runs on a gfx950 GPU only; got tensors on "
                           f"{q.device} (the masked CPU path is the test oracle, not a backend)")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise NotImplementedError("the gfx950 tree-attention kernel is forward-only")
    _check_inputs(q, k, v)
    if scale is not None and not (float(scale) > 0 and math.isfinite(float(scale))):
        raise ValueError(f"scale {scale}: the kernel needs a finite positive softmax scale")
    lib = _native.load()
    h, n, d = q.shape
    hkv = k.shape[0]
    tile_q = _native.tile_q(h, hkv, d, lib=lib)
    if tile_q <= 0:
        raise ValueError(f"unsupported head layout H={h}, Hkv={hkv}")
    groups = _native.head_groups(h, hkv, lib)
    plan = get_plan(segments, n, tile_q, q.device, groups=groups, num_cus=_num_cus(q.device))
    table, _refs = _past_table(plan, layer, hkv, d, q.dtype, q.device)
    if q.dtype == E4M3:
        q_scale, k_scale, v_scale = (_check_scale(t, nm, q.device) for t, nm in zip(fp8_scales, ("q_scale", "k_scale", "v_scale")))
    scales = [q_scale, k_scale, v_scale] if q.dtype == E4M3 else []
    if q.dtype == torch.float32:  # fp16 for the matrix core, with power-of-2 scales
        (q, q_scale), (k, k_scale) = _stage_f16(q), _stage_f16(k)
        scales = [q_scale, k_scale]
    q, k, v = _kernel_view(q), _kernel_view(k), _kernel_view(v)
    units, sched_off, slots = plan.schedule(groups, _num_cus(q.device)) if plan.num_work else (None, None, 0)
    tables = [plan.segs_d, plan.work_d, plan.key_lo_d, plan.col_seg_d, table]
    if plan.num_work:
        tables += [units, sched_off]
    meta = [len(plan.segs), len(plan.past_dicts), plan.num_work, tile_q, plan.vt_cols, slots, phases, int(noalloc)]
    softmax_scale = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    return q, k, v, tables, scales, meta, softmax_scale


def _out_dtype(q, v):
    """The kernel's output type: bf16 for e4m3 inputs, fp32 for fp32 v, else q's."""
    return torch.bfloat16 if q.dtype == E4M3 else v.dtype if v.dtype == torch.float32 else q.dtype


@torch.library.custom_op("dan_amd::tree_attn", mutates_args=("workspace",), device_types="cuda")
def tree_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tables: List[torch.Tensor],
              scales: List[torch.Tensor], meta: List[int], scale: float,
              workspace: Optional[torch.Tensor]) -> torch.Tensor:
    """The kernel launch as a torch operator (``torch.ops.dan_amd.tree_attn``),
    so that fake-tensor tracing and ``torch.compile`` see its output's shape,
    dtype and strides without running it.

    q [H, N, D], k and v [Hkv, N, D] in the kernel's types (q and k bf16,
    fp16 or e4m3; v the same, or fp32 with fp16 q and k), rows 16-byte
    aligned; ``tables``: the plan's device tables (segments, work items,
    key_lo, col_seg), the layer's prefix-cache table and, when there is work,
    the schedule (unit records, slot offsets) and, for a ``BudgetPlan``, the
    batch's device counts; ``scales``: q, k, v scales of
    e4m3 inputs, or the power-of-2 q and k scales of fp32 inputs staged to fp16; ``meta``: [segments, prefix entries, work items, tile_q,
    V^T columns, slots, phases, noalloc]. Returns [H, N, D], a view of
    token-major [N, H, D] storage. The V^T copy goes to ``workspace`` when the
    caller passes one (uint8, at least ``dan_tree_attn_workspace_size`` bytes;
    written by the copy, read by the attention launch), else to a block of
    torch's caching allocator on the current stream (stream-ordered reuse);
    with ``noalloc`` the library's own scratch is used instead."""
    return _launch_tree_attn(q, k, v, tables, scales, meta, scale, workspace)


def _launch_tree_attn(q, k, v, tables, scales, meta, scale, workspace):
    """The body of ``tree_attn``."""
    lib = _native.load()
    h, n, d = q.shape
    hkv = k.shape[0]
    num_segments, num_pasts, num_work, tile_q, vt_cols, slots, phases, noalloc = meta
    out = torch.empty((n, h, d), dtype=_out_dtype(q, v), device=q.device)
    if num_work:
        segs_d, work_d, key_lo_d, col_seg_d, past_table, units, sched_off = tables[:7]
        counts = tables[7] if len(tables) > 7 else None  # budget mode: the batch's device counts
        nbytes = _native.workspace_size(hkv, d, vt_cols, lib)
        ws = None
        if not noalloc:
            ws = workspace if workspace is not None else torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            if ws.dtype != torch.uint8 or ws.device != q.device or not ws.is_contiguous() or ws.numel() < nbytes:
                raise ValueError(f"workspace: a contiguous uint8 tensor of >= {nbytes} bytes on {q.device}")
        a = _native.DanTreeAttnArgs()
        a.abi_version = _native.ABI_VERSION
        a.in_dtype = _DTYPES[q.dtype]
        a.v_dtype = _DTYPES[v.dtype]
        a.out_dtype = _DTYPES[out.dtype]
        a.num_heads, a.num_kv_heads, a.head_dim, a.num_tokens = h, hkv, d, n
        a.scale = scale
        a.q, a.q_stride_tok, a.q_stride_head = q.data_ptr(), q.stride(1), q.stride(0)
        a.k, a.k_stride_tok, a.k_stride_head = k.data_ptr(), k.stride(1), k.stride(0)
        a.v, a.v_stride_tok, a.v_stride_head = v.data_ptr(), v.stride(1), v.stride(0)
        a.out, a.o_stride_tok, a.o_stride_head = out.data_ptr(), out.stride(0), out.stride(1)
        a.segments, a.num_segments = segs_d.data_ptr(), num_segments
        a.pasts, a.num_pasts = past_table.data_ptr(), num_pasts
        a.work, a.num_work = work_d.data_ptr(), num_work
        a.key_lo = key_lo_d.data_ptr()
        a.tile_q = tile_q
        a.vt_cols = vt_cols
        a.col_seg = col_seg_d.data_ptr()
        if ws is not None:
            a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
        if scales:  # e4m3: q, k, v; fp32 staged to fp16: q, k
            a.q_scale, a.k_scale = scales[0].data_ptr(), scales[1].data_ptr()
            if len(scales) == 3:
                a.v_scale = scales[2].data_ptr()
        a.phases = phases
        a.units, a.sched_off, a.num_slots = units.data_ptr(), sched_off.data_ptr(), slots
        if counts is not None:
            a.counts = counts.data_ptr()
        launch = _native.forward_noalloc if noalloc else _native.forward
        launch(a, torch.cuda.current_stream(q.device).cuda_stream, lib)
    return out.transpose(0, 1)


@tree_attn.register_fake
def _tree_attn_fake(q, k, v, tables, scales, meta, scale, workspace):
    h, n, d = q.shape
    return q.new_empty((n, h, d), dtype=_out_dtype(q, v)).transpose(0, 1)


class BudgetPlan:
    """One HIP graph for changing batches under a fixed token budget.

    A batch's ``TilePlan`` is sized by its own counts (work items, V^T
    columns, slots), and those fix the launch grids. A BudgetPlan sizes its
    tables for capacities instead -- ``num_tokens`` packed tokens in at most
    ``max_segments`` segments with ``max_branches`` branches and
    ``max_past_tokens`` prefix-cache tokens over all segments -- keeps them
    at fixed device addresses, and launches with the capacities' grids. The
    planner, the V^T copy and the attention read the batch's own counts from
    device memory, so launches captured once serve every batch that ``load``
    uploads afterwards (the replacement of the per-forward layout,
    dan/attention.py:211-215, for a serving loop that replays one graph):

        bp = BudgetPlan(8192, 32, 8, 128, torch.bfloat16, "cuda", max_segments=16,
                        max_branches=256, max_past_tokens=16 * 1024)
        bp.load(batch)                    # per batch, outside the graph: one upload, one
                                          # planner launch, each layer's prefix table
        out = bp.attend(q, k, v, layer)   # capturable; equals attend(q, k, v, batch, layer)

    q, k, v keep their addresses between replays (copy each batch's values
    into the captured tensors); prefix-cache entries may change freely (they
    are reached through the prefix tables ``load`` rewrites). Rows beyond the
    batch's segments are left as they are. ``load`` waits for its previous
    upload to finish before reusing the host staging buffer."""

    def __init__(self, num_tokens, num_heads, num_kv_heads, head_dim, dtype, device, max_segments, max_branches,
                 max_past_tokens=0):
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("BudgetPlan runs on a gfx950 GPU only")
        lib = _native.load()
        self.n, self.h, self.hkv, self.d, self.dtype, self.device = num_tokens, num_heads, num_kv_heads, head_dim, dtype, device
        self.tile_q = _native.tile_q(num_heads, num_kv_heads, head_dim, lib=lib)
        self.groups = _native.head_groups(num_heads, num_kv_heads, lib)
        if self.tile_q <= 0 or head_dim not in (64, 128, 256) or dtype not in _DTYPES:
            raise ValueError(f"unsupported layout {num_heads}/{num_kv_heads} x {head_dim}, {dtype}")
        self.max_segments, self.max_branches = max_segments, max_branches
        self.max_work = -(-num_tokens // self.tile_q) + max_segments  # sum of ceil(n / tile_q)
        self.max_cols = -(-(num_tokens + max_past_tokens) // _native.KEY_TILE) + max_segments
        self.num_cus = _num_cus(device)
        self.slots = _native.plan_slots(self.max_work, self.groups, self.num_cus, lib)
        if (self.max_work > _native.PLAN_MAX_WORK or self.slots // self.groups > _native.PLAN_MAX_SLOTS
                or max_segments > _native.PLAN_MAX_SEGMENTS or max_branches > _native.PLAN_MAX_BRANCHES):
            raise ValueError(f"capacities ({self.max_work} work items, {max_segments} segments, {max_branches} branches) "
                             "exceed the device planner's limits")
        i32 = dict(dtype=torch.int32, device=device)
        # counts {S, B, W, C}, the segment table, the branch starts: one upload per batch
        size = 4 + 8 * max_segments + max(max_branches, 1)
        self.blob = torch.zeros(size, **i32)
        self.staging = torch.zeros(size, dtype=torch.int32).pin_memory()
        self.counts = self.blob[:4]
        self.segs_d = self.blob[4:4 + 8 * max_segments]
        self.key_lo = torch.zeros(num_tokens, **i32)
        self.col_seg = torch.zeros(self.max_cols, **i32)
        self.work = torch.zeros((self.max_work, 8), **i32)
        self.cost = torch.zeros(self.max_work, **i32)
        self.units = torch.zeros((self.max_work * self.groups, 16), **i32)
        self.sched_off = torch.zeros(self.slots + 1, **i32)
        self.tables = {}  # layer -> (device DanPastDesc table, pinned staging)
        self.refs = []
        self.loaded = None
        self.loaded_layers = set()   # the layers whose prefix tables the last load wrote
        self.loaded_has_past = False  # whether the loaded batch has prefix-cache entries
        self._copied = torch.cuda.Event()
        self._copied.record(torch.cuda.current_stream(device))

    def _table(self, layer):
        if layer not in self.tables:
            nbytes = ctypes.sizeof(_native.DanPastDesc) * self.max_segments
            self.tables[layer] = (torch.zeros(nbytes, dtype=torch.uint8, device=self.device),
                                  torch.zeros(nbytes, dtype=torch.uint8).pin_memory())
        return self.tables[layer][0]

    def load(self, segments, layers=None):
        """Plan ``segments`` (a Batch over this budget's tokens) on the device and
        write the prefix tables of ``layers`` (default: every layer its
        prefix-cache entries hold, and every layer already captured).

        Every check runs and every layer's table is built on the host before
        anything is copied to the device: a batch that fails them (too large,
        a layer its entries lack, a past length or dtype that does not match)
        raises and leaves the previously loaded batch in place."""
        from .plan import device_inputs

        lib = _native.load()
        segs, starts, w, c, past_dicts = device_inputs(segments, self.n, self.tile_q)
        if (len(segs) > self.max_segments or len(starts) > self.max_branches or w > self.max_work
                or c > self.max_cols):
            raise ValueError(f"batch of {len(segs)} segments, {len(starts)} branches, {w} work items, {c} V^T column "
                             f"blocks exceeds the capacities ({self.max_segments}, {self.max_branches}, "
                             f"{self.max_work}, {self.max_cols})")
        if layers is None:
            layers = set(self.tables)
            if past_dicts:
                layers |= set.intersection(*(set(pd) for pd in past_dicts))
        built, refs = {}, []
        for layer in sorted(layers):
            if any(layer not in pd for pd in past_dicts):
                raise KeyError(f"layer {layer}: a prefix-cache entry of this batch holds no such layer")
            raw, r = _past_descs(past_dicts, segs, layer, self.hkv, self.d, self.dtype, self.device, self.max_segments)
            built[layer] = raw
            refs += r
        stream = torch.cuda.current_stream(self.device)
        self._copied.synchronize()  # the previous upload has left the staging buffers
        st = self.staging.numpy()
        st[:4] = (len(segs), len(starts), w, c)
        st[4:4 + segs.size] = segs.ravel()
        st[4 + 8 * self.max_segments:4 + 8 * self.max_segments + len(starts)] = starts
        self.blob.copy_(self.staging, non_blocking=True)
        for layer, raw in built.items():
            table = self._table(layer)
            stage = self.tables[layer][1]
            stage.copy_(raw)
            table.copy_(stage, non_blocking=True)
        a = _native.DanTreePlanArgs()
        a.abi_version = _native.PLAN_ABI_VERSION
        a.num_tokens, a.num_segments, a.num_branches = self.n, self.max_segments, self.max_branches
        a.num_work, a.num_cols, a.tile_q, a.groups, a.num_cus, a.overhead = (self.max_work, self.max_cols, self.tile_q,
                                                                              self.groups, self.num_cus, 1)
        a.segments = self.segs_d.data_ptr()
        a.branch_starts = self.blob.data_ptr() + 4 * (4 + 8 * self.max_segments)
        a.key_lo, a.col_seg, a.work, a.cost = (self.key_lo.data_ptr(), self.col_seg.data_ptr(), self.work.data_ptr(),
                                               self.cost.data_ptr())
        a.units, a.sched_off, a.counts = self.units.data_ptr(), self.sched_off.data_ptr(), self.counts.data_ptr()
        _native.plan(a, stream.cuda_stream, lib)
        self._copied.record(stream)
        self.refs = refs  # the prefix entries (and staged copies) the tables point at
        self.loaded = segments
        self.loaded_layers = set(built)
        self.loaded_has_past = bool(past_dicts)

    def attend(self, q, k, v, layer, scale=None, *, q_scale=None, k_scale=None, v_scale=None):
        """``attend(q, k, v, batch, layer)`` over the batch ``load`` uploaded, with
        the capacities' launch grids (no save side effect): safe to capture in
        a HIP graph and replay after later ``load`` calls."""
        if not q.is_cuda:
            raise RuntimeError("BudgetPlan.attend runs on a gfx950 GPU only")
        _check_inputs(q, k, v)
        if tuple(q.shape) != (self.h, self.n, self.d) or k.shape[0] != self.hkv or q.dtype != self.dtype:
            raise ValueError(f"q {tuple(q.shape)} {q.dtype}: this budget plan is for [{self.h}, {self.n}, {self.d}] "
                             f"{self.dtype} with {self.hkv} kv heads")
        if self.loaded is None:
            raise ValueError("load a batch before attend")
        if self.loaded_has_past and layer not in self.loaded_layers:
            # the layer's prefix table was not written for this batch: the V^T
            # copy and the attention would read prefix entries through it
            raise KeyError(f"layer {layer}: the loaded batch has prefix-cache entries, but load() wrote no prefix "
                           f"table for this layer (loaded: {sorted(self.loaded_layers)})")
        scales = []
        if q.dtype == E4M3:
            scales = [_check_scale(t, nm, q.device) for t, nm in
                      zip((q_scale, k_scale, v_scale), ("q_scale", "k_scale", "v_scale"))]
        if q.dtype == torch.float32:
            (q, qs), (k, ks) = _stage_f16(q), _stage_f16(k)
            scales = [qs, ks]
        q, k, v = _kernel_view(q), _kernel_view(k), _kernel_view(v)
        tables = [self.segs_d, self.work, self.key_lo, self.col_seg, self._table(layer), self.units, self.sched_off,
                  self.counts]
        meta = [self.max_segments, self.max_segments, self.max_work, self.tile_q, self.max_cols * _native.KEY_TILE,
                self.slots, _native.PHASES_ALL, 0]
        softmax_scale = (1.0 / math.sqrt(self.d)) if scale is None else float(scale)
        return _call_op(q, k, v, tables, scales, meta, softmax_scale, None)
