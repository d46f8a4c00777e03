"""dan's Gated DeltaNet layers on gfx950.

``DeltaNet`` mirrors dan/models/qwen3_5.py:161-227: projections, then per tree
phase the causal depthwise conv + silu over gathered windows and the gates
(``conv_phase``, kernel ``dan_gdn_conv``), then the delta rule (kernel
``dan_gdn_fwd``), then the gated RMS norm and the output projection.
``RecurrentLayout`` (dan/models/qwen3_5.py:239-298) holds the phases' index
lists, built once per forward and uploaded in one copy.

``delta_rule`` keeps dan's signature and meaning (dan/models/qwen3_5.py:136-158):
packed runs of consecutive rows, each from its own initial state, returning
the packed output and every run's final state. The tree phases of
``DeltaNet.forward`` (dan/models/qwen3_5.py:198-210: trunk part 1, trunk part
2 from part 1's states, every branch from its trunk's final state) are calls
of it. The recurrence runs in this package's kernel (``dan_gdn_fwd``,
include/dan_gdn.h); there is no CPU path (the chunked and token-by-token CPU
forms are the test oracle, oracle/deltanet.py).
"""
from dataclasses import dataclass

import numpy as np
import torch
from torch import nn

from . import _native
from .attention import _DTYPES, Batch


def _row_ok(t):
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * t.element_size()) % 16 == 0 for s in t.stride()[:-1])


# Calls whose longest run has at least this many tokens go through the chunked
# form (when Dv is a multiple of 32). Measured on gfx950 with 16/16 heads of
# 128, 45 or 200 runs of L tokens: the token form is faster up to L = 24, the
# chunked form from L = 32 on (1.1x at 32, 1.6x at 64, 2.3x at 256).
CHUNK_MIN_RUN = 32


def delta_rule(q, k, v, g, beta, lengths, states, cu=None, form=None, state_index=None):
    """q, k [N, Hk, 128]; v [N, Hv, Dv] (bf16 or fp16, CUDA); g, beta [N, Hv];
    ``lengths``: run lengths summing to N (runs are consecutive rows);
    ``states`` [R, Hv, 128, Dv] fp32, or with ``state_index`` ([R] integer,
    on the device) [S, Hv, 128, Dv] of which run r starts from
    ``states[state_index[r]]`` (``states.index_select(0, state_index)``
    without the copy; an index outside [0, S) is clamped). Returns (out
    [N, Hv, Dv] in q's dtype, final states [R, Hv, 128, Dv] fp32). ``cu``: optional precomputed
    (device, host) cumulative lengths, as dan passes them. ``form``: "token"
    (token by token: a run's results do not depend on how it is split into
    calls), "chunk" (64 tokens per step on the matrix cores, Dv a multiple of
    32), or None to take "chunk" when the longest run has at least
    CHUNK_MIN_RUN tokens and Dv allows it. Both forms compute the same
    recurrence in fp32."""
    if not q.is_cuda:
        raise RuntimeError("dan_amd.deltanet.delta_rule runs on a gfx950 GPU only; got tensors on "
                           f"{q.device} (the CPU forms are the test oracle, not a backend)")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must share bf16 or fp16; got {q.dtype}, {k.dtype}, {v.dtype}")
    n, hk, dk = q.shape
    hv, dv = v.shape[1], v.shape[2]
    r = len(lengths)
    if k.shape != q.shape or v.shape[0] != n or hv % hk:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}: want [N, Hk, Dk], [N, Hv, Dv]")
    if sum(lengths) != n or any(x < 0 for x in lengths):
        raise ValueError(f"run lengths {list(lengths)[:8]}... must be >= 0 and sum to {n}")
    if state_index is None and tuple(states.shape) != (r, hv, dk, dv):
        raise ValueError(f"states {tuple(states.shape)}: want {(r, hv, dk, dv)}")
    if state_index is not None:
        if states.dim() != 4 or tuple(states.shape[1:]) != (hv, dk, dv) or states.shape[0] < 1:
            raise ValueError(f"states {tuple(states.shape)}: want (S >= 1, {hv}, {dk}, {dv}) with state_index")
        if tuple(state_index.shape) != (r,) or state_index.device != q.device or state_index.dtype.is_floating_point:
            raise ValueError(f"state_index {tuple(state_index.shape)} on {state_index.device}: want ({r},) integers "
                             f"on {q.device}")
        state_index = state_index.to(torch.int32).contiguous()
    if form is None:
        form = "chunk" if dv % 32 == 0 and max(lengths, default=0) >= CHUNK_MIN_RUN else "token"
    if form not in ("token", "chunk"):
        raise ValueError(f"form {form!r}: 'token', 'chunk' or None")
    code = _native.GDN_FORM_CHUNK if form == "chunk" else _native.GDN_FORM_TOKEN
    dev = q.device
    # a fresh copy when rows are misaligned (contiguous() keeps a misaligned base)
    q = q if _row_ok(q) else torch.empty_like(q, memory_format=torch.contiguous_format).copy_(q)
    k = k if _row_ok(k) else torch.empty_like(k, memory_format=torch.contiguous_format).copy_(k)
    v = v if v.stride(-1) == 1 else v.contiguous()
    g = g.float().contiguous()
    beta = beta.float().contiguous()
    s_in = states.float().contiguous()
    if cu is None:
        cu_d = torch.zeros(r + 1, dtype=torch.int32)
        cu_d[1:] = torch.cumsum(torch.tensor(list(lengths), dtype=torch.int32), 0)
        cu_d = cu_d.pin_memory().to(dev, non_blocking=True)
    else:
        cu_d = cu[0].to(torch.int32)
    out = torch.empty((n, hv, dv), dtype=q.dtype, device=dev)
    finals = torch.empty((r, hv, dk, dv), dtype=torch.float32, device=dev)
    a = _native.DanGdnArgs()
    a.abi_version = _native.GDN_ABI_VERSION
    a.dtype = _DTYPES[q.dtype]
    a.num_k_heads, a.num_v_heads, a.k_dim, a.v_dim, a.num_runs, a.num_tokens = hk, hv, dk, dv, r, n
    a.cu = cu_d.data_ptr()
    a.q, a.q_stride_tok, a.q_stride_head = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_tok, a.k_stride_head = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_tok, a.v_stride_head = v.data_ptr(), v.stride(0), v.stride(1)
    a.g, a.beta = g.data_ptr(), beta.data_ptr()
    a.states_in, a.states_out = s_in.data_ptr(), finals.data_ptr()
    a.out, a.o_stride_tok, a.o_stride_head = out.data_ptr(), out.stride(0), out.stride(1)
    nbytes = _native.load().dan_gdn_workspace_size(code, n, r, hk, hv, dv)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes, a.form = ws.data_ptr(), nbytes, code
    if state_index is not None:
        a.state_index, a.num_states_in = state_index.data_ptr(), s_in.shape[0]
    _native.gdn(a, torch.cuda.current_stream(dev).cuda_stream)
    return out, finals


def delta_gates(b, a, a_log, dt_bias):
    """beta = sigmoid(b) in b's dtype, g = -exp(a_log) softplus(a + dt_bias)
    in fp32 (dan/fused.py:80-82). Eager torch ops; ``conv_phase`` computes the
    same gates inside its kernel for the rows of a phase."""
    return b.sigmoid(), -a_log.float().exp() * torch.nn.functional.softplus(a.float() + dt_bias.float())


def gated_rms_norm(x, gate, weight, eps):
    """dan/fused.py:52-56: RMS-normalize x in fp32, scale by weight in x's
    dtype, multiply by silu(gate) in fp32."""
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
    y = weight * y.to(x.dtype)
    return (y * torch.nn.functional.silu(gate.float())).to(x.dtype)


@dataclass
class Phase:
    """One batch of runs (dan/models/qwen3_5.py:230-236). Index lists are
    int32 device tensors: ``ext`` the virtual source rows of every run's
    [history; tokens], ``take`` the first ext entry of each run token's conv
    window, ``rows`` the packed row of each run token in run order."""

    ext: torch.Tensor
    take: torch.Tensor
    rows: torch.Tensor
    lens: list
    cu: tuple  # (device int32 cumulative lengths, host list)
    rows_long: torch.Tensor = None  # ``rows`` as int64, for index_copy_


@dataclass
class RecurrentLayout:
    """The recurrent layers' index lists for one forward
    (dan/models/qwen3_5.py:239-298). A segment's virtual sequence is
    ``k1 = kernel - 1`` history rows (the zero row, or its cached conv
    history) followed by its trunk rows; the runs are trunk part 1 (up to the
    save boundary when a prefix-cache entry is made), trunk part 2 (the rest)
    and every branch, whose history is the trunk's last ``k1`` virtual rows.
    Virtual source rows: packed row e < n_rows, the zero row n_rows, and
    n_rows + 1 + k1 p + r for row r of the p-th cached history."""

    rows: int
    trunk1: Phase | None
    trunk2: Phase | None
    branches: Phase | None
    split_segments: torch.Tensor | None  # segments whose trunk is in two parts
    branch_segment: torch.Tensor | None  # segment of each branch
    past_segments: list  # segments with a cached conv history, in history order
    saves: list  # (segment, the k1 virtual rows of its conv tail at the save boundary)

    @classmethod
    def build(cls, segments, k1, n_rows, device):
        past_segments = [i for i, s in enumerate(segments) if s.past]
        hist_base = {i: n_rows + 1 + k1 * p for p, i in enumerate(past_segments)}
        t1, t2, br, split, br_seg, saves = [], [], [], [], [], []
        for i, s in enumerate(segments):
            hist = list(range(hist_base[i], hist_base[i] + k1)) if i in hist_base else [n_rows] * k1
            virtual = np.array(hist + list(range(s.start, s.start + s.trunk)), dtype=np.int64)
            cut = s.save if 0 < s.save < s.trunk else s.trunk
            t1.append((virtual[:k1], virtual[k1:k1 + cut]))
            if cut < s.trunk:
                t2.append((virtual[cut:cut + k1], virtual[k1 + cut:]))
                split.append(i)
            if s.save:
                saves.append((i, virtual[cut:cut + k1].tolist()))
            for a, b in s.branches:
                br.append((virtual[len(virtual) - k1:], np.arange(a, b)))
                br_seg.append(i)
        parts, lists = [], []  # one int32 upload for every phase's lists

        def add(arr):
            lists.append(np.asarray(arr, dtype=np.int32))
            return len(lists) - 1

        for runs in (t1, t2, br):
            if not runs:
                parts.append(None)
                continue
            lens = [len(toks) for _, toks in runs]
            ext = np.concatenate([np.concatenate([h, t]) for h, t in runs])
            starts = np.cumsum([0] + [len(h) + len(t) for h, t in runs[:-1]])
            take = np.concatenate([st + np.arange(len(t)) for st, (_, t) in zip(starts, runs)])
            rows = np.concatenate([t for _, t in runs])
            cu = np.concatenate([[0], np.cumsum(lens)])
            parts.append((add(ext), add(take), add(rows), add(cu), lens))
        extra = [add(split)] if split else []
        extra += [add(br_seg)] if br_seg else []
        sizes = [len(x) for x in lists]
        host = torch.from_numpy(np.concatenate(lists) if lists else np.zeros(0, np.int32))
        blob = (host.pin_memory().to(device, non_blocking=True) if torch.device(device).type == "cuda"
                else host.to(device))
        offs = np.concatenate([[0], np.cumsum(sizes)])
        piece = [blob[offs[j]:offs[j + 1]] for j in range(len(lists))]

        def phase(part):
            if part is None:
                return None
            e, t, r, c, lens = part
            return Phase(piece[e], piece[t], piece[r], lens, (piece[c], lists[c].tolist()), piece[r].long())

        j = len(lists) - len(extra)
        split_d = piece[j].long() if split else None
        br_d = piece[j + (1 if split else 0)].long() if br_seg else None
        return cls(n_rows, phase(parts[0]), phase(parts[1]), phase(parts[2]), split_d, br_d, past_segments, saves)


def conv_phase(qkv, hist, ph, weight, b, a, a_log, dt_bias):
    """The rows of one phase: silu(causal depthwise conv) over each run token's
    window of the virtual source, and the gates (dan/models/qwen3_5.py:216-218,
    223; dan/fused.py:80-82), in one ``dan_gdn_conv`` call. ``qkv`` [N, C]
    packed rows (row stride any multiple of 8), ``hist`` [rows, C] the cached
    histories in layout order or None, ``weight`` [C, 1, K], ``b``/``a``
    [N, Hv], ``a_log``/``dt_bias`` [Hv]. Returns (conv [T, C] in qkv's dtype,
    beta [T, Hv] fp32, g [T, Hv] fp32)."""
    x, outs, _keep = conv_phase_args(qkv, hist, ph, weight, b, a, a_log, dt_bias)
    _native.gdn_conv(x, torch.cuda.current_stream(qkv.device).cuda_stream)
    return outs


def conv_phase_args(qkv, hist, ph, weight, b, a, a_log, dt_bias):
    """``conv_phase``'s ``DanGdnConvArgs``, its outputs (conv, beta, g) and the
    tensors the arguments point at (keep them alive while the call runs), so
    that a caller can launch the same phase again without rebuilding them."""
    if not qkv.is_cuda:
        raise RuntimeError("dan_amd.deltanet.conv_phase runs on a gfx950 GPU only")
    n, c = qkv.shape
    kk = weight.shape[-1]
    hv = b.shape[1]
    dev = qkv.device
    t = len(ph.rows)
    if qkv.stride(1) != 1 or qkv.stride(0) % 8 or qkv.data_ptr() % 16:
        qkv = qkv.contiguous()
    w = weight.reshape(c, kk).to(qkv.dtype).contiguous()
    if w.data_ptr() % 16:
        w = w.clone()
    hist = None if hist is None else hist.to(qkv.dtype).contiguous()
    b = b if b.stride(1) == 1 else b.contiguous()
    a = a if a.stride(1) == 1 else a.contiguous()
    al, dtb = a_log.float().contiguous(), dt_bias.float().contiguous()
    out = torch.empty((t, c), dtype=qkv.dtype, device=dev)
    beta = torch.empty((t, hv), dtype=torch.float32, device=dev)
    g = torch.empty((t, hv), dtype=torch.float32, device=dev)
    x = _native.DanGdnConvArgs()
    x.abi_version = _native.GDN_ABI_VERSION
    x.dtype = _DTYPES[qkv.dtype]
    x.channels, x.kernel, x.num_rows = c, kk, n
    x.num_hist_rows = 0 if hist is None else hist.shape[0]
    x.num_ext, x.num_out = len(ph.ext), t
    x.src, x.src_stride = qkv.data_ptr(), qkv.stride(0)
    x.hist = 0 if hist is None else hist.data_ptr()
    x.ext, x.take, x.weight = ph.ext.data_ptr(), ph.take.data_ptr(), w.data_ptr()
    x.out, x.out_stride = out.data_ptr(), out.stride(0)
    x.num_heads, x.rows = hv, ph.rows.data_ptr()
    x.b, x.b_stride, x.a, x.a_stride = b.data_ptr(), b.stride(0), a.data_ptr(), a.stride(0)
    x.a_log, x.dt_bias, x.beta, x.g = al.data_ptr(), dtb.data_ptr(), beta.data_ptr(), g.data_ptr()
    return x, (out, beta, g), (qkv, w, hist, b, a, al, dtb, ph)


class DeltaNet(nn.Module):
    """dan/models/qwen3_5.py:161-227 with the same parameters and config
    fields (``linear_num_key_heads``, ``linear_num_value_heads``,
    ``linear_key_head_dim`` (128), ``linear_value_head_dim``,
    ``linear_conv_kernel_dim``, ``hidden_size``, ``rms_norm_eps``), so dan's
    checkpoints load into it. Prefix-cache entries: ``past[index] = (conv
    history [K - 1, C], state [Hv, Dk, Dv])``, written to ``saved[index]`` at
    a segment's save boundary."""

    def __init__(self, c, index):
        super().__init__()
        self.index = index
        self.hk, self.hv = c.linear_num_key_heads, c.linear_num_value_heads
        self.dk, self.dv = c.linear_key_head_dim, c.linear_value_head_dim
        self.kernel = c.linear_conv_kernel_dim
        key_dim, value_dim = self.hk * self.dk, self.hv * self.dv
        self.conv_dim = 2 * key_dim + value_dim
        self.eps = c.rms_norm_eps
        self.in_proj_qkv = nn.Linear(c.hidden_size, self.conv_dim, bias=False)
        self.in_proj_z = nn.Linear(c.hidden_size, value_dim, bias=False)
        self.in_proj_b = nn.Linear(c.hidden_size, self.hv, bias=False)
        self.in_proj_a = nn.Linear(c.hidden_size, self.hv, bias=False)
        self.conv1d = nn.Conv1d(self.conv_dim, self.conv_dim, self.kernel, groups=self.conv_dim, bias=False)
        self.dt_bias = nn.Parameter(torch.ones(self.hv))
        self.A_log = nn.Parameter(torch.zeros(self.hv))
        self.norm = nn.Module()
        self.norm.weight = nn.Parameter(torch.ones(self.dv))
        self.out_proj = nn.Linear(value_dim, c.hidden_size, bias=False)

    def forward(self, x, segments):
        n = x.shape[0]
        qkv, z, b, a = self.in_proj_qkv(x), self.in_proj_z(x), self.in_proj_b(x), self.in_proj_a(x)
        k1 = self.kernel - 1
        lay = getattr(segments, "recurrent", None)
        if lay is None or lay.rows != n:
            lay = RecurrentLayout.build(segments, k1, n, x.device)
            if isinstance(segments, Batch):  # every DeltaNet layer of this forward shares it
                segments.recurrent = lay
        hist = (torch.cat([segments[i].past[self.index][0] for i in lay.past_segments])
                if lay.past_segments else None)
        zeros = torch.zeros(self.hv, self.dk, self.dv, device=x.device, dtype=torch.float32)
        init = torch.stack([s.past[self.index][1].float() if s.past else zeros for s in segments])
        out = torch.empty(n, self.hv, self.dv, device=x.device, dtype=x.dtype)
        final = self._phase(lay.trunk1, qkv, hist, b, a, init, out)
        if lay.trunk2 is not None:
            f2 = self._phase(lay.trunk2, qkv, hist, b, a, final, out, lay.split_segments)
            final_end = final.index_copy(0, lay.split_segments, f2)
        else:
            final_end = final
        for i, tail in lay.saves:  # prefix-cache entries at each save boundary
            segments[i].saved[self.index] = (_virtual_rows(qkv, hist, tail), final[i].clone())
        if lay.branches is not None:
            self._phase(lay.branches, qkv, hist, b, a, final_end, out, lay.branch_segment)
        y = gated_rms_norm(out.reshape(-1, self.dv), z.reshape(-1, self.dv), self.norm.weight, self.eps)
        return self.out_proj(y.reshape(n, -1))

    def _phase(self, ph, qkv, hist, b, a, states, out, state_index=None):
        conv, beta, g = conv_phase(qkv, hist, ph, self.conv1d.weight, b, a, self.A_log, self.dt_bias)
        t, kd = conv.shape[0], self.hk * self.dk
        q = conv[:, :kd].view(t, self.hk, self.dk)
        k = conv[:, kd:2 * kd].view(t, self.hk, self.dk)
        v = conv[:, 2 * kd:].view(t, self.hv, self.dv)
        o, f = delta_rule(q, k, v, g, beta, ph.lens, states, ph.cu, state_index=state_index)
        out.index_copy_(0, ph.rows_long, o)
        return f


def _virtual_rows(qkv, hist, idx):
    """Rows ``idx`` of the virtual source (packed rows, the zero row, then the
    cached histories) as a new [len(idx), C] tensor."""
    n = qkv.shape[0]
    parts = []
    for e in idx:
        if e < n:
            parts.append(qkv[e:e + 1])
        elif e == n:
            parts.append(qkv.new_zeros(1, qkv.shape[1]))
        else:
            parts.append(hist[e - n - 1:e - n])
    return torch.cat(parts)
