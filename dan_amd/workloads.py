"""Seeded synthetic workloads for the tree-attention kernel: the five
benchmark configurations and the reference's own differential shapes.

Everything is drawn from ``numpy.random.default_rng(seed)`` in a fixed order
(structure first, then the fused q|k|v activations, then the prefix-cache
block), generated in fp32 and cast with torch's round-to-nearest-even, so the
same seed gives bit-identical inputs on any machine.

q, k, v are laid out as the Llama attention module hands them to ``attend``
(dan/models/llama.py:78-86): strided [H, N, D] / [Hkv, N, D] views of one
token-major fused projection buffer [N, H + 2 Hkv, D].
"""
import hashlib
from dataclasses import dataclass, field, replace

import numpy as np
import torch

from .attention import Batch, segment

LLAMA3_8B = dict(num_heads=32, num_kv_heads=8, head_dim=128)
BUDGET = 8192


@dataclass
class Workload:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    segments: Batch
    layer: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def num_tokens(self):
        return self.q.shape[1]

    @property
    def attend_kwargs(self):
        """Extra arguments of ``attend`` for this workload (the e4m3 scales)."""
        return {k: self.meta[k] for k in ("q_scale", "k_scale", "v_scale") if k in self.meta}

    def digest(self):
        """SHA-256 over q, k, v and every distinct past tensor (raw bytes)."""
        h = hashlib.sha256()
        tensors = [self.q, self.k, self.v]
        seen = set()
        for s in self.segments:
            if s.past and id(s.past) not in seen:
                seen.add(id(s.past))
                tensors += list(s.past[self.layer][:2])
        for t in tensors:
            c = t.detach().to("cpu").contiguous()
            h.update(c.view(torch.uint8).numpy().tobytes() if c.dtype != torch.float8_e4m3fn
                     else c.view(torch.uint8).numpy().tobytes())
        return h.hexdigest()


def branch_ids(trunk, lens):
    return [0] * trunk + [j for j, n in enumerate(lens, 1) for _ in range(n)]


def fifo_pack(requests, budget):
    """Pack (trunk, lens) requests in order as the serving engine does
    (dan/engine.py:83-94), counting new tokens. The first request that does
    not fit keeps its branches and has its trunk trimmed to fill the budget
    exactly (a trunk of at least one token); packing stops there."""
    out, used = [], 0
    for trunk, lens in requests:
        need = trunk + sum(lens)
        if used + need <= budget:
            out.append((trunk, lens))
            used += need
            continue
        room = budget - used - sum(lens)
        if room >= 1:
            out.append((room, lens))
            used += room + sum(lens)
        break
    return out, used


def _to(x, dtype, device):
    return torch.from_numpy(x).to(dtype).to(device)


def _rms_norm_heads(x, eps=1e-6):
    """Per-head RMSNorm with weight 1: normalize in fp32, cast back
    (dan/fused.py:35-40)."""
    y = x.float()
    return (y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


def build(name, structure, num_heads, num_kv_heads, head_dim, dtype, device, rng, std=1.0, past_len=0,
          past_std=1.0, qk_norm=False, v_std=None, per_segment_past=None, meta=None):
    """Materialize a workload. ``structure`` is a list of (trunk, [branch
    lengths]); ``per_segment_past`` (a list of past lengths) gives each
    segment its own prefix-cache entry, otherwise ``past_len > 0`` shares one
    entry across all segments."""
    h, hkv, d = num_heads, num_kv_heads, head_dim
    n = sum(t + sum(ls) for t, ls in structure)
    qkv = rng.standard_normal((n, h + 2 * hkv, d), dtype=np.float32)
    if v_std is None:
        qkv *= std
    else:
        qkv[:, :h + hkv] *= std
        qkv[:, h + hkv:] *= v_std
    fused = _to(qkv, dtype, device)
    q, k, v = fused[:, :h], fused[:, h:h + hkv], fused[:, h + hkv:]
    if qk_norm:
        q, k = _rms_norm_heads(q), _rms_norm_heads(k)
    q, k, v = q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)
    layer = 0
    shared = None
    if past_len and per_segment_past is None:
        pkv = rng.standard_normal((2, hkv, past_len, d), dtype=np.float32) * past_std
        shared = {layer: (_to(pkv[0], dtype, device), _to(pkv[1], dtype, device))}
    segs, start = Batch(), 0
    for i, (trunk, lens) in enumerate(structure):
        ids = branch_ids(trunk, lens)
        past, plen = shared, past_len
        if per_segment_past is not None:
            plen = per_segment_past[i]
            past = None
            if plen:
                pkv = rng.standard_normal((2, hkv, plen, d), dtype=np.float32) * past_std
                past = {layer: (_to(pkv[0], dtype, device), _to(pkv[1], dtype, device))}
        segs.append(segment(start, ids, past, 0, plen if past else 0, str(device)))
        start += len(ids)
    info = dict(meta or {})
    info.update(requests=len(structure), branches=sum(len(ls) for _, ls in structure), packed_tokens=n,
                past_len=past_len if per_segment_past is None else list(per_segment_past))
    return Workload(name, q, k, v, segs, layer, info)


def config1(seed=0, device="cpu"):
    """fp32, 8 q / 2 kv heads, head_dim 64; one request: trunk 256 + 4 branches of 32; no past."""
    rng = np.random.default_rng(seed)
    return build("c1", [(256, [32] * 4)], 8, 2, 64, torch.float32, device, rng)


def config2(seed=0, device="cpu"):
    """Llama-3-8B shape, bf16; 4 requests, trunk ~ U[128, 1024], 3-6 branches of U[16, 64]; N(0,1)*0.5."""
    rng = np.random.default_rng(seed)
    structure = []
    for _ in range(4):
        trunk = int(rng.integers(128, 1025))
        nb = int(rng.integers(3, 7))
        structure.append((trunk, [int(x) for x in rng.integers(16, 65, nb)]))
    return build("c2", structure, dtype=torch.bfloat16, device=device, rng=rng, std=0.5, **LLAMA3_8B)


def config3_structure(rng, candidates=16, budget=BUDGET):
    reqs = []
    for _ in range(candidates):
        trunk = int(rng.integers(200, 2001))
        nb = int(rng.integers(3, 13))
        reqs.append((trunk, [int(x) for x in rng.integers(16, 97, nb)]))
    return fifo_pack(reqs, budget)


def config3(seed=0, device="cpu"):
    """Llama-3-8B shape, bf16, the 8192-token serving budget: 16 candidate
    requests (trunk ~ U[200, 2000], 3-12 branches of U[16, 96]) packed FIFO,
    the first that does not fit trimmed to fill the budget; a shared
    1024-token prefix-cache block ~ N(0,1) before every trunk; new q/k/v
    ~ N(0,1)*0.5."""
    rng = np.random.default_rng(seed)
    structure, used = config3_structure(rng)
    return build("c3", structure, dtype=torch.bfloat16, device=device, rng=rng, std=0.5, past_len=1024,
                 meta=dict(budget=BUDGET, filled=used), **LLAMA3_8B)


def config4(seed=0, device="cpu"):
    """Qwen3-4B-style full attention, bf16, 32/8 heads, head_dim 128: one
    trunk of 7680 tokens + 32 branches of 16; q, k ~ N(0,1) then per-head
    RMSNorm (weight 1, eps 1e-6); v ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    return build("c4", [(7680, [16] * 32)], dtype=torch.bfloat16, device=device, rng=rng, qk_norm=True,
                 **LLAMA3_8B)


def useful_pairs(segments):
    """Visible (query, key) pairs of a batch, counted per query: query i of a
    segment sees its p + i + 1 causal keys except, for a branch query, the
    sibling span between the trunk's end (p + trunk) and its own branch's
    start. Useful FLOPs are 4 * head_dim * num_heads * pairs (QK^T and PV)."""
    total = 0
    for s in segments:
        p = s.past_len if s.past else 0
        n = s.end - s.start
        lo = np.zeros(n, np.int64)
        for a, b in s.branches:
            lo[a - s.start:b - s.start] = p + (a - s.start)
        gap = np.maximum(lo - (p + s.trunk), 0)
        total += int((p + np.arange(n) + 1 - gap).sum())
    return total


E4M3_MAX = 448.0  # torch.finfo(torch.float8_e4m3fn).max (dan/quant.py:15-16)


def quantize_e4m3(x):
    """Per-tensor OCP e4m3 as dan/fused.py:85-91 (rowwise=False) with the
    dan/quant.py:15-16, 28-31 conventions: scale = max(amax|x|, 1e-12) / 448,
    xq = (x / scale) in float8_e4m3fn, so x ~ xq * scale. Returns (xq, scale)
    with scale a one-element fp32 tensor on x's device."""
    xf = x.float()
    scale = xf.abs().amax().clamp(min=1e-12).reshape(1) / E4M3_MAX
    return (xf / scale).to(torch.float8_e4m3fn), scale


def to_e4m3(w):
    """The workload with q, k, v and every prefix-cache entry quantized per
    tensor (each with its own scale). Segments are copied; one shared cache
    entry stays shared. The scales are in ``meta`` (q_scale, k_scale,
    v_scale); an e4m3 cache entry is (k, v, k_scale, v_scale)."""
    (qq, qs), (kq, ks), (vq, vs) = quantize_e4m3(w.q), quantize_e4m3(w.k), quantize_e4m3(w.v)
    entries, segs = {}, Batch()
    for s in w.segments:
        past = None
        if s.past:
            past = entries.get(id(s.past))
            if past is None:
                pk, pv = s.past[w.layer][:2]
                (pkq, pks), (pvq, pvs) = quantize_e4m3(pk), quantize_e4m3(pv)
                past = entries[id(s.past)] = {w.layer: (pkq, pvq, pks, pvs)}
        segs.append(replace(s, past=past, saved={}, _mask=None))
    meta = dict(w.meta, q_scale=qs, k_scale=ks, v_scale=vs, source=w.name)
    return Workload(w.name + "-e4m3", qq, kq, vq, segs, w.layer, meta)


def config5(seed=0, device="cpu"):
    """Config 3's inputs quantized per tensor to OCP e4m3 (q, k, v, and the
    prefix-cache k and v, each with its own fp32 scale); bf16 output."""
    return to_e4m3(config3(seed, device))


def runner_shapes(seed=0, device="cpu", dtype=torch.bfloat16, head_dim=128):
    """The differential shapes of the reference's kernel test
    (tests/test_runner.py:52-55): h=8, hkv=2, (trunk, [branch lengths], past)
    = (40,[5,9,1],0), (7,[30],12), (1,[3]*6,0), (64,[],0), (13,[17,2],20);
    each segment with a past has its own entry."""
    shapes = [(40, [5, 9, 1], 0), (7, [30], 12), (1, [3] * 6, 0), (64, [], 0), (13, [17, 2], 20)]
    rng = np.random.default_rng(seed)
    return build("runner_shapes", [(t, ls) for t, ls, _ in shapes], 8, 2, head_dim, dtype, device, rng,
                 per_segment_past=[p for _, _, p in shapes])


def qwen35_budget(seed=0, device="cpu"):
    """Qwen3.5's gated-attention layout (16 q / 2 kv heads, head_dim 256), bf16,
    at config 3's structure: the 8192-token budget packed FIFO with a shared
    1024-token prefix-cache block; q/k/v ~ N(0,1)*0.5. Not one of the five
    configurations: it measures the head_dim 256 kernel."""
    rng = np.random.default_rng(seed)
    structure, used = config3_structure(rng)
    return build("q35", structure, 16, 2, 256, torch.bfloat16, device, rng, std=0.5, past_len=1024,
                 meta=dict(budget=BUDGET, filled=used))


CONFIGS = {"c1": config1, "c2": config2, "c3": config3, "c4": config4, "c5": config5}
EXTRA = {"q35": qwen35_budget}  # workloads beyond the five configurations (bench.py --workload)
