"""The attention front end on gfx950, one launch (``dan_qkv_front``).

Between the fused qkv projection and ``attend``, the reference runs an eager
chain per layer (dan/models/llama.py:78-86; dan/models/qwen3_5.py:319-326):
split and reshape, optional q/k RMSNorm (dan/fused.py:36-40, or the
zero-centered form of dan/fused.py:44-48), rotate-half RoPE on the whole head
(dan/models/llama.py:43-45) or its first R dims (dan/fused.py:70-76), the
transposes to [H, N, D], and inside ``attend`` the prefix-save clones
(dan/attention.py:202-204). ``qkv_front`` does all of it in one pass over q
and k and returns the tensors the reference hands to ``attend``; with
``segments`` and ``layer`` it also fills ``s.saved[layer]`` for saving
segments, after which ``attend(..., save=False)`` skips its own clones.

Numerics are the eager ops': fp32 arithmetic with each op's result rounded to
the model dtype; only the summation order of the norm's sum of squares
differs from torch.
"""
import numpy as np
import torch

from . import _native
from .attention import _DTYPES

NORMS = {None: _native.FRONT_NORM_NONE, "rms": _native.FRONT_NORM_RMS,
         "zero_centered": _native.FRONT_NORM_RMS_ZERO_CENTERED}


def _row_ok(t):
    es = t.element_size()
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1])


def _view(t):
    """t itself when its rows are 16-byte aligned, else a fresh contiguous copy
    (a new allocation is aligned; ``contiguous()`` would return a contiguous
    but misaligned tensor unchanged)."""
    return t if _row_ok(t) else torch.empty_like(t, memory_format=torch.contiguous_format).copy_(t)


def save_index(segments, num_tokens, device):
    """int32 [N]: for each packed token, the index among the saving segments
    of the one whose saved rows hold it, else -1 (cached on a ``Batch``)."""
    key = ("save_of", num_tokens, str(device))
    cache = getattr(segments, "front_cache", None)
    if cache is not None and key in cache:
        return cache[key]
    idx = np.full(num_tokens, -1, np.int32)
    order = []
    for s in segments:
        if s.save:
            if not 0 < s.save <= s.end - s.start:
                raise ValueError(f"segment save {s.save} outside its {s.end - s.start} new tokens")
            idx[s.start:s.start + s.save] = len(order)
            order.append(s)
    t = torch.from_numpy(idx)
    t = t.pin_memory().to(device, non_blocking=True) if torch.device(device).type == "cuda" else t.to(device)
    out = (t, order)
    if hasattr(segments, "__dict__"):
        if cache is None:
            cache = {}
            try:
                segments.front_cache = cache
            except AttributeError:
                cache = None
        if cache is not None:
            cache[key] = out
    return out


def qkv_front(q, k, v, cos, sin, *, q_norm_weight=None, k_norm_weight=None, eps=1e-6, norm="rms",
              segments=None, layer=None):
    """q: [N, H, D]; k, v: [N, Hkv, D] (views of the projection output: any
    strides with a unit-stride head_dim); cos, sin: [N, R] in the model dtype
    (R: rotary dims, a multiple of 16 up to D; the reference's tables).
    ``norm``: None (no q/k norm), "rms" (dan/fused.py:36-40) or
    "zero_centered" (dan/fused.py:44-48), with ``q_norm_weight``,
    ``k_norm_weight`` [D] and ``eps``.

    Returns ``(q [H, N, D], k [Hkv, N, D], v [Hkv, N, D])``: the first two
    are views of new token-major [N, H, D] / [N, Hkv, D] tensors, v is the
    input's view. With ``segments`` and ``layer``, each segment with
    ``save > 0`` gets ``saved[layer] = (k[:, start:start+save], v[...])`` as
    contiguous copies, written by the same launch."""
    if not q.is_cuda:
        raise RuntimeError("dan_amd.qkv_front runs on a gfx950 GPU only; got tensors on "
                           f"{q.device} (the eager CPU chain is the test oracle, not a backend)")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad):
        raise NotImplementedError("the gfx950 front end is forward-only")
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q must be [N, H, D] and k, v [N, Hkv, D]")
    n, h, d = q.shape
    hkv = k.shape[1]
    if k.shape != (n, hkv, d) or v.shape != (n, hkv, d):
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must be [{n}, Hkv, {d}]")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must share bf16 or fp16; got {q.dtype}, {k.dtype}, {v.dtype}")
    if norm not in NORMS:
        raise ValueError(f"norm {norm!r}: one of {list(NORMS)}")
    r = 0 if cos is None else cos.shape[-1]
    if r:
        if cos.shape != (n, r) or sin is None or sin.shape != (n, r):
            raise ValueError(f"cos and sin must both be [{n}, R]")
        if cos.dtype != q.dtype or sin.dtype != q.dtype:
            raise ValueError("cos and sin must be in the model dtype (the reference casts them, llama.py:158)")
    lib = _native.load()
    dev = q.device
    q_in, k_in, v_in = _view(q), _view(k), _view(v)
    cs = sn = None
    if r:
        cs, sn = cos, sin
        if cs.stride() != sn.stride() or not (_row_ok(cs) and _row_ok(sn)):
            cs, sn = cos.contiguous(), sin.contiguous()
    weights = []
    if norm is not None:
        for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
            if not (isinstance(w, torch.Tensor) and w.shape == (d,) and w.device == dev):
                raise ValueError(f"norm {norm!r} needs {name}: a [{d}] tensor on {dev}")
            weights.append(w.to(q.dtype).contiguous())
    q_out = torch.empty((n, h, d), dtype=q.dtype, device=dev)
    k_out = torch.empty((n, hkv, d), dtype=q.dtype, device=dev)

    a = _native.DanQkvFrontArgs()
    a.abi_version = _native.FRONT_ABI_VERSION
    a.dtype = _DTYPES[q.dtype]
    a.num_tokens, a.num_heads, a.num_kv_heads, a.head_dim, a.rotary_dim = n, h, hkv, d, r
    a.norm, a.eps = NORMS[norm], float(eps)
    a.q, a.q_stride_tok, a.q_stride_head = q_in.data_ptr(), q_in.stride(0), q_in.stride(1)
    a.k, a.k_stride_tok, a.k_stride_head = k_in.data_ptr(), k_in.stride(0), k_in.stride(1)
    a.v, a.v_stride_tok, a.v_stride_head = v_in.data_ptr(), v_in.stride(0), v_in.stride(1)
    if r:
        a.cos, a.sin, a.cs_stride_tok = cs.data_ptr(), sn.data_ptr(), cs.stride(0)
    if weights:
        a.q_norm_weight, a.k_norm_weight = weights[0].data_ptr(), weights[1].data_ptr()
    a.q_out, a.qo_stride_tok, a.qo_stride_head = q_out.data_ptr(), q_out.stride(0), q_out.stride(1)
    a.k_out, a.ko_stride_tok, a.ko_stride_head = k_out.data_ptr(), k_out.stride(0), k_out.stride(1)

    keep = []
    if segments is not None and layer is not None and any(s.save for s in segments):
        save_of, order = save_index(segments, n, dev)
        dst = [(torch.empty((hkv, s.save, d), dtype=q.dtype, device=dev),
                torch.empty((hkv, s.save, d), dtype=q.dtype, device=dev)) for s in order]
        table = (_native.DanFrontSave * len(order))()
        for i, (s, (kd, vd)) in enumerate(zip(order, dst)):
            table[i].start, table[i].len, table[i].k_dst, table[i].v_dst = s.start, s.save, kd.data_ptr(), vd.data_ptr()
        raw = torch.frombuffer(bytearray(table), dtype=torch.uint8)
        table_d = raw.pin_memory().to(dev, non_blocking=True)
        a.save_of, a.saves, a.num_saves = save_of.data_ptr(), table_d.data_ptr(), len(order)
        keep = [table_d]
        for s, kv in zip(order, dst):
            s.saved[layer] = kv
    _native.front(a, torch.cuda.current_stream(dev).cuda_stream, lib)
    if keep:
        # the table must outlive the launch: tie its lifetime to the stream's progress
        keep[0].record_stream(torch.cuda.current_stream(dev))
    return q_out.transpose(0, 1), k_out.transpose(0, 1), v.transpose(0, 1)
