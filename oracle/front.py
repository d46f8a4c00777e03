"""CPU oracle for the attention front end -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg import this module, as the
checker. The product (dan_amd.front) never imports it and has no CPU path.

Contents, each restating the reference's eager ops on CPU tensors, so every
op's result is rounded to the model dtype exactly as torch rounds it:

- ``rms_norm``                 dan/fused.py:36-40 (shared with tree_attention)
- ``rms_norm_zero_centered``   dan/fused.py:44-48
- ``rotate``                   dan/models/llama.py:43-45, rotate-half over the whole head
- ``rotate_partial``           dan/fused.py:70-76, rotate-half over the first R dims
- ``front``                    the chain between the qkv split and attend():
  dan/models/llama.py:82-86 (norms when qk_norm, rotate, transposes) and
  dan/models/qwen3_5.py:322-327 (zero-centered norms, rotate_partial), and the
  prefix-save rows of dan/attention.py:202-204
- ``front_bruteforce``         an fp64 restatement of the same formulas with no
  intermediate rounding; it pins ``front`` (see tests/test_front_oracle.py)
"""
import torch

from .tree_attention import rms_norm


def rms_norm_zero_centered(x, weight, eps):
    """Qwen3.5-style: the weight w is applied as (1 + w), in fp32, one final cast
    (dan/fused.py:44-48)."""
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + weight.float())).to(x.dtype)


def _half_turn(x):
    """rotate-half's partner term: (x1, x2) -> (-x2, x1) over the last dim."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def rotate(x, cos, sin):
    """x [N, H, D], cos/sin broadcastable to it (dan/models/llama.py:43-45)."""
    return x * cos + _half_turn(x) * sin


def rotate_partial(x, cos, sin):
    """Rotate-half on the first R = cos.shape[-1] dims of each head, the rest
    unchanged; x [N, H, D], cos/sin [N, R] (dan/fused.py:70-76)."""
    r = cos.shape[-1]
    head, tail = x[..., :r], x[..., r:]
    return torch.cat([head * cos[:, None] + _half_turn(head) * sin[:, None], tail], dim=-1)


def front(q, k, v, cos, sin, q_norm_weight=None, k_norm_weight=None, eps=1e-6, norm="rms", saves=()):
    """q [N, H, D], k, v [N, Hkv, D] (CPU, model dtype); cos, sin [N, R] or None.
    Returns (q [H, N, D], k [Hkv, N, D], v [Hkv, N, D], saved) where ``saved``
    lists (k rows, v rows) [Hkv, len, D] for each (start, len) in ``saves``."""
    if norm == "rms":
        q, k = rms_norm(q, q_norm_weight, eps), rms_norm(k, k_norm_weight, eps)
    elif norm == "zero_centered":
        q, k = rms_norm_zero_centered(q, q_norm_weight, eps), rms_norm_zero_centered(k, k_norm_weight, eps)
    elif norm is not None:
        raise ValueError(norm)
    if cos is not None and cos.shape[-1]:
        if cos.shape[-1] == q.shape[-1]:
            q, k = rotate(q, cos[:, None], sin[:, None]), rotate(k, cos[:, None], sin[:, None])
        else:
            q, k = rotate_partial(q, cos, sin), rotate_partial(k, cos, sin)
    qt, kt, vt = q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)
    saved = [(kt[:, s:s + n].contiguous(), vt[:, s:s + n].contiguous()) for s, n in saves]
    return qt, kt, vt, saved


def front_bruteforce(x, cos, sin, weight=None, eps=1e-6, norm="rms"):
    """The same formulas in float64 with no intermediate rounding, the
    rotation written index by index: x [N, H, D] -> [N, H, D] float64."""
    x = x.double()
    if norm is not None:
        r = 1.0 / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
        w = weight.double()
        x = x * r * (w if norm == "rms" else 1.0 + w)
    if cos is None or not cos.shape[-1]:
        return x
    rd = cos.shape[-1]
    c, s = cos.double()[:, None, :], sin.double()[:, None, :]
    out = x.clone()
    half = rd // 2
    for i in range(rd):
        partner = -x[..., i + half] if i < half else x[..., i - half]
        out[..., i] = x[..., i] * c[..., i] + partner * s[..., i]
    return out
