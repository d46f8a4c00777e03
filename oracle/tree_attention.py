"""CPU oracle for tree-masked prefill attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or the timed CPU baseline. The product
(dan_amd) never imports it and has no CPU path.

Contents, each restating the reference's algorithm from its source:

- ``tree_mask`` / ``branch_rows_mask``  dan/attention.py:54-59, :62-69
- ``segment_spans``                     dan/attention.py:114-126 (trunk and branch spans)
- ``past_mask``                         dan/attention.py:86-95 (branch rows with the past prepended)
- ``repeat_heads``                      dan/attention.py:273-279
- ``attend_dense``                      dan/attention.py:244-270, the reference's masked CPU path:
  per segment, one causal SDPA for the trunk (bottom-right aligned after the
  cached prefix, :259-264) and one masked SDPA for the branch rows against
  K/V repeated per query head (:265-269). fp32.
- ``attend_bruteforce``                 an independent fp64 numpy restatement of
  softmax(scale * q k^T + M) v with M built key by key from the visibility
  rule; it pins ``attend_dense``.
- ``lse_merge``                          dan/fused.py:94-101
- ``rms_norm``                           dan/fused.py:35-40
- ``fp8_quantize``                       dan/fused.py:85-91 (per-tensor mode) with
  the e4m3 conventions of dan/quant.py:15-16
- ``label_softmax`` / ``readout_probs`` dan/readout.py:13-17 and the read
  position of dan/runner.py:58 (last token of each branch), projected as
  dan/models/llama.py:161-165 does.

Segments are duck-typed: anything with start, end, trunk, branches, past,
past_len, branch_ids (the fields of dan/attention.py:72-84).
"""
import math

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

E4M3 = torch.float8_e4m3fn
E4M3_MAX = torch.finfo(E4M3).max  # 448.0


def tree_mask(branch):
    """[N, N] bool: key j visible to query i iff j <= i and (branch[j] == 0 or
    branch[j] == branch[i]) (dan/attention.py:54-59)."""
    n = branch.shape[0]
    idx = torch.arange(n)
    return (idx[None, :] <= idx[:, None]) & ((branch[None, :] == 0) | (branch[None, :] == branch[:, None]))


def branch_rows_mask(branch, trunk):
    """Rows trunk.. of the tree mask, [N - trunk, N] (dan/attention.py:62-69)."""
    n = branch.shape[0]
    cols = torch.arange(n)
    rows = cols[trunk:]
    own = (branch[None, :] == branch[trunk:, None]) & (cols[None, :] <= rows[:, None])
    return (cols[None, :] < trunk) | own


def segment_spans(branch):
    """(trunk, [(a, b), ...]) of a branch-id list, segment-local: the trunk is
    the index of the first nonzero id, and each maximal run of equal ids after
    it is one branch (dan/attention.py:117-124)."""
    trunk = next((i for i, b in enumerate(branch) if b), len(branch))
    spans, i = [], trunk
    while i < len(branch):
        j = i
        while j < len(branch) and branch[j] == branch[i]:
            j += 1
        spans.append((i, j))
        i = j
    return trunk, spans


def past_mask(branch_ids, trunk, past_len):
    """Branch rows of a segment's mask with ``past_len`` all-visible columns
    prepended, [n - trunk, past_len + n] (dan/attention.py:86-95)."""
    m = branch_rows_mask(torch.tensor(branch_ids), trunk)
    if past_len:
        m = torch.cat([m.new_ones(m.shape[0], past_len), m], dim=1)
    return m


def repeat_heads(x, rep):
    """[N, H, D] -> [N, H * rep, D], head h repeated rep times in place
    (dan/attention.py:273-279)."""
    if rep == 1:
        return x
    n, h, d = x.shape
    return x[:, :, None].expand(n, h, rep, d).reshape(n, h * rep, d)


def _past(seg, layer):
    if not seg.past:
        return None
    pk, pv = seg.past[layer][:2]
    return pk, pv


def attend_dense(q, k, v, segments, layer, scale=None):
    """The reference's masked CPU path (dan/attention.py:244-270), in fp32.

    q: [H, N, D]; k, v: [Hkv, N, D]; past entries (k, v) [Hkv, P, D]. Inputs
    of any float dtype are upcast to fp32 on the CPU. Returns fp32 [H, N, D];
    rows outside every segment are zero."""
    q, k, v = (t.detach().to("cpu", torch.float32) for t in (q, k, v))
    rep = q.shape[0] // k.shape[0]
    out = torch.zeros_like(q)
    for s in segments:
        ks, vs = k[:, s.start:s.end], v[:, s.start:s.end]
        past = 0
        pkv = _past(s, layer)
        if pkv is not None:
            pk, pv = (t.detach().to("cpu", torch.float32) for t in pkv)
            past = pk.shape[1]
            ks, vs = torch.cat([pk, ks], dim=1), torch.cat([pv, vs], dim=1)
        t, mid = s.trunk, s.start + s.trunk
        if t:
            kt, vt = ks[None, :, :past + t], vs[None, :, :past + t]
            mask = causal_lower_right(t, past + t) if past else None
            out[:, s.start:mid] = F.scaled_dot_product_attention(
                q[None, :, s.start:mid], kt, vt, attn_mask=mask, is_causal=not past, scale=scale,
                enable_gqa=rep > 1)[0]
        if s.end > mid:
            kb = repeat_heads(ks.transpose(0, 1), rep).transpose(0, 1)
            vb = repeat_heads(vs.transpose(0, 1), rep).transpose(0, 1)
            m = past_mask(s.branch_ids, s.trunk, past)
            out[:, mid:s.end] = F.scaled_dot_product_attention(
                q[None, :, mid:s.end], kb[None], vb[None], attn_mask=m[None, None], scale=scale)[0]
    return out


def visible(seg_trunk, branch_ids, past_len):
    """[n, P + n] bool visibility of one segment, key by key from the rule
    "key precedes query and (key is past or trunk or in the query's own
    branch)" -- written independently of the tensor masks above."""
    trunk, spans = seg_trunk, segment_spans(branch_ids)[1]
    n = len(branch_ids)
    own = np.full(n, -1)
    for a, b in spans:
        own[a:b] = a
    i = np.arange(n)[:, None]  # query
    j = np.arange(n)[None, :]  # key
    new = (j <= i) & ((j < trunk) | ((own[i] >= 0) & (own[j] == own[i])))
    return np.concatenate([np.ones((n, past_len), bool), new], axis=1)


def attend_bruteforce(q, k, v, segments, layer, scale=None):
    """fp64 numpy attention from the visibility rule (small inputs only).
    Returns float64 [H, N, D]; rows outside every segment are zero."""
    q, k, v = (t.detach().to("cpu", torch.float64).numpy() for t in (q, k, v))
    h, n_tok, d = q.shape
    rep = h // k.shape[0]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros_like(q)
    for s in segments:
        n = s.end - s.start
        pkv = _past(s, layer)
        pk = pkv[0].detach().to("cpu", torch.float64).numpy() if pkv is not None else np.zeros((k.shape[0], 0, d))
        pv = pkv[1].detach().to("cpu", torch.float64).numpy() if pkv is not None else np.zeros((k.shape[0], 0, d))
        vis = visible(s.trunk, list(s.branch_ids), pk.shape[1])
        for hq in range(h):
            g = hq // rep
            keys = np.concatenate([pk[g], k[g, s.start:s.end]], 0)
            vals = np.concatenate([pv[g], v[g, s.start:s.end]], 0)
            logits = scale * q[hq, s.start:s.end] @ keys.T
            logits = np.where(vis, logits, -np.inf)
            logits -= logits.max(axis=1, keepdims=True)
            p = np.exp(logits)
            p /= p.sum(axis=1, keepdims=True)
            out[hq, s.start:s.end] = p @ vals
    return out


def lse_merge(o_a, lse_a, o_b, lse_b):
    """Union of two attentions over disjoint key sets from their natural-log
    LSEs; o: [T, H, D], lse: [H, T] (dan/fused.py:94-101)."""
    la, lb = lse_a.float().t()[..., None], lse_b.float().t()[..., None]
    m = torch.maximum(la, lb)
    wa, wb = (la - m).exp(), (lb - m).exp()
    return ((o_a.float() * wa + o_b.float() * wb) / (wa + wb)).to(o_a.dtype)


def rms_norm(x, weight, eps):
    """Llama-style: normalize in fp32, cast back, then scale (dan/fused.py:35-40)."""
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
    return weight * y.to(x.dtype)


def fp8_quantize(x):
    """Per-tensor e4m3: scale = amax(|x|).clamp(1e-12) / 448, xq = (x / scale)
    cast to float8_e4m3fn (dan/fused.py:85-91 with rowwise=False,
    dan/quant.py:15-16). Returns (xq, scale fp32 [1, 1])."""
    xf = x.float()
    scale = xf.abs().amax().reshape(1, 1).clamp(min=1e-12) / E4M3_MAX
    return (xf / scale).to(E4M3), scale


def dequantize(xq, scale):
    return xq.float() * scale.reshape(())


def label_softmax(xs):
    """Max-subtracted softmax of a list of floats (dan/readout.py:13-17)."""
    mx = max(xs)
    ex = [math.exp(x - mx) for x in xs]
    z = sum(ex)
    return [e / z for e in ex]


def readout_weights(num_branches, width, seed):
    """Per branch b, W_b in R^{K_b x width} ~ N(0,1)/sqrt(width), K_b = 2 + (b mod 7)."""
    rng = np.random.default_rng([seed, 7])
    return [torch.from_numpy(rng.standard_normal((2 + b % 7, width), dtype=np.float32) / math.sqrt(width))
            for b in range(num_branches)]


def read_rows(segments):
    """Packed row read for each branch: its last token (dan/runner.py:58)."""
    return [b - 1 for s in segments for _, b in s.branches]


def readout_probs(out, segments, weights, eps=1e-6):
    """Label probabilities per branch from attention output ``out`` [H, N, D]
    (any dtype): the read row's values as given, h = its RMS normalization
    with weight 1 computed in fp32 (the normalize step of dan/fused.py:35-40,
    as llama.py:161 applies it; the result is kept in fp32 instead of being
    re-rounded to the activation dtype, which would make the comparison a
    function of rounding noise), logits = W_b h in fp32 (llama.py:163-165),
    probabilities by ``label_softmax``."""
    rows = read_rows(segments)
    probs = []
    for w, r in zip(weights, rows):
        y = out[:, r].detach().to("cpu").reshape(-1).float()
        h = y * torch.rsqrt(y.pow(2).mean() + eps)
        probs.append(label_softmax((w.float() @ h).tolist()))
    return probs


def useful_pairs(segments):
    """Visible (query, key) pairs: T*P + T(T+1)/2 + sum_b [L_b (P+T) + L_b(L_b+1)/2]."""
    total = 0
    for s in segments:
        p = s.past_len if s.past else 0
        t = s.trunk
        total += t * p + t * (t + 1) // 2
        for a, b in s.branches:
            lb = b - a
            total += lb * (p + t) + lb * (lb + 1) // 2
    return total
