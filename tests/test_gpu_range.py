"""Magnitudes beyond fp16's range: bf16 / fp32 v and fp32 q, k at |x| up to
~5e5 and down to ~1e-9.

The matrix core runs fp16 for P V (and for fp32 callers' q and k). The V^T
copy holds each (kv head, 64-key) block scaled by a power of 2 chosen from
its largest |v| (unscaled while that lies in [2^-6, 2^15]), and fp32 q and k
are staged to fp16 with per-tensor powers of 2 chosen the same way. Two
inputs that differ by a power of 2 and are both rescaled therefore store the
same fp16 values, which gives exact identities:
    attend(q, k, v * 2^17)  == attend(q, k, v * 2^-30) * 2^47     (bit for bit)
    attend(q * 2^s, k * 2^-s, v) == attend(q * 2^-s, k * 2^s, v)  (fp32, bit for bit)
and every run is also held to the fp32 oracle, with the max-abs bar relative
to the largest |v|, as are blocks of very different scale in one accumulation
and magnitudes that are not powers of 2."""
import math
from dataclasses import replace

import numpy as np
import pytest
import torch

from dan_amd import workloads as W
from dan_amd.attention import Batch, attend
from oracle import tree_attention as O
from test_gpu_parity import random_batch

pytestmark = pytest.mark.gpu

ATOL = 2e-2


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def scaled(w, q=1.0, k=1.0, v=1.0, pk=1.0, pv=1.0, v_rows=None):
    """A copy of workload w with inputs multiplied (in fp32, then cast back);
    ``v_rows`` limits v's factor to those packed rows. Fresh segments, so no
    plan or prefix table is shared with w."""
    def mul(t, f):
        return (t.float() * f).to(t.dtype) if f != 1.0 else t.clone()

    vv = w.v.clone()
    if v_rows is None:
        vv = mul(w.v, v)
    else:
        vv[:, v_rows] = mul(w.v[:, v_rows], v)
    new_past = {}
    segs = Batch()
    for s in w.segments:
        past = None
        if s.past:
            if id(s.past) not in new_past:
                ek, ev = s.past[w.layer][:2]
                new_past[id(s.past)] = {w.layer: (mul(ek, pk), mul(ev, pv))}
            past = new_past[id(s.past)]
        segs.append(replace(s, past=past, saved={}, _mask=None))
    return W.Workload(w.name, mul(w.q, q), mul(w.k, k), vv, segs, w.layer, dict(w.meta))


def run(w):
    out = attend(w.q, w.k, w.v, w.segments, w.layer)
    torch.cuda.synchronize()
    return out


def rows_of(w):
    return torch.cat([torch.arange(s.start, s.end) for s in w.segments])


def check_oracle(w, name, rel):
    out = run(w)
    ref = O.attend_dense(w.q, w.k, w.v, w.segments, w.layer)
    rows = rows_of(w)
    got = out.float().cpu()[:, rows]
    assert torch.isfinite(got).all(), f"{name}: non-finite output"
    err = (got - ref[:, rows]).abs().max().item() / rel
    say(f"{name}: max-abs / {rel:.3g} = {err:.3e}")
    assert err <= ATOL, f"{name}: relative max-abs {err:.3e} > {ATOL}"


def test_bf16_v_power_of_two_is_exact(gpu):
    """|v| up to ~2^19 (> 65504) and down to ~2^-32: both runs match the oracle
    and each other exactly up to the factor 2^47."""
    rng = np.random.default_rng(7)
    w = random_batch(rng, 8, 2, 128, torch.bfloat16, gpu, long=True)
    hi, lo = scaled(w, v=2.0 ** 17, pv=2.0 ** 17), scaled(w, v=2.0 ** -30, pv=2.0 ** -30)
    say(f"bf16 v * 2^17: max |v| {hi.v.float().abs().max().item():.3e}; v * 2^-30: {lo.v.float().abs().max().item():.3e}")
    check_oracle(hi, "bf16 v * 2^17", rel=2.0 ** 17)
    check_oracle(lo, "bf16 v * 2^-30", rel=2.0 ** -30)
    rows = rows_of(w)
    assert torch.equal(run(hi)[:, rows].float(), run(lo)[:, rows].float() * 2.0 ** 47)


def test_bf16_v_mixed_magnitudes(gpu):
    """Half the new tokens' values at |v| ~ 1e5 and the pasts' at ~1e-7 next to
    N(0, 1) rows: blocks with and without an exponent in one accumulation."""
    rng = np.random.default_rng(8)
    w = random_batch(rng, 8, 2, 128, torch.bfloat16, gpu, long=True)
    n = w.num_tokens
    big_rows = torch.arange(0, n, 2)
    m = scaled(w, v=1e5 / 4, v_rows=big_rows, pv=1e-7)
    check_oracle(m, "bf16 v mixed 1e5 / 1 / 1e-7", rel=max(1.0, m.v.float().abs().max().item()))


def test_fp16_v_full_range(gpu):
    """fp16 inputs at the top of fp16's range (|v| up to 60000)."""
    rng = np.random.default_rng(9)
    w = random_batch(rng, 8, 2, 64, torch.float16, gpu)
    m = scaled(w, v=60000.0 / 4, pv=60000.0 / 4)
    check_oracle(m, "fp16 v ~ 6e4", rel=6e4)


def test_fp32_qk_power_of_two_is_exact(gpu):
    """fp32 q * 2^17 with k * 2^-17 (pasts included), and the reverse: q or k
    beyond 65504, the other in fp16's subnormal range. Same scores, so the
    two outputs are identical, and both match the oracle."""
    rng = np.random.default_rng(10)
    for base_w in (W.config1(0, device=gpu), random_batch(rng, 8, 2, 64, torch.float32, gpu)):
        a = scaled(base_w, q=2.0 ** 17, k=2.0 ** -17, pk=2.0 ** -17)
        b = scaled(base_w, q=2.0 ** -17, k=2.0 ** 17, pk=2.0 ** 17)
        say(f"fp32 {base_w.name}: max |q| {a.q.abs().max().item():.3e} / {b.q.abs().max().item():.3e}")
        check_oracle(a, f"fp32 {base_w.name} q * 2^17, k * 2^-17", rel=1.0)
        check_oracle(b, f"fp32 {base_w.name} q * 2^-17, k * 2^17", rel=1.0)
        rows = rows_of(base_w)
        assert torch.equal(run(a)[:, rows], run(b)[:, rows])


def test_fp32_large_q_v_and_past_scale(gpu):
    """fp32 |q| and |v| up to ~1e5 and tiny ones (not powers of 2), with a
    prefix cache whose k has another magnitude than the new keys (its own
    staging scale). The scores stay O(1): fp16 staging keeps ~11 bits of q
    and k, so it is the range that is tested here, not the precision of huge
    scores."""
    rng = np.random.default_rng(11)
    w = random_batch(rng, 8, 2, 128, torch.float32, gpu)
    m = scaled(w, q=1e5 / 4, k=4e-5, v=1e5 / 4, pk=1e-3, pv=1e5 / 4)
    say(f"fp32 max |q| {m.q.abs().max().item():.3e}, max |v| {m.v.abs().max().item():.3e}")
    check_oracle(m, "fp32 q ~ 1e5, k ~ 1e-4, v ~ 1e5, past k ~ 1e-3", rel=max(1.0, m.v.abs().max().item()))
    m = scaled(w, q=1e-4, k=1e4, v=1e-7, pk=1e4, pv=1e-7)
    check_oracle(m, "fp32 q ~ 1e-4, k ~ 3e4, v ~ 1e-7", rel=m.v.abs().max().item())
