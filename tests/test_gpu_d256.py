"""head_dim 256: the layout of Qwen3.5's gated attention layers, which call
attend (dan/models/qwen3_5.py:327) with 16 q / 2 kv heads of 256 after a
zero-centered q/k RMSNorm and a partial rotary embedding.

The kernel runs these with 16 queries per wave on 16x16 products, two
waves per SIMD, and two stage buffers (a 64 KB K + V^T tile pair per
buffer). Same bars as the other parity tests:
max-abs 2e-2 against the fp32 oracle, readout 1e-3 (e4m3: against the
oracle on the dequantized inputs)."""
import numpy as np
import pytest
import torch

from dan_amd import workloads as W
from dan_amd.attention import attend
from dan_amd.front import qkv_front
from oracle import front as OF
from oracle import tree_attention as O
from test_gpu_front import _qkv, _tables
from test_gpu_parity import _fp8_case, check, random_batch, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(6))
def test_random_trees_d256(gpu, seed):
    """Empty trunks, single-token branches, per-segment pasts, ragged tiles."""
    rng = np.random.default_rng(300 + seed)
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    h, hkv = ((16, 2), (8, 2), (4, 4))[seed % 3]
    check(random_batch(rng, h, hkv, 256, dtype, gpu, long=seed % 3 == 0), f"D=256 random tree seed {seed} {h}/{hkv}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_reference_differential_shapes_d256(gpu, dtype):
    """tests/test_runner.py:44-68 of the reference at head_dim 256."""
    check(W.runner_shapes(0, device=gpu, dtype=dtype, head_dim=256), f"runner shapes {dtype} D=256")


def test_fp8_d256(gpu):
    _fp8_case(W.runner_shapes(0, device=gpu, dtype=torch.bfloat16, head_dim=256), "e4m3 runner shapes D=256", gpu,
              vs_original=False)


def test_qwen35_budget_batch(gpu):
    """An 8192-token packed batch of config-3 structure (5 requests, 45
    branches, a shared 1024-token prefix) at Qwen3.5's 16/2 x 256 layout."""
    rng = np.random.default_rng(0)
    structure, _ = W.config3_structure(rng)
    w = W.build("qwen35-budget", structure, 16, 2, 256, torch.bfloat16, gpu, rng, std=0.5, past_len=1024)
    check(w, "Qwen3.5 layout, 8192-token budget")


def test_qwen35_front_then_attend(gpu):
    """The Qwen3.5 chain: q/gate interleaved projection, zero-centered q/k
    RMSNorm, rotary on the first 64 of 256 dims (the front end), then tree
    attention -- against the oracle's eager chain and masked attention."""
    rng = np.random.default_rng(4)
    structure = [(300, [20, 35, 7]), (150, [64, 1]), (90, [])]
    w = W.build("qwen35-chain", structure, 16, 2, 256, torch.bfloat16, gpu, rng)
    n, h, hkv, d, r = w.num_tokens, 16, 2, 256, 64
    say(f"front -> attend: Qwen3.5 layout, N={n}")
    q, k, v = _qkv(n, h, hkv, d, torch.bfloat16, gpu, seed=5, gate=True)
    cos, sin = _tables(n, r, torch.bfloat16, gpu)
    g = torch.Generator().manual_seed(6)
    wq = (torch.randn(d, generator=g) * 0.2).to(torch.bfloat16).to(gpu)
    wk = (torch.randn(d, generator=g) * 0.2).to(torch.bfloat16).to(gpu)
    qo, ko, vo = qkv_front(q, k, v, cos, sin, q_norm_weight=wq, k_norm_weight=wk, norm="zero_centered",
                           segments=w.segments, layer=0)
    out = attend(qo, ko, vo, w.segments, 0, save=False)
    torch.cuda.synchronize()
    rq, rk, rv, _ = OF.front(q.cpu(), k.cpu(), v.cpu(), cos.cpu(), sin.cpu(), wq.cpu(), wk.cpu(), 1e-6, "zero_centered")
    ref = O.attend_dense(rq, rk, rv, w.segments, 0)
    rows = torch.cat([torch.arange(s.start, s.end) for s in w.segments])
    err = (out.float().cpu()[:, rows] - ref[:, rows]).abs().max().item()
    say(f"  max-abs {err:.3e}")
    assert err <= 2e-2
