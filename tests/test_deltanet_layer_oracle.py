"""The DeltaNet layer oracle (oracle/deltanet.py: silu_conv, delta_gates,
gated_rms_norm, path_windows, deltanet_layer) pinned without a GPU, and the
product's RecurrentLayout (host index lists) checked against it.

- silu_conv equals torch's depthwise conv1d (fp32, an independent library
  route) rounded to bf16 then silu, except at rounding ties; one-hot taps give
  the shifted input exactly (tap K-1 is the current token, tap 0 the oldest
  history row), which fails an off-by-one window.
- delta_gates: closed forms at b = 0 (beta = 1/2), a + dt_bias = 0
  (g = -exp(A_log) ln 2) and above softplus's threshold (g = -exp(A_log) x).
- gated_rms_norm: a constant row normalizes to 1 / sqrt(1 + eps / c^2).
- The layer over a tree equals the layer over each root-to-leaf path as a
  plain sequence (branch rows), the tree property the phases exist for.
- A prefix-cache entry saved at a boundary and used as the next forward's
  past continues the sequence: outputs equal the uninterrupted run's.
- A planted mistake (branches starting from the zero state) fails the
  tree-equals-paths check.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from dan_amd.attention import Batch, segment
from dan_amd.deltanet import RecurrentLayout
from deltanet_cases import DK, DV, EPS, HIDDEN, HK, HV, KERNEL, path_batch, tree_batch, weights
from oracle import deltanet as D


def layer(w, x, segs, recurrent=False):
    return D.deltanet_layer(w, x, segs, 0, HK, HV, DK, DV, KERNEL, EPS, recurrent=recurrent)


def test_silu_conv_matches_torch_conv1d():
    g = torch.Generator().manual_seed(0)
    seq = torch.randn(3 + 50, 48, generator=g).bfloat16()
    w = (torch.randn(48, 4, generator=g) * 0.5).bfloat16()
    got = D.silu_conv(seq, w)
    y = F.conv1d(seq.float().t()[None], w.float()[:, None], groups=48)[0].t()
    ref = F.silu(y.bfloat16().float()).bfloat16()
    diff = (got.float() - ref.float()).abs()
    assert (diff <= ref.float().abs() * 2.0 ** -7 + 1e-30).all()  # one bf16 spacing at a tie
    assert (diff == 0).float().mean() > 0.99


@pytest.mark.parametrize("tap", [0, 3])
def test_silu_conv_one_hot_taps_shift_exactly(tap):
    seq = torch.randn(3 + 20, 16).bfloat16()
    w = torch.zeros(16, 4, dtype=torch.bfloat16)
    w[:, tap] = 1
    got = D.silu_conv(seq, w)
    assert torch.equal(got, F.silu(seq[tap:tap + 20].float()).bfloat16())


def test_delta_gates_closed_forms():
    a_log = torch.tensor([0.0, 0.7, -1.2])
    beta, g = D.delta_gates(torch.zeros(3, dtype=torch.bfloat16), -torch.tensor([1.0, 2.0, 3.0]), a_log,
                            torch.tensor([1.0, 2.0, 3.0]))
    assert torch.equal(beta.float(), torch.full((3,), 0.5))
    assert torch.allclose(g, -a_log.exp() * math.log(2), rtol=1e-6)
    _, g = D.delta_gates(torch.zeros(3), torch.full((3,), 25.0), a_log, torch.zeros(3))
    assert torch.allclose(g, -a_log.exp() * 25.0, rtol=1e-6)


def test_gated_rms_norm_constant_row():
    x = torch.full((2, 8), 3.0)
    gate = torch.full((2, 8), 30.0)  # silu(30) = 30 to fp32 precision
    y = D.gated_rms_norm(x, gate, torch.ones(8), 1e-6)
    assert torch.allclose(y, torch.full((2, 8), 30.0 / math.sqrt(1 + 1e-6 / 9)), rtol=1e-6)


def test_tree_equals_paths():
    w = weights(1)
    segs, x = tree_batch(2)
    y, pre, _ = layer(w, x, segs)
    psegs, px, paths = path_batch(segs, x)
    py, ppre, _ = layer(w, px, psegs)
    at = 0
    for p, rows in paths:
        got = pre[rows]
        want = ppre[at:at + len(rows)]
        assert torch.allclose(got, want, rtol=1e-5, atol=1e-5)
        at += len(rows)


def test_saved_entry_continues_the_sequence():
    w = weights(3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(40, HIDDEN, generator=g).bfloat16()
    full = Batch([segment(0, [0] * 40)])
    _, pre, _ = layer(w, x, full)
    first = Batch([segment(0, [0] * 40, save=25)])
    _, pre1, saved = layer(w, x, first)
    assert torch.allclose(pre1, pre, rtol=1e-5, atol=1e-5)  # the split does not change the run
    hist, state = saved[0]
    rest = Batch([segment(0, [0] * 15, past={0: (hist, state)}, past_len=25)])
    _, pre2, _ = layer(w, x[25:], rest)
    assert torch.allclose(pre2, pre[25:], rtol=1e-5, atol=1e-5)


def test_planted_zero_branch_state_fails():
    w = weights(1)
    segs, x = tree_batch(2)
    _, pre, _ = layer(w, x, segs)
    wrong = Batch([segment(s.start, s.branch_ids, past=s.past, save=s.save, past_len=s.past_len) for s in segs])
    for s in wrong:  # planted: every branch as a fresh segment (zero state, zero history)
        s.branches = []
    _, pre_w, _ = layer(w, x, wrong)
    rows = [r for s in segs for a, b in s.branches for r in range(a, b)]
    assert not torch.allclose(pre_w[rows], pre[rows], rtol=1e-3, atol=1e-3)


def test_layout_matches_path_windows():
    """The product's RecurrentLayout (host lists; built on the CPU here)
    gives every token the conv window and phase of the oracle's paths."""
    segs, x = tree_batch(5)
    k1, n = KERNEL - 1, x.shape[0]
    lay = RecurrentLayout.build(segs, k1, n, "cpu")
    want = D.path_windows(segs, k1, n)
    seen = {}
    for phase, ph in ((1, lay.trunk1), (2, lay.trunk2), (3, lay.branches)):
        ext, take, rows = ph.ext.numpy(), ph.take.numpy(), ph.rows.numpy()
        assert sum(ph.lens) == len(rows) == len(take) and ph.cu[1][-1] == len(rows)
        for i, r in enumerate(rows):
            seen[int(r)] = (phase, ext[take[i]:take[i] + k1 + 1].tolist())
    assert seen == want
    assert lay.past_segments == [0] and [i for i, _ in lay.saves] == [0]
    assert lay.saves[0][1] == want[segs[0].start + segs[0].save - 1][1][1:]
    assert lay.split_segments.tolist() == [0]
    assert lay.branch_segment.tolist() == [0, 0, 0, 1, 1]
