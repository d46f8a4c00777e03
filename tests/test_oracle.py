"""The CPU oracle, pinned against the reference's known answers, an independent
fp64 brute force, and invariants the mathematics fixes. A plausible mistake
(dropped past, wrong GQA mapping, sibling branches leaking, wrong causal
alignment) is planted in the oracle and must be caught."""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from hypothesis import given, settings
from hypothesis import strategies as st

from dan_amd import workloads as W
from dan_amd.attention import Batch, segment
from oracle import tree_attention as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_tree_mask_known_answers():
    """tests/test_runner.py:16-22 of the reference, from the committed fixture."""
    with open(os.path.join(GOLDEN, "mask_known_answers.json")) as f:
        ka = json.load(f)
    m = O.tree_mask(torch.tensor(ka["tree_mask"]["branch"]))
    for row, want in ka["tree_mask"]["rows"].items():
        assert m[int(row)].tolist() == want
    case = ka["branch_rows_mask_equals_tree_rows"]
    b = torch.tensor(case["branch"])
    assert torch.equal(O.branch_rows_mask(b, case["trunk"]), O.tree_mask(b)[case["trunk"]:])


def test_masks_match_the_visibility_rule():
    """tree_mask, branch_rows_mask and past_mask against the key-by-key rule."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        trunk = int(rng.integers(0, 6))
        lens = [int(x) for x in rng.integers(1, 5, int(rng.integers(0, 4)))]
        ids = W.branch_ids(trunk, lens)
        if not ids:
            continue
        past = int(rng.integers(0, 4))
        vis = O.visible(trunk, ids, past)
        tm = O.tree_mask(torch.tensor(ids)).numpy()
        assert (tm == vis[:, past:]).all()
        assert (O.past_mask(ids, trunk, past).numpy() == vis[trunk:]).all()


def test_segment_spans_closed_form():
    """trunk = first nonzero id; each maximal run after it is one span (brute force)."""
    rng = np.random.default_rng(4)
    for _ in range(200):
        ids = [0] * int(rng.integers(0, 4)) + sorted(int(x) for x in rng.integers(1, 5, int(rng.integers(0, 8))))
        trunk, spans = O.segment_spans(ids)
        assert trunk == (ids.index(next(b for b in ids if b)) if any(ids) else len(ids))
        flat = [i for a, b in spans for i in range(a, b)]
        assert flat == list(range(trunk, len(ids)))
        for a, b in spans:
            assert len(set(ids[a:b])) == 1
        for (_, b1), (a2, _) in zip(spans, spans[1:]):
            assert ids[b1 - 1] != ids[a2]
        s = segment(10, ids)
        assert s.trunk == trunk and s.branches == [(10 + a, 10 + b) for a, b in spans]


def test_bruteforce_golden_samples():
    """The fp64 brute force reproduces its committed samples (catches drift)."""
    g = np.load(os.path.join(GOLDEN, "bruteforce_samples.npz"))
    for name, w in (("c1", W.config1(0)), ("runner_shapes", W.runner_shapes(0, dtype=torch.float32))):
        rows = g[f"{name}_rows"]
        got = O.attend_bruteforce(w.q, w.k, w.v, w.segments, w.layer)[:, rows]
        np.testing.assert_allclose(got, g[f"{name}_out"], rtol=0, atol=1e-12)


def test_input_digests():
    """The seeded generators are bit-stable."""
    with open(os.path.join(GOLDEN, "input_digests.json")) as f:
        want = json.load(f)
    ws = {"c1": W.config1(0), "c2": W.config2(0), "c3": W.config3(0), "c4": W.config4(0),
          "runner_shapes": W.runner_shapes(0), "runner_shapes_fp32": W.runner_shapes(0, dtype=torch.float32)}
    for name, w in ws.items():
        assert w.digest() == want[name]["digest"], name
        assert w.meta == want[name]["meta"], name


@pytest.mark.parametrize("make", [lambda: W.config1(0), lambda: W.runner_shapes(0, dtype=torch.float32),
                                  lambda: W.runner_shapes(1, dtype=torch.float32, head_dim=64)])
def test_dense_matches_bruteforce(make):
    w = make()
    dense = O.attend_dense(w.q, w.k, w.v, w.segments, w.layer).double().numpy()
    brute = O.attend_bruteforce(w.q, w.k, w.v, w.segments, w.layer)
    assert np.abs(dense - brute).max() < 1e-5


def _random_batch(rng, h=4, hkv=2, d=16, max_segments=3):
    structure, pasts = [], []
    for _ in range(int(rng.integers(1, max_segments + 1))):
        trunk = int(rng.integers(0, 9))
        lens = [int(x) for x in rng.integers(1, 7, int(rng.integers(0, 4)))]
        if trunk + sum(lens) == 0:
            trunk = 1
        structure.append((trunk, lens))
        pasts.append(int(rng.integers(0, 6)) if rng.random() < 0.5 else 0)
    return W.build("random", structure, h, hkv, d, torch.float32, "cpu", rng, per_segment_past=pasts)


@settings(max_examples=40, deadline=None)
@given(st.integers(0, 2 ** 31 - 1))
def test_dense_matches_bruteforce_random_trees(seed):
    """Random trees: empty trunks, single-token branches, no branches, pasts."""
    w = _random_batch(np.random.default_rng(seed))
    dense = O.attend_dense(w.q, w.k, w.v, w.segments, w.layer).double().numpy()
    brute = O.attend_bruteforce(w.q, w.k, w.v, w.segments, w.layer)
    assert np.abs(dense - brute).max() < 1e-5


def test_no_branches_is_causal_attention():
    """A segment without branches is plain causal attention (GQA by repeat)."""
    rng = np.random.default_rng(5)
    w = W.build("causal", [(37, [])], 8, 2, 32, torch.float32, "cpu", rng)
    got = O.attend_dense(w.q, w.k, w.v, w.segments, 0)
    k = w.k.repeat_interleave(4, dim=0)
    v = w.v.repeat_interleave(4, dim=0)
    want = F.scaled_dot_product_attention(w.q[None], k[None], v[None], is_causal=True)[0]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=0)


def test_single_branch_is_causal_over_past_trunk_branch():
    """One branch: every token sees [past; trunk; own prefix] -- causal attention
    over the concatenation, read at the new rows."""
    rng = np.random.default_rng(6)
    w = W.build("one", [(11, [7])], 4, 4, 16, torch.float32, "cpu", rng, per_segment_past=[5])
    got = O.attend_dense(w.q, w.k, w.v, w.segments, 0)
    pk, pv = w.segments[0].past[0]
    k = torch.cat([pk, w.k], 1)
    v = torch.cat([pv, w.v], 1)
    q = torch.cat([torch.zeros(4, 5, 16), w.q], 1)
    want = F.scaled_dot_product_attention(q[None], k[None], v[None], is_causal=True)[0][:, 5:]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=0)


def test_branch_permutation_permutes_rows():
    """Reordering branches (ids remapped) reorders the branch rows' outputs."""
    rng = np.random.default_rng(7)
    trunk, lens = 9, [3, 5, 2]
    w = W.build("perm", [(trunk, lens)], 4, 2, 16, torch.float32, "cpu", rng, per_segment_past=[4])
    base = O.attend_dense(w.q, w.k, w.v, w.segments, 0)
    order = [2, 0, 1]
    starts = np.cumsum([0] + lens)[:-1] + trunk
    rows = list(range(trunk)) + [int(starts[b]) + i for b in order for i in range(lens[b])]
    q, k, v = w.q[:, rows], w.k[:, rows], w.v[:, rows]
    seg = segment(0, W.branch_ids(trunk, [lens[b] for b in order]), w.segments[0].past, 0, 4)
    got = O.attend_dense(q, k, v, Batch([seg]), 0)
    torch.testing.assert_close(got, base[:, rows], atol=1e-5, rtol=0)


def test_lse_merge_of_disjoint_key_sets_is_the_union():
    """dan/fused.py:94-101: two attentions over a split of the keys merge into
    the attention over all keys."""
    torch.manual_seed(0)
    t, h, d, n = 6, 3, 8, 20
    q, k, v = torch.randn(h, t, d), torch.randn(h, n, d), torch.randn(h, n, d)

    def part(ks, vs):
        s = q @ ks.transpose(1, 2) / math.sqrt(d)
        lse = torch.logsumexp(s, -1)
        return (torch.softmax(s, -1) @ vs).transpose(0, 1), lse

    oa, la = part(k[:, :7], v[:, :7])
    ob, lb = part(k[:, 7:], v[:, 7:])
    whole, _ = part(k, v)
    torch.testing.assert_close(O.lse_merge(oa, la, ob, lb), whole, atol=1e-6, rtol=0)


# ---- planted mistakes: the checks above must catch each of them ------------------

def _diff_vs_brute(w):
    dense = O.attend_dense(w.q, w.k, w.v, w.segments, w.layer).double().numpy()
    return np.abs(dense - O.attend_bruteforce(w.q, w.k, w.v, w.segments, w.layer)).max()


def test_planted_wrong_gqa_mapping_is_caught(monkeypatch):
    """h % Hkv instead of h // rep."""
    def bad(x, rep):
        n, h, d = x.shape
        return x.repeat(1, rep, 1) if rep > 1 else x
    monkeypatch.setattr(O, "repeat_heads", bad)
    assert _diff_vs_brute(W.runner_shapes(0, dtype=torch.float32)) > 1e-2


def test_planted_sibling_leak_is_caught(monkeypatch):
    """Branch rows that see every earlier token (siblings included)."""
    def leaky(ids, trunk, past):
        n = len(ids)
        m = torch.ones(n - trunk, past + n, dtype=torch.bool).tril(past + trunk)
        return m
    monkeypatch.setattr(O, "past_mask", leaky)
    assert _diff_vs_brute(W.config1(0)) > 1e-2


def test_planted_top_left_causal_alignment_is_caught(monkeypatch):
    """Trunk rows aligned top-left after a past (j <= i instead of j <= P + i)."""
    from torch.nn.attention.bias import causal_upper_left
    monkeypatch.setattr(O, "causal_lower_right", causal_upper_left)
    assert _diff_vs_brute(W.runner_shapes(0, dtype=torch.float32)) > 1e-2


def test_planted_dropped_past_is_caught():
    w = W.runner_shapes(0, dtype=torch.float32)
    dense = O.attend_dense(w.q, w.k, w.v, w.segments, 0).double().numpy()
    for s in w.segments:
        s.past, s.past_len = None, 0
    brute = O.attend_bruteforce(w.q, w.k, w.v, w.segments, 0)
    assert np.abs(dense - brute).max() > 1e-2


# ---- fp8 and readout conventions -------------------------------------------------

def test_fp8_quantize_closed_form():
    """scale = amax / 448; the amax element maps to exactly 448; e4m3 keeps
    3 mantissa bits, so normal values round within 2^-4 relative."""
    torch.manual_seed(1)
    x = torch.randn(4096) * 3
    xq, s = O.fp8_quantize(x)
    assert xq.dtype == torch.float8_e4m3fn
    assert s.item() == pytest.approx(x.abs().max().item() / 448.0, rel=1e-7)
    assert xq.float().abs().max().item() == 448.0
    deq = O.dequantize(xq, s)
    normal = (x / s).abs() >= 2.0 ** -6
    rel = ((deq - x).abs() / x.abs())[normal]
    assert rel.max().item() <= 2.0 ** -4 + 1e-7


def test_label_softmax_matches_torch():
    xs = [0.3, -1.2, 4.0, 2.5]
    np.testing.assert_allclose(O.label_softmax(xs), torch.softmax(torch.tensor(xs, dtype=torch.float64), 0).numpy(),
                               rtol=1e-12)


def test_useful_pairs_counts_the_mask():
    """The useful-FLOP pair count equals the number of True entries of the
    segment masks (closed form vs brute force)."""
    w = W.runner_shapes(0, dtype=torch.float32)
    total = sum(O.visible(s.trunk, list(s.branch_ids), s.past_len).sum() for s in w.segments)
    assert O.useful_pairs(w.segments) == total


def test_package_useful_pairs_matches_oracle_closed_form():
    """The package's per-query count (used by bench.py) against the oracle's
    closed form, which test_useful_pairs_counts_the_mask pins to the mask."""
    from dan_amd import workloads as W
    for cfg in ("c1", "c2", "c3", "c4"):
        w = W.CONFIGS[cfg](0)
        assert W.useful_pairs(w.segments) == O.useful_pairs(w.segments), cfg
    w = W.runner_shapes(0)
    assert W.useful_pairs(w.segments) == O.useful_pairs(w.segments)


def test_package_e4m3_quantization_matches_oracle():
    """dan_amd.workloads.quantize_e4m3 (the config-5 input generator) against
    the oracle's restatement of dan/fused.py:85-91: same bytes, same scale;
    and a shared prefix-cache entry stays one shared e4m3 entry."""
    from dan_amd import workloads as W
    x = torch.from_numpy(np.random.default_rng(3).standard_normal((4, 100, 64)).astype(np.float32) * 3)
    xq, s = W.quantize_e4m3(x)
    oq, os_ = O.fp8_quantize(x)
    assert torch.equal(xq.view(torch.uint8), oq.view(torch.uint8))
    assert torch.equal(s.reshape(()), os_.reshape(()))
    w = W.to_e4m3(W.config3(0))
    entries = {id(seg.past) for seg in w.segments if seg.past}
    assert len(entries) == 1
    pk, pv, pks, pvs = w.segments[0].past[0]
    assert pk.dtype == pv.dtype == torch.float8_e4m3fn and pks.numel() == pvs.numel() == 1
