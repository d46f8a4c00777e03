"""One HIP graph for changing batches under a fixed token budget
(dan_amd.attention.BudgetPlan): the planner, the V^T copy and the attention
read the batch's counts from device memory and launch with the capacities'
grids, so launches captured over one batch serve later batches after one
upload and one planner launch each.

- Eager: BudgetPlan.attend equals attend bit for bit on c2, the reference's
  differential shapes (per-segment prefix entries), an fp32 batch and an
  e4m3 batch (the same kernels run on the same tables; only the grids and
  the V^T copy's row stride are the capacities').
- Graph: one capture over c3 seed 0 (8192 tokens, a 1024-token prefix entry),
  replayed for seeds 0, 1 and 2 (other structures, other prefix tensors;
  seed 1 fills 7992 of the 8192 rows),
  twice each, with eager attend calls and synchronizations between replays;
  every replay bit-identical to the eager call on the same batch.
- A batch beyond the capacities is refused before anything runs."""
import sys

import pytest
import torch

from dan_amd import workloads as W
from dan_amd.attention import BudgetPlan, attend

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def rows_of(w):
    return torch.cat([torch.arange(s.start, s.end) for s in w.segments])


def plan_for(w, gpu, **caps):
    h, n, d = w.q.shape
    caps = dict(dict(max_segments=16, max_branches=256, max_past_tokens=16 * 1024), **caps)
    return BudgetPlan(n, h, w.k.shape[0], d, w.q.dtype, gpu, **caps)


@pytest.mark.parametrize("name", ["c2", "runner", "fp32", "e4m3"])
def test_budget_attend_equals_attend(gpu, name):
    w = {"c2": lambda: W.config2(0, device=gpu),
         "runner": lambda: W.runner_shapes(0, device=gpu),
         "fp32": lambda: W.runner_shapes(1, device=gpu, dtype=torch.float32),
         "e4m3": lambda: W.to_e4m3(W.runner_shapes(2, device=gpu))}[name]()
    say(f"budget plan, eager: {name} N={w.num_tokens} segments={len(w.segments)}")
    bp = plan_for(w, gpu)
    bp.load(w.segments)
    got = bp.attend(w.q, w.k, w.v, w.layer, **w.attend_kwargs)
    want = attend(w.q, w.k, w.v, w.segments, w.layer, **w.attend_kwargs)
    torch.cuda.synchronize()
    rows = rows_of(w)
    assert torch.equal(got[:, rows], want[:, rows])


def test_one_graph_serves_changing_batches(gpu):
    ws = [W.config3(s, device=gpu) for s in (0, 1, 2)]
    h, _, d = ws[0].q.shape
    n = W.BUDGET
    hkv = ws[0].k.shape[0]
    say(f"budget plan graph: c3 seeds 0-2, {[len(w.segments) for w in ws]} segments")
    # static inputs laid out like the model's fused projection ([N, H + 2 Hkv, D] views)
    fused = torch.empty(n, h + 2 * hkv, d, dtype=torch.bfloat16, device=gpu)
    q, k, v = (fused[:, :h].transpose(0, 1), fused[:, h:h + hkv].transpose(0, 1), fused[:, h + hkv:].transpose(0, 1))
    bp = BudgetPlan(n, h, hkv, d, torch.bfloat16, gpu, max_segments=16, max_branches=256, max_past_tokens=16 * 1024)

    def put(w):  # a batch may fill fewer rows than the budget (c3 seed 1: 7992)
        m = w.num_tokens
        q[:, :m].copy_(w.q)
        k[:, :m].copy_(w.k)
        v[:, :m].copy_(w.v)
        bp.load(w.segments)

    put(ws[0])
    bp.attend(q, k, v, 0)  # first call outside the capture (library load, kernel attributes)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = bp.attend(q, k, v, 0)
    for rep in range(2):
        for i, w in enumerate(ws):
            put(w)
            g.replay()
            want = attend(w.q, w.k, w.v, w.segments, 0)  # eager work between replays
            torch.cuda.synchronize()
            rows = rows_of(w)
            same = torch.equal(out[:, rows], want[:, rows])
            say(f"  replay {rep}, seed {i}: bit-identical {same}")
            assert same


def test_unloaded_layer_is_refused(gpu):
    """A batch with prefix-cache entries: attend on a layer whose prefix table
    load() did not write is refused on the host (its table would point the
    V^T copy at no entry), so is a load of a layer the entries lack, and the
    loaded batch still serves its own layer afterwards."""
    w = W.runner_shapes(0, device=gpu)
    bp = plan_for(w, gpu)
    bp.load(w.segments)
    other = w.layer + 1
    with pytest.raises(KeyError, match="prefix table"):
        bp.attend(w.q, w.k, w.v, other)
    with pytest.raises(KeyError, match="no such layer"):
        bp.load(w.segments, layers=[other])
    got = bp.attend(w.q, w.k, w.v, w.layer)
    want = attend(w.q, w.k, w.v, w.segments, w.layer)
    torch.cuda.synchronize()
    rows = rows_of(w)
    assert torch.equal(got[:, rows], want[:, rows])


def test_failed_load_keeps_the_loaded_batch(gpu):
    """A load whose prefix entry does not match its segment (past length)
    raises before anything is uploaded: the batch loaded before still
    gives its own outputs."""
    w, w2 = W.runner_shapes(0, device=gpu), W.runner_shapes(1, device=gpu)
    bp = plan_for(w, gpu)
    bp.load(w.segments)
    seg = next(s for s in w2.segments if s.past)
    pk, pv = seg.past[w2.layer]
    seg.past[w2.layer] = (pk[:, :-1], pv[:, :-1])
    with pytest.raises(ValueError, match="past"):
        bp.load(w2.segments)
    got = bp.attend(w.q, w.k, w.v, w.layer)
    want = attend(w.q, w.k, w.v, w.segments, w.layer)
    torch.cuda.synchronize()
    rows = rows_of(w)
    assert torch.equal(got[:, rows], want[:, rows])


def test_capacities_are_checked(gpu):
    w = W.config2(0, device=gpu)
    bp = plan_for(w, gpu, max_segments=2)
    with pytest.raises(ValueError, match="capacities"):
        bp.load(w.segments)
    with pytest.raises(ValueError, match="load"):
        plan_for(w, gpu).attend(w.q, w.k, w.v, 0)
