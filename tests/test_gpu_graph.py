"""HIP graph capture of fixed forwards: once a batch's tile plan, past
tables, workspace and recurrent layout are cached (the first call), the
attention call and the DeltaNet layer only allocate and launch, so a serving
loop can capture a forward once and replay it with new activations written
into the captured input buffers.

Each test captures, then replays three times with new inputs. Between
replays the program runs its own eager work and synchronizes, and every
replay is checked against an eager call on the same inputs:
- attention (the c3 batch: 8192 tokens, 1024-token cached prefix, 45
  branches; two layers' calls in one graph): bit-identical, since the same
  kernels run on the same inputs;
- the DeltaNet layer (tree with a cached prefix, a save boundary and
  branches): within 1e-6 of the output's scale, since the library GEMMs may
  pick another algorithm under capture."""
import sys

import pytest
import torch

from dan_amd import workloads
from dan_amd.attention import attend
from deltanet_cases import tree_batch, weights

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def fill(xs, gen):
    for x in xs:
        x.copy_((torch.randn(x.shape, device=x.device, generator=gen) * 0.5).to(x.dtype))


def test_attend_graph_replays_equal_eager(gpu):
    w = workloads.config3(0, device=gpu)
    say(f"graph capture: attend x2 over c3 ({w.num_tokens} tokens, {len(w.segments)} segments)")
    ins = [x.clone() for x in (w.q, w.k, w.v, w.q, w.k, w.v)]
    attend(*ins[:3], w.segments, w.layer)  # first call: plan, past table and workspace are cached
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        o1 = attend(*ins[:3], w.segments, w.layer)
        o2 = attend(*ins[3:], w.segments, w.layer)
    gen = torch.Generator(device=gpu).manual_seed(3)
    for r in range(3):
        fill(ins, gen)
        g.replay()
        e1 = attend(*ins[:3], w.segments, w.layer)
        e2 = attend(*ins[3:], w.segments, w.layer)
        torch.cuda.synchronize()
        say(f"  replay {r}: equal {torch.equal(o1, e1)} {torch.equal(o2, e2)}")
        assert torch.equal(o1, e1) and torch.equal(o2, e2)


def test_deltanet_layer_graph_replays_match_eager(gpu):
    from test_gpu_deltanet_layer import module, on

    segs, x = tree_batch(31)
    on(segs, gpu)
    m = module(weights(32), gpu)
    xs = x.to(gpu).clone()
    say(f"graph capture: DeltaNet layer over a tree of {len(segs)} segments, N {x.shape[0]}")
    with torch.no_grad():
        m(xs, segs)  # first call: the recurrent layout is cached on the batch
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = m(xs, segs)
        gen = torch.Generator(device=gpu).manual_seed(4)
        for r in range(3):
            fill([xs], gen)
            g.replay()
            e = m(xs, segs)
            torch.cuda.synchronize()
            err = (y.float() - e.float()).abs().max().item()
            say(f"  replay {r}: max |graph - eager| {err:.3e}")
            assert err <= 1e-6 * e.float().abs().max().item()
