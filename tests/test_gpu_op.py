"""torch.ops.dan_amd.tree_attn on the GPU: torch.library.opcheck (schema,
fake against real output metadata, dispatch under AOT tracing) and
torch.compile(fullgraph=True) with the plan's tables captured, against the
eager attend call bit for bit."""
import pytest
import torch

from dan_amd import workloads as W
from dan_amd.attention import _op_args, attend

pytestmark = pytest.mark.gpu


def _covered(w):
    rows = sorted((s.start, s.end) for s in w.segments)
    return rows[0][0] == 0 and rows[-1][1] == w.num_tokens and all(a[1] == b[0] for a, b in zip(rows, rows[1:]))


@pytest.mark.parametrize("cfg", ["c2", "c5"])
def test_opcheck(gpu, cfg):
    w = W.CONFIGS[cfg](0, device=gpu)
    assert _covered(w)  # every output row defined, so repeated calls compare equal
    kw = w.attend_kwargs
    fp8 = (kw["q_scale"], kw["k_scale"], kw["v_scale"]) if kw else None
    print(f"[gpu-case] opcheck {cfg}: N={w.num_tokens}", flush=True)
    # opcheck's schema and AOT checks do arithmetic on the inputs, which torch
    # does not implement for float8_e4m3fn: e4m3 gets the fake-tensor check.
    utils = ("test_faketensor",) if fp8 else ("test_schema", "test_autograd_registration", "test_faketensor",
                                               "test_aot_dispatch_dynamic")
    torch.library.opcheck(torch.ops.dan_amd.tree_attn.default, _op_args(w.q, w.k, w.v, w.segments, w.layer, None, fp8) + (None,),
                          test_utils=utils)


def test_compile_fullgraph(gpu):
    w = W.CONFIGS["c2"](0, device=gpu)
    h, n, d = w.q.shape
    q, k, v, tables, scales, meta, sc = _op_args(w.q, w.k, w.v, w.segments, w.layer, None)

    def layer_out(q, k, v):  # the reference's o.transpose(0, 1).reshape(n, H * D)
        return torch.ops.dan_amd.tree_attn(q, k, v, tables, scales, meta, sc, None).transpose(0, 1).reshape(n, h * d)

    print(f"[gpu-case] compile c2: N={n}", flush=True)
    f = torch.compile(layer_out, fullgraph=True, backend="aot_eager")
    want = attend(w.q, w.k, w.v, w.segments, w.layer).transpose(0, 1).reshape(n, h * d)
    for _ in range(2):
        assert torch.equal(f(q, k, v), want)
