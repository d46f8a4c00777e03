"""dan_tree_attn_fwd_noalloc through the C ABI: the V^T copy goes to the
library's per-GPU scratch array instead of a caller workspace, and the output
must equal dan_tree_attn_fwd's bit for bit. Two calls in a row, the second
with a smaller batch (the scratch keeps the first call's contents)."""
import pytest
import torch

from dan_amd import workloads
from dan_amd.attention import _attend_fused

pytestmark = pytest.mark.gpu


def _both(w):
    kw = w.attend_kwargs
    fp8 = (kw["q_scale"], kw["k_scale"], kw["v_scale"]) if kw else None
    ref = _attend_fused(w.q, w.k, w.v, w.segments, w.layer, None, fp8)
    got = _attend_fused(w.q, w.k, w.v, w.segments, w.layer, None, fp8, noalloc=True)
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_equals_workspace_path_two_calls(gpu):
    big = workloads.config3(0, device=gpu)
    small = workloads.config2(1, device=gpu)
    assert small.num_tokens < big.num_tokens
    for w in (big, small):
        print(f"noalloc {w.name}: N={w.num_tokens}", flush=True)
        ref, got = _both(w)
        assert torch.equal(ref, got), f"{w.name}: noalloc output differs from the workspace path"
        assert torch.isfinite(got).all()


def test_noalloc_e4m3(gpu):
    w = workloads.config5(0, device=gpu)
    ref, got = _both(w)
    assert torch.equal(ref, got)


def test_noalloc_refuses_split_phases(gpu):
    """A split (pack-only or attend-only) call would read or leave the V^T
    copy in the shared scratch across operator calls that declare no
    mutation; it is refused on the host before anything is launched."""
    from dan_amd import _native

    w = workloads.config1(0, device=gpu)
    for ph in (_native.PHASE_PACK, _native.PHASE_ATTEND):
        with pytest.raises(ValueError, match="noalloc"):
            _attend_fused(w.q, w.k, w.v, w.segments, w.layer, None, None, phases=ph, noalloc=True)
