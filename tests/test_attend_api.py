"""The drop-in surface without a GPU: names and metadata mirror
dan/attention.py, and the product has no CPU path -- CPU tensors raise."""
import pytest
import torch

import dan_amd
from dan_amd import attention as A
from oracle import tree_attention as O


def test_public_names():
    for name in ("attend", "segment", "Segment", "Batch", "tree_mask", "branch_rows_mask", "repeat_heads", "to_device"):
        assert hasattr(dan_amd, name)


def test_masks_equal_oracle_restatement():
    for ids in ([0, 0, 1, 1, 2], [0, 0, 0, 1, 1, 2, 3, 3], [1, 1, 2], [0, 0, 0]):
        b = torch.tensor(ids)
        assert torch.equal(A.tree_mask(b), O.tree_mask(b))
        t = next((i for i, x in enumerate(ids) if x), len(ids))
        assert torch.equal(A.branch_rows_mask(b, t), O.branch_rows_mask(b, t))


def test_repeat_heads_is_repeat_interleave():
    x = torch.randn(5, 3, 4)
    assert torch.equal(A.repeat_heads(x, 4), x.repeat_interleave(4, dim=1))
    assert A.repeat_heads(x, 1) is x


def test_cpu_tensors_raise():
    """No CPU fallback: the masked CPU path is the oracle, not a backend."""
    q, k, v = torch.randn(8, 10, 64), torch.randn(2, 10, 64), torch.randn(2, 10, 64)
    segs = A.Batch([A.segment(0, [0] * 6 + [1] * 4)])
    with pytest.raises(RuntimeError, match="gfx950"):
        A.attend(q, k, v, segs, 0)


def test_batch_caches():
    b = A.Batch()
    assert b.layout is None and b.recurrent is None and b.tile_plan is None


@pytest.mark.parametrize("qdt,vdt,want", [(torch.bfloat16, torch.bfloat16, torch.bfloat16),
                                          (torch.float16, torch.float16, torch.float16),
                                          (torch.float16, torch.float32, torch.float32),
                                          (torch.float8_e4m3fn, torch.float8_e4m3fn, torch.bfloat16)])
def test_custom_op_fake_output(qdt, vdt, want):
    """torch.ops.dan_amd.tree_attn under fake tensors (no GPU, no launch):
    the output is [H, N, D] in the kernel's output type, a view of
    token-major [N, H, D] storage -- the layout the real op returns."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    h, hkv, n, d = 32, 8, 100, 128
    with FakeTensorMode():
        q = torch.empty(h, n, d, dtype=qdt, device="cuda")
        k = torch.empty(hkv, n, d, dtype=qdt, device="cuda")
        v = torch.empty(hkv, n, d, dtype=vdt, device="cuda")
        tables = [torch.empty(8, dtype=torch.int32, device="cuda") for _ in range(7)]
        scales = [torch.empty(1, device="cuda") for _ in range(3)] if qdt == torch.float8_e4m3fn else []
        o = torch.ops.dan_amd.tree_attn(q, k, v, tables, scales, [1, 0, 1, 64, 128, 1, 0, 0], 0.1, None)
        assert o.shape == (h, n, d) and o.dtype == want and o.device.type == "cuda"
        assert o.stride() == (d, h * d, 1)
