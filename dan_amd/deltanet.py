"""The gated delta rule of dan's Gated DeltaNet layers on gfx950.

``delta_rule`` keeps dan's signature and meaning (dan/models/qwen3_5.py:136-158):
packed runs of consecutive rows, each from its own initial state, returning
the packed output and every run's final state. The tree phases of
``DeltaNet.forward`` (dan/models/qwen3_5.py:198-210: trunk part 1, trunk part
2 from part 1's states, every branch from its trunk's final state) are calls
of it. The recurrence runs in this package's kernel (``dan_gdn_fwd``,
include/dan_gdn.h); there is no CPU path (the chunked and token-by-token CPU
forms are the test oracle, oracle/deltanet.py).
"""
import torch

from . import _native
from .attention import _DTYPES


def _row_ok(t):
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * t.element_size()) % 16 == 0 for s in t.stride()[:-1])


def delta_rule(q, k, v, g, beta, lengths, states, cu=None):
    """q, k [N, Hk, 128]; v [N, Hv, Dv] (bf16 or fp16, CUDA); g, beta [N, Hv];
    ``lengths``: run lengths summing to N (runs are consecutive rows);
    ``states`` [R, Hv, 128, Dv] fp32. Returns (out [N, Hv, Dv] in q's dtype,
    final states [R, Hv, 128, Dv] fp32). ``cu``: optional precomputed
    (device, host) cumulative lengths, as dan passes them."""
    if not q.is_cuda:
        raise RuntimeError("dan_amd.deltanet.delta_rule runs on a gfx950 GPU only; got tensors on "
                           f"{q.device} (the CPU forms are the test oracle, not a backend)")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must share bf16 or fp16; got {q.dtype}, {k.dtype}, {v.dtype}")
    n, hk, dk = q.shape
    hv, dv = v.shape[1], v.shape[2]
    r = len(lengths)
    if k.shape != q.shape or v.shape[0] != n or hv % hk:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}: want [N, Hk, Dk], [N, Hv, Dv]")
    if sum(lengths) != n or any(x < 0 for x in lengths):
        raise ValueError(f"run lengths {list(lengths)[:8]}... must be >= 0 and sum to {n}")
    if tuple(states.shape) != (r, hv, dk, dv):
        raise ValueError(f"states {tuple(states.shape)}: want {(r, hv, dk, dv)}")
    dev = q.device
    q = q if _row_ok(q) else q.contiguous()
    k = k if _row_ok(k) else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    g = g.float().contiguous()
    beta = beta.float().contiguous()
    s_in = states.float().contiguous()
    if cu is None:
        cu_d = torch.zeros(r + 1, dtype=torch.int32)
        cu_d[1:] = torch.cumsum(torch.tensor(list(lengths), dtype=torch.int32), 0)
        cu_d = cu_d.pin_memory().to(dev, non_blocking=True)
    else:
        cu_d = cu[0].to(torch.int32)
    out = torch.empty((n, hv, dv), dtype=q.dtype, device=dev)
    finals = torch.empty((r, hv, dk, dv), dtype=torch.float32, device=dev)
    a = _native.DanGdnArgs()
    a.abi_version = _native.GDN_ABI_VERSION
    a.dtype = _DTYPES[q.dtype]
    a.num_k_heads, a.num_v_heads, a.k_dim, a.v_dim, a.num_runs, a.num_tokens = hk, hv, dk, dv, r, n
    a.cu = cu_d.data_ptr()
    a.q, a.q_stride_tok, a.q_stride_head = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_tok, a.k_stride_head = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_tok, a.v_stride_head = v.data_ptr(), v.stride(0), v.stride(1)
    a.g, a.beta = g.data_ptr(), beta.data_ptr()
    a.states_in, a.states_out = s_in.data_ptr(), finals.data_ptr()
    a.out, a.o_stride_tok, a.o_stride_head = out.data_ptr(), out.stride(0), out.stride(1)
    nbytes = _native.load().dan_gdn_workspace_size(n, hk)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    _native.gdn(a, torch.cuda.current_stream(dev).cuda_stream)
    return out, finals
