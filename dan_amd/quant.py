"""FP8 (OCP e4m3) decoder linears on gfx950, mirroring dan/quant.py.

``FP8Linear`` keeps dan's module interface and conventions (dan/quant.py:23-42):
weights quantized once, per output row (rowwise) or per tensor, activations
quantized on every call with ``scale = max(amax, 1e-12) / 448`` and
``xq = e4m3fn(x / scale)`` (dan/fused.py:85-91), then one scaled fp8 GEMM with
the bias in its epilogue. Both are this package's gfx950 kernels
(include/dan_fp8.h): the quantizer (``dan_fp8_quantize``, one read of x per
call, where dan's eager chain makes five passes) and the scaled GEMM
(``dan_fp8_gemm``, e4m3 x e4m3 on the matrix core with fp32 accumulation),
which takes the place of dan's ``torch._scaled_mm`` call (dan/quant.py:39-41).
FP8Linear hands both operands to the GEMM in its tiled layout (TiledE4M3):
the quantizer writes the activation's codes tiled on every call, and the
weight's tiled copy is made once (dan's row-major ``weight`` stays the
parameter).

There is no CPU path: CPU tensors raise (the eager CPU chain is the test
oracle, oracle/quant.py).
"""
import torch
from torch import nn

from . import _native
from .attention import _DTYPES

E4M3 = torch.float8_e4m3fn
E4M3_MAX = torch.finfo(E4M3).max  # 448 (dan/quant.py:15-16)


class TiledE4M3:
    """e4m3 codes of an [rows, cols] tensor in the GEMM's tiled layout
    (include/dan_fp8.h): 256-row panels of 16 KB k-steps, each k-step 16
    blocks of 16 rows x 64 bytes in the GEMM's LDS order, zero padding to
    whole panels and k-steps. ``data`` is a 1-D uint8 CUDA tensor."""

    def __init__(self, data, rows, cols):
        self.data, self.rows, self.cols = data, rows, cols

    @property
    def shape(self):
        return (self.rows, self.cols)

    @property
    def device(self):
        return self.data.device


def tiled_bytes(rows, cols):
    """Bytes of an [rows, cols] e4m3 tensor in the tiled layout."""
    return -(-rows // 256) * 256 * (-(-cols // 64) * 64)


def tile_codes(codes):
    """[R, K] e4m3 codes (row-major, CUDA) -> TiledE4M3, by index arithmetic on
    the device (for codes that exist only row-major, e.g. a loaded weight)."""
    r, k = codes.shape
    p, ks = -(-r // 256), -(-k // 64)
    padded = torch.zeros((p * 256, ks * 64), dtype=torch.uint8, device=codes.device)
    padded[:r, :k] = codes.view(torch.uint8)
    t = padded.view(p, 16, 16, ks, 4, 16).permute(0, 3, 1, 2, 4, 5)  # panel, k-step, block, row, chunk, byte
    i = torch.arange(16, device=codes.device)
    swz = ((i >> 1) & 3) ^ ((i >> 3) & 1)
    src = torch.arange(4, device=codes.device)[None, :] ^ swz[:, None]  # chunk stored at each position, per row
    out = torch.gather(t, 4, src.view(1, 1, 1, 16, 4, 1).expand(p, ks, 16, 16, 4, 16))
    return TiledE4M3(out.reshape(-1).contiguous(), r, k)


def fp8_quantize(x, fp8_max=E4M3_MAX, rowwise=True, tiled=False):
    """x [M, K] (bf16, fp16 or fp32, CUDA) -> (xq, scale [M, 1] or [1, 1]
    fp32), as dan/fused.py:85-91: xq is [M, K] e4m3fn, or with ``tiled`` the
    same codes as a TiledE4M3 (the GEMM's operand layout). K must be a
    multiple of 16 (dan quantizes only such linears, dan/quant.py:69-70)."""
    if fp8_max != E4M3_MAX:
        raise ValueError(f"fp8_max {fp8_max}: the e4m3fn maximum is {E4M3_MAX}")
    if not x.is_cuda:
        raise RuntimeError("dan_amd.quant.fp8_quantize runs on a gfx950 GPU only; got tensors on "
                           f"{x.device} (the eager CPU chain is the test oracle, not a backend)")
    if x.dim() != 2:
        raise ValueError(f"x must be [M, K]; got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"x dtype {x.dtype}: bf16, fp16 or fp32")
    m, k = x.shape
    es = x.element_size()
    if x.stride(1) != 1 or x.data_ptr() % 16 or (x.stride(0) * es) % 16 or x.stride(0) < k:
        x = torch.empty_like(x, memory_format=torch.contiguous_format).copy_(x)  # a new, aligned allocation
    if tiled:
        xq = torch.empty(tiled_bytes(m, k), dtype=torch.uint8, device=x.device)
    else:
        xq = torch.empty((m, k), dtype=E4M3, device=x.device)
    scale = torch.empty((m, 1) if rowwise else (1, 1), dtype=torch.float32, device=x.device)
    a = _native.DanFp8QuantArgs()
    a.abi_version = _native.FP8_ABI_VERSION
    a.dtype = _DTYPES[x.dtype]
    a.rows, a.cols = m, k
    a.mode = _native.FP8_SCALE_ROW if rowwise else _native.FP8_SCALE_TENSOR
    a.layout = _native.FP8_LAYOUT_TILED if tiled else _native.FP8_LAYOUT_ROWS
    a.x, a.x_stride = x.data_ptr(), x.stride(0)
    a.xq, a.scale = xq.data_ptr(), scale.data_ptr()
    _native.fp8_quantize(a, torch.cuda.current_stream(x.device).cuda_stream)
    return (TiledE4M3(xq, m, k) if tiled else xq), scale


def fp8_gemm(xq, scale_a, wq, scale_b, bias=None, out_dtype=torch.bfloat16):
    """``torch._scaled_mm(xq, wq.t(), scale_a, scale_b, bias, out_dtype)`` as
    dan calls it (dan/quant.py:39-41) on gfx950: y [M, N] = (xq [M, K] wq
    [N, K]^T) * scale_a * scale_b + bias, fp32 accumulation, rounded to
    out_dtype. scale_a is [M, 1] or [1, 1], scale_b [1, N] or [1, 1] (fp32);
    bias [N] of out_dtype or None. N and K are multiples of 16. Either operand
    may be a TiledE4M3 (the layout the GEMM streams fastest)."""
    if not (xq.device.type == "cuda" and wq.device.type == "cuda"):
        raise RuntimeError("dan_amd.quant.fp8_gemm runs on a gfx950 GPU only; got tensors on "
                           f"{xq.device} / {wq.device}")
    for t in (xq, wq):
        if not isinstance(t, TiledE4M3) and t.dtype != E4M3:
            raise ValueError(f"operands must be float8_e4m3fn or TiledE4M3; got {t.dtype}")
        if not isinstance(t, TiledE4M3) and t.dim() != 2:
            raise ValueError(f"operands must be 2-D; got {tuple(t.shape)}")
        if isinstance(t, TiledE4M3) and t.data.numel() != tiled_bytes(t.rows, t.cols):
            raise ValueError(f"a TiledE4M3 of {t.rows} x {t.cols} holds {tiled_bytes(t.rows, t.cols)} bytes, "
                             f"not {t.data.numel()}")
    if xq.shape[1] != wq.shape[1]:
        raise ValueError(f"xq [M, K] and wq [N, K]; got {tuple(xq.shape)} and {tuple(wq.shape)}")
    if out_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"out_dtype {out_dtype}: bf16, fp16 or fp32")
    m, k = xq.shape
    n = wq.shape[0]
    flags = 0
    if scale_a.numel() == 1 and m != 1:
        flags |= _native.FP8_GEMM_X_SCALE_TENSOR
    elif scale_a.numel() != m:
        raise ValueError(f"scale_a has {scale_a.numel()} values for {m} rows")
    if scale_b.numel() == 1 and n != 1:
        flags |= _native.FP8_GEMM_W_SCALE_TENSOR
    elif scale_b.numel() != n:
        raise ValueError(f"scale_b has {scale_b.numel()} values for {n} rows")

    def dense(t, dtype, name):
        if t.dtype != dtype:
            raise ValueError(f"{name} must be {dtype}; got {t.dtype}")
        return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous().clone()

    sa, sb = dense(scale_a, torch.float32, "scale_a"), dense(scale_b, torch.float32, "scale_b")
    if bias is not None:
        bias = dense(bias, out_dtype, "bias")
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} values for {n} outputs")

    def operand(t, tiled_flag):  # (pointer, row stride, flag)
        if isinstance(t, TiledE4M3):
            return t.data.data_ptr(), 0, tiled_flag
        if t.stride(1) != 1 or t.stride(0) % 16 or t.data_ptr() % 16 or t.stride(0) < t.shape[1]:
            t = t.contiguous().clone()
        keep.append(t)
        return t.data_ptr(), t.stride(0), 0

    keep = []
    xp, xs, xf = operand(xq, _native.FP8_GEMM_X_TILED)
    wp, ws, wf = operand(wq, _native.FP8_GEMM_W_TILED)
    y = torch.empty((m, n), dtype=out_dtype, device=xq.device)
    a = _native.DanFp8GemmArgs()
    a.abi_version = _native.FP8_ABI_VERSION
    a.out_dtype = _DTYPES[out_dtype]
    a.m, a.n, a.k, a.flags = m, n, k, flags | xf | wf
    a.xq, a.xq_stride, a.x_scale = xp, xs, sa.data_ptr()
    a.wq, a.wq_stride, a.w_scale = wp, ws, sb.data_ptr()
    a.bias = bias.data_ptr() if bias is not None else None
    a.y, a.y_stride = y.data_ptr(), y.stride(0)
    _native.fp8_gemm(a, torch.cuda.current_stream(y.device).cuda_stream)
    return y


def supported(device=None):
    """gfx950 (OCP e4m3 matrix cores)."""
    if not torch.cuda.is_available():
        return False
    return "gfx950" in torch.cuda.get_device_properties(device).gcnArchName


class FP8Linear(nn.Module):
    """dan/quant.py:23-42 on gfx950: e4m3 weight [out, in] with its scale
    ([1, out] rowwise, [1, 1] per tensor), activations quantized per call."""

    def __init__(self, linear, rowwise=True):
        super().__init__()
        w = linear.weight.detach()
        self.out_features, self.in_features = w.shape
        wq, scale = fp8_quantize(w, E4M3_MAX, rowwise)
        self.weight = nn.Parameter(wq, requires_grad=False)  # [out, in], dan's layout (state dicts)
        self.register_buffer("weight_scale", scale.reshape(1, -1) if rowwise else scale)  # [1, out] or [1, 1]
        self.bias = linear.bias
        self.rowwise = rowwise
        self.out_dtype = w.dtype
        # the same codes in the GEMM's tiled layout, rebuilt if `weight` changes
        self._tiled = fp8_quantize(w, E4M3_MAX, rowwise, tiled=True)[0]
        self._tiled_of = self._weight_key()

    def _weight_key(self):
        return (self.weight.data_ptr(), self.weight._version)

    def tiled_weight(self):
        if self._tiled_of != self._weight_key():
            self._tiled, self._tiled_of = tile_codes(self.weight.detach()), self._weight_key()
        return self._tiled

    def forward(self, x):
        shape = x.shape
        xq, scale = fp8_quantize(x.reshape(-1, shape[-1]), E4M3_MAX, self.rowwise, tiled=True)
        y = fp8_gemm(xq, scale, self.tiled_weight(), self.weight_scale, self.bias, self.out_dtype)
        return y.reshape(*shape[:-1], self.out_features)


def quantize_fp8(model, min_features=16, rowwise=True):
    """Replace the decoder's nn.Linear modules with FP8Linear in place
    (dan/quant.py:60-73; rowwise scaling is fast on gfx950, so it is the
    default)."""
    device = next(model.parameters()).device
    if not supported(device):
        raise RuntimeError("FP8 linears need a gfx950 GPU (OCP e4m3 matrix cores)")
    for layer in model.model.layers:
        for mod in list(layer.modules()):
            for name, child in list(mod.named_children()):
                if isinstance(child, nn.Linear) and min(child.in_features, child.out_features) >= min_features \
                        and child.in_features % 16 == 0 and child.out_features % 16 == 0:
                    setattr(mod, name, FP8Linear(child, rowwise))
    torch.cuda.empty_cache()
    return model
