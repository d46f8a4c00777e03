"""The gfx950 FP8 linear path (dan_amd.quant -> dan_fp8_quantize, then
dan_fp8_gemm) against the CPU oracle (oracle/quant.py) and against dan's own
formulation (torch._scaled_mm, hipBLASLt) on the same GPU.

Bars:
- the quantizer's e4m3 codes and fp32 scales are bit-identical to the
  oracle's (dan/fused.py:85-91) for bf16, fp16 and fp32 inputs, rowwise and
  per tensor, contiguous and strided rows;
- FP8Linear's output is bit-identical to the package's GEMM (dan_fp8_gemm)
  on the oracle's quantized operands, which the quantizer matches bit for bit
  (torch's eager GPU ops are not the reference here: they divide by the
  scalar 448 through a reciprocal, so their scale can differ from dan's CPU
  result in the last bit);
- against the float64 product of the quantized operands, every output is
  within half a bf16 spacing of the result and half of the product before
  the bias (the GEMM may round there too), plus (K + 3) 2^-24 of the sum of
  |terms| (fp32 accumulation of K products, two scale multiplies, the bias
  add), plus the oracle's bound on the e4m3 matrix core's in-group
  truncation (oracle/quant.py mfma_truncation_bound; the model is pinned in
  tests/test_gpu_fp8_gemm.py); dan's own GEMM call (_scaled_mm) on the same
  operands meets the same bar."""
import sys

import numpy as np
import pytest
import torch
from torch import nn

from dan_amd import quant as DQ
from oracle import quant as OQ

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def check_quant(x, rowwise):
    xq, s = DQ.fp8_quantize(x, rowwise=rowwise)
    torch.cuda.synchronize()
    rq, rs = OQ.fp8_quantize(x.cpu(), rowwise)
    same = (xq.cpu().view(torch.uint8) == rq.view(torch.uint8)).float().mean().item()
    say(f"  codes identical {same * 100:.4f} %, scales identical {torch.equal(s.cpu(), rs)}")
    assert torch.equal(s.cpu(), rs)
    assert torch.equal(xq.cpu().view(torch.uint8), rq.view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rowwise", [True, False])
def test_quantize_bit_exact(gpu, dtype, rowwise):
    g = torch.Generator().manual_seed(7)
    say(f"fp8 quantize {dtype}, {'rowwise' if rowwise else 'per tensor'}")
    for m, k, scale in ((1, 16, 1.0), (33, 48, 0.01), (512, 4096, 3.0), (64, 14336, 1e-3)):
        x = (torch.randn(m, k, generator=g) * scale).to(dtype)
        x[0, :5] = torch.tensor([0.0, -0.0, 1e-6, -1e-6, 65.0]).to(dtype)  # zeros and tiny values
        check_quant(x.to(gpu), rowwise)


def test_quantize_strided_rows_and_zero_rows(gpu):
    say("fp8 quantize: strided rows, an all-zero row")
    big = torch.randn(40, 128, dtype=torch.bfloat16, device=gpu)
    big[3] = 0
    check_quant(big[:, 32:96], True)  # row stride 128, 64 columns
    check_quant(big[::2, :64], False)


def test_quantize_propagates_nan(gpu):
    """A NaN in a row makes that row's scale NaN and all its codes NaN, as
    dan's formula does on the CPU (torch's amax and clamp keep NaN,
    dan/fused.py:88); per tensor, one NaN makes every code NaN. Other rows
    keep the oracle's codes and scales bit for bit."""
    say("fp8 quantize: NaN rows")
    g = torch.Generator().manual_seed(11)
    for dtype in (torch.bfloat16, torch.float32):
        for k in (48, 4096, 20480):  # register-resident rows and the two-pass path
            x = torch.randn(6, k, generator=g).to(dtype)
            x[2, 5] = float("nan")
            x[4, k - 1] = float("nan")
            for rowwise in (True, False):
                xq, s = DQ.fp8_quantize(x.to(gpu), rowwise=rowwise)
                torch.cuda.synchronize()
                rq, rs = OQ.fp8_quantize(x, rowwise)
                got_nan = (xq.cpu().view(torch.uint8) & 0x7F) == 0x7F
                want_nan = (rq.view(torch.uint8) & 0x7F) == 0x7F
                assert torch.equal(got_nan, want_nan), (dtype, k, rowwise)
                assert torch.equal(torch.isnan(s.cpu()), torch.isnan(rs))
                ok = ~want_nan
                assert torch.equal(xq.cpu().view(torch.uint8)[ok], rq.view(torch.uint8)[ok])
                fin = ~torch.isnan(rs)
                assert torch.equal(s.cpu()[fin], rs[fin])


def test_fp8_linear_equals_dan_formulation_and_oracle(gpu):
    g = torch.Generator().manual_seed(3)
    for rowwise in (True, False):
        for m, n, k in ((16, 32, 64), (300, 512, 1024), (2048, 1024, 4096)):
            say(f"FP8Linear {'rowwise' if rowwise else 'per tensor'} M {m} N {n} K {k}")
            lin = nn.Linear(k, n, bias=True).to(torch.bfloat16)
            with torch.no_grad():
                lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
                lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
            lin = lin.to(gpu)
            f = DQ.FP8Linear(lin, rowwise=rowwise)
            x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(gpu)
            y = f(x)
            # the oracle's operands (dan/fused.py:85-91, dan/quant.py:27-31) through dan's GEMM call
            xq, sx = OQ.fp8_quantize(x.cpu(), rowwise)
            wq, sw = OQ.fp8_quantize(lin.weight.detach().cpu(), rowwise)
            sw = sw.reshape(1, -1) if rowwise else sw
            same = DQ.fp8_gemm(xq.to(gpu), sx.to(gpu), wq.to(gpu), sw.to(gpu), lin.bias, torch.bfloat16)
            lib = torch._scaled_mm(xq.to(gpu), wq.to(gpu).t(), scale_a=sx.to(gpu), scale_b=sw.to(gpu), bias=lin.bias,
                                   out_dtype=torch.bfloat16)
            torch.cuda.synchronize()
            assert torch.equal(f.weight.cpu().view(torch.uint8), wq.view(torch.uint8))
            assert torch.equal(f.weight_scale.cpu(), sw)
            assert torch.equal(y, same), "same operands, same GEMM"
            exact, mag = OQ.fp8_linear(xq, sx, wq, sw, lin.bias.cpu())
            trunc = OQ.mfma_truncation_bound(xq, sx, wq, sw)

            def spacing(v):  # bf16 spacing at |v|
                return 2.0 ** (torch.floor(torch.log2(v.abs().clamp(min=2.0 ** -126))) - 7)

            for name, out in (("dan_fp8_gemm", y), ("torch._scaled_mm", lib)):
                yd = out.cpu().double()
                # the result may be rounded once before the bias is added and once after (in the next binade)
                half = (spacing(torch.maximum(exact.abs(), yd.abs())) + spacing(exact - lin.bias.cpu().double())) / 2
                err = (yd - exact).abs()
                acc = mag * (k + 3) * 2.0 ** -24 + trunc  # fp32 adds, scale multiplies, bias add; in-group truncation
                assert (err <= half + acc).all(), f"{name}: max excess {(err - half - acc).max()}"
                say(f"  {name}: max |y - exact| {err.max().item():.3e}")


def test_fp8_linear_retiles_a_changed_weight(gpu):
    """FP8Linear streams a tiled copy of its weight; writing new codes into
    `weight` in place (as a state-dict load does) makes the next forward use
    them."""
    say("FP8Linear: re-tiling after an in-place weight change")
    g = torch.Generator().manual_seed(21)
    lin = nn.Linear(512, 256, bias=False).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(256, 512, generator=g) * 0.02)
    f = DQ.FP8Linear(lin.to(gpu))
    x = torch.randn(300, 512, generator=g).to(torch.bfloat16).to(gpu)
    y0 = f(x)
    other, _ = DQ.fp8_quantize((torch.randn(256, 512, generator=g) * 0.02).to(torch.bfloat16).to(gpu))
    with torch.no_grad():
        f.weight.copy_(other)
    y1 = f(x)
    xq, sx = DQ.fp8_quantize(x)
    want = DQ.fp8_gemm(xq, sx, other, f.weight_scale, None, torch.bfloat16)
    torch.cuda.synchronize()
    assert not torch.equal(y0, y1)
    assert torch.equal(y1, want)


def test_module_replacement_and_errors(gpu):
    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj, self.small, self.odd = nn.Linear(64, 64), nn.Linear(64, 8), nn.Linear(64, 40)

    class Body(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList([Layer(), Layer()])

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.model = Body()

    say("quantize_fp8 module replacement")
    m = Model().to(torch.bfloat16).to(gpu)
    DQ.quantize_fp8(m)
    for layer in m.model.layers:
        assert isinstance(layer.q_proj, DQ.FP8Linear)
        assert isinstance(layer.small, nn.Linear) and not isinstance(layer.small, DQ.FP8Linear)  # < 16 features
        assert isinstance(layer.odd, nn.Linear) and not isinstance(layer.odd, DQ.FP8Linear)  # not a multiple of 16
    with pytest.raises(RuntimeError):
        DQ.fp8_quantize(torch.randn(4, 16))
    with pytest.raises(RuntimeError, match="multiple of 16"):
        DQ.fp8_quantize(torch.randn(4, 24, device=gpu))
