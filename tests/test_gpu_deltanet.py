"""The gfx950 gated delta rule (dan_amd.deltanet.delta_rule -> dan_gdn_fwd)
against the float64 token-by-token oracle (oracle/deltanet.py), which the
CPU tests pin against the restated chunked form and closed forms.

Bars (fp32 state, outputs rounded to the model dtype):
- outputs within 2^-8 of |reference| + 2e-3 (bf16; 2^-11 and 5e-4 for fp16);
- final states within 1e-4 + 1e-4 |reference|;
- token form: splitting a run into two calls, the second from the first's
  final state, is bit-identical to one call (the kernel's arithmetic per
  token does not depend on where a run starts); chunked form: the split
  moves the chunk boundaries, and both results stay within the bars above;
- the tree phases (trunk part 1, part 2 from its states, branches from the
  trunk's final state) equal the oracle run over each root-to-leaf path."""
import functools
import sys

import numpy as np
import pytest
import torch

from dan_amd.deltanet import delta_rule
from oracle import deltanet as OD

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def inputs(lengths, hk, hv, dv, dtype, gpu, seed):
    g = torch.Generator().manual_seed(seed)
    n = sum(lengths)
    q = torch.randn(n, hk, 128, generator=g).to(dtype)
    k = torch.randn(n, hk, 128, generator=g).to(dtype)
    v = torch.randn(n, hv, dv, generator=g).to(dtype)
    gg = -(torch.rand(n, hv, generator=g) * 0.3 + 0.01)
    b = torch.rand(n, hv, generator=g)
    st = torch.randn(len(lengths), hv, 128, dv, generator=g) * 0.1
    return [x.to(gpu) for x in (q, k, v, gg, b, st)]


def check(out, fin, ref_o, ref_f, dtype):
    rel, ab = (2.0 ** -8, 2e-3) if dtype == torch.bfloat16 else (2.0 ** -11, 5e-4)
    eo = (out.cpu().double() - ref_o.double()).abs()
    ef = (fin.cpu().double() - ref_f.double()).abs()
    say(f"  max |out - ref| {eo.max().item():.3e}, max |state - ref| {ef.max().item():.3e}")
    assert (eo <= rel * ref_o.double().abs() + ab).all()
    assert (ef <= 1e-4 + 1e-4 * ref_f.double().abs()).all()


@pytest.mark.parametrize("form", ["token", "chunk"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hk,hv,dv", [(2, 2, 128), (2, 4, 128), (1, 3, 64), (1, 2, 256)])
def test_delta_rule_matches_oracle(gpu, form, dtype, hk, hv, dv):
    lengths = [5, 0, 1, 300, 64, 17, 129]
    say(f"delta rule {form} {dtype} Hk {hk} Hv {hv} Dv {dv} runs {lengths}")
    q, k, v, g, b, st = inputs(lengths, hk, hv, dv, dtype, gpu, seed=hk * 10 + hv + dv)
    out, fin = delta_rule(q, k, v, g, b, lengths, st, form=form)
    torch.cuda.synchronize()
    ref_o, ref_f = OD.delta_rule(*(x.cpu() for x in (q, k, v, g, b)), lengths, st.cpu(), recurrent=True)
    check(out, fin, ref_o, ref_f, dtype)
    assert torch.equal(fin[1], st[1])  # empty run: state unchanged


def test_split_run_is_bit_identical(gpu):
    say("delta rule, token form: one run of 400 tokens vs two calls (150 + 250)")
    q, k, v, g, b, st = inputs([400], 2, 2, 128, torch.bfloat16, gpu, seed=1)
    out, fin = delta_rule(q, k, v, g, b, [400], st, form="token")
    o1, f1 = delta_rule(q[:150], k[:150], v[:150], g[:150], b[:150], [150], st, form="token")
    o2, f2 = delta_rule(q[150:], k[150:], v[150:], g[150:], b[150:], [250], f1, form="token")
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([o1, o2]), out) and torch.equal(f2, fin)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lengths", [[600, 1, 0, 700, 65], [40, 3, 64, 100, 17, 1]])
def test_chunk_form_scan_variants(gpu, lengths, dtype):
    """fp16 inputs: calls whose runs average more than 256 tokens take the
    fp32 scan's long-run build (16 state columns per work group), others its
    short-run one (32 columns; DAN_GDN_SHORT_RUN). bf16 inputs take the
    bf16-pair scan either way. All against the recurrence, with ragged and
    empty runs and GQA."""
    say(f"delta rule, chunked form {dtype}: runs {lengths} (mean {sum(lengths) / len(lengths):.0f})")
    q, k, v, g, b, st = inputs(lengths, 1, 2, 128, dtype, gpu, seed=11)
    out, fin = delta_rule(q, k, v, g, b, lengths, st, form="chunk")
    torch.cuda.synchronize()
    ref_o, ref_f = OD.delta_rule(*(x.cpu() for x in (q, k, v, g, b)), lengths, st.cpu(), recurrent=True)
    check(out, fin, ref_o, ref_f, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_chunk_scan_variants_bit_identical(gpu, dtype):
    """Two runs of 300 tokens average 300 (fp16: the fp32 scan's long-run
    build, 16 columns per work group); with two empty runs appended they
    average 150 (its short-run build, 32 columns). Both builds add the same
    products in the same order, so outputs and final states are
    bit-identical. bf16 (one scan for both) must not depend on empty runs
    either."""
    say(f"delta rule, chunked form {dtype}: long-run vs short-run scan on the same runs")
    q, k, v, g, b, st = inputs([300, 300], 2, 2, 128, dtype, gpu, seed=5)
    o8, f8 = delta_rule(q, k, v, g, b, [300, 300], st, form="chunk")
    st4 = torch.cat([st, torch.zeros_like(st)])
    o4, f4 = delta_rule(q, k, v, g, b, [300, 300, 0, 0], st4, form="chunk")
    torch.cuda.synchronize()
    assert torch.equal(o8, o4) and torch.equal(f8, f4[:2])


@pytest.mark.parametrize("form", ["token", "chunk"])
def test_repeated_keys(gpu, form):
    """Every key one of two vectors, beta = 1 and no decay: I + L is as far
    from the identity as it gets (its off-diagonal entries are +-1 and 1), and
    the chunked form's triangular inverse must still follow the recurrence."""
    say(f"delta rule {form}: repeated keys, beta 1, no decay")
    lengths = [200, 70]
    q, k, v, g, b, st = inputs(lengths, 1, 2, 128, torch.bfloat16, gpu, seed=9)
    k = k[:2].repeat((sum(lengths) + 1) // 2, 1, 1)[:sum(lengths)].contiguous()
    g = torch.zeros_like(g)
    b = torch.ones_like(b)
    out, fin = delta_rule(q, k, v, g, b, lengths, st, form=form)
    torch.cuda.synchronize()
    ref_o, ref_f = OD.delta_rule(*(x.cpu() for x in (q, k, v, g, b)), lengths, st.cpu(), recurrent=True)
    check(out, fin, ref_o, ref_f, torch.bfloat16)


def test_chunk_form_split_run(gpu):
    say("delta rule, chunked form: one run of 400 tokens vs two calls (150 + 250)")
    q, k, v, g, b, st = inputs([400], 2, 2, 128, torch.bfloat16, gpu, seed=1)
    out, fin = delta_rule(q, k, v, g, b, [400], st, form="chunk")
    o1, f1 = delta_rule(q[:150], k[:150], v[:150], g[:150], b[:150], [150], st, form="chunk")
    o2, f2 = delta_rule(q[150:], k[150:], v[150:], g[150:], b[150:], [250], f1, form="chunk")
    torch.cuda.synchronize()
    ref_o, ref_f = OD.delta_rule(*(x.cpu() for x in (q, k, v, g, b)), [400], st.cpu(), recurrent=True)
    check(out, fin, ref_o, ref_f, torch.bfloat16)
    check(torch.cat([o1, o2]), f2, ref_o, ref_f, torch.bfloat16)


@pytest.mark.parametrize("form", ["token", "chunk"])
def test_strong_decay(gpu, form):
    """Gates down to -8 per token: within a chunk exp(G) underflows to 0 and
    the state forgets; both forms follow the recurrence."""
    say(f"delta rule {form}: strong decay")
    q, k, v, g, b, st = inputs([3, 250], 1, 2, 128, torch.bfloat16, gpu, seed=7)
    g = g * 25.0
    out, fin = delta_rule(q, k, v, g, b, [3, 250], st, form=form)
    torch.cuda.synchronize()
    ref_o, ref_f = OD.delta_rule(*(x.cpu() for x in (q, k, v, g, b)), [3, 250], st.cpu(), recurrent=True)
    check(out, fin, ref_o, ref_f, torch.bfloat16)


def test_tree_phases_equal_paths(gpu):
    """Trunk of 200 tokens saved at 120 (two parts), two branches of 30 and 7
    tokens: phase calls as dan/models/qwen3_5.py:198-210 makes them."""
    say("delta rule: tree phases vs root-to-leaf paths")
    trunk, cut, br = 200, 120, [30, 7]
    n = trunk + sum(br)
    q, k, v, g, b, st = inputs([n], 2, 2, 128, torch.bfloat16, gpu, seed=4)
    o = torch.empty(n, 2, 128, dtype=torch.bfloat16, device=gpu)
    o[:cut], f1 = delta_rule(q[:cut], k[:cut], v[:cut], g[:cut], b[:cut], [cut], st)
    o[cut:trunk], f2 = delta_rule(q[cut:trunk], k[cut:trunk], v[cut:trunk], g[cut:trunk], b[cut:trunk], [trunk - cut], f1)
    rows = slice(trunk, n)
    ob, fb = delta_rule(q[rows], k[rows], v[rows], g[rows], b[rows], br, f2.expand(len(br), -1, -1, -1).contiguous())
    o[rows] = ob
    torch.cuda.synchronize()
    c = [x.cpu() for x in (q, k, v, g, b)]
    at = trunk
    for i, nb in enumerate(br):
        idx = torch.cat([torch.arange(trunk), torch.arange(at, at + nb)])
        ref_o, ref_f = OD.delta_rule(*(x[idx] for x in c), [trunk + nb], st.cpu(), recurrent=True)
        check(torch.cat([o[:trunk], o[at:at + nb]]), fb[i:i + 1], ref_o, ref_f, torch.bfloat16)
        at += nb


def test_errors(gpu):
    q, k, v, g, b, st = inputs([4], 1, 1, 128, torch.bfloat16, gpu, seed=0)
    with pytest.raises(RuntimeError):
        delta_rule(q.cpu(), k.cpu(), v.cpu(), g.cpu(), b.cpu(), [4], st.cpu())
    with pytest.raises(ValueError):
        delta_rule(q, k, v, g, b, [3], st)
    with pytest.raises(ValueError):
        delta_rule(q.float(), k.float(), v.float(), g, b, [4], st)
    with pytest.raises(ValueError):
        delta_rule(q, k, v, g, b, [4], st, form="chunked")
    q2, k2, v2, g2, b2, st2 = inputs([4], 1, 1, 40, torch.bfloat16, gpu, seed=0)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        delta_rule(q2, k2, v2, g2, b2, [4], st2, form="chunk")


@functools.lru_cache(maxsize=1)
def _c3_case():
    """The c3 tree's DeltaNet inputs (CPU) and the oracle's float64 token
    recurrence over them: trunk phase, then branch phase from its finals."""
    from dan_amd import workloads

    w = workloads.config3(0, device="cpu")
    trunks = [(s.start, s.trunk) for s in w.segments]
    branches = [(a, b - a, i) for i, s in enumerate(w.segments) for a, b in s.branches]
    g = torch.Generator().manual_seed(21)
    n, h, d = w.num_tokens, 16, 128
    q = torch.randn(n, h, d, generator=g).bfloat16()
    k = torch.randn(n, h, d, generator=g).bfloat16()
    v = torch.randn(n, h, d, generator=g).bfloat16()
    gg = -(torch.rand(n, h, generator=g) * 0.1)
    b = torch.rand(n, h, generator=g)
    init = torch.randn(len(trunks), h, d, d, generator=g) * 0.05
    trow = torch.cat([torch.arange(a, a + t) for a, t in trunks])
    brow = torch.cat([torch.arange(a, a + m) for a, m, _ in branches])
    bseg = torch.tensor([i for _, _, i in branches])
    tl, bl = [t for _, t in trunks], [m for _, m, _ in branches]
    torch.set_num_threads(8)
    rt = OD.delta_rule(*(x[trow] for x in (q, k, v, gg, b)), tl, init, recurrent=True)
    rb = OD.delta_rule(*(x[brow] for x in (q, k, v, gg, b)), bl, rt[1].index_select(0, bseg), recurrent=True)
    return (q, k, v, gg, b), init, trow, brow, bseg, tl, bl, rt, rb


@pytest.mark.parametrize("form", ["token", "chunk"])
def test_c3_tree_phases_match_oracle(gpu, form):
    """The c3 tree at full size (5 trunks up to 1843 tokens, 45 branches,
    8192 tokens, 16/16 heads of 128): the trunk phase from random states,
    then the branch phase from the trunk finals, against the oracle's
    float64 token recurrence on the same inputs, with the bf16 bars of the
    small cases."""
    say(f"delta rule c3 ({form}): oracle")
    x, init, trow, brow, bseg, tl, bl, (rt_o, rt_f), (rb_o, rb_f) = _c3_case()
    say(f"delta rule c3 ({form}): {len(tl)} trunks (longest {max(tl)}), {len(bl)} branches")
    dv = [t.to(gpu) for t in x]
    ot, ft = delta_rule(*(t[trow.to(gpu)] for t in dv), tl, init.to(gpu), form=form)
    ob, fb = delta_rule(*(t[brow.to(gpu)] for t in dv), bl, ft.index_select(0, bseg.to(gpu)), form=form)
    torch.cuda.synchronize()
    check(ot, ft, rt_o, rt_f, torch.bfloat16)
    check(ob, fb, rb_o, rb_f, torch.bfloat16)


@pytest.mark.parametrize("form", ["token", "chunk"])
def test_state_index_equals_gathered_states(gpu, form):
    """Runs that start from states[state_index[r]] (the phase gather of
    dan/models/qwen3_5.py:204 and :211 done in the kernels' state load) give
    bit-identical outputs and final states to a call on the gathered states;
    indices outside [0, S) are clamped to the nearest entry."""
    say(f"delta rule {form}: state_index against gathered states")
    lengths = [70, 5, 0, 130, 33]
    q, k, v, g, b, _ = inputs(lengths, 2, 4, 128, torch.bfloat16, gpu, seed=21)
    gen = torch.Generator().manual_seed(22)
    pool = (torch.randn(3, 4, 128, 128, generator=gen) * 0.05).to(gpu)
    idx = torch.tensor([2, 0, 2, -1, 5], dtype=torch.int64)
    want_idx = idx.clamp(0, 2)
    o1, f1 = delta_rule(q, k, v, g, b, lengths, pool, form=form, state_index=idx.to(gpu))
    o2, f2 = delta_rule(q, k, v, g, b, lengths, pool.index_select(0, want_idx.to(gpu)), form=form)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(f1, f2)
