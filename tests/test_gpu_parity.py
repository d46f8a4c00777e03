"""Parity of the gfx950 kernel (through dan_amd.attend -> C ABI) with the CPU
oracle on identical seeded inputs.

Bars: bf16/fp16/fp32 outputs within max-abs 2e-2 of the fp32 oracle; the
label-softmax readout (rms_norm of the read row, seeded label heads,
softmax) within 1e-3 in probability."""
import math
import sys
from dataclasses import replace

import numpy as np
import pytest
import torch

from dan_amd import workloads as W
from dan_amd.attention import Batch, attend, segment
from oracle import tree_attention as O

pytestmark = pytest.mark.gpu

ATOL = 2e-2
READOUT_ATOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def readout_dp(out, ref, segments, width):
    """Max |dp| of the label-softmax readout of two attention outputs."""
    nb = sum(len(s.branches) for s in segments)
    wts = O.readout_weights(nb, width, seed=11)
    pa = O.readout_probs(out, segments, wts)
    pb = O.readout_probs(ref, segments, wts)
    return max(abs(a - b) for x, y in zip(pa, pb) for a, b in zip(x, y))


def check(w, name, atol=ATOL, readout=True, ref=None, readout_atol=READOUT_ATOL):
    """max-abs against the fp32 oracle; readout against the oracle's output
    rounded to the kernel's output dtype. The output tensor has q's dtype (as
    in the reference), and rounding even an exact fp32 result to bf16 moves
    the readout probabilities by up to ~1e-3 against the unrounded oracle, so
    both sides of the readout take that rounding; the figure against the
    unrounded fp32 oracle is reported too."""
    say(f"{name}: N={w.num_tokens} H={w.q.shape[0]} Hkv={w.k.shape[0]} D={w.q.shape[2]} {w.q.dtype} "
        f"segments={len(w.segments)}")
    out = attend(w.q, w.k, w.v, w.segments, w.layer, **w.attend_kwargs)
    torch.cuda.synchronize()
    want_dtype = torch.bfloat16 if w.q.dtype == torch.float8_e4m3fn else w.q.dtype
    assert out.shape == w.q.shape and out.dtype == want_dtype
    if ref is None:
        ref = O.attend_dense(w.q, w.k, w.v, w.segments, w.layer)
    got = out.float().cpu()
    rows = torch.cat([torch.arange(s.start, s.end) for s in w.segments])
    err = (got[:, rows] - ref[:, rows]).abs().max().item()
    dp = dp32 = 0.0
    if readout and any(s.branches for s in w.segments):
        width = w.q.shape[0] * w.q.shape[2]
        dp = readout_dp(out.cpu(), ref.to(out.dtype), w.segments, width)
        dp32 = readout_dp(out.cpu(), ref, w.segments, width)
    say(f"{name}: max-abs {err:.3e}, readout dp {dp:.2e} (vs fp32 oracle output: {dp32:.2e})")
    assert math.isfinite(err) and err <= atol, f"{name}: max-abs {err:.3e} > {atol}"
    assert dp <= readout_atol, f"{name}: readout |dp| {dp:.2e} > {readout_atol}"
    return out, ref


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
def test_config_seed0(gpu, cfg):
    check(W.CONFIGS[cfg](0, device=gpu), f"{cfg} seed 0")


@pytest.mark.parametrize("cfg,seed", [("c2", 1), ("c2", 2), ("c3", 1), ("c3", 2), ("c1", 3)])
def test_config_more_seeds(gpu, cfg, seed):
    check(W.CONFIGS[cfg](seed, device=gpu), f"{cfg} seed {seed}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [128, 64])
def test_reference_differential_shapes(gpu, dtype, head_dim):
    """tests/test_runner.py:44-68 of the reference: h=8, hkv=2, mixed trees with
    per-segment pasts, bf16 and fp16."""
    check(W.runner_shapes(0, device=gpu, dtype=dtype, head_dim=head_dim), f"runner shapes {dtype} D={head_dim}")


def random_batch(rng, h, hkv, d, dtype, device, max_segments=5, long=False):
    structure, pasts = [], []
    for _ in range(int(rng.integers(1, max_segments + 1))):
        trunk = int(rng.integers(0, 700 if long else 150))
        lens = [int(x) for x in rng.integers(1, 100, int(rng.integers(0, 7)))]
        if trunk + sum(lens) == 0:
            trunk = 1
        structure.append((trunk, lens))
        pasts.append(int(rng.integers(1, 300)) if rng.random() < 0.4 else 0)
    return W.build("random", structure, h, hkv, d, dtype, device, rng, std=0.7, per_segment_past=pasts)


@pytest.mark.parametrize("seed", range(12))
def test_random_trees(gpu, seed):
    """Empty trunks, single-token branches, segments without branches,
    per-segment pasts, ragged tiles."""
    rng = np.random.default_rng(100 + seed)
    d = 128 if seed % 3 else 64
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    check(random_batch(rng, 8, 2, d, dtype, gpu, long=seed % 4 == 0), f"random tree seed {seed}")


@pytest.mark.parametrize("h,hkv", [(4, 4), (8, 4), (14, 2), (16, 2), (12, 3)])
def test_head_layouts(gpu, h, hkv):
    """rep = 1, 2, 7 (two head chunks, one idle wave), 8 (two chunks), 4 with 3 kv heads."""
    rng = np.random.default_rng(h * 31 + hkv)
    check(random_batch(rng, h, hkv, 128, torch.bfloat16, gpu), f"heads {h}/{hkv}")


def test_single_tokens_and_tiny_segments(gpu):
    rng = np.random.default_rng(5)
    structure = [(1, []), (0, [1]), (1, [1, 1, 1]), (0, [2, 3]), (65, [1]), (64, [64])]
    w = W.build("tiny", structure, 8, 2, 128, torch.bfloat16, gpu, rng, per_segment_past=[0, 3, 0, 70, 64, 1])
    check(w, "tiny segments")


def _scored_batch(gpu, structure, score_fn, h=8, hkv=2, d=128, seed=0):
    """Inputs whose raw scores q.k follow score_fn(query_token, key_token):
    every key row is unit vector u times a per-key coefficient and every
    query is u times a per-query coefficient, so q.k = a(q) b(k) exactly; v
    is random. Packed one segment after another from ``structure``."""
    rng = np.random.default_rng(seed)
    n = sum(t + sum(ls) for t, ls in structure)
    u = rng.standard_normal(d).astype(np.float32)
    u /= np.linalg.norm(u)
    a, b = score_fn(np.arange(n))
    q = np.broadcast_to((a[:, None, None] * u), (n, h, d)).copy()
    k = np.broadcast_to((b[:, None, None] * u), (n, hkv, d)).copy()
    v = rng.standard_normal((n, hkv, d), dtype=np.float32)
    to = lambda x: torch.from_numpy(x).to(torch.float32).to(gpu).transpose(0, 1)
    segs, start = Batch(), 0
    for trunk, lens in structure:
        ids = W.branch_ids(trunk, lens)
        segs.append(segment(start, ids, None, 0, 0, gpu))
        start += len(ids)
    return W.Workload("scored", to(q), to(k), to(v), segs, 0, {})


# head_dim 256 runs its own step (16 queries per wave, 16x16 products) with its
# own running-max start and per-tile raise: the score-shaped cases run there too.
@pytest.mark.parametrize("d", [128, 256])
def test_running_max_set_by_first_visible_key(gpu, d):
    """Empty trunk, two branches; the second branch's queries share a work
    item with the first branch's tail but see none of key tile 0. All scores
    are near -300 / sqrt(D) * log2 e below zero, so a running max left at 0
    would underflow every probability."""
    w = _scored_batch(gpu, [(0, [80, 70])], lambda t: (np.full(t.shape, -20.0, np.float32),
                                                          np.full(t.shape, 15.0, np.float32) + 0.01 * t), d=d)
    check(w, f"negative scores, first visible key after tile 0, D={d}")


@pytest.mark.parametrize("d", [128, 256])
def test_running_max_raised_by_growing_scores(gpu, d):
    """Scores grow with the key index along a 1000-token trunk, so later
    tiles keep exceeding the running max: the rescale path runs on most
    tiles."""
    w = _scored_batch(gpu, [(1000, [40, 24])], lambda t: (np.full(t.shape, 4.0, np.float32),
                                                          0.1 * t.astype(np.float32)), d=d)
    check(w, f"growing scores, D={d}")


def _as_dtype(w, dtype):
    return W.Workload(f"{w.name}-{dtype}", w.q.to(dtype), w.k.to(dtype), w.v.to(dtype), w.segments, w.layer, {})


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("dtype", ["fp32", "bf16", "e4m3"])
def test_overflowing_units_among_others(gpu, dtype, d):
    """The kernel runs a unit without the per-tile overflow check and runs it
    again with the check when a probability overflowed fp16. Here the first
    segment's scores grow along its 600-token trunk (its units overflow and
    run twice) while the other segments' scores are flat (one pass), so work
    groups mix both kinds and a second pass sits between units whose first
    tiles were prefetched."""
    structure = [(600, [40, 24]), (600, [30]), (300, [20, 20]), (200, [])]
    first = 600 + 64

    def scores(t):
        b = np.where(t < first, 0.1 * t, 0.5).astype(np.float32)
        return np.full(t.shape, 4.0, np.float32), b
    w = _scored_batch(gpu, structure, scores, d=d)
    if dtype == "e4m3":
        _fp8_case(w, f"overflowing units among others (e4m3, D={d})", gpu, vs_original=False)
        return
    check(w if dtype == "fp32" else _as_dtype(w, torch.bfloat16), f"overflowing units among others ({dtype}, D={d})")


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("rise", [15.5, 16.5])
def test_probabilities_near_fp16_limit(gpu, rise, d):
    """Keys 0-63 score 0 and every later key scores `rise` (log2 units) above
    them, so queries past the first tile start from m = 0 and then meet
    p = 2^rise: 2^15.5 fits fp16 (one pass, P up to 46341), 2^16.5 overflows
    it (at head_dim <= 128 the unit runs again with the check, which raises m;
    at 256 the per-tile check raises m on the tile)."""
    raw = rise / (math.log2(math.e) / math.sqrt(d))  # raw q.k giving S * scale * log2(e) = rise

    def scores(t):
        return np.full(t.shape, 4.0, np.float32), np.where(t < 64, 0.0, raw / 4.0).astype(np.float32)
    w = _scored_batch(gpu, [(300, [40, 24])], scores, d=d)
    check(w, f"probabilities near the fp16 limit (rise {rise}, D={d})")


def dequantized(w):
    """An e4m3 workload with q, k, v and every cache entry dequantized to fp32
    (x = xq * scale), for the oracle."""
    m = w.meta
    entries, segs = {}, Batch()
    for s in w.segments:
        past = None
        if s.past:
            past = entries.get(id(s.past))
            if past is None:
                pk, pv, pks, pvs = s.past[w.layer]
                past = entries[id(s.past)] = {w.layer: (O.dequantize(pk, pks), O.dequantize(pv, pvs))}
        segs.append(replace(s, past=past, saved={}, _mask=None))
    return W.Workload(w.name + "-dq", O.dequantize(w.q, m["q_scale"]), O.dequantize(w.k, m["k_scale"]),
                      O.dequantize(w.v, m["v_scale"]), segs, w.layer, {})


def _fp8_case(w_orig, name, gpu, vs_original=True):
    """e4m3 kernel output (1) against the oracle on the dequantized inputs --
    the kernel's own error, held to the bf16 bars (max-abs 2e-2, readout
    1e-3) -- and (2) against the oracle on the original inputs: max-abs 5e-2
    (pre-registered) and readout within 1e-2 of the quantization floor. The
    floor (oracle on dequantized vs oracle on original inputs) is what
    quantizing q, k, v to e4m3 costs before any kernel runs; on config 5 its
    readout |dp| (2.6e-2 at seed 0) already exceeds the pre-registered 1e-2,
    so that bar is applied on top of it."""
    w8 = W.to_e4m3(w_orig)
    ref = O.attend_dense(w_orig.q, w_orig.k, w_orig.v, w_orig.segments, w_orig.layer)
    wd = dequantized(w8)
    ref_dq = O.attend_dense(wd.q, wd.k, wd.v, wd.segments, wd.layer)
    rows = torch.cat([torch.arange(s.start, s.end) for s in w_orig.segments])
    floor = (ref_dq[:, rows] - ref[:, rows]).abs().max().item()
    dpf = 0.0
    if any(s.branches for s in w_orig.segments):
        dpf = readout_dp(ref_dq, ref, w_orig.segments, w_orig.q.shape[0] * w_orig.q.shape[2])
    say(f"{name}: quantization floor (oracle, dequantized vs original inputs): max-abs {floor:.3e}, readout dp {dpf:.2e}")
    check(w8, f"{name} vs oracle on dequantized inputs", atol=ATOL, ref=ref_dq)
    if vs_original:
        check(w8, f"{name} vs oracle on original inputs", atol=5e-2, ref=ref, readout_atol=dpf + 1e-2)


def test_fp8_config5(gpu):
    """Config 5: config 3 quantized per tensor to OCP e4m3."""
    _fp8_case(W.config3(0, device=gpu), "c5 seed 0 (e4m3)", gpu)


@pytest.mark.parametrize("head_dim", [128, 64])
def test_fp8_reference_shapes(gpu, head_dim):
    """The differential shapes with per-segment e4m3 cache entries (12 and 20
    keys: tiles holding both cache and new keys take the k-scale fix-up).
    Held to the oracle on the dequantized inputs only: with N(0,1) inputs and
    rows of a few keys the quantization floor itself is ~0.18 max-abs."""
    _fp8_case(W.runner_shapes(0, device=gpu, dtype=torch.bfloat16, head_dim=head_dim),
              f"e4m3 runner shapes D={head_dim}", gpu, vs_original=False)


def test_fp8_needs_scales(gpu):
    w8 = W.to_e4m3(W.config1(0, device=gpu))
    with pytest.raises(ValueError, match="scale"):
        attend(w8.q, w8.k, w8.v, w8.segments, 0)


def test_fp32_config1_layout(gpu):
    """fp32 in, fp32 out (staged through fp16 for the matrix cores)."""
    out, _ = check(W.config1(1, device=gpu), "c1 seed 1")
    assert out.dtype == torch.float32


def test_output_is_token_major_view(gpu):
    w = W.config2(0, device=gpu)
    say("output layout")
    out = attend(w.q, w.k, w.v, w.segments, 0)
    h, n, d = w.q.shape
    assert out.shape == (h, n, d) and out.stride() == (d, h * d, 1)
    flat = out.transpose(0, 1).reshape(n, h * d)  # the o_proj input of dan/models/llama.py:87
    assert flat.data_ptr() == out.data_ptr()


def test_deterministic(gpu):
    w = W.config3(0, device=gpu)
    say("determinism c3")
    a = attend(w.q, w.k, w.v, w.segments, 0)
    b = attend(w.q, w.k, w.v, w.segments, 0)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_save_side_effect(gpu):
    """dan/attention.py:202-204: saved[layer] holds clones of the first `save` keys/values."""
    w = W.config2(0, device=gpu)
    w.segments[1].save = 50
    say("save side effect")
    attend(w.q, w.k, w.v, w.segments, 3)
    s = w.segments[1]
    sk, sv = s.saved[3]
    assert torch.equal(sk, w.k[:, s.start:s.start + 50]) and torch.equal(sv, w.v[:, s.start:s.start + 50])
    assert sk.data_ptr() != w.k.data_ptr()


def test_misaligned_and_contiguous_inputs(gpu):
    """Views whose rows are not 16-byte aligned take a contiguous copy; fully
    contiguous [H, N, D] inputs work as they are."""
    w = W.config2(1, device=gpu)
    ref = attend(w.q, w.k, w.v, w.segments, 0).float()
    say("misaligned views")
    big = torch.empty(w.q.numel() + 1, dtype=w.q.dtype, device=gpu)
    q_odd = big[1:].view(w.q.shape).copy_(w.q)  # base 2 bytes off
    got = attend(q_odd, w.k.contiguous(), w.v.contiguous(), w.segments, 0).float()
    torch.cuda.synchronize()
    assert (got - ref).abs().max().item() == 0.0


def test_side_stream(gpu):
    """The launch goes to the caller's current stream."""
    w = W.config2(2, device=gpu)
    say("side stream")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = attend(w.q, w.k, w.v, w.segments, 0)
    s.synchronize()
    ref = attend(w.q, w.k, w.v, w.segments, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_plan_is_cached_on_batch(gpu):
    w = W.config2(0, device=gpu)
    say("plan cache")
    attend(w.q, w.k, w.v, w.segments, 0)
    plan = w.segments.tile_plan
    attend(w.q, w.k, w.v, w.segments, 0)
    assert w.segments.tile_plan is plan
    assert 0 in plan.past_tables


def test_errors_are_python_exceptions(gpu):
    w = W.config2(0, device=gpu)
    say("error paths")
    with pytest.raises(NotImplementedError):
        with torch.enable_grad():
            attend(w.q.detach().requires_grad_(), w.k, w.v, w.segments, 0)
    with pytest.raises(ValueError):
        attend(w.q, w.k[:, :10], w.v[:, :10], w.segments, 0)
    bad = Batch([segment(0, [0] * 10 + [1] * 5)])
    bad[0].end = w.num_tokens + 5
    with pytest.raises(ValueError):
        attend(w.q, w.k, w.v, bad, 0)


def test_full_size_invariants(gpu):
    """At the 8192-token budget: outputs are convex combinations of visible
    values (|o| <= max |v| per head group), and permuting whole segments of the
    packed batch permutes the output rows exactly."""
    w = W.config3(0, device=gpu)
    say("full-size invariants c3")
    out = attend(w.q, w.k, w.v, w.segments, 0).float()
    vmax = max(w.v.float().abs().max().item(), w.segments[0].past[0][1].float().abs().max().item())
    assert out.abs().max().item() <= vmax * (1 + 2 ** -7)
    order = list(range(len(w.segments)))[::-1]
    rows, segs, start = [], Batch(), 0
    for i in order:
        s = w.segments[i]
        rows += range(s.start, s.end)
        segs.append(segment(start, s.branch_ids, s.past, 0, s.past_len, str(gpu)))
        start += s.end - s.start
    rows = torch.tensor(rows, device=gpu)
    got = attend(w.q[:, rows], w.k[:, rows], w.v[:, rows], segs, 0).float()
    torch.cuda.synchronize()
    assert torch.equal(got, out[:, rows])


def test_phases_split_equals_one_call(gpu):
    """The V^T copy and the attention launched by two calls (phases 1, 2)
    give the one-call result bit for bit."""
    from dan_amd import _native
    from dan_amd.attention import _attend_fused, workspace_bytes
    w = W.config2(0, device=gpu)
    say("phases split")
    full = attend(w.q, w.k, w.v, w.segments, 0).clone()
    ws = torch.empty(workspace_bytes(w.q, w.k, w.segments), dtype=torch.uint8, device=gpu)
    _attend_fused(w.q, w.k, w.v, w.segments, 0, None, phases=_native.PHASE_PACK, workspace=ws)
    out = _attend_fused(w.q, w.k, w.v, w.segments, 0, None, phases=_native.PHASE_ATTEND, workspace=ws)
    with pytest.raises(ValueError, match="workspace"):
        _attend_fused(w.q, w.k, w.v, w.segments, 0, None, phases=_native.PHASE_ATTEND)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(s.start, s.end) for s in w.segments])
    assert torch.equal(out[:, rows], full[:, rows])


def test_schedule_order_is_invisible(gpu):
    """Units are independent: the planned persistent schedule, one unit per
    work group in natural order, one work group per head group walking all
    of its units, and every list reversed give the same output bit for bit."""
    from dan_amd import _native
    from dan_amd import plan as plan_mod
    from dan_amd.attention import _num_cus, get_plan
    w = W.config3(0, device=gpu)
    say("schedule variants c3")
    h, hkv = w.q.shape[0], w.k.shape[0]
    plan = plan_mod.TilePlan.build(w.segments, w.num_tokens, _native.tile_q(h, hkv), w.q.device)  # host tables
    w.segments.tile_plan = plan
    ref = attend(w.q, w.k, w.v, w.segments, 0).clone()
    assert get_plan(w.segments, w.num_tokens, _native.tile_q(h, hkv), w.q.device) is plan
    groups = _native.head_groups(h, hkv)
    key = (groups, _num_cus(w.q.device))
    planned = plan.schedules[key]
    units = len(plan.work) * groups
    sched, off = plan_mod.schedule(plan.cost, groups, key[1])
    lists = [sched[off[s]:off[s + 1]] for s in range(len(off) - 1)]
    variants = {
        "one unit per work group": [[u] for u in range(units)],
        "one work group per head group": [[u for u in range(units) if u % groups == g] for g in range(groups)],
        "reversed lists": [x[::-1] for x in lists],
    }
    try:
        for name, lst in variants.items():
            say(f"schedule variant: {name}")
            flat = np.array([u for x in lst for u in x], np.int32)
            offs = np.zeros(len(lst) + 1, np.int32)
            offs[1:] = np.cumsum([len(x) for x in lst])
            units = plan_mod.unit_records(plan.segs, plan.work, flat, groups)
            plan.schedules[key] = (plan_mod._upload(units, w.q.device), plan_mod._upload(offs, w.q.device), len(lst))
            out = attend(w.q, w.k, w.v, w.segments, 0)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), name
    finally:
        plan.schedules[key] = planned
