"""Pins the front-end oracle (oracle/front.py) on the CPU: closed forms of
rotate-half, invariants of the norms, an fp64 restatement, and planted
mistakes that those checks catch. The reference's own tests cover these ops
only through model-level parity with checkpoints this build cannot load."""
import math

import pytest
import torch

from oracle import front as F

BF16 = torch.bfloat16


def _inputs(n=37, h=3, d=128, r=128, dtype=BF16, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, h, d, generator=g).to(dtype)
    pos = torch.arange(n, dtype=torch.float32) * 3 + 5
    inv = 1.0 / (10000.0 ** (torch.arange(0, r, 2, dtype=torch.float64) / r)).float()
    ang = pos[:, None] * inv[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    return x, ang.cos().to(dtype), ang.sin().to(dtype)


def _ulps(a, b):
    """|a - b| in units of the bf16 spacing at b (b float64)."""
    spacing = torch.where(b.abs() > 0, 2.0 ** (torch.floor(torch.log2(b.abs())) - 7), torch.full_like(b, 2.0 ** -133))
    return ((a.double() - b).abs() / spacing)


def _bound(x, c, s, w, norm):
    """Error bound of the eager chain against fp64: each op rounds to bf16
    (unit roundoff 2^-8): up to two roundings in the norm, then x*cos, rot*sin
    and their sum -- so the bound scales with the magnitudes of both terms,
    which matters where they nearly cancel."""
    u = 2.0 ** -8
    n = F.front_bruteforce(x, None, None, w, 1e-6, norm)
    if c is None:
        return 2 * u * n.abs() + 1e-30
    r = c.shape[-1]
    nh = n[..., :r]
    partner = torch.cat((nh[..., r // 2:], nh[..., :r // 2]), -1).abs()
    t1 = nh.abs() * c.double().abs()[:, None]
    t2 = partner * s.double().abs()[:, None]
    out = torch.cat((3 * u * (t1 + t2) + u * (t1 + t2), 2 * u * n[..., r:].abs()), -1)
    return out + 1e-30


def test_rotation_identity_and_quarter_turn():
    x, c, s = _inputs()
    one, zero = torch.ones_like(c), torch.zeros_like(s)
    assert torch.equal(F.rotate(x, one[:, None], zero[:, None]), x)
    # two quarter turns (cos 0, sin 1) negate every element
    twice = F.rotate(F.rotate(x, zero[:, None], one[:, None]), zero[:, None], one[:, None])
    assert torch.equal(twice, -x)
    # partial: the first R dims turn, the rest pass through untouched
    y = F.rotate_partial(x, zero[:, :64], one[:, :64])
    assert torch.equal(y[..., 64:], x[..., 64:])
    assert torch.equal(y[..., :32], -x[..., 32:64]) and torch.equal(y[..., 32:64], x[..., :32])


def test_position_zero_is_identity():
    x, c, s = _inputs()
    ang = torch.zeros(1, 128)
    y = F.rotate(x[:1], ang.cos().to(BF16)[:, None], ang.sin().to(BF16)[:, None])
    assert torch.equal(y, x[:1])


@pytest.mark.parametrize("norm", [None, "rms", "zero_centered"])
@pytest.mark.parametrize("r", [128, 64, 0])
def test_front_matches_fp64_restatement(norm, r):
    x, c, s = _inputs(r=max(r, 16))
    if r == 0:
        c = s = None
    else:
        c, s = c[:, :r], s[:, :r]
    w = (torch.randn(128, generator=torch.Generator().manual_seed(1)) * 0.3 + (1.0 if norm == "rms" else 0.0)).to(BF16)
    q, _, _, _ = F.front(x, x[:, :1], x[:, :1], c, s, w, w, 1e-6, norm)
    ref = F.front_bruteforce(x, c, s, w, 1e-6, norm).transpose(0, 1)
    err = (q.double() - ref).abs()
    assert err.max().item() <= _bound(x, c, s, w, norm).transpose(0, 1).max().item() * 4  # sanity
    assert (err <= _bound(x, c, s, w, norm).transpose(0, 1)).all()
    # and most elements are within one bf16 spacing of the unrounded result
    assert (_ulps(q, ref) <= 1.0).float().mean().item() > 0.75


def test_norm_invariants():
    x, _, _ = _inputs()
    one = torch.ones(128, dtype=BF16)
    y = F.rms_norm(x, one, 1e-6).double()
    rms = y.pow(2).mean(-1).sqrt()
    assert (rms - 1).abs().max().item() < 1e-2
    # zero-centered with w = 0 is the Llama form with w = 1, bit for bit
    assert torch.equal(F.rms_norm_zero_centered(x, torch.zeros(128, dtype=BF16), 1e-6), y.to(BF16))
    # a constant vector normalizes to ones (sign kept)
    cst = torch.full((1, 1, 128), -3.0, dtype=BF16)
    assert torch.equal(F.rms_norm(cst, one, 0.0), torch.full_like(cst, -1.0))


def test_rotation_keeps_pair_norms():
    x, c, s = _inputs()
    y = F.rotate(x, c[:, None], s[:, None]).double()
    xd = x.double()
    before = xd[..., :64] ** 2 + xd[..., 64:] ** 2
    after = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert ((after - before).abs() <= 0.03 * before + 1e-3).all()


def test_saved_rows_are_k_and_v_rows():
    x, c, s = _inputs(n=40, h=2)
    v = x.flip(0).contiguous()
    q, k, vt, saved = F.front(x, x, v, c, s, None, None, 1e-6, None, saves=[(3, 10), (20, 5)])
    assert torch.equal(saved[0][0], k[:, 3:13]) and torch.equal(saved[1][1], vt[:, 20:25])
    assert saved[0][0].is_contiguous()


@pytest.mark.parametrize("mistake", ["sign", "no_eps_scale", "half_swap"])
def test_planted_mistakes_are_caught(mistake, monkeypatch):
    x, c, s = _inputs()
    w = torch.ones(128, dtype=BF16)
    ref = F.front_bruteforce(x, c, s, w, 1e-6, "rms").transpose(0, 1)
    if mistake == "sign":
        monkeypatch.setattr(F, "_half_turn", lambda t: torch.cat((t.chunk(2, -1)[1], -t.chunk(2, -1)[0]), -1))
    elif mistake == "half_swap":
        monkeypatch.setattr(F, "_half_turn", lambda t: torch.cat((-t.chunk(2, -1)[0], t.chunk(2, -1)[1]), -1))
    else:
        monkeypatch.setattr(F, "rms_norm", lambda t, wt, eps: wt * (t.float() / t.float().abs().max()).to(t.dtype))
    q, _, _, _ = F.front(x, x[:, :1], x[:, :1], c, s, w, w, 1e-6, "rms")
    assert not (( q.double() - ref).abs() <= _bound(x, c, s, w, "rms").transpose(0, 1)).all()
