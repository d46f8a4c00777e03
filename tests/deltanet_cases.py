"""Shared DeltaNet layer cases of the CPU and GPU tests: a small head shape,
random weights, a tree batch with a cached prefix, a save boundary and
branches, and its root-to-leaf paths as separate segments."""
import torch

from dan_amd.attention import Batch, segment

HK, HV, DK, DV, KERNEL, HIDDEN, EPS = 2, 4, 128, 64, 4, 64, 1e-6
C = 2 * HK * DK + HV * DV


def weights(seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)

    def r(*shape, s=1.0):
        return (torch.randn(*shape, generator=g) * s).to(dtype)

    return {"in_proj_qkv": r(C, HIDDEN, s=HIDDEN ** -0.5), "in_proj_z": r(HV * DV, HIDDEN, s=HIDDEN ** -0.5),
            "in_proj_b": r(HV, HIDDEN, s=HIDDEN ** -0.5), "in_proj_a": r(HV, HIDDEN, s=HIDDEN ** -0.5),
            "conv1d": r(C, 1, KERNEL, s=0.5), "dt_bias": r(HV, s=0.5), "A_log": r(HV, s=0.5),
            "norm": (1 + r(DV, s=0.1).float()).to(dtype), "out_proj": r(HIDDEN, HV * DV, s=(HV * DV) ** -0.5)}


def tree_batch(seed, with_past=True):
    """Two segments: one after a cached prefix (history + state) with a save
    boundary inside its trunk and three branches, one fresh with two."""
    g = torch.Generator().manual_seed(seed)
    past = {0: ((torch.randn(KERNEL - 1, C, generator=g)).bfloat16(), torch.randn(HV, DK, DV, generator=g) * 0.1)}
    b1 = [0] * 23 + [1] * 6 + [2] * 1 + [3] * 9
    b2 = [0] * 17 + [1] * 5 + [2] * 8
    s1 = segment(0, b1, past=past if with_past else None, save=11, past_len=5)
    s2 = segment(len(b1), b2)
    n = len(b1) + len(b2)
    x = torch.randn(n, HIDDEN, generator=g).bfloat16()
    return Batch([s1, s2]), x


def path_batch(segs, x):
    """Each root-to-leaf path of the tree as its own branch-free segment."""
    rows, out, at = [], [], 0
    for s in segs:
        trunk = list(range(s.start, s.start + s.trunk))
        for a, b in s.branches or [(s.end, s.end)]:
            r = trunk + list(range(a, b))
            out.append((segment(at, [0] * len(r), past=s.past, past_len=s.past_len), r))
            rows += r
            at += len(r)
    return Batch([p for p, _ in out]), x[rows], out
