"""The gated delta rule oracle (oracle/deltanet.py) pinned without a GPU.

- The chunked form (a restatement of dan/models/qwen3_5.py:103-133) and the
  token-by-token form written from the recurrence's definition agree to
  float64 rounding on random runs, with and without grouped key heads.
- Closed forms: with beta = 0 nothing is written, so the state only decays
  (S_T = exp(sum g) S_0, o_t = exp(sum_{<=t} g) S_0^T q_t); with g = 0,
  beta = 1 and orthonormal keys the state stores each value exactly
  (o for a query equal to key j is Dk^-1/2 v_j once token j is written).
- Splitting a run into two calls, the second starting from the first's
  final state, gives the single call's output and state (the property the
  tree phases rely on: trunk part 2 and the branches start from trunk
  states).
- A planted mistake (the decay applied after the write) fails the closed
  forms."""
import torch

from oracle import deltanet as D

DT = torch.float64


def rand(t, h, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(t, h, dk, generator=g), torch.randn(t, h, dk, generator=g), torch.randn(t, h, dv, generator=g),
            -torch.rand(t, h, generator=g) * 0.7, torch.rand(t, h, generator=g), torch.randn(h, dk, dv, generator=g) * 0.2)


def test_chunked_equals_recurrent():
    for t, h, dk, dv, seed in ((1, 1, 8, 4, 0), (63, 2, 16, 8, 1), (64, 2, 16, 8, 2), (200, 3, 32, 16, 3)):
        q, k, v, g, b, s = rand(t, h, dk, dv, seed)
        oc, fc = D.delta_rule_chunked(q, k, v, g, b, s, dtype=DT)
        orr, fr = D.delta_rule_recurrent(q, k, v, g, b, s)
        assert (oc - orr).abs().max() < 1e-12 and (fc - fr).abs().max() < 1e-12


def test_packed_runs_with_grouped_key_heads():
    g = torch.Generator().manual_seed(5)
    lengths = [7, 0, 65, 1]
    n, hk, hv, dk, dv = sum(lengths), 2, 4, 16, 8
    q, k = torch.randn(n, hk, dk, generator=g), torch.randn(n, hk, dk, generator=g)
    v, gg, b = torch.randn(n, hv, dv, generator=g), -torch.rand(n, hv, generator=g), torch.rand(n, hv, generator=g)
    st = torch.randn(len(lengths), hv, dk, dv, generator=g) * 0.1
    oc, fc = D.delta_rule(q.double(), k.double(), v.double(), gg.double(), b.double(), lengths, st.double())
    orr, fr = D.delta_rule(q, k, v, gg, b, lengths, st, recurrent=True)
    assert (oc - orr).abs().max() < 1e-6 and (fc - fr).abs().max() < 1e-6
    assert torch.equal(fr[1], st[1].float())  # an empty run keeps its state
    # value head 3 reads key head 1
    o3, _ = D.delta_rule_recurrent(q[:7, 1:2], k[:7, 1:2], v[:7, 3:4], gg[:7, 3:4], b[:7, 3:4], st[0, 3:4])
    assert (o3[:, 0].float() - orr[:7, 3]).abs().max() < 1e-6


def test_closed_form_no_write_only_decays():
    q, k, v, g, _, s = rand(30, 2, 16, 8, 7)
    b = torch.zeros(30, 2)
    o, f = D.delta_rule_recurrent(q, k, v, g, b, s)
    cg = g.double().cumsum(0)
    assert torch.allclose(f, s.double() * cg[-1].exp()[:, None, None], rtol=0, atol=1e-13)
    qn = D.l2norm(q.double()) * 16 ** -0.5
    want = torch.einsum("thk,hkv->thv", qn, s.double()) * cg.exp()[..., None]
    assert torch.allclose(o, want, rtol=0, atol=1e-12)


def test_closed_form_orthonormal_keys_store_values_exactly():
    dk, dv, t = 16, 8, 10
    keys = torch.eye(dk)[:t]  # e_0 .. e_9
    v = torch.randn(t, 1, dv, generator=torch.Generator().manual_seed(9))
    q = keys[torch.tensor([3, 3, 3, 3, 0, 5, 9, 9, 2, 1])]  # query key 3 before and after it is written, ...
    o, f = D.delta_rule_recurrent(q[:, None], keys[:, None], v, torch.zeros(t, 1), torch.ones(t, 1), torch.zeros(1, dk, dv))
    for tt, j in enumerate([3, 3, 3, 3, 0, 5, 9, 9, 2, 1]):
        want = v[j, 0].double() * dk ** -0.5 if j <= tt else torch.zeros(dv, dtype=DT)
        assert torch.allclose(o[tt, 0], want, atol=1e-14), (tt, j)
    assert torch.allclose(f[0][:t], v[:, 0].double(), atol=1e-14) and f[0][t:].abs().max() == 0


def test_split_runs_match_one_run():
    q, k, v, g, b, s = rand(150, 2, 16, 8, 11)
    o, f = D.delta_rule_recurrent(q, k, v, g, b, s)
    o1, f1 = D.delta_rule_recurrent(q[:57], k[:57], v[:57], g[:57], b[:57], s)
    o2, f2 = D.delta_rule_recurrent(q[57:], k[57:], v[57:], g[57:], b[57:], f1)
    assert torch.equal(torch.cat([o1, o2]), o) and torch.equal(f2, f)
    oc1, fc1 = D.delta_rule_chunked(q[:57], k[:57], v[:57], g[:57], b[:57], s, dtype=DT)
    oc2, fc2 = D.delta_rule_chunked(q[57:], k[57:], v[57:], g[57:], b[57:], fc1, dtype=DT)
    assert (torch.cat([oc1, oc2]) - o).abs().max() < 1e-12 and (fc2 - f).abs().max() < 1e-12


def test_planted_decay_after_write_fails():
    q, k, v, g, _, s = rand(12, 1, 8, 4, 13)
    b = torch.ones(12, 1)

    def wrong(q, k, v, g, b, s):  # decay applied after the write
        q, k = D.l2norm(q.double()) * 8 ** -0.5, D.l2norm(k.double())
        s = s.double().clone()
        outs = []
        for t in range(q.shape[0]):
            u = torch.einsum("hk,hkv->hv", k[t], s)
            s = s + k[t][:, :, None] * (b[t].double()[:, None] * (v[t].double() - u))[:, None, :]
            s = s * g[t].double().exp()[:, None, None]
            outs.append(torch.einsum("hk,hkv->hv", q[t], s))
        return torch.stack(outs), s

    o, f = D.delta_rule_recurrent(q, k, v, g, b, s)
    ow, fw = wrong(q, k, v, g, b, s)
    assert (o - ow).abs().max() > 1e-3
