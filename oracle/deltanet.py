"""CPU oracle for the gated delta rule -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg import this module, as the
checker. The product (dan_amd.deltanet) never imports it and has no CPU path.

- ``l2norm``             dan/models/qwen3_5.py:99-100
- ``delta_rule_chunked`` dan/models/qwen3_5.py:103-133 (delta_rule_torch): the
                         chunked form of one sequence, restated with torch CPU
                         ops in fp32 (or float64 with ``dtype``)
- ``delta_rule_recurrent`` the same recurrence token by token, written from
                         its definition: with q, k l2-normalized and q scaled
                         by Dk^-1/2, per head
                             S <- exp(g_t) S
                             S <- S + k_t (beta_t (v_t - S^T k_t))^T
                             o_t = S^T q_t
                         (S: [Dk, Dv]). It pins the chunked form.
- ``delta_rule``         packed sequences from per-sequence states, as
                         dan/models/qwen3_5.py:136-158 does without fla
"""
import torch
import torch.nn.functional as F


def l2norm(x, eps=1e-6):
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def delta_rule_chunked(q, k, v, g, beta, state, chunk=64, dtype=torch.float32):
    """q, k [T, H, Dk]; v [T, H, Dv]; g, beta [T, H]; state [H, Dk, Dv].
    Returns (out [T, H, Dv] in ``dtype``, final state [H, Dk, Dv])."""
    t = q.shape[0]
    q, k, v, beta, g = (x.transpose(0, 1).to(dtype) for x in (q, k, v, beta, g))
    state = state.to(dtype)
    q, k = l2norm(q), l2norm(k)
    q = q * q.shape[-1] ** -0.5
    pad = (chunk - t % chunk) % chunk
    q, k, v = (F.pad(x, (0, 0, 0, pad)) for x in (q, k, v))
    beta, g = F.pad(beta, (0, pad)), F.pad(g, (0, pad))
    h, n = q.shape[0], (t + pad) // chunk
    v_beta, k_beta = v * beta[..., None], k * beta[..., None]
    q, k, k_beta, v_beta = (x.reshape(h, n, chunk, x.shape[-1]) for x in (q, k, k_beta, v_beta))
    g = g.reshape(h, n, chunk).cumsum(-1)
    upper = torch.ones(chunk, chunk, dtype=torch.bool).triu(1)
    decay = (g[..., :, None] - g[..., None, :]).masked_fill(upper, float("-inf")).exp()
    system = (k_beta @ k.transpose(-1, -2)) * decay
    intra = (q @ k.transpose(-1, -2)) * decay
    new_v = torch.linalg.solve_triangular(system, v_beta, upper=False, unitriangular=True)
    k_cum = torch.linalg.solve_triangular(system, k_beta * g.exp()[..., None], upper=False, unitriangular=True)
    q = q * g.exp()[..., None]
    k = k * (g[..., -1:] - g).exp()[..., None]
    chunk_decay = g[..., -1].exp()[..., None, None]
    out = torch.zeros_like(new_v)
    for i in range(n):
        vi = new_v[:, i] - k_cum[:, i] @ state
        out[:, i] = q[:, i] @ state + intra[:, i] @ vi
        state = state * chunk_decay[:, i] + k[:, i].transpose(-1, -2) @ vi
    out = out.reshape(h, -1, out.shape[-1])[:, :t].transpose(0, 1)
    return out, state


def delta_rule_recurrent(q, k, v, g, beta, state, dtype=torch.float64):
    """Token by token (see module docstring); same arguments and returns."""
    q, k = l2norm(q.to(dtype)), l2norm(k.to(dtype))
    q = q * q.shape[-1] ** -0.5
    v, g, beta, s = v.to(dtype), g.to(dtype), beta.to(dtype), state.to(dtype).clone()
    out = torch.empty(v.shape, dtype=dtype)
    for t in range(q.shape[0]):
        s = s * g[t].exp()[:, None, None]
        u = torch.einsum("hk,hkv->hv", k[t], s)
        s = s + k[t][:, :, None] * (beta[t][:, None] * (v[t] - u))[:, None, :]
        out[t] = torch.einsum("hk,hkv->hv", q[t], s)
    return out, s


def repeat_heads(x, rep):
    """[N, Hk, D] -> [N, Hk * rep, D], head h reading key head h // rep
    (dan/attention.py repeat_heads)."""
    return x if rep == 1 else x.repeat_interleave(rep, dim=1)


def delta_rule(q, k, v, g, beta, lengths, states, recurrent=False):
    """Packed sequences: q, k [N, Hk, Dk], v [N, Hv, Dv], g, beta [N, Hv],
    states [R, Hv, Dk, Dv]. Returns (out [N, Hv, Dv] fp32, finals [R, Hv, Dk, Dv])."""
    rep = v.shape[1] // q.shape[1]
    q, k = repeat_heads(q, rep), repeat_heads(k, rep)
    fn = delta_rule_recurrent if recurrent else delta_rule_chunked
    outs, finals, i = [], [], 0
    for n, s in zip(lengths, states):
        o, f = fn(q[i:i + n], k[i:i + n], v[i:i + n], g[i:i + n], beta[i:i + n], s)
        outs.append(o.float())
        finals.append(f.float())
        i += n
    return torch.cat(outs), torch.stack(finals)
