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
- ``delta_gates``        dan/fused.py:80-82
- ``gated_rms_norm``     dan/fused.py:52-56
- ``silu_conv``          the causal depthwise conv + silu of one sequence
                         (dan/models/qwen3_5.py:216-217: conv1d in the model
                         dtype, then silu), with the sum taken in float64 and
                         rounded once to the model dtype
- ``path_windows``       every token's conv window of virtual rows, from the
                         tree's paths (dan/models/qwen3_5.py:239-259: a
                         segment's sequence is its k1 history rows then its
                         trunk; a branch continues from the trunk's last k1
                         rows). It pins the product's RecurrentLayout.
- ``deltanet_layer``     dan/models/qwen3_5.py:183-210 restated per path: each
                         trunk as one sequence from its initial state and conv
                         history (split at the save boundary, where the cache
                         entry is taken), each branch from the trunk's final
                         state and last k1 conv rows
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


def delta_gates(b, a, a_log, dt_bias):
    return b.sigmoid(), -a_log.float().exp() * F.softplus(a.float() + dt_bias.float())


def gated_rms_norm(x, gate, weight, eps):
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
    y = weight * y.to(x.dtype)
    return (y * F.silu(gate.float())).to(x.dtype)


def silu_conv(seq, weight):
    """seq [K - 1 + n, C] (model dtype), weight [C, K] -> [n, C]: output t is
    silu(sum_j weight[:, j] seq[t + j]), the sum rounded to the model dtype."""
    kk = weight.shape[1]
    n = seq.shape[0] - kk + 1
    s64, w64 = seq.double(), weight.double()
    y = sum(w64[:, j] * s64[j:j + n] for j in range(kk))
    return F.silu(y.to(seq.dtype).float()).to(seq.dtype)


def _virtual(seg, k1, n_rows, hist_base):
    if seg.past:
        base = hist_base[id(seg)]
        hist = list(range(base, base + k1))
    else:
        hist = [n_rows] * k1
    return hist + list(range(seg.start, seg.start + seg.trunk))


def path_windows(segments, k1, n_rows):
    """{packed row: (phase, its k1 + 1 virtual conv rows)} with phase 1 (trunk
    up to the save boundary), 2 (the rest of the trunk) or 3 (a branch).
    Virtual rows: packed rows, the zero row n_rows, then n_rows + 1 + k1 p + r
    for row r of the p-th segment with a cached history."""
    hist_base, p = {}, 0
    for s in segments:
        if s.past:
            hist_base[id(s)] = n_rows + 1 + k1 * p
            p += 1
    win = {}
    for s in segments:
        v = _virtual(s, k1, n_rows, hist_base)
        cut = s.save if 0 < s.save < s.trunk else s.trunk
        for t in range(s.trunk):
            win[s.start + t] = (1 if t < cut else 2, v[t:t + k1 + 1])
        for a, b in s.branches:
            path = v[len(v) - k1:] + list(range(a, b))
            for t in range(b - a):
                win[a + t] = (3, path[t:t + k1 + 1])
    return win


def deltanet_layer(w, x, segments, index, hk, hv, dk, dv, kernel, eps, recurrent=False):
    """One DeltaNet layer over a packed tree batch, path by path. ``w``: dict
    of the module's parameters (in_proj_qkv, in_proj_z, in_proj_b, in_proj_a
    [out, hidden], conv1d [C, 1, K], dt_bias, A_log, norm, out_proj). The
    linears multiply in fp32 and round to x's dtype. Returns (y [N, hidden],
    pre-norm out [N, Hv, Dv] fp32, {segment: (conv tail, state)} saved)."""
    dt = x.dtype

    def lin(name, inp):
        return (inp.float() @ w[name].float().t()).to(dt)

    qkv, z, b, a = lin("in_proj_qkv", x), lin("in_proj_z", x), lin("in_proj_b", x), lin("in_proj_a", x)
    beta, g = delta_gates(b, a, w["A_log"], w["dt_bias"])
    cw = w["conv1d"].reshape(qkv.shape[1], kernel).to(dt)
    k1, kd = kernel - 1, hk * dk
    out = torch.zeros(x.shape[0], hv, dv)
    saved = {}

    def run(conv, rows, state):
        t = conv.shape[0]
        q, k, v = (conv[:, :kd].reshape(t, hk, dk), conv[:, kd:2 * kd].reshape(t, hk, dk),
                   conv[:, 2 * kd:].reshape(t, hv, dv))
        o, f = delta_rule(q, k, v, g[rows], beta[rows], [t], state[None], recurrent=recurrent)
        out[rows] = o
        return f[0]

    for i, s in enumerate(segments):
        if s.past:
            hist, state = s.past[index][0].to(dt), s.past[index][1].float()
        else:
            hist, state = torch.zeros(k1, qkv.shape[1], dtype=dt), torch.zeros(hv, dk, dv)
        seq = torch.cat([hist, qkv[s.start:s.start + s.trunk]])
        conv = silu_conv(seq, cw)
        rows = torch.arange(s.start, s.start + s.trunk)
        cut = s.save if 0 < s.save < s.trunk else s.trunk
        f = run(conv[:cut], rows[:cut], state)
        if s.save:
            saved[i] = (seq[cut:cut + k1].clone(), f.clone())
        if cut < s.trunk:
            f = run(conv[cut:], rows[cut:], f)
        for a0, b0 in s.branches:
            conv_b = silu_conv(torch.cat([seq[seq.shape[0] - k1:], qkv[a0:b0]]), cw)
            run(conv_b, torch.arange(a0, b0), f)
    y = gated_rms_norm(out.to(dt).reshape(-1, dv), z.reshape(-1, dv), w["norm"].to(dt), eps)
    return lin("out_proj", y.reshape(x.shape[0], -1)), out, saved
