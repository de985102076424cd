"""CPU oracle of the Gated DeltaNet (GDN) mixer ops -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker / the timed CPU
baseline.  The product path (the HIP library behind the ``wy_lib::gdn_*``
ops) never calls it.

Each function restates the reference semantics in fp32 PyTorch on the CPU and
cites the reference lines it follows (sujuyu/qwen3_5-triton-inference-engine,
``triton_kernels/``).  ``PINNED`` lists the independent checks that pin each
function; tests/test_oracle_gdn.py implements them.
"""

from __future__ import annotations

import torch

PINNED = {
    "gdn_sequential": "pure-Python brute force (nested loops, DK=DV=4); explicit transition-"
                      "matrix form S_t = e_t (I - beta k k^T) S_{t-1} + beta k v^T; delta-rule "
                      "invariant k^T S_new = v for unit k, beta=1, g=0; g=-inf & beta=1 -> "
                      "S = k v^T, out = (q.k) v; packed batch == per-sequence runs",
    "gdn_decode": "decode chain from a prefix state == one sequential run; beta=0 -> pure "
                  "decay e^g S",
    "gdn_qk_norm_gates": "pure-Python brute force (math.sqrt, math.exp, math.log1p); "
                         "softplus(x) == log(1+e^x) for moderate x; q/k rows have unit norm "
                         "(q scaled by D^-1/2)",
    "conv4_decode": "direct 4-tap formula on a shifted window; decode chain == causal "
                    "conv over the whole sequence (torch conv1d, padding 3)",
    "gdn_gated_rmsnorm": "pure-Python brute force; z=0 -> 0; scale invariance of x",
    "conv4_prefill": "torch conv1d (padding 3) per sequence of a packed batch",
    "conv_state_from_packed": "direct row selection by index (last 4 rows, zero on top)",
    "gdn_chunk_prepare_wy / gdn_chunk_state / gdn_chunk_output": "the three stages chained "
        "(fp64) == gdn_sequential for T in {1, 63, 64, 65, 200, 300} (out and final state); "
        "u_base / w solve (I + L) X = B (residual ~1e-15 against the explicit matrix); "
        "chunk_state[0] == 0 and chunk_state[c] == the sequential state after 64 c tokens",
}


def gdn_sequential(q, k, v, beta, g, cu_seqlens=None, state0=None):
    """Delta-rule recurrence (gdn_recurrent_prefill.py:52-143 kernel body,
    :1537-1560 the reference's own torch restatement).  q, k ``[T, H, DK]``,
    v ``[T, H, DV]``, beta, g ``[T, H]``.  Per sequence (``cu_seqlens`` or one
    sequence) from ``state0`` (``[B, H, DK, DV]``, default zero).
    Returns ``(out fp32 [T, H, DV], state fp32 [B, H, DK, DV])``."""
    T, H, DK = q.shape
    DV = v.shape[-1]
    if cu_seqlens is None:
        cu = [0, T]
    else:
        cu = [int(x) for x in cu_seqlens]
    B = len(cu) - 1
    qf, kf, vf = q.float(), k.float(), v.float()
    bf, gf = beta.float(), g.float()
    out = torch.zeros(T, H, DV)
    states = torch.zeros(B, H, DK, DV)
    for b in range(B):
        s = torch.zeros(H, DK, DV) if state0 is None else state0[b].float().clone()
        for t in range(cu[b], cu[b + 1]):
            s = torch.exp(gf[t])[:, None, None] * s                      # decay
            mem = torch.einsum("hk,hkv->hv", kf[t], s)                    # k^T S
            delta = bf[t][:, None] * (vf[t] - mem)                        # beta (v - mem)
            s = s + kf[t][:, :, None] * delta[:, None, :]                 # S += k delta^T
            out[t] = torch.einsum("hk,hkv->hv", qf[t], s)                 # q^T S
        states[b] = s
    return out, states


def gdn_decode(q, k, v, beta, g, state):
    """One token per sequence from the cached state (gdn_recurrent_prefill.py:151-246):
    q, k ``[B, H, DK]``, v ``[B, H, DV]``, beta, g ``[B, H]``, state
    ``[B, H, DK, DV]``.  Returns ``(out fp32 [B, H, DV], new state)``."""
    B = q.shape[0]
    outs, states = [], []
    for b in range(B):
        o, s = gdn_sequential(q[b:b + 1], k[b:b + 1], v[b:b + 1], beta[b:b + 1], g[b:b + 1],
                              None, state[b:b + 1])
        outs.append(o[0])
        states.append(s[0])
    return torch.stack(outs), torch.stack(states)


def gdn_qk_norm_gates(q, k, a, b, a_log, dt_bias):
    """gdn_qk_norm_gates.py:19-115 (kernel), :231-247 (torch restatement):
    q_n = bf16(q * rsqrt(sum q^2 + 1e-6) * D^-0.5), k_n = bf16(k * rsqrt(sum k^2 + 1e-6)),
    beta = sigmoid(b), g = -exp(a_log) * softplus(a + dt_bias), all fp32 math."""
    D = q.shape[-1]
    qf, kf = q.float(), k.float()
    qn = qf * torch.rsqrt((qf * qf).sum(-1, keepdim=True) + 1e-6) * (D ** -0.5)
    kn = kf * torch.rsqrt((kf * kf).sum(-1, keepdim=True) + 1e-6)
    beta = torch.sigmoid(b.float())
    x = a.float() + dt_bias.float()[None, :]
    softplus = torch.clamp(x, min=0.0) + torch.log1p(torch.exp(-x.abs()))
    g = -torch.exp(a_log.float())[None, :] * softplus
    return qn.to(torch.bfloat16), kn.to(torch.bfloat16), beta, g


def conv4_decode(x, state, weight):
    """depthwise_causal_conv4_decode.py:86-150: state ``[B, 4, D]`` holds the
    last 4 conv inputs; shift in x ``[B, D]``, y = silu(sum_r w[r] * state[r])
    in fp32 -> bf16.  weight ``[4, D]``.  Returns ``(y bf16, new state)``."""
    new = torch.cat([state[:, 1:], x[:, None, :]], dim=1)
    acc = (new.float() * weight.float()[None]).sum(1)
    y = acc * torch.sigmoid(acc)
    return y.to(torch.bfloat16), new


def conv4_prefill(x, weight_dc, seq_start=None):
    """depthwise_causal_conv4_prefill.py:23-92: out[t, c] = bf16(silu(sum_r
    w[c, r] x[t-3+r, c])) with taps before seq_start[t] (or 0) read as zero.
    x ``[T, D]``, weight ``[D, 4]``."""
    T, D = x.shape
    xf, wf = x.float(), weight_dc.float()
    lo = torch.zeros(T, dtype=torch.long) if seq_start is None else seq_start.long()
    acc = torch.zeros(T, D)
    for r in range(4):
        src = torch.arange(T) - 3 + r
        ok = (src >= lo) & (src >= 0)
        tap = torch.where(ok[:, None], xf[src.clamp(min=0)], torch.zeros(()))
        acc = acc + tap * wf[:, r][None, :]
    return (acc * torch.sigmoid(acc)).to(torch.bfloat16)


def conv_state_from_packed(x, cu_seqlens):
    """depthwise_causal_conv4_decode.py:253-330: state[b, r] = x[end_b - 4 + r]
    or zero before the sequence start."""
    cu = [int(c) for c in cu_seqlens]
    B, D = len(cu) - 1, x.shape[1]
    st = torch.zeros(B, 4, D, dtype=x.dtype)
    for b in range(B):
        for r in range(4):
            t = cu[b + 1] - 4 + r
            if t >= cu[b]:
                st[b, r] = x[t]
    return st


def gdn_gated_rmsnorm(x, z, weight):
    """gdn_gated_rmsnorm.py:21-76: out = bf16(x * rsqrt(mean(x^2) + 1e-6) * w * z * sigmoid(z))
    over the last dim, fp32 math; weight fp32."""
    xf, zf = x.float(), z.float()
    inv = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + 1e-6)
    return (xf * inv * weight.float() * (zf * torch.sigmoid(zf))).to(torch.bfloat16)


def make_gdn_inputs(T, H, DK, DV, gen):
    """The reference's input distribution (gdn_recurrent_prefill.py:1285-1299):
    L2-normalised q (scaled by DK^-0.5) and k, beta = sigmoid(N(0,1)),
    g = -softplus(N(0,1))."""
    q = torch.randn(T, H, DK, generator=gen)
    k = torch.randn(T, H, DK, generator=gen)
    v = torch.randn(T, H, DV, generator=gen).to(torch.bfloat16)
    q = (q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * DK ** -0.5).to(torch.bfloat16)
    k = (k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, H, generator=gen))
    g = -torch.nn.functional.softplus(torch.randn(T, H, generator=gen))
    return q, k, v, beta, g


# ------------------------------------------------------------ chunked (WY) prefill
CHUNK = 64


def gdn_chunk_prepare_wy(k, v, beta, g):
    """Per 64-token chunk and head (gdn_recurrent_prefill.py:249-402):
    G = cumsum(g) in the chunk; L[t, i] = beta_t exp(G_t - G_i) <k_t, k_i> for
    i < t; P = (I + L)^-1; u_base = P (beta v), w = P (beta exp(G) k).
    Tokens past T count as beta = g = 0 and k = v = 0.  fp64.  Returns
    ``(w [N, H, 64, DK], u_base [N, H, 64, DV], g_cumsum [N, H, 64])``."""
    T, H, DK = k.shape
    DV = v.shape[-1]
    N = -(-T // CHUNK)
    pad = N * CHUNK - T
    kf = torch.nn.functional.pad(k.double(), (0, 0, 0, 0, 0, pad))
    vf = torch.nn.functional.pad(v.double(), (0, 0, 0, 0, 0, pad))
    bf = torch.nn.functional.pad(beta.double(), (0, 0, 0, pad))
    gf = torch.nn.functional.pad(g.double(), (0, 0, 0, pad))
    kc = kf.view(N, CHUNK, H, DK).permute(0, 2, 1, 3)     # [N, H, 64, DK]
    vc = vf.view(N, CHUNK, H, DV).permute(0, 2, 1, 3)
    bc = bf.view(N, CHUNK, H).permute(0, 2, 1)            # [N, H, 64]
    G = gf.view(N, CHUNK, H).permute(0, 2, 1).cumsum(-1)
    kkt = kc @ kc.transpose(-1, -2)
    strict = torch.tril(torch.ones(CHUNK, CHUNK, dtype=torch.bool), -1)
    decay = torch.exp(torch.where(strict, G[..., :, None] - G[..., None, :],
                                  torch.full((), -float("inf"), dtype=torch.float64)))
    L = bc[..., :, None] * decay * kkt
    eye = torch.eye(CHUNK, dtype=torch.float64)
    rhs = torch.cat([bc[..., None] * vc, (bc * torch.exp(G))[..., None] * kc], dim=-1)
    X = torch.linalg.solve_triangular(eye + L, rhs, upper=False, unitriangular=True)
    return X[..., DV:].contiguous(), X[..., :DV].contiguous(), G


def gdn_chunk_state(k, w, u_base, g_cumsum):
    """Chunk recurrence (gdn_recurrent_prefill.py:405-562): chunk_state[c] =
    the state entering chunk c; delta = u_base - w S; S = exp(G_last) S +
    k^T (delta * exp(G_last - G_t)), tokens past T masked.  fp64.
    Returns ``(delta [N, H, 64, DV], chunk_state [N, H, DK, DV], final [H, DK, DV])``."""
    T, H, DK = k.shape
    N, _, _, DV = u_base.shape
    pad = N * CHUNK - T
    kc = torch.nn.functional.pad(k.double(), (0, 0, 0, 0, 0, pad)).view(
        N, CHUNK, H, DK).permute(0, 2, 1, 3)
    valid = (torch.arange(N * CHUNK) < T).view(N, CHUNK).double()
    S = torch.zeros(H, DK, DV, dtype=torch.float64)
    delta = torch.empty(N, H, CHUNK, DV, dtype=torch.float64)
    chunk_state = torch.empty(N, H, DK, DV, dtype=torch.float64)
    for c in range(N):
        chunk_state[c] = S
        d = u_base[c].double() - w[c].double() @ S
        delta[c] = d
        G = g_cumsum[c].double()
        to_end = torch.exp(G[:, -1:] - G) * valid[c][None, :]
        S = torch.exp(G[:, -1])[:, None, None] * S + kc[c].transpose(-1, -2) @ (d * to_end[..., None])
    return delta, chunk_state, S


def gdn_chunk_output(q, k, delta, g_cumsum, chunk_state):
    """Chunk outputs (gdn_recurrent_prefill.py:565-690): out_t = exp(G_t) q_t S_c
    + sum_{i <= t} exp(G_t - G_i) <q_t, k_i> delta_i.  fp64 ``[T, H, DV]``."""
    T, H, DK = q.shape
    N, _, _, DV = delta.shape
    pad = N * CHUNK - T
    qc = torch.nn.functional.pad(q.double(), (0, 0, 0, 0, 0, pad)).view(
        N, CHUNK, H, DK).permute(0, 2, 1, 3)
    kc = torch.nn.functional.pad(k.double(), (0, 0, 0, 0, 0, pad)).view(
        N, CHUNK, H, DK).permute(0, 2, 1, 3)
    G = g_cumsum.double()
    causal = torch.tril(torch.ones(CHUNK, CHUNK, dtype=torch.bool))
    decay = torch.exp(torch.where(causal, G[..., :, None] - G[..., None, :],
                                  torch.full((), -float("inf"), dtype=torch.float64)))
    att = (qc @ kc.transpose(-1, -2)) * decay
    out = torch.exp(G)[..., None] * (qc @ chunk_state.double()) + att @ delta.double()
    return out.permute(0, 2, 1, 3).reshape(N * CHUNK, H, DV)[:T]


def gdn_chunked(q, k, v, beta, g):
    """The three stages chained (call_gdn_recurrent_prefill_chunked_triton,
    gdn_recurrent_prefill.py:1026-1048): ``(out fp64 [T, H, DV], state [H, DK, DV])``."""
    w, u, G = gdn_chunk_prepare_wy(k, v, beta, g)
    delta, cs, final = gdn_chunk_state(k, w, u, G)
    return gdn_chunk_output(q, k, delta, G, cs), final
