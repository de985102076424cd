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
