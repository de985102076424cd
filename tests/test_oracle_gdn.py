"""Pins the GDN oracle with checks that do not restate its formulas:
pure-Python brute force, the explicit transition-matrix form of the delta
rule, closed-form special cases and torch's own conv1d.  CPU only."""

import math

import pytest
import torch

from oracle import gdn_oracle as go


def _inputs(T, H, DK, DV, seed):
    return go.make_gdn_inputs(T, H, DK, DV, torch.Generator().manual_seed(seed))


def test_sequential_matches_python_brute_force():
    T, H, DK, DV = 6, 2, 4, 4
    q, k, v, beta, g = _inputs(T, H, DK, DV, 1)
    out, st = go.gdn_sequential(q, k, v, beta, g)
    for h in range(H):
        S = [[0.0] * DV for _ in range(DK)]
        for t in range(T):
            e = math.exp(float(g[t, h]))
            S = [[e * S[i][j] for j in range(DV)] for i in range(DK)]
            kk = [float(k[t, h, i]) for i in range(DK)]
            qq = [float(q[t, h, i]) for i in range(DK)]
            mem = [sum(kk[i] * S[i][j] for i in range(DK)) for j in range(DV)]
            d = [float(beta[t, h]) * (float(v[t, h, j]) - mem[j]) for j in range(DV)]
            S = [[S[i][j] + kk[i] * d[j] for j in range(DV)] for i in range(DK)]
            o = [sum(qq[i] * S[i][j] for i in range(DK)) for j in range(DV)]
            for j in range(DV):
                assert abs(o[j] - float(out[t, h, j])) < 1e-5
        for i in range(DK):
            for j in range(DV):
                assert abs(S[i][j] - float(st[0, h, i, j])) < 1e-5


def test_sequential_matches_transition_matrix_form():
    """S_t = e_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T, as dense
    matrix products (float64)."""
    T, H, DK, DV = 9, 3, 8, 16
    q, k, v, beta, g = _inputs(T, H, DK, DV, 2)
    out, st = go.gdn_sequential(q, k, v, beta, g)
    for h in range(H):
        S = torch.zeros(DK, DV, dtype=torch.float64)
        for t in range(T):
            kk = k[t, h].double()[:, None]
            A = math.exp(float(g[t, h])) * (torch.eye(DK, dtype=torch.float64)
                                            - float(beta[t, h]) * kk @ kk.T)
            # (I - b k k^T)(e S) + b k v^T  ==  e (I - b k k^T) S + b k v^T
            S = A @ S + float(beta[t, h]) * kk @ v[t, h].double()[None, :]
            o = q[t, h].double()[None, :] @ S
            assert torch.allclose(o[0].float(), out[t, h], atol=1e-5, rtol=1e-5)
        assert torch.allclose(S.float(), st[0, h], atol=1e-5, rtol=1e-5)


def test_delta_rule_writes_the_value_for_a_unit_key():
    """beta = 1, g = 0, |k| = 1: after the update k^T S = v exactly (up to
    rounding), whatever S held before."""
    gen = torch.Generator().manual_seed(3)
    H, DK, DV = 2, 16, 8
    k = torch.randn(1, H, DK, generator=gen, dtype=torch.float64)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(1, H, DV, generator=gen)
    s0 = torch.randn(1, H, DK, DV, generator=gen)
    q = k.clone()
    _, st = go.gdn_sequential(q, k, v, torch.ones(1, H), torch.zeros(1, H), None, s0)
    mem = torch.einsum("hk,hkv->hv", k[0].float(), st[0])
    assert torch.allclose(mem, v[0], atol=1e-5)


def test_full_decay_and_unit_beta_give_outer_product():
    gen = torch.Generator().manual_seed(4)
    H, DK, DV = 2, 8, 8
    q, k, v, _, _ = _inputs(1, H, DK, DV, 5)
    s0 = torch.randn(1, H, DK, DV, generator=gen)
    out, st = go.gdn_sequential(q, k, v, torch.ones(1, H), torch.full((1, H), -math.inf),
                                None, s0)
    kf, vf, qf = k[0].float(), v[0].float(), q[0].float()
    assert torch.allclose(st[0], kf[:, :, None] * vf[:, None, :], atol=1e-6)
    assert torch.allclose(out[0], (qf * kf).sum(-1)[:, None] * vf, atol=1e-6)


def test_zero_beta_is_pure_decay():
    gen = torch.Generator().manual_seed(6)
    B, H, DK, DV = 3, 2, 8, 16
    q, k, v, _, g = _inputs(B, H, DK, DV, 7)
    s0 = torch.randn(B, H, DK, DV, generator=gen)
    out, st = go.gdn_decode(q, k, v, torch.zeros(B, H), g, s0)
    e = torch.exp(g)[:, :, None, None]
    assert torch.allclose(st, e * s0, atol=1e-6)
    assert torch.allclose(out, torch.einsum("bhk,bhkv->bhv", q.float(), e * s0), atol=1e-5)


def test_packed_batch_equals_per_sequence_and_decode_chain():
    lengths = [5, 1, 12, 3]
    T, H, DK, DV = sum(lengths), 2, 8, 8
    q, k, v, beta, g = _inputs(T, H, DK, DV, 8)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    out, st = go.gdn_sequential(q, k, v, beta, g, cu)
    for b, n in enumerate(lengths):
        s, e = int(cu[b]), int(cu[b + 1])
        o1, s1 = go.gdn_sequential(q[s:e], k[s:e], v[s:e], beta[s:e], g[s:e])
        assert torch.equal(o1, out[s:e]) and torch.equal(s1[0], st[b])
        # prefix prefill, then token-by-token decode (gdn_recurrent_prefill.py:1603-1650)
        if n > 1:
            _, sp = go.gdn_sequential(q[s:s + 1], k[s:s + 1], v[s:s + 1], beta[s:s + 1],
                                      g[s:s + 1])
            for t in range(s + 1, e):
                o, sp = go.gdn_decode(q[t:t + 1], k[t:t + 1], v[t:t + 1], beta[t:t + 1],
                                      g[t:t + 1], sp)
                assert torch.allclose(o[0], out[t], atol=1e-6)
            assert torch.allclose(sp[0], st[b], atol=1e-6)


def test_qk_norm_gates_brute_force():
    gen = torch.Generator().manual_seed(9)
    T, H, D = 3, 4, 8
    q = torch.randn(T, H, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(T, H, D, generator=gen).to(torch.bfloat16)
    a = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    b = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    a_log = torch.randn(H, generator=gen)
    dt = torch.randn(H, generator=gen).to(torch.bfloat16)
    qn, kn, beta, g = go.gdn_qk_norm_gates(q, k, a, b, a_log, dt)
    for t in range(T):
        for h in range(H):
            qq = [float(x) for x in q[t, h]]
            kk = [float(x) for x in k[t, h]]
            rq = 1.0 / math.sqrt(sum(x * x for x in qq) + 1e-6)
            rk = 1.0 / math.sqrt(sum(x * x for x in kk) + 1e-6)
            for d in range(D):
                assert abs(float(qn[t, h, d]) - qq[d] * rq / math.sqrt(D)) <= 2 ** -8 * abs(
                    qq[d] * rq / math.sqrt(D)) + 1e-7
                assert abs(float(kn[t, h, d]) - kk[d] * rk) <= 2 ** -8 * abs(kk[d] * rk) + 1e-7
            assert abs(float(beta[t, h]) - 1 / (1 + math.exp(-float(b[t, h])))) < 1e-6
            x = float(a[t, h]) + float(dt[h])
            ref = -math.exp(float(a_log[h])) * math.log1p(math.exp(x))
            assert abs(float(g[t, h]) - ref) <= 1e-5 * max(1.0, abs(ref))
    # normalised rows: |k_n| = 1, |q_n| = D^-1/2 (to bf16 precision)
    assert torch.allclose(kn.float().norm(dim=-1), torch.ones(T, H), atol=1e-2)
    assert torch.allclose(qn.float().norm(dim=-1), torch.full((T, H), D ** -0.5), atol=1e-2)


def test_conv4_decode_chain_equals_causal_conv():
    """Decoding token by token from a zero state gives torch's causal depthwise
    conv1d (left padding 3) followed by SiLU."""
    gen = torch.Generator().manual_seed(10)
    B, T, D = 2, 7, 12
    x = torch.randn(B, T, D, generator=gen).to(torch.bfloat16)
    w = torch.randn(4, D, generator=gen).to(torch.bfloat16)
    ref = torch.nn.functional.conv1d(x.float().transpose(1, 2), w.float().T[:, None, :],
                                     padding=3, groups=D)[:, :, :T]
    ref = torch.nn.functional.silu(ref).transpose(1, 2)
    state = torch.zeros(B, 4, D, dtype=torch.bfloat16)
    for t in range(T):
        y, state = go.conv4_decode(x[:, t], state, w)
        assert torch.allclose(y.float(), ref[:, t], atol=1e-2, rtol=1e-2)
    assert torch.equal(state, x[:, T - 4:])


def test_gated_rmsnorm_brute_force_and_special_cases():
    gen = torch.Generator().manual_seed(11)
    T, H, D = 2, 3, 16
    x = torch.randn(T, H, D, generator=gen).to(torch.bfloat16)
    z = torch.randn(T, H, D, generator=gen).to(torch.bfloat16)
    w = torch.randn(D, generator=gen)
    out = go.gdn_gated_rmsnorm(x, z, w)
    for t in range(T):
        for h in range(H):
            xx = [float(c) for c in x[t, h]]
            r = 1 / math.sqrt(sum(c * c for c in xx) / D + 1e-6)
            for d in range(D):
                zz = float(z[t, h, d])
                ref = xx[d] * r * float(w[d]) * zz / (1 + math.exp(-zz))
                assert abs(float(out[t, h, d]) - ref) <= 2 ** -8 * abs(ref) + 1e-6
    assert torch.equal(go.gdn_gated_rmsnorm(x, torch.zeros_like(z), w).float(),
                       torch.zeros(T, H, D))
    x2 = (x.float() * 4).to(torch.bfloat16)  # power-of-two scale: same output
    assert torch.allclose(go.gdn_gated_rmsnorm(x2, z, w).float(), out.float(), atol=1e-2)


def test_conv4_prefill_packed_equals_per_sequence_conv1d():
    gen = torch.Generator().manual_seed(12)
    lengths, D = [5, 1, 9, 2], 6
    T = sum(lengths)
    x = torch.randn(T, D, generator=gen).to(torch.bfloat16)
    w = torch.randn(D, 4, generator=gen).to(torch.bfloat16)
    starts = torch.repeat_interleave(torch.tensor([0, 5, 6, 15], dtype=torch.int32),
                                     torch.tensor(lengths))
    out = go.conv4_prefill(x, w, starts)
    s = 0
    for n in lengths:
        seg = x[s:s + n].float().T[None]
        ref = torch.nn.functional.conv1d(seg, w.float()[:, None, :], padding=3, groups=D)
        ref = torch.nn.functional.silu(ref[0, :, :n]).T
        assert torch.allclose(out[s:s + n].float(), ref, atol=1e-2, rtol=1e-2)
        s += n


def test_conv_state_from_packed_selects_rows():
    x = torch.arange(10 * 3, dtype=torch.float32).view(10, 3).to(torch.bfloat16)
    st = go.conv_state_from_packed(x, torch.tensor([0, 2, 10], dtype=torch.int32))
    assert torch.equal(st[0, :2], torch.zeros(2, 3, dtype=torch.bfloat16))
    assert torch.equal(st[0, 2:], x[0:2])
    assert torch.equal(st[1], x[6:10])


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200, 300])
def test_chunked_stages_equal_sequential(T):
    """The chunk-64 WY form (three stages) equals the sequential recurrence,
    which the brute-force tests above pin: any wrong term of L, w, u_base, the
    chunk state or the intra-chunk output shows here."""
    gen = torch.Generator().manual_seed(T)
    q, k, v, beta, g = go.make_gdn_inputs(T, 3, 16, 8, gen)
    out, st = go.gdn_chunked(q, k, v, beta, g)
    ref_o, ref_s = go.gdn_sequential(q, k, v, beta, g)
    torch.testing.assert_close(out.float(), ref_o, atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(st.float(), ref_s[0], atol=2e-5, rtol=2e-5)


def test_chunk_prepare_solves_the_triangular_system_and_states_chain():
    gen = torch.Generator().manual_seed(11)
    T, H, DK, DV = 150, 2, 16, 8
    q, k, v, beta, g = go.make_gdn_inputs(T, H, DK, DV, gen)
    w, u, G = go.gdn_chunk_prepare_wy(k, v, beta, g)
    # (I + L) [u | w] = [beta v | beta exp(G) k] row by row, L built explicitly
    for c in range(w.shape[0]):
        for h in range(H):
            n = min(64, T - 64 * c)
            kk = k[64 * c:64 * c + n, h].double()
            b = beta[64 * c:64 * c + n, h].double()
            Gc = G[c, h, :n]
            L = torch.zeros(n, n, dtype=torch.float64)
            for t in range(n):
                for i in range(t):
                    L[t, i] = b[t] * math.exp(Gc[t] - Gc[i]) * float(kk[t] @ kk[i])
            A = torch.eye(n, dtype=torch.float64) + L
            assert torch.allclose(A @ u[c, h, :n], b[:, None] * v[64 * c:64 * c + n, h].double(),
                                  atol=1e-12)
            assert torch.allclose(A @ w[c, h, :n], (b * torch.exp(Gc))[:, None] * kk, atol=1e-12)
    delta, cs, final = go.gdn_chunk_state(k, w, u, G)
    assert not cs[0].any()
    for c in (1, 2):
        _, s_ref = go.gdn_sequential(q[:64 * c], k[:64 * c], v[:64 * c], beta[:64 * c],
                                     g[:64 * c])
        torch.testing.assert_close(cs[c].float(), s_ref[0], atol=2e-5, rtol=2e-5)
