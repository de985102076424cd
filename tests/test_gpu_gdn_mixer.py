"""GPU parity of the GDN decode mixer ops (conv4 decode, q/k norm + gates,
gated RMSNorm) against the CPU oracle, and of the one-launch decode block
(wy_lib::gdn_decode_block) against the four-op sequence (bit-identical) and
the oracle chain.  bf16 outputs: atol 1e-2 / rtol 1e-2 against fp32 math
(the reference's own self-test bounds); the conv state shift is bit-exact."""

import sys

import pytest
import torch

from oracle import gdn_oracle as go

pytestmark = pytest.mark.gpu

H, D = 16, 128
C = 3 * H * D


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close(got, ref, atol=1e-2, rtol=1e-2):
    torch.testing.assert_close(got.float().cpu(), ref.float(), atol=atol, rtol=rtol)


def mixer_inputs(B, seed):
    gen = torch.Generator().manual_seed(seed)
    fused = torch.randn(B, 4 * H * D + 2 * H, generator=gen).to(torch.bfloat16)
    conv_state = torch.randn(B, 4, C, generator=gen).to(torch.bfloat16)
    conv_w = (torch.randn(4, C, generator=gen) * 0.5).to(torch.bfloat16)
    a_log = torch.log(torch.rand(H, generator=gen) * 15 + 1)
    dt_bias = torch.randn(H, generator=gen).to(torch.bfloat16)
    norm_w = 1 + 0.1 * torch.randn(D, generator=gen)
    state = torch.randn(B, H, D, D, generator=gen) * 0.1
    return fused, conv_state, conv_w, a_log, dt_bias, norm_w, state


def oracle_chain(fused, conv_state, conv_w, a_log, dt_bias, norm_w, state):
    B = fused.shape[0]
    HD = H * D
    y, new_conv = go.conv4_decode(fused[:, :3 * HD], conv_state, conv_w)
    q = y[:, :HD].view(B, H, D)
    k = y[:, HD:2 * HD].view(B, H, D)
    v = y[:, 2 * HD:].view(B, H, D)
    a = fused[:, 4 * HD:4 * HD + H]
    b = fused[:, 4 * HD + H:]
    qn, kn, beta, g = go.gdn_qk_norm_gates(q, k, a, b, a_log, dt_bias)
    core, new_state = go.gdn_decode(qn, kn, v, beta, g, state)
    z = fused[:, 3 * HD:4 * HD].view(B, H, D)
    out = go.gdn_gated_rmsnorm(core.to(torch.bfloat16), z, norm_w)
    return out.view(B, HD), new_conv, new_state


@pytest.mark.parametrize("B", [1, 5, 32])
def test_conv4_decode_vs_oracle(pkg, dev, B):
    say(f"conv4 decode B={B}")
    fused, conv_state, conv_w, *_ = mixer_inputs(B, B)
    y_ref, st_ref = go.conv4_decode(fused[:, :C], conv_state, conv_w)
    fd, st = fused.to(dev), conv_state.to(dev)
    y = pkg.depthwise_causal_conv4_decode(fd[:, :C], st, conv_w.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(st.cpu(), st_ref)
    close(y, y_ref)


def test_conv4_decode_chain_equals_causal_conv(pkg, dev):
    say("conv4 decode chain")
    gen = torch.Generator().manual_seed(3)
    B, T, Cs = 2, 9, 384
    x = torch.randn(B, T, Cs, generator=gen).to(torch.bfloat16)
    w = torch.randn(4, Cs, generator=gen).to(torch.bfloat16)
    ref = torch.nn.functional.conv1d(x.float().transpose(1, 2), w.float().T[:, None, :],
                                     padding=3, groups=Cs)[:, :, :T]
    ref = torch.nn.functional.silu(ref).transpose(1, 2)
    st = torch.zeros(B, 4, Cs, dtype=torch.bfloat16, device=dev)
    xd, wd = x.to(dev), w.to(dev)
    for t in range(T):
        close(pkg.depthwise_causal_conv4_decode(xd[:, t].contiguous(), st, wd), ref[:, t])
    assert torch.equal(st.cpu(), x[:, T - 4:])


@pytest.mark.parametrize("T", [1, 3, 17, 130])
def test_qk_norm_gates_vs_oracle(pkg, dev, T):
    say(f"gdn qk norm gates T={T}")
    gen = torch.Generator().manual_seed(T)
    qk = torch.randn(T, 2 * H * D, generator=gen).to(torch.bfloat16)  # strided views
    a = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    b = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    a_log = torch.log(torch.rand(H, generator=gen) * 15 + 1)
    dt = torch.randn(H, generator=gen).to(torch.bfloat16)
    q, k = qk[:, :H * D].view(T, H, D), qk[:, H * D:].view(T, H, D)
    refs = go.gdn_qk_norm_gates(q, k, a, b, a_log, dt)
    qkd = qk.to(dev)
    got = pkg.gdn_qk_norm_gates(qkd[:, :H * D].view(T, H, D), qkd[:, H * D:].view(T, H, D),
                                a.to(dev), b.to(dev), a_log.to(dev), dt.to(dev))
    torch.cuda.synchronize()
    close(got[0], refs[0])
    close(got[1], refs[1])
    close(got[2], refs[2], atol=1e-5, rtol=1e-5)
    close(got[3], refs[3], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("T", [1, 7, 64])
def test_gated_rmsnorm_vs_oracle(pkg, dev, T):
    say(f"gdn gated rmsnorm T={T}")
    gen = torch.Generator().manual_seed(50 + T)
    x = torch.randn(T, H, D, generator=gen).to(torch.bfloat16)
    zbuf = torch.randn(T, 2 * H * D, generator=gen).to(torch.bfloat16)
    z = zbuf[:, H * D:].view(T, H, D)
    w = 1 + 0.1 * torch.randn(D, generator=gen)
    ref = go.gdn_gated_rmsnorm(x, z, w)
    got = pkg.gdn_gated_rmsnorm(x.to(dev), zbuf.to(dev)[:, H * D:].view(T, H, D), w.to(dev))
    torch.cuda.synchronize()
    close(got, ref)


@pytest.mark.parametrize("B", [1, 32])
def test_decode_block_equals_op_sequence_and_oracle(pkg, dev, B):
    say(f"gdn decode block B={B}")
    inp = mixer_inputs(B, 1000 + B)
    out_ref, conv_ref, st_ref = oracle_chain(*inp)
    fused, conv_state, conv_w, a_log, dt_bias, norm_w, state = (x.to(dev) for x in inp)
    cs1, st1 = conv_state.clone(), state.clone()
    cs2, st2 = conv_state.clone(), state.clone()
    seq = pkg.gdn_decode_ops(fused, cs1, conv_w, a_log, dt_bias, norm_w, st1)
    blk = pkg.gdn_decode_block(fused, cs2, conv_w, a_log, dt_bias, norm_w, st2)
    torch.cuda.synchronize()
    assert torch.equal(blk, seq), (blk.float() - seq.float()).abs().max().item()
    assert torch.equal(cs2, cs1) and torch.equal(st2, st1)
    assert torch.equal(cs2.cpu(), conv_ref)
    close(blk, out_ref, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(st2.cpu(), st_ref, atol=2e-4, rtol=2e-4)


def test_decode_block_chain_and_graph_replays(pkg, dev):
    """Six decode steps as graph replays (both states advance in the graph)
    equal six eager block calls bit for bit."""
    say("gdn decode block graph replays")
    B = 4
    fused, conv_state, conv_w, a_log, dt_bias, norm_w, state = (
        x.to(dev) for x in mixer_inputs(B, 77))
    cs_e, st_e = conv_state.clone(), state.clone()
    eager = [pkg.gdn_decode_block(fused, cs_e, conv_w, a_log, dt_bias, norm_w, st_e).clone()
             for _ in range(6)]
    cs, st = conv_state.clone(), state.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pkg.gdn_decode_block(fused, cs.clone(), conv_w, a_log, dt_bias, norm_w, st.clone())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.gdn_decode_block(fused, cs, conv_w, a_log, dt_bias, norm_w, st)
    for i in range(6):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i]), f"replay {i}"
    assert torch.equal(cs, cs_e) and torch.equal(st, st_e)


@pytest.mark.parametrize("lengths", [[5], [3, 6, 2], [1, 1, 40], [100, 17]])
def test_conv4_prefill_vs_oracle_and_decode_chain(pkg, dev, lengths):
    """Packed prefill conv vs the oracle; each sequence's outputs equal the
    decode step chain from a zero state bit for bit; the packed conv-state
    write equals the last four rows of each sequence (zero-padded on top)."""
    say(f"conv4 prefill lengths={lengths}")
    gen = torch.Generator().manual_seed(sum(lengths))
    T, Cs = sum(lengths), 640
    x = torch.randn(T, Cs, generator=gen).to(torch.bfloat16)
    w = torch.randn(Cs, 1, 4, generator=gen).to(torch.bfloat16)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    starts = torch.repeat_interleave(cu[:-1], torch.tensor(lengths))
    ref = go.conv4_prefill(x, w[:, 0], starts)
    xd, wd = x.to(dev), w.to(dev)
    out = pkg.depthwise_causal_conv4_prefill(xd, wd, starts.to(dev))
    torch.cuda.synchronize()
    close(out, ref)
    w_dec = w[:, 0].T.contiguous().to(dev)  # [4, C] decode layout
    for b, n in enumerate(lengths):
        st = torch.zeros(1, 4, Cs, dtype=torch.bfloat16, device=dev)
        for t in range(int(cu[b]), int(cu[b + 1])):
            y = pkg.depthwise_causal_conv4_decode(xd[t:t + 1], st, w_dec)
            assert torch.equal(y[0], out[t]), (b, t)
    state = torch.full((len(lengths), 4, Cs), 7.0, dtype=torch.bfloat16, device=dev)
    pkg.conv_state_from_packed_prefill(state, xd, cu.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(state.cpu(), go.conv_state_from_packed(x, cu))


def test_row_vectorised_norms_equal_per_row_kernels(pkg, dev):
    """From 256 (token, head) rows the q/k norm + gates and the gated RMSNorm
    take the 16-lanes-per-row kernels; token by token (16 rows) they take one
    block per row.  Same pairing of the sum of squares either way: the results
    agree bit for bit."""
    say("gdn row-vectorised norms == per-row kernels")
    T = 40
    gen = torch.Generator().manual_seed(77)
    qk = torch.randn(T, 2 * H * D, generator=gen).to(torch.bfloat16).to(dev)
    a = torch.randn(T, H, generator=gen).to(torch.bfloat16).to(dev)
    b = torch.randn(T, H, generator=gen).to(torch.bfloat16).to(dev)
    a_log = torch.log(torch.rand(H, generator=gen) * 15 + 1).to(dev)
    dt = torch.randn(H, generator=gen).to(torch.bfloat16).to(dev)
    q, k = qk[:, :H * D].view(T, H, D), qk[:, H * D:].view(T, H, D)
    assert T * H >= 256
    big = pkg.gdn_qk_norm_gates(q, k, a, b, a_log, dt)
    rows = [pkg.gdn_qk_norm_gates(q[t:t + 1], k[t:t + 1], a[t:t + 1], b[t:t + 1], a_log, dt)
            for t in range(T)]
    x = torch.randn(T, H, D, generator=gen).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(D, generator=gen)).to(dev)
    nbig = pkg.gdn_gated_rmsnorm(x, k, w)
    nrows = [pkg.gdn_gated_rmsnorm(x[t:t + 1], k[t:t + 1], w) for t in range(T)]
    torch.cuda.synchronize()
    for i in range(4):
        assert torch.equal(big[i], torch.cat([r[i] for r in rows])), i
    assert torch.equal(nbig, torch.cat(nrows))
