"""GPU parity of the Gated DeltaNet recurrence (wy_lib::gdn_recurrent_decode,
wy_lib::gdn_recurrent_prefill_sequential) against the CPU oracle.

Tolerances follow the reference's own self-test (gdn_recurrent_prefill.py:
1590-1592): out (bf16) atol = rtol = 1e-2, fp32 state atol = rtol = 2e-4.
Packed vs per-sequence runs of the HIP kernel are bit-identical (each
wavefront's arithmetic does not depend on the batch).
"""

import sys

import pytest
import torch

from oracle import gdn_oracle as go

pytestmark = pytest.mark.gpu

H, DK, DV = 16, 128, 128


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check(out, state, out_ref, state_ref):
    out, state = out.float().cpu(), state.float().cpu()
    assert torch.isfinite(out).all() and torch.isfinite(state).all()
    torch.testing.assert_close(out, out_ref.float(), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(state, state_ref, rtol=2e-4, atol=2e-4)


def inputs(T, seed, heads=H):
    return go.make_gdn_inputs(T, heads, DK, DV, torch.Generator().manual_seed(seed))


@pytest.mark.parametrize("T", [1, 3, 17, 65])
@pytest.mark.parametrize("strided", [False, True])
def test_prefill_sequential_vs_oracle(pkg, dev, T, strided):
    say(f"gdn prefill sequential T={T} strided={strided}")
    q, k, v, beta, g = inputs(T, T)
    out_ref, st_ref = go.gdn_sequential(q, k, v, beta, g)
    if strided:
        # every other element of a wider buffer (gdn_recurrent_prefill.py:1570-1583)
        def spread(x):
            buf = torch.zeros(*x.shape[:-1], 2 * x.shape[-1], dtype=x.dtype)
            buf[..., ::2] = x
            return buf.to(dev)[..., ::2]
        qd, kd, vd = spread(q), spread(k), spread(v)
    else:
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out, st = pkg.gdn_recurrent_prefill_sequential(qd, kd, vd, beta.to(dev), g.to(dev))
    torch.cuda.synchronize()
    assert out.shape == (T, H, DV) and st.shape == (H, DK, DV)
    check(out, st, out_ref, st_ref[0])


@pytest.mark.parametrize("lengths", [[5], [3, 6, 2], [1, 1, 1, 1], [17, 3], [64, 1, 100],
                                     [0, 7], [33, 0, 2]])
def test_prefill_packed_vs_oracle_and_per_sequence(pkg, dev, lengths):
    say(f"gdn prefill packed lengths={lengths}")
    total = sum(lengths)
    q, k, v, beta, g = inputs(total, 100 + total)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    out_ref, st_ref = go.gdn_sequential(q, k, v, beta, g, cu)
    qd, kd, vd, bd, gd = (x.to(dev) for x in (q, k, v, beta, g))
    out, st = pkg.gdn_recurrent_prefill_sequential(qd, kd, vd, bd, gd, cu.to(dev))
    torch.cuda.synchronize()
    assert st.shape == (len(lengths), H, DK, DV)
    check(out, st, out_ref, st_ref)
    for b, n in enumerate(lengths):
        if n == 0:
            assert torch.equal(st[b].cpu(), torch.zeros(H, DK, DV))
            continue
        s, e = int(cu[b]), int(cu[b + 1])
        o1, s1 = pkg.gdn_recurrent_prefill_sequential(qd[s:e], kd[s:e], vd[s:e], bd[s:e],
                                                      gd[s:e])
        assert torch.equal(o1, out[s:e]) and torch.equal(s1, st[b])


def test_prefill_none_equals_single_range(pkg, dev):
    say("gdn prefill cu_seqlens None vs [0, T]")
    q, k, v, beta, g = (x.to(dev) for x in inputs(19, 19))
    o1, s1 = pkg.gdn_recurrent_prefill_sequential(q, k, v, beta, g)
    o2, s2 = pkg.gdn_recurrent_prefill_sequential(
        q, k, v, beta, g, torch.tensor([0, 19], dtype=torch.int32, device=dev))
    assert torch.equal(o1, o2) and torch.equal(s1, s2[0])


def test_prefill_then_decode_equals_full_sequence(pkg, dev):
    """gdn_recurrent_prefill.py:1603-1650: prefix prefill then token-by-token
    decode equals the whole sequence through the recurrence."""
    say("gdn prefill 17 + decode 48")
    T, prefix = 65, 17
    q, k, v, beta, g = inputs(T, 65)
    out_ref, st_ref = go.gdn_sequential(q, k, v, beta, g)
    qd, kd, vd, bd, gd = (x.to(dev) for x in (q, k, v, beta, g))
    o, st = pkg.gdn_recurrent_prefill_sequential(qd[:prefix], kd[:prefix], vd[:prefix],
                                                 bd[:prefix], gd[:prefix])
    st = st.unsqueeze(0).contiguous()
    parts = [o]
    for t in range(prefix, T):
        parts.append(pkg.gdn_recurrent_decode(qd[t:t + 1], kd[t:t + 1], vd[t:t + 1],
                                              bd[t:t + 1], gd[t:t + 1], st))
    torch.cuda.synchronize()
    check(torch.cat(parts), st[0], out_ref, st_ref[0])


@pytest.mark.parametrize("B", [1, 32])
def test_decode_batch_vs_oracle(pkg, dev, B):
    say(f"gdn decode B={B}")
    gen = torch.Generator().manual_seed(200 + B)
    q, k, v, beta, g = inputs(B, 300 + B)
    s0 = torch.randn(B, H, DK, DV, generator=gen) * 0.5
    out_ref, st_ref = go.gdn_decode(q, k, v, beta, g, s0)
    st = s0.to(dev)
    out = pkg.gdn_recurrent_decode(q.to(dev), k.to(dev), v.to(dev), beta.to(dev), g.to(dev), st)
    torch.cuda.synchronize()
    check(out, st, out_ref, st_ref)


def test_decode_strided_views_of_a_fused_buffer(pkg, dev):
    """The runner's layout: q/k/v are column slices of the conv output [B, 6144]
    viewed as [B, 16, 128] (engine/runner.py:433-437)."""
    say("gdn decode strided conv-output slices")
    B = 8
    gen = torch.Generator().manual_seed(7)
    q, k, v, beta, g = inputs(B, 8)
    conv = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], 1).to(dev)
    qd = conv[:, :H * DK].view(B, H, DK)
    kd = conv[:, H * DK:2 * H * DK].view(B, H, DK)
    vd = conv[:, 2 * H * DK:].view(B, H, DV)
    s0 = torch.randn(B, H, DK, DV, generator=gen) * 0.5
    out_ref, st_ref = go.gdn_decode(q, k, v, beta, g, s0)
    st = s0.to(dev)
    out = pkg.gdn_recurrent_decode(qd, kd, vd, beta.to(dev), g.to(dev), st)
    torch.cuda.synchronize()
    check(out, st, out_ref, st_ref)


def test_decode_graph_replays(pkg, dev):
    """Captured decode step replayed 5 times, each replay advancing the state
    in place; every replay equals the eager chain bit for bit."""
    say("gdn decode graph replays")
    B = 4
    gen = torch.Generator().manual_seed(11)
    q, k, v, beta, g = (x.to(dev) for x in inputs(B, 12))
    s0 = (torch.randn(B, H, DK, DV, generator=gen) * 0.5).to(dev)
    eager_state = s0.clone()
    eager = [pkg.gdn_recurrent_decode(q, k, v, beta, g, eager_state).clone() for _ in range(5)]
    state = s0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        warm = state.clone()
        pkg.gdn_recurrent_decode(q, k, v, beta, g, warm)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.gdn_recurrent_decode(q, k, v, beta, g, state)
    state.copy_(s0)
    for i in range(5):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i]), f"replay {i}"
    assert torch.equal(state, eager_state)
