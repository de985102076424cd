"""GPU parity of the Gated DeltaNet chunk-64 (WY) prefill ops
(wy_lib::gdn_chunk_prepare_wy / gdn_chunk_state / gdn_chunk_output and
their chain) against the CPU oracle: each stage against the oracle's stage
on the same inputs (fp64 there; bounds below), and the chain against the
sequential recurrence at the reference's own bounds (out atol/rtol 1e-2,
final state 2e-4) and against this build's sequential kernel.  The oracle's
chunked form is pinned to the sequential one in tests/test_oracle_gdn.py."""

import sys

import pytest
import torch

from oracle import gdn_oracle as go

pytestmark = pytest.mark.gpu

H, DK, DV = 16, 128, 128


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def inputs(T, seed, heads=H):
    return go.make_gdn_inputs(T, heads, DK, DV, torch.Generator().manual_seed(seed))


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
def test_chunk_stages_vs_oracle(pkg, dev, T):
    say(f"gdn chunk stages T={T}")
    q, k, v, beta, g = inputs(T, 100 + T, heads=4)
    qd, kd, vd, bd, gd = (x.to(dev) for x in (q, k, v, beta, g))
    w, u, G = pkg.gdn_chunk_prepare_wy(kd, vd, bd, gd)
    w_r, u_r, G_r = go.gdn_chunk_prepare_wy(k, v, beta, g)
    torch.testing.assert_close(G.cpu().double(), G_r, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(u.cpu().double(), u_r, atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(w.cpu().double(), w_r, atol=2e-5, rtol=1e-4)
    # stage 2 and 3 on this build's own stage-1 outputs
    delta, cs, fin = pkg.gdn_chunk_state(kd, w, u, G)
    d_r, cs_r, fin_r = go.gdn_chunk_state(k, w.cpu(), u.cpu(), G.cpu())
    torch.testing.assert_close(delta.cpu().double(), d_r, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(cs.cpu().double(), cs_r, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(fin.cpu().double(), fin_r, atol=1e-4, rtol=1e-4)
    out = pkg.gdn_chunk_output(qd, kd, delta, G, cs)
    o_r = go.gdn_chunk_output(q, k, delta.cpu(), G.cpu(), cs.cpu())
    assert out.dtype == torch.bfloat16 and out.shape == (T, 4, DV)
    torch.testing.assert_close(out.float().cpu().double(), o_r, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("T", [300, 2048, 4096])
def test_chunked_prefill_vs_sequential(pkg, dev, T):
    """The chain against the sequential recurrence (oracle and this build's
    sequential kernel); T = 4096 is the single long prompt the runner sends
    down the chunked path (engine/runner.py:151-153, 272)."""
    say(f"gdn chunked prefill T={T}")
    q, k, v, beta, g = inputs(T, T)
    qd, kd, vd, bd, gd = (x.to(dev) for x in (q, k, v, beta, g))
    out, st = pkg.call_gdn_recurrent_prefill_chunked_triton(qd, kd, vd, bd, gd)
    torch.cuda.synchronize()
    assert out.shape == (T, H, DV) and st.shape == (H, DK, DV)
    o_seq, s_seq = pkg.gdn_recurrent_prefill_sequential(qd, kd, vd, bd, gd)
    torch.testing.assert_close(out.float(), o_seq.float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(st, s_seq, atol=2e-4, rtol=2e-4)
    # the fp64 oracle at every length, the routed T = 4096 included (about a
    # second of CPU time for 16 heads)
    o_r, s_r = go.gdn_sequential(q, k, v, beta, g)
    torch.testing.assert_close(out.float().cpu(), o_r, atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(st.cpu(), s_r[0], atol=2e-4, rtol=2e-4)


def test_chunked_prefill_strided_inputs(pkg, dev):
    """q, k, v as column slices of wider rows (the runner's views of the conv
    output): same result as contiguous copies."""
    say("gdn chunked prefill strided inputs")
    T = 130
    q, k, v, beta, g = inputs(T, 5)
    wide = torch.cat([q, k, v], dim=-1).to(dev)          # [T, H, 384]
    qv, kv, vv = wide[..., :DK], wide[..., DK:2 * DK], wide[..., 2 * DK:]
    bd, gd = beta.to(dev), g.to(dev)
    out, st = pkg.call_gdn_recurrent_prefill_chunked_triton(qv, kv, vv, bd, gd)
    out2, st2 = pkg.call_gdn_recurrent_prefill_chunked_triton(
        qv.contiguous(), kv.contiguous(), vv.contiguous(), bd, gd)
    assert torch.equal(out, out2) and torch.equal(st, st2)
