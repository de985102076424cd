"""The queue launch of the varlen prefill (persistent grid drawing query
blocks from a ticket counter) against the one-workgroup-per-block launch and
the CPU oracle.

Both launches run the same per-block code, so their outputs must be
bit-identical; the oracle check uses the attention tolerance (max-abs 2e-2,
mean-abs 2e-3).  The ticket counters must be left at zero by every launch.
"""

import sys

import pytest
import torch

from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

HQ, HKV, D = 8, 2, 256


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bf(shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def case(lengths, seed):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    q, k, v = bf((total, HQ, D), gen), bf((total, HKV, D), gen), bf((total, HKV, D), gen)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    return q, k, v, cu


def direct(pkg, q, k, v, cu, max_seqlen):
    """The same op through the C ABI without a workspace: one workgroup per block."""
    lib = pkg._lib
    out = torch.empty_like(q)
    lib.call("wy_varlen_causal_prefill", lib.ptr(q), lib.strides(q), lib.ptr(k),
             lib.strides(k), lib.ptr(v), lib.strides(v), lib.ptr(out), lib.strides(out),
             lib.ptr(cu), cu.numel() - 1, q.shape[1], k.shape[1], q.shape[2], max_seqlen,
             q.shape[0], None, 0, lib.stream(q.device))
    return out


def queue_bytes(pkg, lengths):
    return pkg._lib.load().wy_varlen_causal_prefill_workspace_bytes(len(lengths), HKV,
                                                                    max(lengths))


def counters(pkg, dev):
    return pkg._lib.stream_workspace(dev, "prefill_queue", 8).view(torch.int32)


@pytest.mark.parametrize("lengths", [
    [1, 3, 17, 64, 1000, 2000, 5],
    [4096, 1, 33, 32, 31, 600, 2, 64, 65],
    [16] * 200,
    [257] * 40,
    [16] * 1100,   # 2200 one-tile blocks, a plan of 2200 slices x sequences
])
def test_queue_launch_equals_direct_launch(pkg, dev, lengths):
    say(f"prefill queue vs direct, lengths={lengths[:12]} (B={len(lengths)})")
    assert queue_bytes(pkg, lengths) == 8, "case must take the queue launch"
    q, k, v, cu = (t.to(dev) for t in case(lengths, len(lengths)))
    got = pkg.gqa_attention_varlen_causal(q, k, v, cu, max(lengths))
    ref = direct(pkg, q, k, v, cu, max(lengths))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert counters(pkg, dev).tolist() == [0, 0]
    again = pkg.gqa_attention_varlen_causal(q, k, v, cu, max(lengths))
    assert torch.equal(again, ref)
    assert counters(pkg, dev).tolist() == [0, 0]


def test_queue_launch_vs_oracle(pkg, dev):
    lengths = [1, 3, 17, 64, 700, 900, 5, 130, 31, 32, 33] + [2] * 20
    say(f"prefill queue vs oracle, B={len(lengths)}")
    assert queue_bytes(pkg, lengths) == 8
    q, k, v, cu = case(lengths, 7)
    out = pkg.gqa_attention_varlen_causal(q.to(dev), k.to(dev), v.to(dev), cu.to(dev),
                                          max(lengths))
    ref = orc.varlen_causal(q, k, v, cu)
    got = out.float().cpu()
    err = (got - ref.float()).abs()
    assert torch.isfinite(got).all()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, err.max().item()


def test_queue_launch_exact_fallback(pkg, dev):
    """A block that takes the exact two-pass path inside the persistent loop
    leaves the following blocks of that workgroup correct."""
    lengths = [200, 70] + [1] * 20
    say("prefill queue exact fallback")
    assert queue_bytes(pkg, lengths) == 8
    q, k, v, cu = case(lengths, 41)
    q[:200] = 1.0
    k[:200] = (k[:200].float() * 0.05).to(torch.bfloat16)
    k[130, :, :] = 4.0  # score 92 (log2 units) above the first tile's maximum
    qd, kd, vd, cud = q.to(dev), k.to(dev), v.to(dev), cu.to(dev)
    out = pkg.gqa_attention_varlen_causal(qd, kd, vd, cud, 200)
    assert torch.equal(out, direct(pkg, qd, kd, vd, cud, 200))
    ref = orc.varlen_causal(q, k, v, cu)
    err = (out.float().cpu() - ref.float()).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, err.max().item()


def test_queue_launch_graph_replays(pkg, dev):
    """Captured in a graph, every replay (eager launches in between) matches
    the eager result and leaves the counters at zero."""
    lengths = [1, 3, 17, 64, 1000, 2000, 5]
    say("prefill queue graph replays")
    q, k, v, cu = (t.to(dev) for t in case(lengths, 3))
    ref = pkg.gqa_attention_varlen_causal(q, k, v, cu, max(lengths))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.gqa_attention_varlen_causal(q, k, v, cu, max(lengths))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = pkg.gqa_attention_varlen_causal(q, k, v, cu, max(lengths))
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        eager = pkg.gqa_attention_varlen_causal(q, k, v, cu, max(lengths))
        torch.cuda.synchronize()
        assert torch.equal(eager, ref)
