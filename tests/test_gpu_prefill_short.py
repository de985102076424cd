"""The eight-wave short-sequence prefill kernel (one-round grids of sequences
of at most 128 tokens, csrc/prefill_short.hip) against the CPU oracle
(max-abs 2e-2, mean-abs 2e-3) and against the four-wave kernel on the same
inputs (which it agrees with to rounding: the scale multiplies the scores
instead of a bf16-rounded q, and the exponentials use an exact row max
instead of the first tile's).  The launch picks it by shape;
wy_prefill_set_short_path(0) sends the same launch to the four-wave kernel.
"""

import sys

import pytest
import torch

from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

HQ, HKV, D = 8, 2, 256
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def case(lengths, seed):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    bf = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16)
    q, k, v = bf(total, HQ, D), bf(total, HKV, D), bf(total, HKV, D)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    return q, k, v, cu


def close(got, ref, what):
    err = (got.float().cpu() - ref.float().cpu()).abs()
    assert torch.isfinite(got.float()).all(), f"{what}: non-finite output"
    assert err.max().item() <= MAX_ABS, f"{what}: max abs err {err.max().item():.3e}"
    assert err.mean().item() <= MEAN_ABS, f"{what}: mean abs err {err.mean().item():.3e}"


def four_wave(pkg, fn):
    lib = pkg._lib.load()
    lib.wy_prefill_set_short_path(0)
    try:
        out = fn()
        torch.cuda.synchronize()
    finally:
        lib.wy_prefill_set_short_path(1)
    return out


SHORT = [
    [128] * 32,                                              # config 3
    [1, 2, 5, 17, 31, 32, 33, 63, 64, 65, 100, 127, 128],    # every tile edge
    [64] * 3 + [1],
    [7],
    [128] * 2 + [96] * 30,                                   # 256 blocks: one round
]


@pytest.mark.parametrize("lengths", SHORT)
def test_short_kernel_vs_oracle_and_four_wave(pkg, dev, lengths):
    say(f"prefill short kernel lengths={lengths[:14]} (B={len(lengths)})")
    assert pkg._lib.load().wy_varlen_causal_prefill_workspace_bytes(len(lengths), HKV,
                                                                   max(lengths)) == 0
    q, k, v, cu = case(lengths, len(lengths) + 7)
    qd, kd, vd, cud = (t.to(dev) for t in (q, k, v, cu))
    got = pkg.gqa_attention_varlen_causal(qd, kd, vd, cud, max(lengths))
    torch.cuda.synchronize()
    close(got, orc.varlen_causal(q, k, v, cu), "short kernel vs oracle")
    ref4 = four_wave(pkg, lambda: pkg.gqa_attention_varlen_causal(qd, kd, vd, cud, max(lengths)))
    d = (got.float() - ref4.float()).abs()
    # the same math to rounding (the scale on the scores instead of on a
    # bf16-rounded q): a few bf16 ulps at most
    assert d.max().item() <= 2e-2 and d.mean().item() <= 1e-3, (d.max().item(), d.mean().item())
    if sum(lengths) >= 1024:
        # the two kernels round apart: equal outputs would mean the launch did
        # not take the eight-wave kernel
        assert d.max().item() > 0
    again = pkg.gqa_attention_varlen_causal(qd, kd, vd, cud, max(lengths))
    assert torch.equal(again, got)


def test_short_kernel_outlier_scores(pkg, dev):
    """A key whose score exceeds the first tile's by far more than 2^64 (the
    four-wave kernel's exact-fallback case): the eight-wave kernel's exact
    row max handles it in its one pass."""
    say("prefill short kernel outlier score")
    gen = torch.Generator().manual_seed(43)
    lengths = [128, 70, 16]
    total = sum(lengths)
    q = torch.randn(total, HQ, D, generator=gen).to(torch.bfloat16)
    k = (torch.randn(total, HKV, D, generator=gen) * 0.05).to(torch.bfloat16)
    v = torch.randn(total, HKV, D, generator=gen).to(torch.bfloat16)
    q[:128] = 1.0
    k[100] = 4.0  # q.k = 1024: 92 above the first tile in log2 units
    cu = torch.tensor([0, 128, 198, 214], dtype=torch.int32)
    got = pkg.gqa_attention_varlen_causal(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), 128)
    torch.cuda.synchronize()
    close(got, orc.varlen_causal(q, k, v, cu), "outlier")
    torch.testing.assert_close(got[110:128].float().cpu(),
                               v[100].float().repeat_interleave(4, 0).expand(18, HQ, D),
                               atol=2e-2, rtol=0)


def test_short_kernel_strided_views(pkg, dev):
    """q / k / v / out as views with row strides larger than their heads'
    span (the runner's packed projections)."""
    say("prefill short kernel strided views")
    lengths = [128, 40, 99]
    gen = torch.Generator().manual_seed(44)
    total = sum(lengths)
    big = torch.randn(total, HQ * D + 2 * HKV * D + 64, generator=gen).to(torch.bfloat16)
    q = big[:, : HQ * D].view(total, HQ, D)
    k = big[:, HQ * D: HQ * D + HKV * D].view(total, HKV, D)
    v = big[:, HQ * D + HKV * D: HQ * D + 2 * HKV * D].view(total, HKV, D)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    bd = big.to(dev)
    qd = bd[:, : HQ * D].view(total, HQ, D)
    kd = bd[:, HQ * D: HQ * D + HKV * D].view(total, HKV, D)
    vd = bd[:, HQ * D + HKV * D: HQ * D + 2 * HKV * D].view(total, HKV, D)
    got = pkg.gqa_attention_varlen_causal(qd, kd, vd, cu.to(dev), max(lengths))
    torch.cuda.synchronize()
    close(got, orc.varlen_causal(q.contiguous(), k.contiguous(), v.contiguous(), cu), "strided")


def test_short_kernel_graph_replays(pkg, dev):
    say("prefill short kernel graph replays")
    lengths = [128] * 16 + [50] * 8
    q, k, v, cu = (t.to(dev) for t in case(lengths, 45))
    eager = pkg.gqa_attention_varlen_causal(q, k, v, cu, 128)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.gqa_attention_varlen_causal(q, k, v, cu, 128)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = pkg.gqa_attention_varlen_causal(q, k, v, cu, 128)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
