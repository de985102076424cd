"""GPU parity of wy_lib::gemm_2d (the attention projections) against the fp64
oracle.  The kernel sums in fp32 and rounds to bf16 once, so each output is
within one bf16 rounding of the exact product (relative 2^-8) plus the fp32
summation-order error; the bound below is written for that.  Every test prints
its case before touching the GPU."""

import sys

import pytest
import torch

from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check(y, x, w):
    ref = orc.gemm_2d(x.cpu(), w.cpu())
    got = y.float().cpu().double()
    assert y.dtype == torch.bfloat16 and y.shape == ref.shape and y.is_contiguous()
    assert torch.isfinite(got).all()
    # one bf16 rounding (2^-8 relative) + fp32 accumulation of K terms
    tol = 2.0 ** -8 * ref.abs() + 1e-6 * x.shape[1] * 4 + 1e-3
    bad = (got - ref).abs() > tol
    assert not bad.any(), f"{int(bad.sum())} elements off, max err {(got - ref).abs().max():.3e}"


SHAPES = [
    # decode (M = batch) on the block's projections, engine/runner.py:464, :518
    (1, 5120, 1024), (5, 5120, 1024), (16, 5120, 1024), (32, 5120, 1024), (64, 1024, 2048),
    (33, 16, 1024), (7, 100, 128),
    # prefill (M = tokens), engine/runner.py:329-332, :365; ragged M and N tails
    (65, 2048, 1024), (300, 512, 1024), (1000, 1024, 2048), (129, 100, 256), (4096, 2048, 1024),
    # fewer 128 x 128 tiles than CUs take 128 x 64 tiles (k_proj at 4096 tokens; ragged N)
    (4096, 512, 1024), (2000, 900, 256),
    # grids of >= 384 256x256 tiles take the 8-wave 256 x 256 kernel; ragged edges
    (8292, 8132, 128), (8192, 8192, 128), (8192 + 255, 8192 + 129, 384),
    (4096, 8224, 256),  # the GDN in_proj width at 4096 tokens (last 32 columns: a second launch)
    (8192 + 100, 4128, 256), (8292, 8200, 128),  # narrow last columns (32, 8) with ragged M
    # deeper LDS rings: 128 x 128 tiles with 4 stages (o_proj at 4096 tokens; ragged, K
    # steps not a multiple of the ring), 128 x 64 with 4 stages down to K = 128 (two steps)
    (4096, 1024, 2048), (3000, 1000, 1152), (1000, 1024, 128),
    # 256 x 256 tiles when they make one nearly full round of the CUs (ragged M)
    (8192 - 100, 2048, 384),
]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_2d_vs_oracle(pkg, dev, M, N, K):
    say(f"gemm_2d M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    y = pkg.gemm_2d(x.to(dev), w.to(dev))
    check(y, x, w)


def test_gemm_2d_identity_is_exact(pkg, dev):
    say("gemm_2d identity weight, M=100 and M=3")
    g = torch.Generator().manual_seed(5)
    eye = torch.eye(256).bfloat16().to(dev)
    for M in (3, 100):
        x = torch.randn(M, 256, generator=g).bfloat16()
        assert torch.equal(pkg.gemm_2d(x.to(dev), eye).cpu(), x)


def test_gemm_2d_strided_inputs(pkg, dev):
    say("gemm_2d row-strided x (slice of a wider row) and transposed weight, M=40 and M=300")
    g = torch.Generator().manual_seed(6)
    wt = (torch.randn(1024, 512, generator=g) * 0.05).bfloat16()   # weight^T storage
    for M in (40, 300):
        wide = torch.randn(M, 1536, generator=g).bfloat16()
        x = wide[:, 256:1280]                  # row stride 1536, K contiguous
        y = pkg.gemm_2d(wide.to(dev)[:, 256:1280], wt.to(dev).t())  # weight K-strided
        check(y, x, wt.t())


def test_gemm_2d_graph_replays(pkg, dev):
    say("gemm_2d captured in a graph, replayed 4x with eager work between")
    g = torch.Generator().manual_seed(8)
    x = torch.randn(32, 1024, generator=g).bfloat16().to(dev)
    xl = torch.randn(256, 1024, generator=g).bfloat16().to(dev)
    w = (torch.randn(5120, 1024, generator=g) * 0.05).bfloat16().to(dev)
    ref_s, ref_l = pkg.gemm_2d(x, w), pkg.gemm_2d(xl, w)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ys, yl = pkg.gemm_2d(x, w), pkg.gemm_2d(xl, w)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, ref_s) and torch.equal(yl, ref_l)
        _ = (xl * 2).sum().item()


def _gemm_no_workspace(pkg, x, w):
    """gemm_2d through the C ABI without a workspace: no K split."""
    lib = pkg._lib
    y = torch.empty((x.shape[0], w.shape[0]), dtype=torch.bfloat16, device=x.device)
    lib.call("wy_gemm_2d", lib.ptr(x), lib.i64_array(x.stride()), lib.ptr(w),
             lib.i64_array(w.stride()), lib.ptr(y), lib.i64_array(y.stride()), x.shape[0],
             w.shape[0], x.shape[1], None, 0, lib.stream(x.device))
    return y


@pytest.mark.parametrize("M,N,K", [(32, 1024, 2048), (64, 1024, 2048), (1, 1024, 2048), (33, 16, 1024)])
def test_gemm_2d_split_k(pkg, dev, M, N, K):
    """Shapes that split K across workgroups: the split result and the
    unsplit one both meet the oracle bound, repeated calls are bit-identical
    (partials are added in split order whichever workgroup finishes last),
    and the split counters are left at zero, also inside a graph."""
    say(f"gemm_2d split-K M={M} N={N} K={K}")
    lib = pkg._lib.load()
    nbytes = lib.wy_gemm_2d_workspace_bytes(M, N, K)
    assert nbytes > 16384, "shape must take the split path"
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    xd, wd = x.to(dev), w.to(dev)
    y = pkg.gemm_2d(xd, wd)
    check(y, x, w)
    check(_gemm_no_workspace(pkg, xd, wd), x, w)
    for _ in range(3):
        assert torch.equal(pkg.gemm_2d(xd, wd), y)
    ws = pkg._lib.stream_workspace(dev, "gemm_split", nbytes)
    torch.cuda.synchronize()
    assert not ws[:16384].any(), "split counters not reset"
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        yg = pkg.gemm_2d(xd, wd)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y)
        assert torch.equal(pkg.gemm_2d(xd, wd), y)


@pytest.mark.parametrize("M", [1, 5, 16, 32, 64])
@pytest.mark.parametrize("N", [1024, 7168])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_gemm_equals_separate_ops(pkg, dev, M, N, with_residual):
    """wy_gemm_2d_rmsnorm == residual_add -> qwen_rmsnorm -> gemm_2d, bit for
    bit, including the residual-stream output (N=1024 takes the split-K path)."""
    print(f"rmsnorm_gemm M={M} N={N} residual={with_residual}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M * 7 + N)
    K = 1024
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    r = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16) if with_residual else None
    nw = (torch.randn(K, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    w = (torch.randn(N, K, device=dev, generator=g) * 0.03).to(torch.bfloat16)
    y, t = pkg.rmsnorm_gemm_2d(x, r, nw, 1e-6, w)
    t_ref = pkg.residual_add(x, r) if with_residual else x
    y_ref = pkg.gemm_2d(pkg.qwen_rmsnorm(t_ref, nw, 1e-6), w)
    torch.cuda.synchronize()
    assert torch.equal(t, t_ref)
    assert torch.equal(y, y_ref), (y.float() - y_ref.float()).abs().max().item()


@pytest.mark.parametrize("M", [1, 8, 32])
def test_swiglu_gemm_equals_separate_ops(pkg, dev, M):
    """wy_gemm_2d_swiglu == swiglu -> gemm_2d bit for bit (down projection
    [1024, 3584], the split-K path)."""
    print(f"swiglu_gemm M={M}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M)
    I, N = 3584, 1024
    gu = torch.randn(M, 2 * I, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, I, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    y = pkg.swiglu_gemm_2d(gu, w)
    y_ref = pkg.gemm_2d(pkg.swiglu(gu[:, :I], gu[:, I:]), w)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), (y.float() - y_ref.float()).abs().max().item()


@pytest.mark.parametrize("M", [1, 17, 32, 64, 100, 300, 4096])
def test_gate_up_swiglu_equals_separate_ops(pkg, dev, M):
    """wy_gemm_2d_gate_up_swiglu == gemm_2d -> swiglu bit for bit on the
    model's gate/up projection ([7168, 1024]): the skinny kernel's pair
    epilogue for M <= 64, the tile kernel's (ragged last row tile at 100 and
    300) above."""
    say(f"gate_up_swiglu M={M}")
    g = torch.Generator(device=dev).manual_seed(M)
    I, K = 3584, 1024
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    y = pkg.gate_up_swiglu(x, w)
    gu = pkg.gemm_2d(x, w)
    y_ref = pkg.swiglu(gu[:, :I], gu[:, I:])
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), (y.float() - y_ref.float()).abs().max().item()


@pytest.mark.parametrize("M,I,K", [(32, 1024, 2048), (5, 1000, 512), (64, 256, 4096),
                                   (200, 384, 512), (130, 1000, 256)])
def test_gate_up_swiglu_small_and_split(pkg, dev, M, I, K):
    """Pair plans unlike the plain GEMM's (2I < 4096; split K with fp32
    partials for I <= 1024): against the fp64 projection rounded to bf16,
    then SwiGLU in fp64 (atol/rtol 2e-2, bf16 rounding of gate and up)."""
    say(f"gate_up_swiglu M={M} I={I} K={K}")
    g = torch.Generator(device=dev).manual_seed(I + K)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * I, K, device=dev, generator=g) * 0.03).to(torch.bfloat16)
    for rep in range(2):  # the split counters must be left zero for the next call
        y = pkg.gate_up_swiglu(x, w)
        torch.cuda.synchronize()
        gu = (x.double() @ w.double().T).to(torch.bfloat16).double()
        gate, up = gu[:, :I], gu[:, I:]
        ref = up * gate * torch.sigmoid(gate)
        torch.testing.assert_close(y.double(), ref, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("M", [1, 32, 64])
@pytest.mark.parametrize("N,K", [(1024, 1152), (1024, 1408), (512, 2304), (5120, 1152)])
def test_gemm_2d_skinny_odd_k(pkg, dev, M, N, K):
    """K values whose per-wave slice is not a power-of-two multiple of 128:
    the wave count must keep every wave's slice a multiple of 32 columns, or
    the 32-column tail loop would run into the next wave's slice (and past
    the row end on the last row).  Oracle bound, split and unsplit."""
    say(f"gemm_2d skinny odd K M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M * 3 + N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    xd, wd = x.to(dev), w.to(dev)
    check(pkg.gemm_2d(xd, wd), x, w)
    check(_gemm_no_workspace(pkg, xd, wd), x, w)


@pytest.mark.parametrize("M", [1, 32, 64])
def test_rmsnorm_gemm_odd_k_vs_oracle(pkg, dev, M):
    """wy_gemm_2d_rmsnorm at K=2304 (nine 256-column chunks, a width the
    standalone qwen_rmsnorm op does not take) against the oracle chain
    rmsnorm -> fp64 GEMM.  The normed operand may differ from the oracle's by
    one bf16 rounding where the fp32 sums of squares round differently, so the
    bound adds 1e-2 absolute to the one-rounding relative term."""
    say(f"rmsnorm_gemm K=2304 M={M}")
    g = torch.Generator().manual_seed(M + 2304)
    K, N = 2304, 1024
    x = torch.randn(M, K, generator=g).bfloat16()
    r = torch.randn(M, K, generator=g).bfloat16()
    nw = (torch.randn(K, generator=g) * 0.1).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.03).bfloat16()
    y, t = pkg.rmsnorm_gemm_2d(x.to(dev), r.to(dev), nw.to(dev), 1e-6, w.to(dev))
    t_ref = (x.float() + r.float()).bfloat16()
    assert torch.equal(t.cpu(), t_ref)
    ref = orc.gemm_2d(orc.qwen_rmsnorm(t_ref, nw, 1e-6), w)
    got = y.cpu().double()
    err = (got - ref).abs()
    assert (err <= 2.0 ** -8 * ref.abs() + 1e-2).all(), f"max err {err.max():.3e}"


def test_fused_prologue_gemms_accept_unaligned_row_views(pkg, dev):
    """Row views that start off a 16-byte boundary (a column slice at an odd
    offset) are copied to aligned rows by the ops, not rejected."""
    say("rmsnorm_gemm / swiglu_gemm on unaligned row views")
    g = torch.Generator(device=dev).manual_seed(11)
    wide = torch.randn(8, 1024 + 3, device=dev, generator=g).to(torch.bfloat16)
    x = wide[:, 3:]
    nw = (torch.randn(1024, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    w = (torch.randn(512, 1024, device=dev, generator=g) * 0.03).to(torch.bfloat16)
    y, _ = pkg.rmsnorm_gemm_2d(x, None, nw, 1e-6, w)
    assert torch.equal(y, pkg.gemm_2d(pkg.qwen_rmsnorm(x.contiguous(), nw, 1e-6), w))
    y_r, t_r = pkg.rmsnorm_gemm_2d(x, x, nw, 1e-6, w)
    t_ref = pkg.residual_add(x.contiguous(), x.contiguous())
    assert torch.equal(t_r, t_ref)
    assert torch.equal(y_r, pkg.gemm_2d(pkg.qwen_rmsnorm(t_ref, nw, 1e-6), w))
    gu_wide = torch.randn(8, 2 * 1024 + 5, device=dev, generator=g).to(torch.bfloat16)
    gu = gu_wide[:, 5:]
    y2 = pkg.swiglu_gemm_2d(gu, w)
    assert torch.equal(y2, pkg.gemm_2d(pkg.swiglu(gu[:, :1024].contiguous(),
                                                  gu[:, 1024:].contiguous()), w))
