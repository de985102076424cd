"""GPU parity of the decode step's model-level ops: embedding gather and
residual add bit-exact, SwiGLU within bf16 rounding (atol/rtol 1e-2), the
fused LM head argmax equal to the float64 argmax (exact index; the model's
vocabulary 248320 x 1024 included)."""

import sys

import pytest
import torch

from oracle import model_oracle as mo

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_embedding_gather_exact(pkg, dev):
    say("embedding gather")
    gen = torch.Generator().manual_seed(1)
    w = torch.randn(1000, 1024, generator=gen).to(torch.bfloat16)
    for dtype in (torch.int32, torch.int64):
        ids = torch.randint(0, 1000, (37,), generator=gen).to(dtype)
        out = pkg.embedding_gather(ids.to(dev), w.to(dev))
        assert torch.equal(out.cpu(), mo.embedding_gather(ids, w))


@pytest.mark.parametrize("n", [1024 * 32, 1000 * 3 + 5])
def test_residual_add_exact(pkg, dev, n):
    say(f"residual add n={n}")
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=gen).to(torch.bfloat16)
    r = torch.randn(n, generator=gen).to(torch.bfloat16)
    out = pkg.residual_add(x.to(dev), r.to(dev))
    assert torch.equal(out.cpu(), mo.residual_add(x, r))


@pytest.mark.parametrize("rows,d", [(32, 1024), (1, 1024), (4099, 1024), (13, 256)])
def test_add_rmsnorm_equals_add_then_norm(pkg, dev, rows, d):
    """The fused residual add + RMSNorm equals residual_add -> qwen_rmsnorm bit
    for bit (both outputs), and the oracle's add + norm within bf16 rounding."""
    from oracle import attention_oracle as ao

    say(f"add_rmsnorm rows={rows} d={d}")
    gen = torch.Generator().manual_seed(rows + d)
    h = (torch.randn(rows, d, generator=gen) * 3).to(torch.bfloat16)
    x = torch.randn(rows, d, generator=gen).to(torch.bfloat16)
    w = (torch.randn(d, generator=gen) * 0.1).to(torch.bfloat16)
    hd, xd, wd = h.to(dev), x.to(dev), w.to(dev)
    s, normed = pkg.add_rmsnorm(hd, xd, wd, 1e-6)
    s_ref = pkg.residual_add(hd, xd)
    assert torch.equal(s, s_ref)
    assert torch.equal(normed, pkg.qwen_rmsnorm(s_ref, wd, 1e-6))
    assert torch.equal(s.cpu(), mo.residual_add(h, x))
    ref = ao.qwen_rmsnorm(mo.residual_add(h, x).float(), w, 1e-6)
    torch.testing.assert_close(normed.float().cpu(), ref.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("M", [1, 32])
def test_swiglu_vs_oracle(pkg, dev, M):
    say(f"swiglu M={M}")
    gen = torch.Generator().manual_seed(M)
    gu = torch.randn(M, 2 * 3584, generator=gen).to(torch.bfloat16)
    ref = mo.swiglu(gu[:, :3584], gu[:, 3584:])
    gd = gu.to(dev)
    out = pkg.swiglu(gd[:, :3584], gd[:, 3584:])
    torch.testing.assert_close(out.float().cpu(), ref.float(), atol=1e-2, rtol=1e-2)
    # element-wise path (non-unit inner stride)
    out2 = pkg.swiglu(gd[:, :3584:2], gd[:, 3584::2])
    torch.testing.assert_close(out2.float().cpu(), mo.swiglu(gu[:, :3584:2], gu[:, 3584::2]).float(),
                               atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("rows,vocab,hidden", [(3, 1025, 256), (1, 248320, 1024),
                                               (32, 248320, 1024), (64, 5000, 1024),
                                               (17, 40000, 512)])
def test_lm_head_argmax_vs_float64(pkg, dev, rows, vocab, hidden):
    say(f"lm_head_argmax rows={rows} vocab={vocab} hidden={hidden}")
    gen = torch.Generator().manual_seed(rows + vocab)
    h = torch.randn(rows, hidden, generator=gen).to(torch.bfloat16)
    w = (torch.randn(vocab, hidden, generator=gen) * 0.05).to(torch.bfloat16)
    ref = mo.lm_head_argmax(h, w)
    got = pkg.lm_head_argmax(h.to(dev), w.to(dev), False)
    torch.cuda.synchronize()
    assert got.dtype == torch.int64 and got.shape == (rows,)
    assert torch.equal(got.cpu(), ref)
    last = pkg.lm_head_argmax(h.to(dev), w.to(dev))
    assert last.shape == () and int(last) == int(ref[-1])


def test_lm_head_argmax_first_index_on_ties(pkg, dev):
    say("lm_head_argmax ties")
    gen = torch.Generator().manual_seed(9)
    w = torch.randn(3000, 256, generator=gen).to(torch.bfloat16)
    h = torch.randn(4, 256, generator=gen).to(torch.bfloat16)
    best = mo.lm_head_argmax(h, w)
    # copy each row's winner to an earlier and a later index: the earliest copy wins
    for i, b in enumerate(best.tolist()):
        w[b + 7 if b + 7 < 3000 else b - 7] = w[b]
    ref = torch.argmax(mo.lm_head_logits(h, w), dim=-1)
    got = pkg.lm_head_argmax(h.to(dev), w.to(dev), False)
    assert torch.equal(got.cpu(), ref)


def test_lm_head_argmax_nan_and_inf_rows_give_valid_index(pkg, dev):
    """Rows whose logits are all NaN or all -inf, and a vocabulary with NaN
    rows: the index is torch.argmax's (NaN ranks highest, first one wins; an
    all -inf row gives 0), never an out-of-range id that the next step's
    embedding gather would follow."""
    say("lm_head_argmax NaN / -inf rows")
    gen = torch.Generator().manual_seed(13)
    V, K = 3000, 256
    w = torch.randn(V, K, generator=gen).to(torch.bfloat16)
    h = torch.randn(4, K, generator=gen).to(torch.bfloat16)
    h[1] = float("nan")
    got = pkg.lm_head_argmax(h.to(dev), w.to(dev), False).cpu()
    ref = torch.argmax(mo.lm_head_logits(h, w), dim=-1)
    assert int(got[1]) == 0 and torch.equal(got, ref)
    w_nan = w.clone()
    w_nan[1777] = float("nan")
    w_nan[2500] = float("nan")
    got = pkg.lm_head_argmax(h.to(dev), w_nan.to(dev), False).cpu()
    assert torch.equal(got, torch.argmax(mo.lm_head_logits(h, w_nan), dim=-1))
    assert got.tolist() == [1777, 0, 1777, 1777]
    w_inf = torch.full((V, K), float("-inf")).to(torch.bfloat16)
    h_pos = (torch.rand(3, K, generator=gen) + 0.5).to(torch.bfloat16)
    got = pkg.lm_head_argmax(h_pos.to(dev), w_inf.to(dev), False).cpu()
    assert got.tolist() == [0, 0, 0]


def test_embedding_gather_out_of_range_ids_give_zero_rows(pkg, dev):
    say("embedding gather out-of-range ids")
    gen = torch.Generator().manual_seed(2)
    w = torch.randn(100, 256, generator=gen).to(torch.bfloat16)
    ids = torch.tensor([5, -1, 100, 2 ** 31 - 1, 99], dtype=torch.int64)
    out = pkg.embedding_gather(ids.to(dev), w.to(dev)).cpu()
    assert torch.equal(out[0], w[5]) and torch.equal(out[4], w[99])
    assert not out[1:4].any()
