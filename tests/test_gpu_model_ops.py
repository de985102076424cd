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
