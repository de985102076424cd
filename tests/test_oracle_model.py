"""Pins the model-op oracle with independent checks.  CPU only."""

import math

import torch

from oracle import model_oracle as mo


def test_embedding_matches_functional():
    gen = torch.Generator().manual_seed(1)
    w = torch.randn(50, 16, generator=gen).to(torch.bfloat16)
    ids = torch.randint(0, 50, (9,), generator=gen, dtype=torch.int32)
    assert torch.equal(mo.embedding_gather(ids, w), torch.nn.functional.embedding(ids.long(), w))


def test_residual_add_dyadic_exact():
    x = torch.tensor([1.0, 0.5, -2.0, 3.0]).to(torch.bfloat16)
    r = torch.tensor([0.25, 0.5, 2.0, -1.0]).to(torch.bfloat16)
    assert torch.equal(mo.residual_add(x, r).float(), torch.tensor([1.25, 1.0, 0.0, 2.0]))


def test_swiglu_brute_force():
    gen = torch.Generator().manual_seed(2)
    g = torch.randn(3, 5, generator=gen).to(torch.bfloat16)
    u = torch.randn(3, 5, generator=gen).to(torch.bfloat16)
    out = mo.swiglu(g, u)
    ref = torch.nn.functional.silu(g.float()) * u.float()
    assert torch.allclose(out.float(), ref, atol=1e-2, rtol=1e-2)
    for i in range(3):
        for j in range(5):
            gg, uu = float(g[i, j]), float(u[i, j])
            assert abs(float(out[i, j]) - uu * gg / (1 + math.exp(-gg))) <= 1e-2


def test_lm_head_argmax_special_cases():
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(40, 8, generator=gen).to(torch.bfloat16)
    w[17] = w[5]  # duplicate rows: the first index wins
    h = torch.zeros(8, dtype=torch.bfloat16)
    h[2] = 1.0  # one-hot hidden: logits = column 2
    col = w[:, 2].float().clone()
    col[17] = -1e9
    expect = int(torch.argmax(col))
    assert int(mo.lm_head_argmax(h[None], w)[0]) == expect
