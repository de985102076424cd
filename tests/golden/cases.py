"""Seeded inputs of the golden cases.  Inputs are regenerated from CPU
``torch.Generator`` seeds; ``golden.npz`` stores a checksum of every input and
the oracle's expected outputs."""

from __future__ import annotations

import hashlib

import torch

HQ, HKV, D, PAGE = 8, 2, 256, 16
THETA = 1e7
ROTARY = 64


def bf(shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def digest(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes() if t.dtype != torch.bool
                 else t.numpy().tobytes())
    return h.hexdigest()


def inv_freq():
    return 1.0 / (THETA ** (torch.arange(0, ROTARY, 2, dtype=torch.float32) / ROTARY))


def decode_case(lens=(1, 37, 90, 256), seed=100):
    """Decode step: pools pre-filled with noise, shuffled table, append at pos."""
    gen = torch.Generator().manual_seed(seed)
    B = len(lens)
    max_pages = -(-max(lens) // PAGE) + 1
    num_pages = B * max_pages + 5
    bt = torch.randperm(num_pages, generator=gen)[: B * max_pages].view(B, max_pages)
    bt = bt.to(torch.int32).contiguous()
    kc, vc = bf((num_pages, HKV, PAGE, D), gen), bf((num_pages, HKV, PAGE, D), gen)
    q = bf((B, HQ, D), gen)
    kn, vn = bf((B, HKV, D), gen), bf((B, HKV, D), gen)
    pos = torch.tensor([n - 1 for n in lens], dtype=torch.int64)
    return dict(q=q, kc=kc, vc=vc, kn=kn, vn=vn, bt=bt, pos=pos)


def prefill_case(lengths=(7, 16, 1, 33, 70), seed=200):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    q, k, v = bf((total, HQ, D), gen), bf((total, HKV, D), gen), bf((total, HKV, D), gen)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32)
    return dict(q=q, k=k, v=v, cu=cu, max_seqlen=max(lengths))


def rope_case(seed=300):
    gen = torch.Generator().manual_seed(seed)
    x = bf((1, 33, HQ, D), gen).permute(0, 2, 1, 3)  # the runner's permuted view
    pos = torch.randint(0, 4096, (1, 33), generator=gen, dtype=torch.int64)
    return dict(x=x, pos=pos, inv_freq=inv_freq())


def gate_case(seed=400):
    gen = torch.Generator().manual_seed(seed)
    x = bf((1, 17, HQ, D), gen).permute(0, 2, 1, 3)
    g = bf((1, 17, HQ, D), gen, 3.0).permute(0, 2, 1, 3)
    return dict(x=x, gate=g)


def fill_case(lengths=(17, 1, 40), seed=500):
    gen = torch.Generator().manual_seed(seed)
    B, total = len(lengths), sum(lengths)
    max_pages = -(-max(lengths) // PAGE)
    num_pages = B * max_pages + 4
    bt = torch.randperm(num_pages, generator=gen)[: B * max_pages].view(B, max_pages)
    bt = bt.to(torch.int32).contiguous()
    # [T, H, D] memory seen as [H, T, D] (strides (D, H*D, 1)), as the runner passes k4[0]
    k = bf((total, HKV, D), gen).permute(1, 0, 2)
    v = bf((total, HKV, D), gen).permute(1, 0, 2)
    kc, vc = bf((num_pages, HKV, PAGE, D), gen), bf((num_pages, HKV, PAGE, D), gen)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0).tolist()), dtype=torch.int32)
    return dict(k=k, v=v, kc=kc, vc=vc, bt=bt, cu=cu, max_seqlen=max(lengths))
