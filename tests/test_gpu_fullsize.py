"""Parity at BASELINE.json's full sizes (configs 4 and 5).  The oracle cannot
run whole 4 GiB workloads on the host in seconds, so these tests check, on the
full-size device state:
  * bit-exact page writes (the append of every sequence, the varlen scatter of
    every token) against the address formula;
  * the attention outputs of a sample of sequences against the fp32 oracle on
    that sequence's gathered pages (max-abs 2e-2 / mean-abs 2e-3);
  * decode of token L after prefill of 0..L-1 == row L of the prefill, for every
    sequence (a size-independent identity).
Every test prints its case before touching the GPU."""

import math
import sys

import pytest
import torch

from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

HQ, HKV, D, P = 8, 2, 256, 16


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close(got, ref, what, max_abs=2e-2, mean_abs=2e-3):
    got, ref = got.float().cpu(), ref.float().cpu()
    assert torch.isfinite(got).all(), what
    err = (got - ref).abs()
    assert err.max().item() <= max_abs, f"{what}: max abs {err.max().item():.3e}"
    assert err.mean().item() <= mean_abs, f"{what}: mean abs {err.mean().item():.3e}"


def dev_randn(shape, gen, dev, scale=1.0):
    return (torch.randn(*shape, device=dev, generator=gen) * scale).to(torch.bfloat16)


def sequence_pages(kc, vc, bt_row, n_pages):
    """One sequence's pages as a contiguous host pool + identity table."""
    idx = bt_row[:n_pages].long()
    return kc[idx].cpu(), vc[idx].cpu(), torch.arange(n_pages, dtype=torch.int32).view(1, -1)


def test_config5_full_size(pkg, dev):
    """B=64 x 32768 tokens (4 GiB of K/V), randperm pages, K/V ~ N(0, 0.5)."""
    say("config5 full size: B=64, L=32768")
    B, L = 64, 32768
    pages = L // P + 1
    num_pages = B * pages
    g = torch.Generator(device=dev).manual_seed(5)
    bt = torch.randperm(num_pages, device=dev, generator=g).view(B, pages).to(torch.int32)
    kc = dev_randn((num_pages, HKV, P, D), g, dev, 0.5)
    vc = dev_randn((num_pages, HKV, P, D), g, dev, 0.5)
    q, kn, vn = dev_randn((B, HQ, D), g, dev), dev_randn((B, HKV, D), g, dev), \
        dev_randn((B, HKV, D), g, dev)
    pos = torch.full((B,), L - 1, dtype=torch.int64, device=dev)
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    out = pkg.call_paged_gqa_attention_decode_triton(q, kn, vn, kc, vc, bt, pos, sc)
    torch.cuda.synchronize()
    # the append of every sequence landed at (bt[b, pos // 16], :, pos % 16)
    rows = bt[:, (L - 1) // P].long()
    assert torch.equal(kc[rows, :, (L - 1) % P], kn) and torch.equal(vc[rows, :, (L - 1) % P], vn)
    assert int(sc.counters.abs().sum()) == 0
    for b in (0, 37, 63):
        kp, vp, tab = sequence_pages(kc, vc, bt[b], -(-L // P))
        ref = orc.paged_decode(q[b:b + 1].cpu(), kp, vp, tab, torch.tensor([L]))
        close(out[b:b + 1], ref, f"config5 sequence {b}")
    del kc, vc, sc
    torch.cuda.empty_cache()


def test_config4_full_size(pkg, dev):
    """24 sequences, log-uniform [16, 4096] (seed 4, ~18.6k tokens): packed
    prefill, scatter into a shuffled pool, then one decode step per sequence."""
    g4 = torch.Generator().manual_seed(4)
    lens = torch.exp(torch.empty(24).uniform_(math.log(16), math.log(4096), generator=g4))
    lens = [int(x) for x in lens.round().tolist()]
    say(f"config4 full size: {len(lens)} sequences, {sum(lens)} tokens")
    B = len(lens)
    ext = [n + 1 for n in lens]
    total = sum(ext)
    g = torch.Generator(device=dev).manual_seed(44)
    q = dev_randn((total, HQ, D), g, dev)
    k = dev_randn((total, HKV, D), g, dev)
    v = dev_randn((total, HKV, D), g, dev)
    cu_ext = torch.tensor([0] + torch.tensor(ext).cumsum(0).tolist(), dtype=torch.int32)
    full = pkg.gqa_attention_varlen_causal(q, k, v, cu_ext.to(dev), max(ext))
    # oracle on three sequences: the longest, a mid one, the shortest
    order = sorted(range(B), key=lambda b: ext[b])
    for b in (order[-1], order[B // 2], order[0]):
        s0, s1 = int(cu_ext[b]), int(cu_ext[b + 1])
        ref = orc.varlen_causal(q[s0:s1].cpu(), k[s0:s1].cpu(), v[s0:s1].cpu(),
                                torch.tensor([0, s1 - s0], dtype=torch.int32))
        close(full[s0:s1], ref, f"config4 prefill sequence {b} (L={s1 - s0})")
    # scatter the first L tokens of every sequence into a shuffled pool
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    idx = torch.cat([torch.arange(int(cu_ext[b]), int(cu_ext[b]) + lens[b]) for b in range(B)])
    idx_d = idx.to(dev)
    max_pages = -(-max(ext) // P)
    num_pages = B * max_pages + 5
    bt = torch.randperm(num_pages, generator=g4)[:B * max_pages].view(B, max_pages).to(torch.int32)
    kg = torch.zeros(num_pages, HKV, P, D, dtype=torch.bfloat16, device=dev)
    vg = torch.zeros_like(kg)
    pkg.paged_kv_fill_varlen(kg, vg, k[idx_d].permute(1, 0, 2), v[idx_d].permute(1, 0, 2),
                             bt.to(dev), cu.to(dev), max(lens))
    torch.cuda.synchronize()
    # every token at its closed-form row: bit-exact
    rows = torch.cat([bt[b].long()[torch.arange(lens[b]) // P] * (HKV * P) +
                      torch.arange(lens[b]) % P for b in range(B)])  # head 0 rows
    kf, vf = kg.view(-1, D).cpu(), vg.view(-1, D).cpu()
    kpk, vpk = k[idx_d].cpu(), v[idx_d].cpu()
    for h in range(HKV):
        assert torch.equal(kf[rows + h * P], kpk[:, h]) and torch.equal(vf[rows + h * P], vpk[:, h])
    # untouched slots stay zero: exactly sum(lens) * HKV rows were written
    assert int((kf.abs().sum(-1) != 0).sum()) <= sum(lens) * HKV
    # decode token L of every sequence from those pages == prefill row L
    last = (cu_ext[1:].long() - 1).to(dev)
    ctx = pkg.call_paged_gqa_attention_decode_triton(
        q[last], k[last], v[last], kg, vg, bt.to(dev),
        torch.tensor(lens, dtype=torch.int64, device=dev))
    close(ctx, full[last], "config4 decode after prefill vs prefill row")


def test_config4_lengths_gdn_prefill(pkg, dev):
    """The config-4 length set (24 prompts, log-uniform [16, 4096], seed 4,
    ~18.6k tokens) through the packed GDN sequential prefill (16 heads of
    128): every sequence equals its own unpacked run bit for bit; the
    shortest, a middle and the longest sequence match the CPU oracle (out
    atol/rtol 1e-2, state 2e-4, the reference's bounds)."""
    from oracle import gdn_oracle as go
    g4 = torch.Generator().manual_seed(4)
    lens = torch.exp(torch.empty(24).uniform_(math.log(16), math.log(4096), generator=g4))
    lens = [int(x) for x in lens.round().tolist()]
    total = sum(lens)
    say(f"gdn config4 lengths: {total} tokens")
    q, k, v, beta, g = go.make_gdn_inputs(total, 16, 128, 128, torch.Generator().manual_seed(44))
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    qd, kd, vd, bd, gd = (x.to(dev) for x in (q, k, v, beta, g))
    out, st = pkg.gdn_recurrent_prefill_sequential(qd, kd, vd, bd, gd, cu.to(dev))
    torch.cuda.synchronize()
    for b in range(len(lens)):
        s, e = int(cu[b]), int(cu[b + 1])
        o1, s1 = pkg.gdn_recurrent_prefill_sequential(qd[s:e], kd[s:e], vd[s:e], bd[s:e], gd[s:e])
        assert torch.equal(o1, out[s:e]) and torch.equal(s1, st[b]), b
    order = sorted(range(len(lens)), key=lambda i: lens[i])
    for b in (order[0], order[len(order) // 2], order[-1]):
        s, e = int(cu[b]), int(cu[b + 1])
        say(f"gdn oracle sequence {b} ({lens[b]} tokens)")
        o_ref, s_ref = go.gdn_sequential(q[s:e], k[s:e], v[s:e], beta[s:e], g[s:e])
        torch.testing.assert_close(out[s:e].float().cpu(), o_ref, atol=1e-2, rtol=1e-2)
        torch.testing.assert_close(st[b].cpu(), s_ref[0], atol=2e-4, rtol=2e-4)
