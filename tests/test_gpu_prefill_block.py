"""The prefill attention block (two launches) against the reference op
sequence it replaces (partial RoPE of q and k, varlen causal attention,
sigmoid gate pack, K/V page scatter), run through this package's own ops on
the same inputs: the o_proj input and both page pools must be bit-identical.
The op sequence itself is checked against the CPU oracle elsewhere; one case
here also checks the block directly against the oracle (max-abs 2e-2,
mean-abs 2e-3)."""

import sys

import pytest
import torch

from oracle import attention_oracle as orc
from tests.golden import cases as C

pytestmark = pytest.mark.gpu

HQ, HKV, D = 8, 2, 256


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make(pkg, dev, lengths, seed, pos64=False):
    gen = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    bf = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16)
    q, k, v, gate = bf(T, HQ, D), bf(T, HKV, D), bf(T, HKV * D), bf(T, HQ * D)
    packed = pkg.build_packed_batch(lengths, device=dev)
    if pos64:
        packed = packed.__class__(**{**packed.__dict__,
                                     "position_ids": packed.position_ids.to(torch.int64)})
    max_pages = -(-max(lengths) // 16) + 1
    num_pages = len(lengths) * max_pages + 5
    bt = torch.randperm(num_pages, generator=gen)[: len(lengths) * max_pages]
    bt = bt.view(len(lengths), max_pages).to(torch.int32)
    kc, vc = bf(num_pages, HKV, 16, D), bf(num_pages, HKV, 16, D)
    return [t.to(dev) for t in (q, k, v, gate, bt, kc, vc)] + [packed]


CASES = [
    ([128] * 8, 1, False),                      # config 3's shape, fewer sequences
    ([1, 3, 17, 64, 100, 300, 65, 63], 2, True),  # ragged, partial tiles, int64 positions
    ([1, 3, 17, 64, 1000, 2000, 5], 3, False),  # queue launch (grid larger than the chip)
]


@pytest.mark.parametrize("lengths,seed,pos64", CASES)
def test_block_equals_op_sequence(pkg, dev, lengths, seed, pos64):
    say(f"prefill block vs op sequence lengths={lengths} pos64={pos64}")
    q, k, v, gate, bt, kc, vc, packed = make(pkg, dev, lengths, seed, pos64)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    ref = pkg.prefill_attention_packed(q, k, v, gate, inv, 64, packed, kc1, vc1, bt)
    got = pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc2, vc2, bt)
    torch.cuda.synchronize()
    assert got.shape == ref.shape == (sum(lengths), HQ * D)
    assert torch.equal(got, ref)
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1)


def test_block_vs_oracle(pkg, dev):
    lengths = [5, 70, 130]
    say(f"prefill block vs oracle lengths={lengths}")
    q, k, v, gate, bt, kc, vc, packed = make(pkg, dev, lengths, 9)
    inv = C.inv_freq().to(dev)
    got = pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc, vc, bt)
    pos = packed.position_ids.cpu()
    T = sum(lengths)
    qc, kcpu, vcpu = q.cpu(), k.cpu(), v.cpu().view(T, HKV, D)
    q4 = orc.partial_rope(qc.unsqueeze(0).permute(0, 2, 1, 3), pos, inv.cpu(), 64)
    k4 = orc.partial_rope(kcpu.unsqueeze(0).permute(0, 2, 1, 3), pos, inv.cpu(), 64)
    ctx = orc.varlen_causal(q4[0].permute(1, 0, 2).contiguous(), k4[0].permute(1, 0, 2).contiguous(),
                            vcpu, packed.cu_seqlens.cpu()).to(torch.bfloat16)
    ref = orc.gate_pack(ctx.permute(1, 0, 2).unsqueeze(0),
                        gate.cpu().view(1, T, HQ, D).permute(0, 2, 1, 3))
    err = (got.float().cpu() - ref.float()).abs()
    assert torch.isfinite(got).all()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, err.max().item()
    # the roped K rows sit in the pages at the page-table address: dims past
    # the rotary width bit-exact, rotated dims within bf16 rounding of the
    # oracle's fp32 cos/sin
    kr = k4[0].permute(1, 0, 2)
    for b, n in enumerate(lengths):
        s0 = packed.offsets[b]
        for t in (0, n - 1):
            phys = int(bt[b, t // 16])
            row = kc[phys, :, t % 16].cpu()
            assert torch.equal(row[:, 64:], kr[s0 + t][:, 64:])
            torch.testing.assert_close(row[:, :64].float(), kr[s0 + t][:, :64].float(),
                                       atol=2e-2, rtol=1e-2)
            assert torch.equal(vc[phys, :, t % 16].cpu(), vcpu[s0 + t])


def test_block_gate_view_offsets(pkg, dev):
    """The gate as a view of a wider projection output, at a 16-byte-aligned
    offset (read in place) and at an 8-byte offset (copied first): the same
    bytes as with a contiguous gate."""
    say("prefill block gate views")
    lengths = [40, 130, 7]
    q, k, v, gate, bt, kc, vc, packed = make(pkg, dev, lengths, 12)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    T = sum(lengths)
    ref = pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc.clone(), vc.clone(), bt)
    for off in (8, 4):
        wide = torch.zeros(T, HQ * D + 16, dtype=torch.bfloat16, device=dev)
        wide[:, off:off + HQ * D] = gate
        view = wide[:, off:off + HQ * D]
        got = pkg.prefill_attention_block(q, k, v, view, inv, 64, packed, kc.clone(), vc.clone(),
                                          bt)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), off


@pytest.mark.parametrize("seed", range(6))
def test_block_equals_op_sequence_random_lengths(pkg, dev, seed):
    """Random packed batches (2..24 sequences, lengths log-uniform in
    [1, 4096]; most take the queue launch): the block and the op sequence
    agree bit for bit, pages included."""
    import random
    rng = random.Random(1000 + seed)
    lengths = [max(1, int(2 ** rng.uniform(0, 12))) for _ in range(rng.randint(2, 24))]
    say(f"prefill block vs op sequence, random lengths seed={seed}: {lengths}")
    q, k, v, gate, bt, kc, vc, packed = make(pkg, dev, lengths, 50 + seed)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    ref = pkg.prefill_attention_packed(q, k, v, gate, inv, 64, packed, kc1, vc1, bt)
    got = pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc2, vc2, bt)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1)


@pytest.mark.parametrize("lengths,seed", [
    ([1, 3, 17, 64, 1000, 2000, 5], 3),         # queue launch
    ([128] * 32, 7),                            # config 3: one-workgroup-per-block launch
    ([16, 4096, 1500, 33, 700, 2500, 90, 1200], 11),  # queue launch, long and short
])
def test_block_independent_of_block_order(pkg, dev, lengths, seed):
    """The attention block with its query blocks handed out heaviest first,
    lightest first and alternately from both ends (wy_prefill_set_ticket_order):
    bit-identical to one another and to the op sequence.  Any dependence of a
    block's result on what ran before it on the same workgroup (LDS or
    register state left by an earlier block) or on which workgroups run
    together would show here."""
    lib = pkg._lib.load()
    say(f"prefill block order independence lengths={lengths}")
    q, k, v, gate, bt, kc, vc, packed = make(pkg, dev, lengths, seed)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    ref = pkg.prefill_attention_packed(q, k, v, gate, inv, 64, packed, kc.clone(), vc.clone(),
                                       bt)
    try:
        for order in (0, 1, 2):
            lib.wy_prefill_set_ticket_order(order)
            got = pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc.clone(),
                                              vc.clone(), bt)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"order {order}"
            plain = pkg.gqa_attention_varlen_causal(
                q, k, v.view(-1, HKV, D), packed.cu_seqlens, max(lengths))
            torch.cuda.synchronize()
            if order == 0:
                plain0 = plain
            assert torch.equal(plain, plain0), f"plain op, order {order}"
    finally:
        lib.wy_prefill_set_ticket_order(0)
