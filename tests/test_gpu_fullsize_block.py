"""The runner's whole prefill attention (partial RoPE theta 1e7 on dims
0..63, varlen causal attention, sigmoid gate, K/V page scatter into a
shuffled pool) at BASELINE.json's full sizes, configs 3 (32 x 128) and 4 (24
prompts log-uniform in [16, 4096], ~18.6k tokens), followed by one decode
step per sequence from those pages (engine/runner.py:336-384, :444-518).

Checked on the full-size device state:
  * the two-launch prefill attention block == the reference op sequence
    (RoPE q, RoPE k, attention, gate pack, scatter), output and both pools
    bit for bit;
  * every token's roped K and its V at the closed-form page row, bit-exact
    against the RoPE op's output (and dims 64..255 against the raw input);
    the rotated dims of every token within bf16 rounding of the fp32
    oracle's RoPE; pages outside the table untouched;
  * the shortest, a middle and the longest sequence against the CPU oracle
    chain RoPE -> causal attention -> gate (max-abs 2e-2, mean-abs 2e-3);
  * decode of token L_b (RoPE at position L_b, append, split-K, merge,
    gate) from those pages == row L_b of a prefill of L_b + 1 tokens, for
    every sequence, and the decoded rows of three sequences against the
    oracle on their gathered pages.
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


def config_lengths(name):
    if name == "config3":
        return [128] * 32
    g4 = torch.Generator().manual_seed(4)
    lens = torch.exp(torch.empty(24).uniform_(math.log(16), math.log(4096), generator=g4))
    return [int(x) for x in lens.round().tolist()]


def oracle_sequence(q, k, v, gate, pos, inv):
    """Oracle chain of one sequence: q [n, Hq, D], k/v [n, Hkv, D], gate
    [n, Hq*D] (host bf16), positions [n] -> gated [n, Hq*D] bf16."""
    n = q.shape[0]
    pid = pos.view(1, n)
    q4 = orc.partial_rope(q.unsqueeze(0).permute(0, 2, 1, 3), pid, inv, 64)
    k4 = orc.partial_rope(k.unsqueeze(0).permute(0, 2, 1, 3), pid, inv, 64)
    ctx = orc.varlen_causal(q4[0].permute(1, 0, 2).contiguous(),
                            k4[0].permute(1, 0, 2).contiguous(), v,
                            torch.tensor([0, n], dtype=torch.int32)).to(torch.bfloat16)
    return orc.gate_pack(ctx.permute(1, 0, 2).unsqueeze(0),
                         gate.view(1, n, HQ, D).permute(0, 2, 1, 3))


@pytest.mark.parametrize("config", ["config3", "config4"])
def test_prefill_attention_full_size_with_rope_gate_then_decode(pkg, dev, config):
    lens = config_lengths(config)
    B = len(lens)
    ext = [n + 1 for n in lens]          # each prompt plus the token decoded next
    say(f"{config} full-size prefill attention + decode: {B} sequences, {sum(lens)} tokens")
    g = torch.Generator(device=dev).manual_seed(300 + B)
    te = sum(ext)
    bf = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)
    q_e, k_e, v_e, gate_e = bf(te, HQ, D), bf(te, HKV, D), bf(te, HKV * D), bf(te, HQ * D)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    inv_c = inv.cpu()
    packed_e = pkg.build_packed_batch(ext, device=dev)
    cu_e = packed_e.offsets
    idx = torch.cat([torch.arange(cu_e[b], cu_e[b] + lens[b]) for b in range(B)]).to(dev)
    last = torch.tensor([cu_e[b + 1] - 1 for b in range(B)], device=dev)
    q, k, v, gate = q_e[idx], k_e[idx], v_e[idx], gate_e[idx]
    packed = pkg.build_packed_batch(lens, device=dev)

    # shuffled pool pre-filled with noise, 5 pages outside every table
    max_pages = -(-max(ext) // P) + 1
    num_pages = B * max_pages + 5
    gc = torch.Generator().manual_seed(400 + B)
    perm = torch.randperm(num_pages, generator=gc)
    bt = perm[:B * max_pages].view(B, max_pages).to(torch.int32).to(dev)
    outside = perm[B * max_pages:].to(dev)
    kc0, vc0 = bf(num_pages, HKV, P, D), bf(num_pages, HKV, P, D)

    # block == op sequence, output and pools bit for bit
    kc1, vc1, kc2, vc2 = kc0.clone(), vc0.clone(), kc0.clone(), vc0.clone()
    trace = {}
    ref = pkg.prefill_attention_packed(q, k, v, gate, inv, 64, packed, kc1, vc1, bt, trace=trace)
    got = pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc2, vc2, bt)
    torch.cuda.synchronize()
    assert got.shape == (sum(lens), HQ * D)
    assert torch.equal(got, ref), "block != op sequence"
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), "block pools != op sequence pools"
    del kc1, vc1, ref

    # every token at its closed-form row
    k_roped = trace["rope_k"][0].permute(1, 0, 2)        # [T, Hkv, D]
    lp = torch.cat([torch.arange(n) for n in lens]).to(dev)
    seq_of = torch.cat([torch.full((n,), b) for b, n in enumerate(lens)]).to(dev)
    phys = bt[seq_of, lp // P].long()
    slot = lp % P
    k_rows = kc2[phys, :, slot]                            # [T, Hkv, D]
    v_rows = vc2[phys, :, slot]
    assert torch.equal(k_rows, k_roped), "K page rows != roped K"
    assert torch.equal(k_rows[..., 64:], k[..., 64:]), "K tail dims not verbatim"
    assert torch.equal(v_rows, v.view(-1, HKV, D)), "V page rows != V"
    assert torch.equal(kc2[outside], kc0[outside]) and torch.equal(vc2[outside], vc0[outside])
    pos_all = packed.position_ids.cpu()
    k_orc = orc.partial_rope(k.cpu().unsqueeze(0).permute(0, 2, 1, 3), pos_all, inv_c, 64)
    close(k_rows[..., :64], k_orc[0].permute(1, 0, 2)[..., :64], f"{config} roped K dims 0..63",
          max_abs=3e-2, mean_abs=2e-3)
    del trace, k_roped, k_orc

    # three sequences against the oracle chain
    order = sorted(range(B), key=lambda b: lens[b])
    for b in (order[0], order[B // 2], order[-1]):
        s = packed.slice_of(b)
        say(f"{config} oracle sequence {b} (L={lens[b]})")
        ref_b = oracle_sequence(q[s].cpu(), k[s].cpu(), v[s].cpu().view(-1, HKV, D),
                                gate[s].cpu(), torch.arange(lens[b]), inv_c)
        close(got[s], ref_b, f"{config} prefill sequence {b}")

    # decode token L_b from those pages == row L_b of the prefill of L_b + 1
    say(f"{config} decode after prefill")
    kc_full, vc_full = kc0.clone(), vc0.clone()
    full = pkg.prefill_attention_block(q_e, k_e, v_e, gate_e, inv, 64, packed_e, kc_full,
                                       vc_full, bt)
    del kc_full, vc_full
    pos = torch.tensor(lens, dtype=torch.int64, device=dev)
    scratch = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    kc_d, vc_d = kc2.clone(), vc2.clone()
    dec = pkg.decode_attention_step(q_e[last], k_e[last], v_e[last], gate_e[last], inv, 64, pos,
                                    kc_d, vc_d, bt, scratch)
    torch.cuda.synchronize()
    close(dec, full[last], f"{config} decode vs prefill row L")
    assert int(scratch.counters.abs().sum()) == 0
    # the appended K/V landed at row L_b
    rows = bt[torch.arange(B, device=dev), pos // P].long()
    assert torch.equal(vc_d[rows, :, pos % P], v_e[last].view(B, HKV, D))
    assert torch.equal(kc_d[rows, :, pos % P][..., 64:], k_e[last][..., 64:])
    for b in (order[0], order[-1]):
        n = lens[b] + 1
        s0 = cu_e[b]
        ref_b = oracle_sequence(q_e[s0:s0 + n].cpu(), k_e[s0:s0 + n].cpu(),
                                v_e[s0:s0 + n].cpu().view(-1, HKV, D), gate_e[s0:s0 + n].cpu(),
                                torch.arange(n), inv_c)
        close(dec[b:b + 1], ref_b[-1:], f"{config} decode sequence {b} vs oracle")
