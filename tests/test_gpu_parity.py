"""GPU parity of the HIP path against the CPU oracle and the golden fixtures.

Tolerance for attention math (north star): max-abs 2e-2 and mean-abs 2e-3 vs
the fp32 oracle, bf16 outputs.  Page scatter / append / RoPE tail: bit-exact.
Every test prints the case it runs before touching the GPU.
"""

import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from tests.golden import cases as C

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
HQ, HKV, D = 8, 2, 256
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close(got, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    got = got.float().cpu()
    ref = ref.float().cpu()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    err = (got - ref).abs()
    assert err.max().item() <= max_abs, f"{what}: max abs err {err.max().item():.3e}"
    assert err.mean().item() <= mean_abs, f"{what}: mean abs err {err.mean().item():.3e}"
    return err.max().item()


def golden():
    return np.load(ROOT / "tests" / "golden" / "golden.npz", allow_pickle=False)


def bf(shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def rand_table(B, max_pages, num_pages, gen):
    return torch.randperm(num_pages, generator=gen)[: B * max_pages].view(B, max_pages).to(
        torch.int32).contiguous()


def test_library_is_the_native_hip_build(pkg, dev):
    lib = pkg._lib.load()
    assert lib.wy_build_info().decode().endswith("gfx950")


# ------------------------------------------------------------------ scatter / append

@pytest.mark.parametrize("lengths", [[16], [17], [1], [16, 16], [7, 100, 1, 64], [128] * 8,
                                     [1, 1, 1, 1000], [0, 3]])
@pytest.mark.parametrize("shuffle", [False, True])
def test_fill_varlen_bit_exact(pkg, dev, lengths, shuffle):
    say(f"fill_varlen lengths={lengths} shuffle={shuffle}")
    gen = torch.Generator().manual_seed(sum(lengths) + shuffle)
    B, total = len(lengths), sum(lengths)
    max_pages = max(1, -(-max(lengths) // 16))
    num_pages = B * max_pages + 8
    order = torch.randperm(num_pages, generator=gen) if shuffle else torch.arange(num_pages)
    bt = order[: B * max_pages].view(B, max_pages).to(torch.int32).contiguous()
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    # the runner's k4[0]: [H, T, D] view of [T, H, D] memory
    k = bf((total, HKV, D), gen).permute(1, 0, 2)
    v = bf((total, HKV, D), gen).permute(1, 0, 2)
    kc0, vc0 = bf((num_pages, HKV, 16, D), gen), bf((num_pages, HKV, 16, D), gen)
    kr, vr = kc0.clone(), vc0.clone()
    orc.paged_kv_fill_varlen(kr, vr, k, v, bt, cu)
    kg, vg = kc0.to(dev), vc0.to(dev)
    pkg.paged_kv_fill_varlen(kg, vg, k.permute(1, 0, 2).contiguous().to(dev).permute(1, 0, 2),
                             v.permute(1, 0, 2).contiguous().to(dev).permute(1, 0, 2),
                             bt.to(dev), cu.to(dev), max(lengths))
    assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)
    unused = order[B * max_pages:]
    assert torch.equal(kg.cpu()[unused], kc0[unused])


def test_fill_varlen_generic_strides(pkg, dev):
    """Non-unit innermost stride takes the element-wise path; still bit-exact."""
    say("fill_varlen generic strides")
    gen = torch.Generator().manual_seed(77)
    lengths = [5, 40]
    total = sum(lengths)
    kfull = bf((HKV, D, total), gen)
    k = kfull.permute(0, 2, 1)  # stride_d = total
    v = bf((HKV, total, D), gen)
    bt = rand_table(2, 3, 9, gen)
    cu = torch.tensor([0, 5, 45], dtype=torch.int32)
    kc0, vc0 = bf((9, HKV, 16, D), gen), bf((9, HKV, 16, D), gen)
    kr, vr = kc0.clone(), vc0.clone()
    orc.paged_kv_fill_varlen(kr, vr, k, v, bt, cu)
    kg, vg = kc0.to(dev), vc0.to(dev)
    pkg.paged_kv_fill_varlen(kg, vg, kfull.to(dev).permute(0, 2, 1), v.to(dev), bt.to(dev),
                             cu.to(dev), 40)
    assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)


def test_fill_varlen_golden(pkg, dev):
    say("fill_varlen golden")
    f = C.fill_case()
    kg, vg = f["kc"].to(dev), f["vc"].to(dev)
    pkg.paged_kv_fill_varlen(kg, vg, f["k"].permute(1, 0, 2).contiguous().to(dev).permute(1, 0, 2),
                             f["v"].permute(1, 0, 2).contiguous().to(dev).permute(1, 0, 2),
                             f["bt"].to(dev), f["cu"].to(dev), f["max_seqlen"])
    assert C.digest(kg.cpu(), vg.cpu()) == str(golden()["fill_pool_after_sha"])


def test_paged_kv_fill_single_sequence(pkg, dev):
    say("paged_kv_fill single sequence")
    gen = torch.Generator().manual_seed(5)
    T = 37
    bt = torch.randperm(10, generator=gen)[:3].to(torch.int32)
    k, v = bf((HKV, T, D), gen), bf((HKV, T, D), gen)
    kc0 = bf((10, HKV, 16, D), gen)
    kr, vr = kc0.clone(), kc0.clone()
    orc.paged_kv_fill_varlen(kr, vr, k, v, bt[None], torch.tensor([0, T]))
    kg, vg = kc0.to(dev), kc0.to(dev)
    pkg.paged_kv_fill(kg, vg, k.to(dev), v.to(dev), bt.to(dev))
    assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)


@pytest.mark.parametrize("B", [1, 3, 32])
def test_append_bit_exact(pkg, dev, B):
    say(f"append B={B}")
    gen = torch.Generator().manual_seed(B)
    max_pages = 9
    num_pages = B * max_pages + 2
    bt = rand_table(B, max_pages, num_pages, gen)
    pos = torch.randint(0, max_pages * 16, (B,), generator=gen)
    kc0 = bf((num_pages, HKV, 16, D), gen)
    # k_new as a strided slice of a fused [B, 5120] projection, like the runner's
    fused = bf((B, 5120), gen)
    kn = fused[:, 4096:4608].view(B, HKV, D)
    vn = fused[:, 4608:].view(B, HKV, D)
    kr, vr = kc0.clone(), kc0.clone()
    orc.paged_kv_append(kr, vr, kn, vn, bt, pos)
    fg = fused.to(dev)
    kg, vg = kc0.to(dev), kc0.to(dev)
    pkg.paged_kv_append(kg, vg, fg[:, 4096:4608].view(B, HKV, D), fg[:, 4608:].view(B, HKV, D),
                        bt.to(dev), pos.to(dev))
    assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)


# ------------------------------------------------------------------ RoPE / gate

def test_rope_golden(pkg, dev):
    say("rope golden")
    r = C.rope_case()
    x = r["x"].permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    out = pkg.partial_rope(x, r["pos"].to(dev), r["inv_freq"].to(dev), C.ROTARY)
    assert out.stride() == x.stride()
    ref = torch.from_numpy(golden()["rope_out"])
    close(out, ref, max_abs=2e-2, mean_abs=1e-4, what="rope")
    assert torch.equal(out.cpu()[..., 64:], r["x"][..., 64:])


@pytest.mark.parametrize("shape,R,pos_dtype", [((1, 8, 1, 256), 64, torch.int64),
                                               ((1, 2, 17, 256), 64, torch.int32),
                                               ((2, 3, 65, 128), 64, torch.int32),
                                               ((1, 4, 33, 160), 96, torch.int64),
                                               ((32, 8, 1, 256), 64, torch.int64),
                                               # rotary over the whole head: no tail
                                               ((3, 5, 19, 64), 64, torch.int32),
                                               ((1, 2, 17, 128), 128, torch.int64)])
def test_rope_shapes(pkg, dev, shape, R, pos_dtype):
    say(f"rope shape={shape} R={R}")
    gen = torch.Generator().manual_seed(R + shape[2])
    x = bf(shape, gen)
    B, H, T, Dd = shape
    pos = torch.randint(0, 4096, (B, T), generator=gen).to(pos_dtype)
    inv = C.inv_freq() if R == 64 else 1.0 / (1e7 ** (torch.arange(0, R, 2).float() / R))
    ref = orc.partial_rope(x, pos, inv, R)
    out = pkg.partial_rope(x.to(dev), pos.to(dev), inv.to(dev), R)
    close(out, ref, mean_abs=1e-4, what="rope")
    assert torch.equal(out.cpu()[..., R:], x[..., R:])
    # bf16 rounding of the same fp32 formula: nearly all elements identical
    same = (out.cpu() == ref).float().mean().item()
    assert same > 0.98, same


def test_gate_golden_and_layouts(pkg, dev):
    say("gate golden")
    g = C.gate_case()
    xd = g["x"].permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    gd = g["gate"].permute(0, 2, 1, 3).contiguous().to(dev).permute(0, 2, 1, 3)
    out = pkg.attention_gate_pack(xd, gd)
    assert out.is_contiguous() and out.shape == (17, 2048)
    close(out, torch.from_numpy(golden()["gate_out"]), mean_abs=1e-4, what="gate")
    for T in (1, 3, 17, 65, 129):
        gen = torch.Generator().manual_seed(T)
        x = bf((1, T, 8, 256), gen).permute(0, 2, 1, 3)
        gt = bf((1, T, 8, 256), gen).permute(0, 2, 1, 3)
        ref = orc.gate_pack(x, gt)
        got = pkg.attention_gate_pack(x.to(dev), gt.to(dev))
        close(got, ref, mean_abs=1e-4, what=f"gate T={T}")
        assert (got.cpu() == ref).float().mean().item() > 0.98
    # generic path: non-unit innermost stride
    gen = torch.Generator().manual_seed(1)
    x = bf((1, 8, 256, 5), gen).permute(0, 1, 3, 2)
    gt = bf((1, 8, 5, 256), gen)
    close(pkg.attention_gate_pack(x.to(dev), gt.to(dev)), orc.gate_pack(x, gt), mean_abs=1e-4)


# ------------------------------------------------------------------ decode

def _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos, scratch=None):
    kg, vg = kc.to(dev), vc.to(dev)
    out = pkg.call_paged_gqa_attention_decode_triton(
        q.to(dev), kn.to(dev), vn.to(dev), kg, vg, bt.to(dev), pos.to(dev), scratch)
    return out, kg, vg


def test_decode_golden(pkg, dev):
    say("decode golden")
    d = C.decode_case()
    out, kg, vg = _decode(pkg, dev, d["q"], d["kc"], d["vc"], d["kn"], d["vn"], d["bt"], d["pos"])
    assert C.digest(kg.cpu(), vg.cpu()) == str(golden()["decode_pool_after_sha"])
    close(out, torch.from_numpy(golden()["decode_out"]), what="decode golden")


@pytest.mark.parametrize("lens", [[256], [1], [16], [17], [1, 2, 3, 4, 5],
                                  [31, 2047, 128, 900], [5000], [2048 * 4 + 3]])
def test_decode_vs_oracle(pkg, dev, lens):
    say(f"decode lens={lens}")
    gen = torch.Generator().manual_seed(len(lens) * 1000 + lens[0])
    B = len(lens)
    max_pages = -(-max(lens) // 16) + 1
    num_pages = B * max_pages + 3
    bt = rand_table(B, max_pages, num_pages, gen)
    kc, vc = bf((num_pages, HKV, 16, D), gen), bf((num_pages, HKV, 16, D), gen)
    q, kn, vn = bf((B, HQ, D), gen), bf((B, HKV, D), gen), bf((B, HKV, D), gen)
    pos = torch.tensor([n - 1 for n in lens])
    out, kg, vg = _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos)
    orc.paged_kv_append(kc, vc, kn, vn, bt, pos)
    assert torch.equal(kg.cpu(), kc)
    close(out, orc.paged_decode(q, kc, vc, bt, pos + 1), what=f"decode {lens}")


def test_decode_config2_shape(pkg, dev):
    """B=32, contexts U[128,2048], randperm page table (config 2)."""
    say("decode config2")
    gen = torch.Generator().manual_seed(2)
    lens = torch.randint(128, 2049, (32,), generator=gen).tolist()
    max_pages = 2048 // 16 + 1
    num_pages = 32 * max_pages
    bt = rand_table(32, max_pages, num_pages, gen)
    kc, vc = bf((num_pages, HKV, 16, D), gen), bf((num_pages, HKV, 16, D), gen)
    q, kn, vn = bf((32, HQ, D), gen), bf((32, HKV, D), gen), bf((32, HKV, D), gen)
    pos = torch.tensor([n - 1 for n in lens])
    out, _, _ = _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos)
    orc.paged_kv_append(kc, vc, kn, vn, bt, pos)
    close(out, orc.paged_decode(q, kc, vc, bt, pos + 1), what="config2")


def test_decode_nan_past_pos_does_not_leak(pkg, dev):
    say("decode NaN past pos")
    gen = torch.Generator().manual_seed(11)
    L = 21  # last page partly filled
    bt = rand_table(1, 3, 6, gen)
    kc, vc = bf((6, HKV, 16, D), gen), bf((6, HKV, 16, D), gen)
    q, kn, vn = bf((1, HQ, D), gen), bf((1, HKV, D), gen), bf((1, HKV, D), gen)
    pos = torch.tensor([L - 1])
    clean, _, _ = _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos)
    for t in range(L, 48):
        kc[int(bt[0, t // 16]), :, t % 16] = float("nan")
        vc[int(bt[0, t // 16]), :, t % 16] = float("nan")
    dirty, _, _ = _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos)
    assert torch.isfinite(dirty.cpu().float()).all()
    assert torch.equal(clean.cpu(), dirty.cpu())


def test_decode_dirty_scratch_reuse(pkg, dev):
    """A long sequence leaves every split dirty; a short one must ignore it
    (gqa_attention_decode.py:1115-1131)."""
    say("decode dirty scratch")
    gen = torch.Generator().manual_seed(12)
    scratch = pkg.allocate_split_scratch(HQ, D, batch=1, device=dev)
    for L in (3000, 5):
        bt = rand_table(1, 200, 210, gen)
        kc, vc = bf((210, HKV, 16, D), gen), bf((210, HKV, 16, D), gen)
        q, kn, vn = bf((1, HQ, D), gen), bf((1, HKV, D), gen), bf((1, HKV, D), gen)
        pos = torch.tensor([L - 1])
        out, _, _ = _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos, scratch)
        orc.paged_kv_append(kc, vc, kn, vn, bt, pos)
        close(out, orc.paged_decode(q, kc, vc, bt, pos + 1), what=f"scratch L={L}")


def test_decode_batch_equals_single(pkg, dev):
    say("decode batch == single")
    gen = torch.Generator().manual_seed(13)
    lens = [40, 700, 129]
    B = 3
    bt = rand_table(B, 50, 160, gen)
    kc, vc = bf((160, HKV, 16, D), gen), bf((160, HKV, 16, D), gen)
    q, kn, vn = bf((B, HQ, D), gen), bf((B, HKV, D), gen), bf((B, HKV, D), gen)
    pos = torch.tensor([n - 1 for n in lens])
    full, _, _ = _decode(pkg, dev, q, kc, vc, kn, vn, bt, pos)
    for b in range(B):
        one, _, _ = _decode(pkg, dev, q[b:b + 1], kc, vc, kn[b:b + 1], vn[b:b + 1],
                            bt[b:b + 1], pos[b:b + 1])
        assert torch.equal(one.cpu()[0], full.cpu()[b])


def test_decode_graph_capture_replays(pkg, dev):
    """Capture append+split+combine+gate once; replay with in-graph pos += 1
    (gqa_attention_decode.py:1133-1206).  Each replay is checked."""
    say("decode graph capture")
    gen = torch.Generator().manual_seed(14)
    B, steps = 4, 6
    lens0 = [10, 100, 33, 250]
    bt = rand_table(B, 20, 90, gen)
    kc, vc = bf((90, HKV, 16, D), gen), bf((90, HKV, 16, D), gen)
    q = bf((B, HQ, D), gen)
    gate = bf((1, HQ, B, D), gen)
    kns = [bf((B, HKV, D), gen) for _ in range(steps)]
    vns = [bf((B, HKV, D), gen) for _ in range(steps)]
    kg, vg, btg = kc.to(dev), vc.to(dev), bt.to(dev)
    qg, gateg = q.to(dev), gate.to(dev)
    kn_buf, vn_buf = torch.empty(B, HKV, D, dtype=torch.bfloat16, device=dev), \
        torch.empty(B, HKV, D, dtype=torch.bfloat16, device=dev)
    pos = torch.tensor([n - 1 for n in lens0], device=dev)
    scratch = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)

    def step():
        ctx = pkg.call_paged_gqa_attention_decode_triton(qg, kn_buf, vn_buf, kg, vg, btg, pos,
                                                         scratch)
        o = pkg.attention_gate_pack(ctx.permute(1, 0, 2).unsqueeze(0), gateg)
        pos.add_(1)
        return o

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    kn_buf.copy_(kns[0].to(dev))
    vn_buf.copy_(vns[0].to(dev))
    kg_save, vg_save, pos_save = kg.clone(), vg.clone(), pos.clone()
    with torch.cuda.stream(s):
        step()  # warm up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    kg.copy_(kg_save)
    vg.copy_(vg_save)
    pos.copy_(pos_save)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    kg.copy_(kg_save)
    vg.copy_(vg_save)
    pos.copy_(pos_save)
    torch.cuda.synchronize()
    kr, vr = kc.clone(), vc.clone()
    posr = torch.tensor([n - 1 for n in lens0])
    for i in range(steps):
        kn_buf.copy_(kns[i].to(dev))
        vn_buf.copy_(vns[i].to(dev))
        graph.replay()
        torch.cuda.synchronize()
        orc.paged_kv_append(kr, vr, kns[i], vns[i], bt, posr)
        ctx = orc.paged_decode(q, kr, vr, bt, posr + 1)
        ref = orc.gate_pack(ctx.permute(1, 0, 2).unsqueeze(0).to(torch.bfloat16), gate)
        close(out, ref, what=f"replay {i}")
        assert torch.equal(kg.cpu(), kr)
        posr += 1
        assert torch.equal(pos.cpu(), posr)


# ------------------------------------------------------------------ prefill

def test_prefill_golden(pkg, dev):
    say("prefill golden")
    p = C.prefill_case()
    out = pkg.gqa_attention_varlen_causal(p["q"].to(dev), p["k"].to(dev), p["v"].to(dev),
                                          p["cu"].to(dev), p["max_seqlen"])
    close(out, torch.from_numpy(golden()["prefill_out"]), what="prefill golden")


@pytest.mark.parametrize("lengths", [[7], [16, 16], [1, 3, 17, 64], [3, 100, 1, 64],
                                     [1, 1, 1, 1000], [128] * 32, [300, 65, 64, 63]])
def test_prefill_vs_oracle(pkg, dev, lengths):
    say(f"prefill lengths={lengths}")
    gen = torch.Generator().manual_seed(sum(lengths))
    total = sum(lengths)
    q, k, v = bf((total, HQ, D), gen), bf((total, HKV, D), gen), bf((total, HKV, D), gen)
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    out = pkg.gqa_attention_varlen_causal(q.to(dev), k.to(dev), v.to(dev), cu.to(dev),
                                          max(lengths))
    close(out, orc.varlen_causal(q, k, v, cu), what=f"prefill {lengths}")


def test_prefill_exact_fallback(pkg, dev):
    """Rows whose later scores exceed the first KV tile's maximum by more than
    2^64 (log2 units > 64) take the kernel's exact two-pass path; rows before
    the outlier key and the second sequence take the one-pass path."""
    say("prefill exact fallback")
    gen = torch.Generator().manual_seed(41)
    lengths = [200, 70]
    total = sum(lengths)
    q, k, v = bf((total, HQ, D), gen), bf((total, HKV, D), gen), bf((total, HKV, D), gen)
    q[:200] = 1.0
    k[:200] = (k[:200].float() * 0.05).to(torch.bfloat16)
    k[130, :, :] = 4.0  # q.k = 1024 -> score 64 * log2(e) = 92 above tile 0
    cu = torch.tensor([0, 200, 270], dtype=torch.int32)
    out = pkg.gqa_attention_varlen_causal(q.to(dev), k.to(dev), v.to(dev), cu.to(dev), 200)
    ref = orc.varlen_causal(q, k, v, cu)
    close(out, ref, what="prefill fallback")
    # rows from 130 on attend almost only to token 130
    torch.testing.assert_close(out[140:200].float().cpu(),
                               v[130].float().repeat_interleave(4, 0).expand(60, HQ, D),
                               atol=2e-2, rtol=0)


def test_prefill_strided_inputs(pkg, dev):
    """q/k/v as row-strided views (stride_t != H*D) are addressed correctly."""
    say("prefill strided")
    gen = torch.Generator().manual_seed(21)
    lengths = [50, 90]
    total = sum(lengths)
    big = bf((total, 12, D), gen)
    q, k, v = big[:, :8], big[:, 8:10], big[:, 10:12]
    cu = torch.tensor([0, 50, 140], dtype=torch.int32)
    bg = big.to(dev)
    out = pkg.gqa_attention_varlen_causal(bg[:, :8], bg[:, 8:10], bg[:, 10:12], cu.to(dev), 90)
    close(out, orc.varlen_causal(q, k, v, cu), what="prefill strided")


def test_prefill_then_decode_consistency(pkg, dev):
    """Config-4 shape, scaled down: packed prefill + page scatter into a shuffled
    pool, then one decode step per sequence from those pages.  Decode of token
    L after prefilling 0..L-1 must equal row L of a prefill over 0..L."""
    say("prefill -> decode consistency")
    gen = torch.Generator().manual_seed(31)
    lengths = [16, 1, 77, 300, 1500, 33]
    B = len(lengths)
    ext = [n + 1 for n in lengths]
    total = sum(ext)
    q, k, v = bf((total, HQ, D), gen), bf((total, HKV, D), gen), bf((total, HKV, D), gen)
    cu_ext = torch.tensor([0] + torch.tensor(ext).cumsum(0).tolist(), dtype=torch.int32)
    full = pkg.gqa_attention_varlen_causal(q.to(dev), k.to(dev), v.to(dev), cu_ext.to(dev),
                                           max(ext))
    close(full, orc.varlen_causal(q, k, v, cu_ext), what="full prefill")
    # prefill the first L tokens of every sequence, scatter K/V into pages
    idx = torch.cat([torch.arange(int(cu_ext[b]), int(cu_ext[b]) + lengths[b]) for b in range(B)])
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    max_pages = -(-max(ext) // 16)
    num_pages = B * max_pages + 7
    bt = rand_table(B, max_pages, num_pages, gen)
    kg = torch.zeros(num_pages, HKV, 16, D, dtype=torch.bfloat16, device=dev)
    vg = torch.zeros_like(kg)
    kpk = k[idx].to(dev)
    vpk = v[idx].to(dev)
    pkg.paged_kv_fill_varlen(kg, vg, kpk.permute(1, 0, 2), vpk.permute(1, 0, 2), bt.to(dev),
                             cu.to(dev), max(lengths))
    kr = torch.zeros(num_pages, HKV, 16, D, dtype=torch.bfloat16)
    vr = torch.zeros_like(kr)
    orc.paged_kv_fill_varlen(kr, vr, k[idx].permute(1, 0, 2), v[idx].permute(1, 0, 2), bt, cu)
    assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)
    last = cu_ext[1:].long() - 1
    ctx = pkg.call_paged_gqa_attention_decode_triton(
        q[last].to(dev), k[last].to(dev), v[last].to(dev), kg, vg, bt.to(dev),
        torch.tensor(lengths, dtype=torch.int64, device=dev))
    close(ctx, full.cpu()[last].float(), max_abs=2e-2, mean_abs=2e-3, what="decode vs prefill row")


# ------------------------------------------------------------------ fused decode step

def _lens(n, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


# batches of 16..256 take the balanced workgroup order (one to four chunks of
# 64 sequences in its pass over pos), as do smaller ones over tables of 1024+
# pages (the last two cases); other small batches the direct order.  A
# sequence of more than 16 splits merges in two levels (B=1 x 8195 tokens:
# 128 splits; one 35129-token sequence among 31 short ones: 92 splits).
@pytest.mark.parametrize("lens", [[1], [17, 64, 65], [256], [5000, 3, 700], [2048 * 4 + 3],
                                  _lens(16, 1, 3000, 1), _lens(80, 1, 1000, 2) + [2600],
                                  _lens(256, 1, 300, 3), [35129] + [128] * 31,
                                  [32768], [16400, 1, 60, 33]])
def test_fused_step_equals_three_op_path(pkg, dev, lens):
    """One-launch step == append + split + combine (same device math, same
    rounding): bit-identical output and pools; counters return to zero."""
    say(f"fused vs 3-op B={len(lens)} lens={lens[:8]}")
    gen = torch.Generator().manual_seed(sum(lens))
    B = len(lens)
    max_pages = -(-max(lens) // 16) + 1
    # the step's device-side floor from the total length, where it applies,
    # leaves every sequence's partition as the split op's
    floor = pkg.gqa_attention_decode_paged.min_pages_per_split(B)
    if B <= 256 and (B >= 16 or max_pages >= 1024):
        step_floor = max(floor, -(-HKV * sum(-(-n // 16) for n in lens) // 256))
        assert all(orc.split_partition(n, floor) == orc.split_partition(n, step_floor)
                   for n in lens)
    num_pages = B * max_pages + 3
    bt = rand_table(B, max_pages, num_pages, gen)
    kc, vc = bf((num_pages, HKV, 16, D), gen), bf((num_pages, HKV, 16, D), gen)
    q, kn, vn = bf((B, HQ, D), gen), bf((B, HKV, D), gen), bf((B, HKV, D), gen)
    pos = torch.tensor([n - 1 for n in lens], device=dev)
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    k1, v1 = kc.to(dev), vc.to(dev)
    fused = pkg.call_paged_gqa_attention_decode_triton(q.to(dev), kn.to(dev), vn.to(dev), k1,
                                                       v1, bt.to(dev), pos, sc)
    k2, v2 = kc.to(dev), vc.to(dev)
    plain = pkg.call_paged_gqa_attention_decode_triton(q.to(dev), kn.to(dev), vn.to(dev), k2,
                                                       v2, bt.to(dev), pos, tuple(sc))
    torch.cuda.synchronize()
    assert torch.equal(fused.cpu(), plain.cpu())
    assert torch.equal(k1.cpu(), k2.cpu()) and torch.equal(v1.cpu(), v2.cpu())
    assert int(sc.counters.abs().sum()) == 0
    orc.paged_kv_append(kc, vc, kn, vn, bt, pos.cpu())
    close(fused, orc.paged_decode(q, kc, vc, bt, pos.cpu() + 1), what=f"fused {lens}")


def test_fused_step_split_floor_from_total_length(pkg, dev):
    """B=16 at 24k..32k tokens: the one-launch step raises its split floor
    from the batch's total pages (ceil(2 * sum(npg) / 256) > the 24-page
    floor), a partition the three-op path does not use, so it is checked
    against the oracle (and the three-op path within tolerance)."""
    lens = _lens(16, 24000, 32768, 5)
    say(f"fused work floor B=16 lens={lens[:4]}")
    gen = torch.Generator().manual_seed(5)
    B = len(lens)
    max_pages = -(-max(lens) // 16) + 1
    num_pages = B * max_pages + 3
    bt = rand_table(B, max_pages, num_pages, gen)
    kc, vc = bf((num_pages, HKV, 16, D), gen), bf((num_pages, HKV, 16, D), gen)
    q, kn, vn = bf((B, HQ, D), gen), bf((B, HKV, D), gen), bf((B, HKV, D), gen)
    npg = [-(-n // 16) for n in lens]
    assert -(-2 * sum(npg) // 256) > 24
    pos = torch.tensor([n - 1 for n in lens], device=dev)
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    k1, v1 = kc.to(dev), vc.to(dev)
    fused = pkg.call_paged_gqa_attention_decode_triton(q.to(dev), kn.to(dev), vn.to(dev), k1,
                                                       v1, bt.to(dev), pos, sc)
    k2, v2 = kc.to(dev), vc.to(dev)
    plain = pkg.call_paged_gqa_attention_decode_triton(q.to(dev), kn.to(dev), vn.to(dev), k2,
                                                       v2, bt.to(dev), pos, tuple(sc))
    torch.cuda.synchronize()
    assert int(sc.counters.abs().sum()) == 0
    orc.paged_kv_append(kc, vc, kn, vn, bt, pos.cpu())
    assert torch.equal(k1.cpu(), kc) and torch.equal(v1.cpu(), vc)
    ref = orc.paged_decode(q, kc, vc, bt, pos.cpu() + 1)
    close(fused, ref, what="fused work floor")
    close(fused, plain.float(), what="fused vs 3-op")


def test_decode_attention_step_with_gate(pkg, dev):
    """Runner glue (RoPE + fused append/attention/gate) vs the reference op
    sequence computed by the oracle, on the runner's strided fused-GEMV views."""
    say("decode_attention_step gated")
    gen = torch.Generator().manual_seed(41)
    lens = [33, 1000, 129, 2]
    B = len(lens)
    max_pages = 70
    num_pages = B * max_pages
    bt = rand_table(B, max_pages, num_pages, gen)
    kc, vc = bf((num_pages, HKV, 16, D), gen), bf((num_pages, HKV, 16, D), gen)
    fused_gemv = bf((B, 5120), gen)  # [q 2048 | gate 2048 | k 512 | v 512]
    pos = torch.tensor([n - 1 for n in lens])
    inv = C.inv_freq()
    fg = fused_gemv.to(dev)
    kg, vg = kc.to(dev), vc.to(dev)
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    out = pkg.decode_attention_step(fg[:, :2048].view(B, HQ, D), fg[:, 4096:4608].view(B, HKV, D),
                                    fg[:, 4608:], fg[:, 2048:4096], inv.to(dev), 64, pos.to(dev),
                                    kg, vg, bt.to(dev), sc)
    # reference sequence on the CPU oracle
    q = orc.partial_rope(fused_gemv[:, :2048].view(B, HQ, 1, D), pos.view(B, 1), inv, 64)[:, :, 0]
    k = orc.partial_rope(fused_gemv[:, 4096:4608].view(B, HKV, 1, D), pos.view(B, 1), inv, 64)[:, :, 0]
    v = fused_gemv[:, 4608:].reshape(B, HKV, D)
    orc.paged_kv_append(kc, vc, k, v, bt, pos)
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)
    ctx = orc.paged_decode(q, kc, vc, bt, pos + 1).to(torch.bfloat16)
    gate4 = fused_gemv[:, 2048:4096].reshape(B, HQ, D).permute(1, 0, 2).unsqueeze(0)
    ref = orc.gate_pack(ctx.permute(1, 0, 2).unsqueeze(0), gate4)
    assert out.shape == (B, 2048)
    close(out, ref, what="gated step")


# ------------------------------------------------------------------ q/k norm + attention block

@pytest.mark.parametrize("shape,strided", [((5, 8, 256), True), ((3, 2, 256), True),
                                           ((40, 1024), False), ((7, 3, 256), False)])
def test_qwen_rmsnorm_vs_oracle(pkg, dev, shape, strided):
    say(f"qwen_rmsnorm {shape} strided={strided}")
    gen = torch.Generator().manual_seed(sum(shape))
    d = shape[-1]
    w = bf((d,), gen, 0.3)
    if strided:  # a [B, H, D] view of a wider row, as the fused projection gives
        B, H, _ = shape
        wide = bf((B, 5120), gen, 2.0)
        x = wide[:, 256:256 + H * d].view(B, H, d)
        out = pkg.qwen_rmsnorm(wide.to(dev)[:, 256:256 + H * d].view(B, H, d), w.to(dev), 1e-6)
    else:
        x = bf(shape, gen, 2.0)
        out = pkg.qwen_rmsnorm(x.to(dev), w.to(dev), 1e-6)
    ref = orc.qwen_rmsnorm(x, w, 1e-6)
    assert out.shape == ref.shape and out.is_contiguous()
    # fp32 math rounded to bf16 once: at most one bf16 ulp apart
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=1e-6, rtol=2 ** -7)


def _block_case(gen, lens):
    B = len(lens)
    # the table must cover every sequence's pages: pos is not range-checked on
    # the device (the host allocates pages before the step, engine/paging.py)
    max_pages = -(-max(lens) // 16) + 1
    num_pages = B * max_pages
    return dict(
        B=B, bt=rand_table(B, max_pages, num_pages, gen),
        kc=bf((num_pages, HKV, 16, D), gen), vc=bf((num_pages, HKV, 16, D), gen),
        fused=bf((B, 5120), gen, 1.5), qw=bf((D,), gen, 0.3), kw=bf((D,), gen, 0.3),
        pos=torch.tensor([n - 1 for n in lens]))


def test_decode_block_equals_op_sequence(pkg, dev):
    """One-launch attention block == qwen_rmsnorm -> partial_rope -> fused
    step with gate, bit for bit (output and both caches)."""
    say("decode attention block == op sequence")
    gen = torch.Generator().manual_seed(51)
    c = _block_case(gen, [33, 1000, 129, 2, 16, 17, 512, 1111])
    B = c["B"]
    inv = C.inv_freq().to(dev)
    fg, bt, pos = c["fused"].to(dev), c["bt"].to(dev), c["pos"].to(dev)
    qw, kw = c["qw"].to(dev), c["kw"].to(dev)
    kc1, vc1 = c["kc"].to(dev), c["vc"].to(dev)
    kc2, vc2 = kc1.clone(), vc1.clone()
    sc1 = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    sc2 = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    out1 = pkg.decode_attention_block(fg, qw, kw, 1e-6, inv, 64, pos, kc1, vc1, bt, sc1)
    q = pkg.qwen_rmsnorm(fg[:, :2048].view(B, HQ, D), qw, 1e-6)
    k = pkg.qwen_rmsnorm(fg[:, 4096:4608].view(B, HKV, D), kw, 1e-6)
    out2 = pkg.decode_attention_step(q, k, fg[:, 4608:], fg[:, 2048:4096], inv, 64, pos,
                                     kc2, vc2, bt, sc2)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(out1, out2)
    assert int(sc1.counters.abs().sum()) == 0


def test_decode_block_vs_oracle(pkg, dev):
    """The block against the reference op sequence computed by the oracle."""
    say("decode attention block vs oracle")
    gen = torch.Generator().manual_seed(52)
    c = _block_case(gen, [300, 1, 64, 2000])
    B = c["B"]
    inv = C.inv_freq()
    kg, vg = c["kc"].to(dev), c["vc"].to(dev)
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    out = pkg.decode_attention_block(c["fused"].to(dev), c["qw"].to(dev), c["kw"].to(dev), 1e-6,
                                     inv.to(dev), 64, c["pos"].to(dev), kg, vg, c["bt"].to(dev), sc)
    fused, pos = c["fused"], c["pos"]
    q = orc.qwen_rmsnorm(fused[:, :2048].view(B, HQ, D), c["qw"], 1e-6)
    k = orc.qwen_rmsnorm(fused[:, 4096:4608].view(B, HKV, D), c["kw"], 1e-6)
    q = orc.partial_rope(q.unsqueeze(2), pos.view(B, 1), inv, 64)[:, :, 0]
    k = orc.partial_rope(k.unsqueeze(2), pos.view(B, 1), inv, 64)[:, :, 0]
    v = fused[:, 4608:].reshape(B, HKV, D)
    kc, vc = c["kc"].clone(), c["vc"].clone()
    orc.paged_kv_append(kc, vc, k, v, c["bt"], pos)
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)
    ctx = orc.paged_decode(q, kc, vc, c["bt"], pos + 1).to(torch.bfloat16)
    gate4 = fused[:, 2048:4096].reshape(B, HQ, D).permute(1, 0, 2).unsqueeze(0)
    ref = orc.gate_pack(ctx.permute(1, 0, 2).unsqueeze(0), gate4)
    close(out, ref, what="attention block")


def test_decode_block_graph_replays(pkg, dev):
    """The block captured with an in-graph pos += 1, replayed 4 times with
    eager work in between; every replay equals the eager block."""
    say("decode attention block graph replays")
    gen = torch.Generator().manual_seed(53)
    c = _block_case(gen, [100, 15, 700])
    B = c["B"]
    inv = C.inv_freq().to(dev)
    fg, bt = c["fused"].to(dev), c["bt"].to(dev)
    qw, kw = c["qw"].to(dev), c["kw"].to(dev)
    kc_g, vc_g = c["kc"].to(dev), c["vc"].to(dev)
    kc_e, vc_e = kc_g.clone(), vc_g.clone()
    pos_g, pos_e = c["pos"].to(dev), c["pos"].to(dev)
    sc_g = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    sc_e = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up outside the graph on a throwaway copy
        pkg.decode_attention_block(fg, qw, kw, 1e-6, inv, 64, pos_g.clone(), kc_g.clone(),
                                   vc_g.clone(), bt, pkg.allocate_split_scratch(HQ, D, batch=B,
                                                                                device=dev))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = pkg.decode_attention_block(fg, qw, kw, 1e-6, inv, 64, pos_g, kc_g, vc_g, bt, sc_g)
        pos_g.add_(1)
    for rep in range(4):
        g.replay()
        out_e = pkg.decode_attention_block(fg, qw, kw, 1e-6, inv, 64, pos_e, kc_e, vc_e, bt, sc_e)
        pos_e.add_(1)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), rep
        assert torch.equal(kc_g, kc_e) and torch.equal(vc_g, vc_e), rep


@pytest.mark.parametrize("lens", [[300, 2048, 129, 17, 1000, 1], [5], [4096] * 20])
def test_page_stream_read_reads_each_attended_page_once(pkg, dev, lens):
    """The measurement kernel reads exactly the pages a decode step attends:
    K rows hold 1, V rows 2, every other page 1000, so the total of the
    per-wave sums is 3 * 4096 * (attended pages x heads) exactly (integers in
    fp32 per wave, added in fp64 here) and any extra or missing page shows."""
    say(f"page stream read lens={lens}")
    gen = torch.Generator().manual_seed(len(lens))
    B = len(lens)
    max_pages = -(-max(lens) // 16) + 1
    num_pages = B * max_pages + 3
    bt = torch.randperm(num_pages, generator=gen)[:B * max_pages].view(B, max_pages)
    kc = torch.full((num_pages, HKV, 16, D), 1000.0, dtype=torch.bfloat16)
    vc = kc.clone()
    units = 0
    for b, n in enumerate(lens):
        npg = -(-n // 16)
        units += npg * HKV
        kc[bt[b, :npg].long()] = 1.0
        vc[bt[b, :npg].long()] = 2.0
    pos = torch.tensor([n - 1 for n in lens])
    sums = pkg.page_stream_read(kc.to(dev), vc.to(dev), bt.to(torch.int32).to(dev), pos.to(dev))
    assert float(sums.double().sum()) == 3.0 * 16 * D * units
