"""Pins the CPU oracle with checks that do not restate its formulas:
direct tensor indexing for the page layout, torch SDPA / HF transformers'
RoPE / pure-Python brute force for the float math, and closed-form special
cases.  CPU only."""

import math

import pytest
import torch

from oracle import attention_oracle as orc

HQ, HKV, D = 8, 2, 256


def _bf(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def _table(B, max_pages, num_pages, gen):
    return torch.randperm(num_pages, generator=gen)[: B * max_pages].view(B, max_pages).to(
        torch.int32)


# ------------------------------------------------------------------ page layout

def test_row_index_matches_tensor_indexing():
    gen = torch.Generator().manual_seed(1)
    num_pages, H, Dd = 11, 3, 4
    kc = torch.arange(num_pages * H * 16 * Dd, dtype=torch.float32).view(num_pages, H, 16, Dd)
    bt = torch.randperm(num_pages, generator=gen)[:5].to(torch.int32)
    flat = kc.view(-1, Dd)
    for t in range(5 * 16):
        for h in range(H):
            r = orc.row_index(bt, t, h, H)
            assert torch.equal(flat[r], kc[int(bt[t // 16]), h, t % 16])


@pytest.mark.parametrize("lengths", [[16], [17], [1], [16, 16], [7, 100, 1, 64],
                                     [128] * 8, [1, 1, 1, 1000], [0, 5]])
def test_fill_varlen_oracle_by_indexing(lengths):
    """Every token lands at kc[bt[b, t//16], h, t%16]; nothing else changes
    (reference self-test lengths, gqa_attention_decode_paged.py:1092-1100)."""
    gen = torch.Generator().manual_seed(2)
    B, total = len(lengths), sum(lengths)
    max_pages = max(1, -(-max(lengths) // 16))
    num_pages = B * max_pages + 8
    bt = _table(B, max_pages, num_pages, gen)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32)
    kp, vp = _bf(HKV, total, 8, gen=gen), _bf(HKV, total, 8, gen=gen)
    kc0, vc0 = _bf(num_pages, HKV, 16, 8, gen=gen), _bf(num_pages, HKV, 16, 8, gen=gen)
    kc, vc = kc0.clone(), vc0.clone()
    orc.paged_kv_fill_varlen(kc, vc, kp, vp, bt, cu)
    touched = torch.zeros(num_pages, HKV, 16, dtype=torch.bool)
    for b, n in enumerate(lengths):
        for t in range(n):
            p = int(bt[b, t // 16])
            touched[p, :, t % 16] = True
            for h in range(HKV):
                assert torch.equal(kc[p, h, t % 16], kp[h, int(cu[b]) + t])
                assert torch.equal(vc[p, h, t % 16], vp[h, int(cu[b]) + t])
    assert torch.equal(kc[~touched], kc0[~touched])
    assert torch.equal(vc[~touched], vc0[~touched])


def test_append_oracle_by_indexing():
    gen = torch.Generator().manual_seed(3)
    B, max_pages = 3, 4
    num_pages = B * max_pages + 2
    bt = _table(B, max_pages, num_pages, gen)
    pos = torch.tensor([0, 17, 63])
    kc0 = _bf(num_pages, HKV, 16, 8, gen=gen)
    kc, vc = kc0.clone(), kc0.clone()
    kn, vn = _bf(B, HKV, 8, gen=gen), _bf(B, HKV, 8, gen=gen)
    orc.paged_kv_append(kc, vc, kn, vn, bt, pos)
    diff = (kc != kc0).any(-1)
    assert int(diff.sum()) <= B * HKV
    for b in range(B):
        p = int(pos[b])
        assert torch.equal(kc[int(bt[b, p // 16]), :, p % 16], kn[b])
        assert torch.equal(vc[int(bt[b, p // 16]), :, p % 16], vn[b])


# ------------------------------------------------------------------ decode

def _decode_case(lens, gen, Dd=D, hq=HQ, hkv=HKV):
    B = len(lens)
    max_pages = -(-max(lens) // 16)
    num_pages = B * max_pages + 3
    bt = _table(B, max_pages, num_pages, gen)
    kc, vc = _bf(num_pages, hkv, 16, Dd, gen=gen), _bf(num_pages, hkv, 16, Dd, gen=gen)
    q = _bf(B, hq, Dd, gen=gen)
    return q, kc, vc, bt


def test_decode_oracle_vs_sdpa():
    gen = torch.Generator().manual_seed(4)
    lens = [1, 16, 17, 300]
    q, kc, vc, bt = _decode_case(lens, gen)
    got = orc.paged_decode(q, kc, vc, bt, lens)
    for b, L in enumerate(lens):
        # gather by plain indexing, independent of gather_kv
        k = torch.stack([kc[int(bt[b, t // 16]), :, t % 16] for t in range(L)], 1).float()
        v = torch.stack([vc[int(bt[b, t // 16]), :, t % 16] for t in range(L)], 1).float()
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[b].float()[:, None, :], k, v, enable_gqa=True)[:, 0]
        torch.testing.assert_close(got[b], ref, rtol=1e-5, atol=1e-5)


def test_decode_oracle_brute_force():
    gen = torch.Generator().manual_seed(5)
    Dd, hq, hkv, L = 8, 4, 2, 21
    q, kc, vc, bt = _decode_case([L], gen, Dd, hq, hkv)
    got = orc.paged_decode(q, kc, vc, bt, [L])[0]
    for hh in range(hq):
        kvh = hh // (hq // hkv)
        rows = [(int(bt[0, t // 16]), t % 16) for t in range(L)]
        s = [sum(float(q[0, hh, d]) * float(kc[p, kvh, sl, d]) for d in range(Dd)) / math.sqrt(Dd)
             for p, sl in rows]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        for d in range(Dd):
            ref = sum(w[i] * float(vc[p, kvh, sl, d]) for i, (p, sl) in enumerate(rows)) / z
            assert abs(float(got[hh, d]) - ref) < 1e-5


def test_decode_oracle_uniform_keys_give_mean_of_v():
    gen = torch.Generator().manual_seed(6)
    q, kc, vc, bt = _decode_case([40], gen)
    kc[:] = kc[0, :, 0:1, :]  # every key identical -> uniform softmax
    got = orc.paged_decode(q, kc, vc, bt, [40])[0]
    _, v = orc.gather_kv(kc, vc, bt[0], 40)
    mean = v.mean(1).repeat_interleave(HQ // HKV, 0)
    torch.testing.assert_close(got, mean, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("L", [1, 7, 64, 65, 200, 511, 2100, 4097])
@pytest.mark.parametrize("min_pps", [1, 4, 16, 32])
def test_split_merge_equals_one_shot(L, min_pps):
    """gqa_attention_decode.py:1083-1097: split-K merge == one-shot softmax."""
    gen = torch.Generator().manual_seed(7)
    q, kc, vc, bt = _decode_case([L], gen)
    pos = torch.tensor([L - 1])
    one = orc.paged_decode(q, kc, vc, bt, [L])
    parts = orc.paged_decode_split(q, kc, vc, bt, pos, min_pps)
    assert len(parts[0]) <= orc.MAX_SPLITS
    torch.testing.assert_close(orc.paged_decode_combine(parts), one, rtol=1e-5, atol=1e-5)


def test_split_partition_matches_reference_formula():
    # reference: pps = cdiv(cdiv(L,16),128); splits cover [s*pps, min(..)) (:675-682)
    for L in range(1, 5000, 37):
        npg = -(-L // 16)
        pps = -(-npg // 128)
        parts = orc.split_partition(L, 1)
        assert parts[0][0] == 0 and parts[-1][1] == npg
        assert all(a1 == b0 for (_, a1), (b0, _) in zip(parts, parts[1:]))
        assert all(p1 - p0 <= pps for p0, p1 in parts)


# ------------------------------------------------------------------ prefill

@pytest.mark.parametrize("lengths", [[7], [16, 16], [1, 3, 17, 64], [3, 100, 1, 64]])
def test_varlen_oracle_vs_sdpa(lengths):
    gen = torch.Generator().manual_seed(8)
    total = sum(lengths)
    q, k, v = _bf(total, HQ, D, gen=gen), _bf(total, HKV, D, gen=gen), _bf(total, HKV, D, gen=gen)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32)
    got = orc.varlen_causal(q, k, v, cu)
    s = 0
    for n in lengths:
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[s:s + n].permute(1, 0, 2).float(), k[s:s + n].permute(1, 0, 2).float(),
            v[s:s + n].permute(1, 0, 2).float(), is_causal=True, enable_gqa=True)
        torch.testing.assert_close(got[s:s + n], ref.permute(1, 0, 2), rtol=1e-5, atol=1e-5)
        # first token of each sequence attends only to itself
        torch.testing.assert_close(got[s], v[s].float().repeat_interleave(HQ // HKV, 0))
        s += n


def test_varlen_oracle_brute_force():
    gen = torch.Generator().manual_seed(9)
    lengths, Dd, hq, hkv = [3, 5], 4, 2, 1
    total = sum(lengths)
    q, k, v = _bf(total, hq, Dd, gen=gen), _bf(total, hkv, Dd, gen=gen), _bf(total, hkv, Dd, gen=gen)
    cu = torch.tensor([0, 3, 8], dtype=torch.int32)
    got = orc.varlen_causal(q, k, v, cu)
    for s0, n in ((0, 3), (3, 5)):
        for i in range(n):
            for hh in range(hq):
                sc = [sum(float(q[s0 + i, hh, d]) * float(k[s0 + j, 0, d]) for d in range(Dd))
                      / math.sqrt(Dd) for j in range(i + 1)]
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                for d in range(Dd):
                    ref = sum(w[j] * float(v[s0 + j, 0, d]) for j in range(i + 1)) / sum(w)
                    assert abs(float(got[s0 + i, hh, d]) - ref) < 1e-5


# ------------------------------------------------------------------ elementwise

def _inv_freq(R, theta=1e7):
    return 1.0 / (theta ** (torch.arange(0, R, 2, dtype=torch.float32) / R))


@pytest.mark.parametrize("shape,R", [((1, 8, 33, 256), 64), ((2, 3, 65, 128), 64),
                                     ((1, 4, 33, 160), 96)])
def test_rope_oracle_vs_transformers(shape, R):
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

    gen = torch.Generator().manual_seed(10)
    B, H, T, Dd = shape
    x = _bf(*shape, gen=gen)
    pos = torch.randint(0, 5000, (B, T), generator=gen)
    inv = _inv_freq(R)
    got = orc.partial_rope(x, pos, inv, R)
    ang = pos.float()[..., None] * inv
    emb = torch.cat([ang, ang], -1)
    qe, _ = apply_rotary_pos_emb(x.float(), x.float(), emb.cos(), emb.sin())
    assert torch.equal(got, qe.to(torch.bfloat16))
    assert torch.equal(got[..., R:], x[..., R:])


def test_rope_oracle_special_cases():
    gen = torch.Generator().manual_seed(11)
    x = _bf(1, 2, 9, 256, gen=gen)
    inv = _inv_freq(64)
    zero = orc.partial_rope(x, torch.zeros(1, 9, dtype=torch.int64), inv, 64)
    assert torch.equal(zero, x)  # position 0: identity
    pos = torch.arange(9)[None] * 1000
    xf = x.float()
    out = orc.partial_rope(xf, pos, inv, 64)  # fp32 in -> fp32 out, norm of each pair kept
    n_in = xf[..., :32] ** 2 + xf[..., 32:64] ** 2
    n_out = out[..., :32] ** 2 + out[..., 32:64] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=1e-5, atol=1e-5)


def test_gate_pack_oracle_special_cases():
    gen = torch.Generator().manual_seed(12)
    x = _bf(1, 13, 8, 256, gen=gen).permute(0, 2, 1, 3)
    g0 = torch.zeros_like(x)
    out = orc.gate_pack(x, g0)
    assert out.shape == (13, 8 * 256)
    # sigmoid(0) = 1/2 exactly: halving a bf16 is exact
    assert torch.equal(out, (x.float() / 2).to(torch.bfloat16).permute(0, 2, 1, 3).reshape(13, -1))
    big = torch.full_like(x, 100.0)
    out = orc.gate_pack(x, big)
    for t in (0, 7, 12):
        for h in (0, 5):
            assert torch.equal(out[t, h * 256:(h + 1) * 256], x[0, h, t])


# ------------------------------------------------------------------ qwen_rmsnorm

def test_rmsnorm_oracle_brute_force():
    """Pure-Python restatement with math.sqrt on a few small rows."""
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 256, generator=gen) * 3).to(torch.bfloat16)
    w = (torch.randn(256, generator=gen) * 0.2).to(torch.bfloat16)
    got = orc.qwen_rmsnorm(x, w, 1e-6).float()
    for r in range(3):
        xs = [float(v) for v in x[r]]
        inv = 1.0 / math.sqrt(sum(v * v for v in xs) / 256 + 1e-6)
        for d in range(256):
            want = xs[d] * inv * (1.0 + float(w[d]))
            assert abs(got[r, d].item() - want) <= 2 ** -7 * abs(want) + 1e-6


def test_rmsnorm_oracle_special_cases():
    gen = torch.Generator().manual_seed(6)
    w = (torch.randn(256, generator=gen) * 0.2).to(torch.bfloat16)
    # constant rows: x / rms(x) = sign(c), so y = sign(c) * (1 + w) up to bf16
    for c in (0.5, -3.0, 40.0):
        x = torch.full((2, 256), c, dtype=torch.bfloat16)
        want = (math.copysign(1.0, c) * (1.0 + w.float())).to(torch.bfloat16)
        torch.testing.assert_close(orc.qwen_rmsnorm(x, w, 1e-6), want.expand(2, 256),
                                   atol=0, rtol=2 ** -7)
    # weight 0: every output row has unit RMS
    x = (torch.randn(16, 1024, generator=gen) * 7).to(torch.bfloat16)
    y = orc.qwen_rmsnorm(x, torch.zeros(1024, dtype=torch.bfloat16), 1e-6).float()
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(16), atol=1e-2)
    # power-of-two scaling of the input leaves the output unchanged
    x = torch.randn(4, 256, generator=gen).to(torch.bfloat16)
    assert torch.equal(orc.qwen_rmsnorm(x, w, 1e-12), orc.qwen_rmsnorm(x * 8, w, 1e-12))


def test_gemm_oracle_brute_force():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, 5, generator=g).bfloat16()
    w = torch.randn(4, 5, generator=g).bfloat16()
    ref = orc.gemm_2d(x, w)
    for m in range(3):
        for n in range(4):
            acc = 0.0
            for k in range(5):
                acc += float(x[m, k]) * float(w[n, k])
            assert abs(acc - float(ref[m, n])) < 1e-12


def test_gemm_oracle_special_cases():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(6, 128, generator=g).bfloat16()
    eye = torch.eye(128).bfloat16()
    assert torch.equal(orc.gemm_2d(x, eye).bfloat16(), x)  # identity weight
    sel = torch.zeros(3, 128).bfloat16()
    for n, c in enumerate((7, 0, 127)):
        sel[n, c] = 1.0
    assert torch.equal(orc.gemm_2d(x, sel).bfloat16(), x[:, [7, 0, 127]])  # one-hot rows
    w = torch.randn(9, 128, generator=g).bfloat16()
    x2 = torch.randn(6, 128, generator=g).bfloat16()
    lhs = orc.gemm_2d(x.double() + x2.double(), w)
    assert torch.allclose(lhs, orc.gemm_2d(x, w) + orc.gemm_2d(x2, w), atol=1e-9)
