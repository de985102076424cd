"""CPU oracle of the full-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker / the timed CPU
baseline.  The product path (the HIP library behind ``wy_lib::`` ops) never
calls it.

Every function restates the reference semantics from the mathematics, in
fp32 PyTorch on the CPU (integer/byte work as plain index arithmetic), and
cites the reference lines it follows (sujuyu/qwen3_5-triton-inference-engine).
How each function is pinned by checks independent of this file is listed in
``PINNED``; the tests in tests/test_oracle.py implement those checks.
"""

from __future__ import annotations

import math

import torch

PAGE = 16
MAX_SPLITS = 128

PINNED = {
    "row_index": "brute-force enumeration of the page layout; shuffled-table round trip",
    "paged_kv_append": "row_index closed form; untouched-slot invariant",
    "paged_kv_fill_varlen": "per-sequence append loop equivalence; untouched pages; "
                            "reference length sets (gqa_attention_decode_paged.py:1092-1100)",
    "paged_decode": "torch SDPA (enable_gqa) on gathered K/V; pure-Python brute force; "
                    "uniform-K closed form (mean of V); NaN past pos does not leak",
    "paged_decode_split/combine": "merge == one-shot softmax for every partition",
    "varlen_causal": "per-sequence SDPA is_causal; brute force; row 0 == v_0",
    "partial_rope": "HF transformers qwen3_5 apply_rotary_pos_emb with fp32 cos/sin; "
                    "pos 0 identity; norm preservation; tail bit-exact",
    "gate_pack": "gate=0 -> x/2 exactly; large gate -> x; layout by index identity",
    "qwen_rmsnorm": "pure-Python brute force (math.sqrt); power-of-two scale invariance; "
                    "constant rows -> (1+w)*sign; weight 0 -> unit RMS",
    "gemm_2d": "pure-Python triple loop; identity weight returns x; one-hot weight rows "
               "select columns; linearity in x",
}


# ------------------------------------------------------------------ page layout

def row_index(bt_row: torch.Tensor, t: int, h: int, num_kv_heads: int) -> int:
    """Row of ``k_cache.view(-1, D)`` holding token t, head h
    (engine/paging.py:23, gqa_attention_decode_paged.py:127-144)."""
    return (int(bt_row[t // PAGE]) * num_kv_heads + h) * PAGE + t % PAGE


def paged_kv_append(kc, vc, k_new, v_new, bt, pos) -> None:
    """In place: ``kc[bt[b, p//16], h, p%16] = k_new[b, h]`` with p = pos[b]
    (gqa_attention_decode_paged.py:213-250)."""
    B, H, D = k_new.shape
    kf, vf = kc.view(-1, D), vc.view(-1, D)
    for b in range(B):
        p = int(pos[b])
        for h in range(H):
            r = row_index(bt[b], p, h, H)
            kf[r] = k_new[b, h]
            vf[r] = v_new[b, h]


def paged_kv_fill_varlen(kc, vc, k_packed, v_packed, bt, cu) -> None:
    """In place scatter of packed ``[H, total, D]`` K/V
    (gqa_attention_decode_paged.py:440-489, torch loop :571-588)."""
    H, _, D = k_packed.shape
    kf, vf = kc.view(-1, D), vc.view(-1, D)
    cu = [int(x) for x in cu]
    for b in range(len(cu) - 1):
        start, n = cu[b], cu[b + 1] - cu[b]
        rows = torch.tensor([[row_index(bt[b], t, h, H) for t in range(n)] for h in range(H)],
                            dtype=torch.int64)
        for h in range(H):
            if n:
                kf[rows[h]] = k_packed[h, start:start + n]
                vf[rows[h]] = v_packed[h, start:start + n]


def gather_kv(kc, vc, bt_row, length: int):
    """``[H, L, D]`` fp32 K and V of one sequence through its block table."""
    H, D = kc.shape[1], kc.shape[3]
    t = torch.arange(length)
    phys = bt_row[t // PAGE].to(torch.int64)
    k = kc[phys, :, t % PAGE, :].permute(1, 0, 2).float()
    v = vc[phys, :, t % PAGE, :].permute(1, 0, 2).float()
    return k, v


# ------------------------------------------------------------------ decode

def paged_decode(q, kc, vc, bt, seq_lens) -> torch.Tensor:
    """``[B, Hq, D]`` fp32: ``softmax(q K^T / sqrt(D)) V`` per sequence over its
    first ``seq_lens[b]`` tokens, GQA group Hq/Hkv
    (torch_paged_reference, gqa_attention_decode_paged.py:999-1031)."""
    B, HQ, D = q.shape
    HKV = kc.shape[1]
    G = HQ // HKV
    out = torch.empty(B, HQ, D)
    for b in range(B):
        L = int(seq_lens[b])
        k, v = gather_kv(kc, vc, bt[b], L)
        k = k.repeat_interleave(G, 0)
        v = v.repeat_interleave(G, 0)
        s = torch.einsum("hd,hld->hl", q[b].float(), k) / math.sqrt(D)
        out[b] = torch.einsum("hl,hld->hd", torch.softmax(s, -1), v)
    return out


def split_partition(seq_len: int, min_pps: int = 1):
    """Page ranges of the active splits: npg = ceil(L/16),
    pps = max(ceil(npg/128), min_pps) (gqa_attention_decode_paged.py:675-682)."""
    npg = -(-seq_len // PAGE)
    pps = max(-(-npg // MAX_SPLITS), min_pps)
    nact = -(-npg // pps)
    return [(s * pps, min(s * pps + pps, npg)) for s in range(nact)]


def paged_decode_split(q, kc, vc, bt, pos, min_pps: int = 1):
    """Per-split online-softmax state (m, l, acc) in natural-log units
    (gqa_attention_decode_paged.py:663-733).  Returns lists per sequence."""
    B, HQ, D = q.shape
    HKV = kc.shape[1]
    G = HQ // HKV
    states = []
    for b in range(B):
        L = int(pos[b]) + 1
        k, v = gather_kv(kc, vc, bt[b], L)
        k = k.repeat_interleave(G, 0)
        v = v.repeat_interleave(G, 0)
        s = torch.einsum("hd,hld->hl", q[b].float(), k) / math.sqrt(D)
        per = []
        for p0, p1 in split_partition(L, min_pps):
            t0, t1 = p0 * PAGE, min(p1 * PAGE, L)
            ss = s[:, t0:t1]
            m = ss.max(-1).values
            p = torch.exp(ss - m[:, None])
            per.append((m, p.sum(-1), torch.einsum("hl,hld->hd", p, v[:, t0:t1])))
        states.append(per)
    return states


def paged_decode_combine(states) -> torch.Tensor:
    """``out = sum_s a_s acc_s / sum_s a_s l_s``, ``a_s = exp(m_s - max m)``
    (gqa_attention_decode_paged.py:776-812)."""
    outs = []
    for per in states:
        m = torch.stack([x[0] for x in per])
        l = torch.stack([x[1] for x in per])
        acc = torch.stack([x[2] for x in per])
        a = torch.exp(m - m.max(0).values)
        outs.append((a[:, :, None] * acc).sum(0) / (a * l).sum(0)[:, None])
    return torch.stack(outs)


# ------------------------------------------------------------------ prefill

def varlen_causal(q, k, v, cu) -> torch.Tensor:
    """``[total, Hq, D]`` fp32 causal GQA attention per packed sequence
    (torch_varlen_reference, gqa_attention_varlen_causal.py:301-330)."""
    total, HQ, D = q.shape
    G = HQ // k.shape[1]
    out = torch.empty(total, HQ, D)
    cu = [int(x) for x in cu]
    for b in range(len(cu) - 1):
        s0, s1 = cu[b], cu[b + 1]
        n = s1 - s0
        if n == 0:
            continue
        qs = q[s0:s1].permute(1, 0, 2).float()
        ks = k[s0:s1].permute(1, 0, 2).float().repeat_interleave(G, 0)
        vs = v[s0:s1].permute(1, 0, 2).float().repeat_interleave(G, 0)
        sc = qs @ ks.transpose(1, 2) / math.sqrt(D)
        mask = torch.triu(torch.ones(n, n, dtype=torch.bool), 1)
        sc = sc.masked_fill(mask, float("-inf"))
        out[s0:s1] = (torch.softmax(sc, -1) @ vs).permute(1, 0, 2)
    return out


# ------------------------------------------------------------------ elementwise

def partial_rope(x, position_ids, inv_freq, rotary_dim: int) -> torch.Tensor:
    """bf16 ``[B, H, T, D]``: rotate-half on ``[0, R)`` with fp32
    ``cos/sin(float(pos) * inv_freq)``, tail copied (partial_rope.py:60-132,
    reference torch version :220-236)."""
    half = rotary_dim // 2
    ang = position_ids.float().unsqueeze(-1) * inv_freq.view(1, 1, half)
    cos = torch.cos(ang).unsqueeze(1)
    sin = torch.sin(ang).unsqueeze(1)
    x1 = x[..., :half].float()
    x2 = x[..., half:rotary_dim].float()
    out = x.clone()
    out[..., :half] = (x1 * cos - x2 * sin).to(x.dtype)
    out[..., half:rotary_dim] = (x1 * sin + x2 * cos).to(x.dtype)
    return out


def qwen_rmsnorm(x, weight, eps: float) -> torch.Tensor:
    """bf16 ``x * rsqrt(mean(x^2) + eps) * (1 + weight)`` over the last dim in
    fp32 (qwen_rmsnorm.py:69-73, torch version :165-174)."""
    xf = x.float()
    ms = (xf * xf).mean(dim=-1, keepdim=True)
    return (xf * torch.rsqrt(ms + eps) * (1.0 + weight.float())).to(x.dtype)


def gate_pack(x, gate) -> torch.Tensor:
    """bf16 ``[T, H*D]`` = ``x * sigmoid(gate)`` of ``[1, H, T, D]`` inputs
    (attention_gate_pack.py:34-63, torch version :148-157)."""
    B, H, T, D = x.shape
    out = x.float() * torch.sigmoid(gate.float())
    return out.permute(0, 2, 1, 3).reshape(B * T, H * D).to(x.dtype)


def gemm_2d(x, weight) -> torch.Tensor:
    """fp64 ``x @ weight.T`` of bf16 inputs (the reference's own check,
    ``torch.nn.functional.linear``, gemm_2d.py:240-250); the kernel rounds its
    fp32 sum to bf16 once."""
    return x.double() @ weight.double().T
