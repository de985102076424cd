"""The whole decode step (decoder.DecodeModel / GraphedDecoder) on the GPU.

* fused mixer blocks == the reference op sequence, bit for bit, over several
  steps (tokens, hidden, every cache);
* a 2-layer model (one GDN, one attention layer) against a CPU chain of the
  pinned oracles: hidden within bf16 tolerance, the greedy token within
  0.05 of the best float64 logit;
* the captured graph (step + argmax + pos += 1 + token feedback) replayed
  N times == N eager steps, bit for bit.
"""

import sys

import pytest
import torch

from oracle import attention_oracle as ao
from oracle import gdn_oracle as go
from oracle import model_oracle as mo

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def tiny_cfg(pkg, layers=2, vocab=4096):
    from qwen35_amd.decoder import DecoderConfig
    return DecoderConfig(num_layers=layers, full_attention_interval=2, vocab=vocab)


def build(pkg, dev, cfg, B, max_len, fused, seed=0):
    from qwen35_amd.decoder import DecodeModel, random_weights
    w = random_weights(cfg, seed=seed, device=dev)
    return DecodeModel(cfg, w, batch=B, max_len=max_len, device=dev, fused_mixers=fused)


def states(m):
    ts = [m.attn.pos, *m.attn.k_caches, *m.attn.v_caches]
    return ts + [t for t in m.conv_states + m.rec_states if t is not None]


@pytest.mark.parametrize("B", [5, 20])
def test_fused_blocks_equal_op_sequence(pkg, dev, B):
    """B=5 runs the fused RMSNorm / SwiGLU GEMM prologues, B=20 the separate
    launches with the mixer blocks; both equal the op sequence."""
    say(f"decoder fused vs op sequence, 4 layers, B={B}, 4 steps")
    cfg = tiny_cfg(pkg, layers=4)
    a = build(pkg, dev, cfg, B, 64, True)
    b = build(pkg, dev, cfg, B, 64, False)
    tok = torch.arange(B, dtype=torch.int64, device=dev) * 97 % 4096
    ta, tb = tok.clone(), tok.clone()
    for step in range(4):
        ha, hb = a.decode_step(ta), b.decode_step(tb)
        assert torch.equal(ha, hb), f"hidden differs at step {step}"
        ta = pkg.lm_head_argmax(ha, a.embed, False)
        tb = pkg.lm_head_argmax(hb, b.embed, False)
        a.pos.add_(1)
        b.pos.add_(1)
        assert torch.equal(ta, tb)
    for x, y in zip(states(a), states(b)):
        assert torch.equal(x, y)


def gm(x, w):
    """gemm_2d as the kernel returns it: the float64 product rounded to bf16 once."""
    return ao.gemm_2d(x, w).to(torch.bfloat16)


def oracle_step(m, tokens, kcs, vcs, convs, recs):
    """CPU chain of the oracles for one decode step of DecodeModel m (its
    weights copied to the host); mutates the host caches."""
    cfg = m.cfg
    B = tokens.shape[0]
    pos = m.pos.cpu()
    bt = m.attn.block_table.cpu()
    inv = m.inv_freq.cpu()
    x = mo.embedding_gather(tokens.cpu(), m.embed.cpu())
    for i, w in enumerate(m.layers):
        res = x
        h = ao.qwen_rmsnorm(x, w.input_layernorm.cpu(), cfg.eps)
        fused = gm(h, w.in_proj.cpu())
        if cfg.is_attention(i):
            a = m.attn_index[i]
            qd, kd = cfg.num_q_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
            q = ao.qwen_rmsnorm(fused[:, :qd].reshape(B, cfg.num_q_heads, cfg.head_dim),
                                w.extra["q_norm"].cpu(), cfg.eps)
            k = ao.qwen_rmsnorm(fused[:, 2 * qd:2 * qd + kd].reshape(B, cfg.num_kv_heads,
                                                                     cfg.head_dim),
                                w.extra["k_norm"].cpu(), cfg.eps)
            v = fused[:, 2 * qd + kd:].reshape(B, cfg.num_kv_heads, cfg.head_dim)
            gate = fused[:, qd:2 * qd].reshape(B, cfg.num_q_heads, cfg.head_dim)
            q = ao.partial_rope(q[:, :, None], pos[:, None], inv, cfg.rotary_dim)[:, :, 0]
            k = ao.partial_rope(k[:, :, None], pos[:, None], inv, cfg.rotary_dim)[:, :, 0]
            ao.paged_kv_append(kcs[a], vcs[a], k, v, bt, pos)
            o = ao.paged_decode(q, kcs[a], vcs[a], bt, pos + 1).to(torch.bfloat16)
            o = ao.gate_pack(o.permute(1, 0, 2)[None], gate.permute(1, 0, 2)[None])
            h = gm(o, w.out_proj.cpu())
        else:
            HD = cfg.lin_heads * cfg.lin_head_dim
            H, D = cfg.lin_heads, cfg.lin_head_dim
            y, convs[i] = go.conv4_decode(fused[:, :3 * HD], convs[i], w.extra["conv"].cpu())
            qn, kn, beta, g = go.gdn_qk_norm_gates(
                y[:, :HD].reshape(B, H, D), y[:, HD:2 * HD].reshape(B, H, D),
                fused[:, 4 * HD:4 * HD + H], fused[:, 4 * HD + H:], w.extra["a_log"].cpu(),
                w.extra["dt_bias"].cpu())
            core, recs[i] = go.gdn_decode(qn, kn, y[:, 2 * HD:].reshape(B, H, D), beta, g,
                                          recs[i])
            normed = go.gdn_gated_rmsnorm(core.to(torch.bfloat16),
                                          fused[:, 3 * HD:4 * HD].reshape(B, H, D),
                                          w.extra["norm"].cpu())
            h = gm(normed.reshape(B, HD), w.out_proj.cpu())
        x = mo.residual_add(h, res)
        res = x
        h = ao.qwen_rmsnorm(x, w.post_attention_layernorm.cpu(), cfg.eps)
        gu = gm(h, w.gate_up.cpu())
        h = mo.swiglu(gu[:, :cfg.intermediate], gu[:, cfg.intermediate:])
        h = gm(h, w.down_proj.cpu())
        x = mo.residual_add(h, res)
    return ao.qwen_rmsnorm(x, m.final_norm.cpu(), cfg.eps)


def test_two_layer_model_vs_oracle_chain(pkg, dev):
    say("decoder 2 layers vs oracle chain, B=3, 3 steps")
    cfg = tiny_cfg(pkg, layers=2)
    m = build(pkg, dev, cfg, 3, 48, True, seed=5)
    m.pos.fill_(5)  # a few zero-valued cached tokens precede the decode
    kcs = [k.cpu().clone() for k in m.attn.k_caches]
    vcs = [v.cpu().clone() for v in m.attn.v_caches]
    convs = [c.cpu().clone() if c is not None else None for c in m.conv_states]
    recs = [r.cpu().clone() if r is not None else None for r in m.rec_states]
    tok = torch.tensor([11, 2000, 4000], dtype=torch.int64, device=dev)
    for step in range(3):
        ref = oracle_step(m, tok, kcs, vcs, convs, recs)
        hid = m.decode_step(tok)
        torch.cuda.synchronize()
        torch.testing.assert_close(hid.float().cpu(), ref.float(), atol=5e-2, rtol=5e-2)
        logits = mo.lm_head_logits(ref, m.embed.cpu())
        nxt = pkg.lm_head_argmax(hid, m.embed, False)
        for r, t in enumerate(nxt.cpu().tolist()):
            assert logits[r, t] >= logits[r].max() - 0.05, (step, r)
        m.pos.add_(1)
        tok = nxt
    for a, k in enumerate(m.attn.k_caches):
        torch.testing.assert_close(k.cpu().float(), kcs[a].float(), atol=5e-2, rtol=5e-2)


@pytest.mark.parametrize("B", [4, 20])
def test_graphed_decoder_replays_equal_eager_steps(pkg, dev, B):
    """B=4: the GEMM prologue fusions; B=20: the mixer blocks with add_rmsnorm
    and the gate/up SwiGLU epilogue, whose split-K counters must be back at
    zero for every replay."""
    say(f"graphed decoder 4 layers, B={B}, 5 replays")
    from qwen35_amd.decoder import GraphedDecoder
    cfg = tiny_cfg(pkg, layers=4)
    eager = build(pkg, dev, cfg, B, 32, True, seed=3)
    graphed = build(pkg, dev, cfg, B, 32, True, seed=3)
    tok = torch.arange(5, 5 + B, dtype=torch.int64, device=dev)
    g = GraphedDecoder(graphed, tok)
    t = tok.clone()
    for i in range(5):
        t = eager.next_tokens(t)
        got = g.step()
        torch.cuda.synchronize()
        assert torch.equal(got, t), f"replay {i}"
    for x, y in zip(states(eager), states(graphed)):
        assert torch.equal(x, y)


def test_prefill_then_decode_equals_token_by_token_decode(pkg, dev):
    """Packed prefill of three prompts then two decode steps, against feeding
    the same prompts through the decode step one token at a time: the same
    caches (K/V pages, conv and recurrent states) up to kernel rounding, and
    the same greedy tokens where the float64 margin is clear."""
    say("decoder prefill [5, 17, 33] + 2 decode steps vs token-by-token decode")
    cfg = tiny_cfg(pkg, layers=4)
    lengths = [5, 17, 33]
    B = len(lengths)
    a = build(pkg, dev, cfg, B, 48, True, seed=21)
    b = build(pkg, dev, cfg, B, 48, True, seed=21)
    gen = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen) for n in lengths]
    first = a.prefill(torch.cat(prompts).to(dev), lengths)
    assert torch.equal(a.pos.cpu(), torch.tensor(lengths))
    # token by token: all sequences step together; a finished prompt repeats
    # its last step on a scratch model copy, so only the per-sequence caches
    # of the final step of each prompt are compared
    hid_b = {}
    for t in range(max(lengths)):
        tok = torch.tensor([p[min(t, len(p) - 1)] for p in prompts], device=dev)
        snap = [x.clone() for x in states(b)]
        h = b.decode_step(tok)
        for r, n in enumerate(lengths):
            if t >= n:  # restore sequence r: it is already complete
                for x, y in zip(states(b), snap):
                    if x.ndim > 0 and x.shape[0] == B:
                        x[r].copy_(y[r])
            elif t == n - 1:
                hid_b[r] = h[r].clone()
        b.pos.add_(torch.tensor([1 if t < n else 0 for n in lengths], device=dev))
    assert torch.equal(b.pos.cpu(), torch.tensor(lengths))
    for r in range(B):
        logits = mo.lm_head_logits(hid_b[r].cpu()[None], a.embed.cpu())[0]
        assert logits[int(first[r])] >= logits.max() - 0.05, r
    for i in range(cfg.num_layers):
        if a.conv_states[i] is not None:
            torch.testing.assert_close(a.conv_states[i].float(), b.conv_states[i].float(),
                                       atol=3e-2, rtol=3e-2)
            torch.testing.assert_close(a.rec_states[i], b.rec_states[i], atol=2e-2, rtol=2e-2)
    # the prompt positions of every K/V page (slot n of a finished prompt was
    # rewritten by its repeated steps and is excluded)
    bt = a.attn.block_table.cpu()
    for pool_a, pool_b in ((a.attn.k_caches, b.attn.k_caches), (a.attn.v_caches, b.attn.v_caches)):
        for ka, kb in zip(pool_a, pool_b):
            for r, n in enumerate(lengths):
                t = torch.arange(n)
                pages = bt[r, t // 16].long()
                ga = ka.cpu()[pages, :, t % 16].float()
                gb = kb.cpu()[pages, :, t % 16].float()
                # two kernel paths through 4 layers of bf16 activations:
                # mean error within 1% of the mean magnitude, max within 0.1
                err = (ga - gb).abs()
                scale = gb.abs().mean()
                assert err.max() <= 0.1 and err.mean() <= 1e-2 * scale, (err.max(), err.mean(),
                                                                          scale)
    # decode continues from both states the same way
    ta, tb = first.clone(), first.clone()
    for step in range(2):
        ha, hb = a.decode_step(ta), b.decode_step(tb)
        torch.testing.assert_close(ha.float(), hb.float(), atol=5e-2, rtol=5e-2)
        ta = pkg.lm_head_argmax(ha, a.embed, False)
        tb = ta.clone()
        a.pos.add_(1)
        b.pos.add_(1)


def test_long_prompt_prefill_chunked_equals_sequential(pkg, dev, monkeypatch):
    """One 2100-token prompt takes the chunk-64 GDN prefill (engine/runner.py:
    272-273); the same prompt with the routing threshold raised takes the
    sequential kernel: the recurrent and conv states, the K/V pages and the
    next decode step agree within the kernels' rounding."""
    say("decoder long-prompt prefill: chunked vs sequential GDN")
    import qwen35_amd.decoder as dmod
    cfg = tiny_cfg(pkg, layers=4)
    L = 2100
    gen = torch.Generator().manual_seed(8)
    prompt = torch.randint(0, cfg.vocab, (L,), generator=gen).to(dev)
    a = build(pkg, dev, cfg, 1, L + 8, True, seed=31)
    b = build(pkg, dev, cfg, 1, L + 8, True, seed=31)
    assert dmod.GDN_CHUNKED_PREFILL_MIN_TOKENS <= L
    ta = a.prefill(prompt, [L])
    monkeypatch.setattr(dmod, "GDN_CHUNKED_PREFILL_MIN_TOKENS", L + 1)
    tb = b.prefill(prompt, [L])
    torch.cuda.synchronize()
    # the first GDN layer sees identical inputs: the kernels' own bound; later
    # layers see activations that already differ by bf16 roundings
    first = True
    for i in range(cfg.num_layers):
        if a.rec_states[i] is not None:
            tol = 2e-4 if first else 3e-2
            torch.testing.assert_close(a.rec_states[i], b.rec_states[i], atol=tol, rtol=tol)
            if first:
                assert torch.equal(a.conv_states[i], b.conv_states[i])
            first = False
    # K/V pages written from those activations: two kernel paths through 4
    # layers of bf16 activations, the bound of the packed-prefill test above
    # with the max widened for 2100 tokens' worth of extremes (0.1 -> 0.15)
    for ka, kb in zip(a.attn.k_caches + a.attn.v_caches, b.attn.k_caches + b.attn.v_caches):
        ka, kb = ka.float(), kb.float()
        err = (ka - kb).abs()
        scale = kb.abs().mean()
        assert err.max() <= 0.15 and err.mean() <= 1e-2 * scale, (err.max(), err.mean(), scale)
    ha, hb = a.decode_step(ta), b.decode_step(ta)
    torch.testing.assert_close(ha.float(), hb.float(), atol=5e-2, rtol=5e-2)
