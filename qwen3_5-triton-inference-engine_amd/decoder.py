"""A whole Qwen3.5 decode step on the MI355X kernels, and its graph-captured
form (the reference's ``Runner.decode_step`` and ``GraphedDecoder``,
engine/runner.py:520-567 and :859-954).

The model here is built from random weights with the checkpoint's shapes (no
checkpoint is available offline): 24 layers, every 4th a full-attention
layer (8 q / 2 kv heads of 256, partial RoPE on 64 dims, theta 1e7), the
others Gated DeltaNet layers (16 heads of 128), hidden 1024, MLP 3584, a tied
248320 x 1024 embedding / LM head.  Per layer a decode step runs

    rmsnorm -> fused projection GEMV -> mixer block (one launch) -> out GEMV
    -> residual add -> rmsnorm -> gate_up GEMV -> SwiGLU -> down GEMV -> residual add

where the mixer block is ``wy_lib::paged_gqa_attention_decode_block`` or
``wy_lib::gdn_decode_block`` (``fused_mixers=True``) or the reference's op
sequence (``False``; bit-identical).  ``GraphedDecoder`` captures the step,
the LM-head argmax, ``pos += 1`` and the feedback of the new token into one
HIP graph, so generating a token is one graph replay.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .attention import (
    build_packed_batch,
    decode_attention_block,
    decode_attention_step,
    prefill_attention_block,
)
from .depthwise_causal_conv4_decode import conv_state_from_packed_prefill
from .depthwise_causal_conv4_prefill import depthwise_causal_conv4_prefill
from .gdn_gated_rmsnorm import gdn_gated_rmsnorm
from .gdn_qk_norm_gates import gdn_qk_norm_gates
from .gdn_recurrent_prefill import (
    call_gdn_recurrent_prefill_chunked_triton,
    gdn_prefill_sequential_into,
)

# A single prompt at least this long takes the chunk-64 GDN prefill (the
# reference's routing threshold, engine/runner.py:151-153); packed batches and
# shorter prompts take the sequential kernel.
GDN_CHUNKED_PREFILL_MIN_TOKENS = 2048
from .cache import allocate_attn_caches
from .embedding_gather import embedding_gather
from .gemm_2d import gate_up_swiglu, gemm_2d, rmsnorm_gemm_2d, swiglu_gemm_2d
from .gdn_mixer import gdn_decode_block, gdn_decode_ops
from .partial_rope import rope_inv_freq
from .qwen_rmsnorm import add_rmsnorm, qwen_rmsnorm
from .residual_add import residual_add
from .swiglu import swiglu
from .vocab_argmax import lm_head_argmax


# Above this batch the skinny GEMM's per-workgroup re-reads of its A rows
# (every column block reads all M rows) make the fused RMSNorm / SwiGLU
# prologues cost more than the launches they save (measured: B=32 step
# 1.83 -> 2.02 ms with them, B=1 1.23 -> 1.15 ms).
FUSED_PROLOGUE_MAX_BATCH = 16


@dataclass
class DecoderConfig:
    """Qwen3.5 text-model shapes (the reference loader's text_config,
    engine/loader.py:240-262)."""
    hidden: int = 1024
    num_layers: int = 24
    full_attention_interval: int = 4
    vocab: int = 248320
    intermediate: int = 3584
    lin_heads: int = 16
    lin_head_dim: int = 128
    num_q_heads: int = 8
    num_kv_heads: int = 2
    head_dim: int = 256
    rotary_dim: int = 64
    rope_theta: float = 1e7
    eps: float = 1e-6

    def is_attention(self, i: int) -> bool:
        return (i + 1) % self.full_attention_interval == 0


@dataclass
class LayerWeights:
    input_layernorm: torch.Tensor
    post_attention_layernorm: torch.Tensor
    gate_up: torch.Tensor        # [2*I, H]
    down_proj: torch.Tensor      # [H, I]
    in_proj: torch.Tensor        # attention: q|gate|k|v [5120, H]; GDN: qkv|z|a|b [8224, H]
    out_proj: torch.Tensor       # attention o_proj [H, 2048]; GDN out_proj [H, 2048]
    extra: dict = field(default_factory=dict)  # q_norm/k_norm or conv/a_log/dt_bias/norm


def random_weights(cfg: DecoderConfig, *, seed: int = 0, device="cuda"):
    """Random-init weights with the checkpoint's shapes and dtypes; projection
    scales keep the activations O(1) through 24 layers."""
    gen = torch.Generator(device=device).manual_seed(seed)

    def rnd(*shape, scale=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=gen, device=device) * scale).to(dtype)

    H = cfg.hidden
    layers = []
    for i in range(cfg.num_layers):
        common = dict(
            input_layernorm=rnd(H, scale=0.1), post_attention_layernorm=rnd(H, scale=0.1),
            gate_up=rnd(2 * cfg.intermediate, H, scale=H ** -0.5),
            down_proj=rnd(H, cfg.intermediate, scale=cfg.intermediate ** -0.5 * 0.5))
        if cfg.is_attention(i):
            qd, kd = cfg.num_q_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
            layers.append(LayerWeights(
                **common, in_proj=rnd(2 * qd + 2 * kd, H, scale=H ** -0.5),
                out_proj=rnd(H, qd, scale=qd ** -0.5 * 0.5),
                extra=dict(q_norm=rnd(cfg.head_dim, scale=0.1),
                           k_norm=rnd(cfg.head_dim, scale=0.1))))
        else:
            hd = cfg.lin_heads * cfg.lin_head_dim
            layers.append(LayerWeights(
                **common, in_proj=rnd(4 * hd + 2 * cfg.lin_heads, H, scale=H ** -0.5),
                out_proj=rnd(H, hd, scale=hd ** -0.5 * 0.5),
                extra=dict(
                    conv=rnd(4, 3 * hd, scale=0.5),
                    a_log=torch.log(torch.rand(cfg.lin_heads, generator=gen, device=device)
                                    * 15 + 1),
                    dt_bias=rnd(cfg.lin_heads),
                    norm=1 + 0.1 * torch.randn(cfg.lin_head_dim, generator=gen,
                                               device=device))))
    embed = rnd(cfg.vocab, H, scale=0.05)
    final_norm = rnd(H, scale=0.1)
    return layers, embed, final_norm


class DecodeModel:
    """Decode-time model state: weights plus the per-sequence caches (paged
    KV per attention layer, conv and recurrent state per GDN layer)."""

    def __init__(self, cfg: DecoderConfig, weights, *, batch: int, max_len: int,
                 device="cuda", fused_mixers: bool = True):
        self.cfg = cfg
        self.layers, self.embed, self.final_norm = weights
        self.batch = batch
        self.fused_mixers = fused_mixers
        self.device = torch.device(device)
        n_attn = sum(cfg.is_attention(i) for i in range(cfg.num_layers))
        self.attn = allocate_attn_caches(n_attn, max_len, batch=batch,
                                         num_q_heads=cfg.num_q_heads,
                                         num_kv_heads=cfg.num_kv_heads,
                                         head_dim=cfg.head_dim, device=device)
        self.attn.reserve(max_len)
        hd = cfg.lin_heads * cfg.lin_head_dim
        self.conv_states, self.rec_states, self.attn_index = [], [], []
        a = 0
        for i in range(cfg.num_layers):
            if cfg.is_attention(i):
                self.conv_states.append(None)
                self.rec_states.append(None)
                self.attn_index.append(a)
                a += 1
            else:
                self.conv_states.append(torch.zeros(batch, 4, 3 * hd, dtype=torch.bfloat16,
                                                    device=device))
                self.rec_states.append(torch.zeros(batch, cfg.lin_heads, cfg.lin_head_dim,
                                                   cfg.lin_head_dim, dtype=torch.float32,
                                                   device=device))
                self.attn_index.append(-1)
        self.inv_freq = rope_inv_freq(cfg.rotary_dim, cfg.rope_theta, device=device)

    @property
    def pos(self) -> torch.Tensor:
        return self.attn.pos

    # ------------------------------------------------------------------ mixers
    def _attention(self, h, w: LayerWeights, a: int):
        cfg, B = self.cfg, h.shape[0]
        fused = gemm_2d(h, w.in_proj)
        kc, vc = self.attn.k_caches[a], self.attn.v_caches[a]
        if self.fused_mixers:
            o = decode_attention_block(fused, w.extra["q_norm"], w.extra["k_norm"], cfg.eps,
                                       self.inv_freq, cfg.rotary_dim, self.attn.pos, kc, vc,
                                       self.attn.block_table, self.attn.split_scratch)
        else:
            qd, kd = cfg.num_q_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
            q = qwen_rmsnorm(fused[:, :qd].view(B, cfg.num_q_heads, cfg.head_dim),
                             w.extra["q_norm"], cfg.eps)
            k = qwen_rmsnorm(fused[:, 2 * qd:2 * qd + kd].view(B, cfg.num_kv_heads,
                                                               cfg.head_dim),
                             w.extra["k_norm"], cfg.eps)
            o = decode_attention_step(q, k, fused[:, 2 * qd + kd:], fused[:, qd:2 * qd],
                                      self.inv_freq, cfg.rotary_dim, self.attn.pos, kc, vc,
                                      self.attn.block_table, self.attn.split_scratch)
        return gemm_2d(o, w.out_proj)

    def _gdn(self, h, w: LayerWeights, i: int):
        fused = gemm_2d(h, w.in_proj)
        fn = gdn_decode_block if self.fused_mixers else gdn_decode_ops
        normed = fn(fused, self.conv_states[i], w.extra["conv"], w.extra["a_log"],
                    w.extra["dt_bias"], w.extra["norm"], self.rec_states[i])
        return gemm_2d(normed, w.out_proj)

    # -------------------------------------------------------------- one step
    def decode_step(self, token_ids: torch.Tensor) -> torch.Tensor:
        """Advance every sequence by one token: ``token_ids [B]`` -> final-norm
        hidden ``[B, H]``.  Writes K/V at ``pos`` and advances the GDN states;
        does not advance ``pos`` (engine/runner.py:520-567).  With
        ``fused_mixers`` each residual add + RMSNorm runs inside the next
        projection's launch and SwiGLU inside the down projection's
        (bit-identical to the separate ops)."""
        if not self.fused_mixers:
            return self._decode_step_ops(token_ids)
        if self.batch > FUSED_PROLOGUE_MAX_BATCH:
            return self._decode_step_blocks(token_ids)
        cfg = self.cfg
        x = embedding_gather(token_ids, self.embed)
        h = None  # the previous sub-block's output, not yet added to x
        for i, w in enumerate(self.layers):
            fused, x = rmsnorm_gemm_2d(x, h, w.input_layernorm, cfg.eps, w.in_proj)
            if cfg.is_attention(i):
                h = self._attention_from(fused, w, self.attn_index[i])
            else:
                h = self._gdn_from(fused, w, i)
            gate_up, x = rmsnorm_gemm_2d(h, x, w.post_attention_layernorm, cfg.eps, w.gate_up)
            h = swiglu_gemm_2d(gate_up, w.down_proj)
        x = residual_add(h, x)
        return qwen_rmsnorm(x, self.final_norm, cfg.eps)

    def _attention_from(self, fused, w: LayerWeights, a: int):
        cfg = self.cfg
        o = decode_attention_block(fused, w.extra["q_norm"], w.extra["k_norm"], cfg.eps,
                                   self.inv_freq, cfg.rotary_dim, self.attn.pos,
                                   self.attn.k_caches[a], self.attn.v_caches[a],
                                   self.attn.block_table, self.attn.split_scratch)
        return gemm_2d(o, w.out_proj)

    def _gdn_from(self, fused, w: LayerWeights, i: int):
        normed = gdn_decode_block(fused, self.conv_states[i], w.extra["conv"], w.extra["a_log"],
                                  w.extra["dt_bias"], w.extra["norm"], self.rec_states[i])
        return gemm_2d(normed, w.out_proj)

    def _decode_step_blocks(self, token_ids: torch.Tensor) -> torch.Tensor:
        """Mixer blocks with plain GEMMs: the residual add and the RMSNorm after
        it share a launch, and SwiGLU runs in the gate/up GEMM's epilogue
        (all bit-identical to the op sequence)."""
        cfg = self.cfg
        x = embedding_gather(token_ids, self.embed)
        h = None  # the previous sub-block's output, not yet added to x
        for i, w in enumerate(self.layers):
            if h is None:
                normed = qwen_rmsnorm(x, w.input_layernorm, cfg.eps)
            else:
                x, normed = add_rmsnorm(h, x, w.input_layernorm, cfg.eps)
            fused = gemm_2d(normed, w.in_proj)
            if cfg.is_attention(i):
                h = self._attention_from(fused, w, self.attn_index[i])
            else:
                h = self._gdn_from(fused, w, i)
            x, normed = add_rmsnorm(h, x, w.post_attention_layernorm, cfg.eps)
            h = gemm_2d(gate_up_swiglu(normed, w.gate_up), w.down_proj)
        return add_rmsnorm(h, x, self.final_norm, cfg.eps)[1]

    def _decode_step_ops(self, token_ids: torch.Tensor) -> torch.Tensor:
        """The reference runner's op sequence, one op per launch."""
        cfg = self.cfg
        x = embedding_gather(token_ids, self.embed)
        for i, w in enumerate(self.layers):
            residual = x
            h = qwen_rmsnorm(x, w.input_layernorm, cfg.eps)
            if cfg.is_attention(i):
                h = self._attention(h, w, self.attn_index[i])
            else:
                h = self._gdn(h, w, i)
            x = residual_add(h, residual)
            residual = x
            h = qwen_rmsnorm(x, w.post_attention_layernorm, cfg.eps)
            gate_up = gemm_2d(h, w.gate_up)
            h = swiglu(gate_up[:, :cfg.intermediate], gate_up[:, cfg.intermediate:])
            h = gemm_2d(h, w.down_proj)
            x = residual_add(h, residual)
        return qwen_rmsnorm(x, self.final_norm, cfg.eps)

    # ------------------------------------------------------------ prefill
    def prefill(self, token_ids: torch.Tensor, lengths: list[int]) -> torch.Tensor:
        """Packed prefill of B prompts (``token_ids`` ``[sum(lengths)]``, one
        prompt per sequence slot, engine/runner.py:570-667): fills the K/V
        pages, the GDN conv and recurrent states, sets ``pos[b] = lengths[b]``
        and returns each prompt's greedy next token ``[B]`` int64."""
        cfg = self.cfg
        assert len(lengths) == self.batch and min(lengths) >= 1
        assert max(lengths) <= self.attn.max_len
        packed = build_packed_batch(list(lengths), device=self.device)
        T = packed.total_tokens
        x = embedding_gather(token_ids, self.embed)
        h = None  # the previous sub-block's output, not yet added to x
        for i, w in enumerate(self.layers):
            if h is None:
                normed = qwen_rmsnorm(x, w.input_layernorm, cfg.eps)
            else:
                x, normed = add_rmsnorm(h, x, w.input_layernorm, cfg.eps)
            fused = gemm_2d(normed, w.in_proj)
            if cfg.is_attention(i):
                h = self._attention_prefill(fused, w, self.attn_index[i], packed)
            else:
                h = self._gdn_prefill(fused, w, i, packed)
            x, normed = add_rmsnorm(h, x, w.post_attention_layernorm, cfg.eps)
            h = gemm_2d(gate_up_swiglu(normed, w.gate_up), w.down_proj)
        # only each prompt's last row reaches the LM head
        last = packed.cu_seqlens[1:].long() - 1
        hidden = add_rmsnorm(h[last].contiguous(), x[last].contiguous(), self.final_norm,
                             cfg.eps)[1]
        self.attn.pos.copy_(torch.tensor(lengths, dtype=torch.int64, device=self.device))
        assert T == token_ids.shape[0]
        return lm_head_argmax(hidden, self.embed, False)

    def _attention_prefill(self, fused, w: LayerWeights, a: int, packed):
        cfg = self.cfg
        T = fused.shape[0]
        qd, kd = cfg.num_q_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
        q = qwen_rmsnorm(fused[:, :qd].view(T, cfg.num_q_heads, cfg.head_dim),
                         w.extra["q_norm"], cfg.eps)
        k = qwen_rmsnorm(fused[:, 2 * qd:2 * qd + kd].view(T, cfg.num_kv_heads, cfg.head_dim),
                         w.extra["k_norm"], cfg.eps)
        v = fused[:, 2 * qd + kd:].view(T, cfg.num_kv_heads, cfg.head_dim)
        gate = fused[:, qd:2 * qd].view(T, cfg.num_q_heads, cfg.head_dim)
        o = prefill_attention_block(q, k, v, gate, self.inv_freq, cfg.rotary_dim, packed,
                                    self.attn.k_caches[a], self.attn.v_caches[a],
                                    self.attn.block_table)
        return gemm_2d(o, w.out_proj)

    def _gdn_prefill(self, fused, w: LayerWeights, i: int, packed):
        cfg = self.cfg
        T = fused.shape[0]
        H, D = cfg.lin_heads, cfg.lin_head_dim
        HD = H * D
        qkv = fused[:, :3 * HD]
        # the decode conv weight [4, C] read as the prefill layout [C, 4]
        conv = depthwise_causal_conv4_prefill(qkv, w.extra["conv"].t(), packed.seq_start)
        q = conv[:, :HD].view(T, H, D)
        k = conv[:, HD:2 * HD].view(T, H, D)
        v = conv[:, 2 * HD:].view(T, H, D)
        qn, kn, beta, g = gdn_qk_norm_gates(q, k, fused[:, 4 * HD:4 * HD + H],
                                            fused[:, 4 * HD + H:], w.extra["a_log"],
                                            w.extra["dt_bias"])
        if packed.batch == 1 and T >= GDN_CHUNKED_PREFILL_MIN_TOKENS:
            # one long prompt: the chunk-64 WY path (engine/runner.py:272-273)
            core, state = call_gdn_recurrent_prefill_chunked_triton(qn, kn, v, beta, g)
            state = state.unsqueeze(0)
            self.rec_states[i].copy_(state)
        else:
            core = gdn_prefill_sequential_into(qn, kn, v, beta, g, packed.cu_seqlens,
                                               self.rec_states[i])
        conv_state_from_packed_prefill(self.conv_states[i], qkv, packed.cu_seqlens)
        normed = gdn_gated_rmsnorm(core, fused[:, 3 * HD:4 * HD].view(T, H, D), w.extra["norm"])
        return gemm_2d(normed.view(T, HD), w.out_proj)

    def next_tokens(self, token_ids: torch.Tensor) -> torch.Tensor:
        """One step plus the greedy pick: ``[B]`` -> ``[B]`` int64; advances pos."""
        hidden = self.decode_step(token_ids)
        nxt = lm_head_argmax(hidden, self.embed, False)
        self.attn.pos.add_(1)
        return nxt


class GraphedDecoder:
    """The whole decode step as one captured HIP graph (engine/runner.py:859-954):
    replay = embedding -> 24 layers -> final norm -> LM-head argmax -> pos += 1
    -> the new token fed back as the next input.  ``tokens`` is the static
    input/output buffer."""

    def __init__(self, model: DecodeModel, first_tokens: torch.Tensor):
        self.model = model
        self.tokens = first_tokens.to(torch.int64).clone()
        # warm up on the stream the capture will use: the per-stream zeroed
        # workspaces (split-K and argmax partials, queue counters) are then
        # allocated and cleared here, outside the graph; afterwards restore
        # every state the warm-up advanced
        saved = self._snapshot()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self._restore(saved)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            self._step()
        torch.cuda.synchronize()
        self._restore(saved)

    def _step(self):
        nxt = self.model.next_tokens(self.tokens)
        self.tokens.copy_(nxt)

    def _snapshot(self):
        m = self.model
        ts = [m.attn.pos, self.tokens, *m.attn.k_caches, *m.attn.v_caches]
        ts += [t for t in m.conv_states + m.rec_states if t is not None]
        return [(t, t.clone()) for t in ts]

    @staticmethod
    def _restore(saved):
        for t, c in saved:
            t.copy_(c)

    def step(self) -> torch.Tensor:
        """Generate one token per sequence; returns the token buffer."""
        self.graph.replay()
        return self.tokens
