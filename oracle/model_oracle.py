"""CPU oracle of the decode step's model-level ops -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
path (the HIP library behind ``wy_lib::`` ops) never calls it.  Each function
cites the reference lines it restates (sujuyu/qwen3_5-triton-inference-engine,
``triton_kernels/``); ``PINNED`` names the independent checks in
tests/test_oracle_model.py.
"""

from __future__ import annotations

import torch

PINNED = {
    "embedding_gather": "torch.nn.functional.embedding",
    "residual_add": "exact bf16 sums of dyadic values",
    "swiglu": "torch.nn.functional.silu(gate) * up; pure-Python brute force",
    "lm_head_argmax": "float64 matmul + argmax; duplicate weight rows -> first index; "
                      "one-hot hidden picks the largest weight column",
}


def embedding_gather(ids, weight):
    """embedding_gather.py:20-50: out[t] = weight[ids[t]]."""
    return weight[ids.long()]


def residual_add(x, r):
    """residual_add.py:8-20: bf16(x + r) with fp32 arithmetic."""
    return (x.float() + r.float()).to(torch.bfloat16)


def swiglu(gate, up):
    """swiglu.py:22-60: bf16(up * gate * sigmoid(gate)), fp32 math."""
    g, u = gate.float(), up.float()
    return (u * g * torch.sigmoid(g)).to(torch.bfloat16)


def lm_head_logits(hidden, weight):
    """vocab_argmax.py:243-248: logits = weight @ hidden (float64 here)."""
    return hidden.double() @ weight.double().T


def lm_head_argmax(hidden, weight):
    """argmax over the vocabulary per row (first index on ties)."""
    return torch.argmax(lm_head_logits(hidden, weight), dim=-1)
