"""Strict-FP32 oracle for the causal pre-LN Transformer forward (TEST INFRASTRUCTURE).

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped forward path lives in ``tiktoktechjam2026_amd`` and
runs hand-written HIP kernels only.

It restates, in plain PyTorch FP32, the reference's numerics definition:

* ``BaselineTransformer`` / ``BaselineTransformerBlock`` /
  ``BaselineSelfAttention`` - ``torch_transformer_benchmark.py:136-249``.
  Pre-LN block ``x = x + attn(LN1(x)); x = x + W2 gelu_erf(W1 LN2(x))``,
  separate q/k/v projections, materialized S x S scores in FP32, causal
  ``-inf`` mask (``triu(1)``), key-padding mask, softmax in FP32, final LN,
  and masked zero-fill of padded tokens (``:176-198, :211-222, :239-249``).
* Parameter creation: ``seeded_state_dict`` draws the same PyTorch default
  initialisation in the same order as the reference's module construction
  (``torch_transformer_benchmark.py:149-152, 205-209, 229-237``): per layer
  q, k, v, out projections, then ffn_in and ffn_out; each ``nn.Linear``
  draws its weight (kaiming-uniform, a=sqrt(5)) and then its bias
  (U(+-1/sqrt(fan_in))); LayerNorms draw nothing (gamma=1, beta=0).

Pinning (see ``tests/test_oracle.py``):

* the parameters against ``tests/golden/seeded_weights_tiny.npz`` and
  ``seeded_weight_fingerprints.json``, written by executing the reference's
  own ``BaselineTransformer.__init__`` (``tests/golden/make_golden.py``);
* the forward against closed forms: a float64 brute-force per-query softmax
  loop, ``torch.nn.functional.scaled_dot_product_attention``,
  ``F.layer_norm``, causality (output t independent of inputs after t),
  batch independence, and LN row statistics.

The forward is written functionally over a state dict whose keys are the
reference's (``layers.{i}.attention.q_proj.weight`` ...), so a reference
``state_dict()`` loads without translation.
"""

from __future__ import annotations

import math
from typing import Dict, Iterable, Optional

import torch
import torch.nn.functional as F

LN_EPS = 1e-5

# Linear sub-modules of one block, in reference construction order
# (torch_transformer_benchmark.py:149-152 then :208-209).
_BLOCK_LINEARS = (
    ("attention.q_proj", "d", "d"),
    ("attention.k_proj", "d", "d"),
    ("attention.v_proj", "d", "d"),
    ("attention.out_proj", "d", "d"),
    ("ffn_in", "d", "f"),
    ("ffn_out", "f", "d"),
)


def _dims(config) -> Dict[str, int]:
    return {"d": int(config.d_model), "f": int(config.ffn_dim)}


def _default_linear(fan_in: int, fan_out: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Draw one nn.Linear default init: weight first, then bias."""
    weight = torch.empty(fan_out, fan_in, dtype=torch.float32)
    torch.nn.init.kaiming_uniform_(weight, a=math.sqrt(5))
    bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
    bias = torch.empty(fan_out, dtype=torch.float32).uniform_(-bound, bound)
    return weight, bias


def seeded_state_dict(config, seed: Optional[int] = 1234) -> Dict[str, torch.Tensor]:
    """Return the reference model's parameters for ``config`` after ``manual_seed(seed)``.

    ``seed=None`` draws from the current global RNG state instead of reseeding.
    Keys and order match ``BaselineTransformer(config).state_dict()``.
    """
    if seed is not None:
        torch.manual_seed(seed)
    dims = _dims(config)
    d = dims["d"]
    state: Dict[str, torch.Tensor] = {}
    for layer in range(int(config.num_layers)):
        prefix = f"layers.{layer}."
        drawn = {}
        for name, fan_in, fan_out in _BLOCK_LINEARS:
            drawn[name] = _default_linear(dims[fan_in], dims[fan_out])
        # state_dict order of a block: norm1, attention.{q,k,v,out}, norm2, ffn_in, ffn_out
        state[prefix + "norm1.weight"] = torch.ones(d)
        state[prefix + "norm1.bias"] = torch.zeros(d)
        for name in ("attention.q_proj", "attention.k_proj", "attention.v_proj", "attention.out_proj"):
            state[prefix + name + ".weight"], state[prefix + name + ".bias"] = drawn[name]
        state[prefix + "norm2.weight"] = torch.ones(d)
        state[prefix + "norm2.bias"] = torch.zeros(d)
        for name in ("ffn_in", "ffn_out"):
            state[prefix + name + ".weight"], state[prefix + name + ".bias"] = drawn[name]
    state["final_norm.weight"] = torch.ones(d)
    state["final_norm.bias"] = torch.zeros(d)
    return state


# The three library routines below are the ones the reference's modules call
# (nn.Linear -> F.linear, nn.LayerNorm -> F.layer_norm, F.gelu(approximate="none")),
# so the restatement rounds exactly as the reference does on the same PyTorch build.
def _linear(x: torch.Tensor, state: Dict[str, torch.Tensor], name: str) -> torch.Tensor:
    return F.linear(x, state[name + ".weight"], state[name + ".bias"])


def _layer_norm(x: torch.Tensor, state: Dict[str, torch.Tensor], name: str) -> torch.Tensor:
    weight = state[name + ".weight"]
    return F.layer_norm(x, (weight.shape[0],), weight, state[name + ".bias"], LN_EPS)


def _gelu_erf(x: torch.Tensor) -> torch.Tensor:
    return F.gelu(x, approximate="none")


def self_attention(
    x: torch.Tensor,
    state: Dict[str, torch.Tensor],
    prefix: str,
    num_heads: int,
    valid_token_mask: Optional[torch.Tensor],
    causal: bool,
) -> torch.Tensor:
    """Explicit multi-head attention with materialized FP32 scores.

    Follows ``torch_transformer_benchmark.py:162-199``.
    """
    batch, seq_len, d_model = x.shape
    head_dim = d_model // num_heads
    scale = head_dim ** -0.5

    def heads(t: torch.Tensor) -> torch.Tensor:
        return t.reshape(batch, seq_len, num_heads, head_dim).permute(0, 2, 1, 3).contiguous()

    q = heads(_linear(x, state, prefix + "q_proj"))
    k = heads(_linear(x, state, prefix + "k_proj"))
    v = heads(_linear(x, state, prefix + "v_proj"))
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if causal:
        future = torch.ones(seq_len, seq_len, dtype=torch.bool, device=x.device).triu(1)
        scores = scores.masked_fill(future, float("-inf"))
    if valid_token_mask is not None:
        scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
    probs = torch.softmax(scores.float(), dim=-1)
    context = torch.matmul(probs, v).permute(0, 2, 1, 3).reshape(batch, seq_len, d_model)
    out = _linear(context, state, prefix + "out_proj")
    if valid_token_mask is not None:
        out = out.masked_fill(~valid_token_mask[..., None], 0)
    return out


def forward(
    x: torch.Tensor,
    state: Dict[str, torch.Tensor],
    config,
    valid_token_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Strict-FP32 forward of the whole stack (``torch_transformer_benchmark.py:239-249``)."""
    if x.dtype != torch.float32:
        raise ValueError("the strict oracle takes FP32 input")
    for layer in range(int(config.num_layers)):
        p = f"layers.{layer}."
        x = x + self_attention(
            _layer_norm(x, state, p + "norm1"), state, p + "attention.", int(config.num_heads),
            valid_token_mask, bool(config.causal),
        )
        hidden = _gelu_erf(_linear(_layer_norm(x, state, p + "norm2"), state, p + "ffn_in"))
        x = x + _linear(hidden, state, p + "ffn_out")
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
    x = _layer_norm(x, state, "final_norm")
    if valid_token_mask is not None:
        x = x.masked_fill(~valid_token_mask[..., None], 0)
    return x


class BaselineTransformer(torch.nn.Module):
    """Module wrapper with the reference's call signature ``forward(x, valid_token_mask=None)``.

    Parameters are buffers holding the seeded state dict; ``state_dict()``
    therefore has the reference's keys.
    """

    def __init__(self, config, seed: Optional[int] = None) -> None:
        super().__init__()
        self.config = config
        for key, value in seeded_state_dict(config, seed).items():
            self.register_buffer(key.replace(".", "__"), value)

    def named_state(self) -> Dict[str, torch.Tensor]:
        return {name.replace("__", "."): buf for name, buf in self.named_buffers()}

    def state_dict(self, *args, **kwargs):  # type: ignore[override]
        return dict(self.named_state())

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        return forward(x, self.named_state(), self.config, valid_token_mask)


def forward_in_slices(
    x: torch.Tensor,
    state: Dict[str, torch.Tensor],
    config,
    slice_size: int,
    rows: Optional[Iterable[int]] = None,
) -> torch.Tensor:
    """Run the oracle over batch slices (exact: batch elements are independent).

    Mirrors the microbatching precedent at ``torch_transformer_benchmark.py:808-833``
    to bound the ``[b,H,S,S]`` FP32 score memory.  ``rows`` restricts the
    evaluation to selected batch indices (returned in that order).
    """
    index = list(range(x.shape[0])) if rows is None else list(rows)
    outputs = []
    for start in range(0, len(index), slice_size):
        chunk = index[start:start + slice_size]
        outputs.append(forward(x[chunk], state, config))
    return torch.cat(outputs, dim=0)
