"""Pins the strict-FP32 oracle (CPU only).

* Seeded parameters against fixtures written by executing the reference's own
  ``BaselineTransformer.__init__`` (tests/golden/make_golden.py).
* The forward against independent closed forms: a float64 per-query loop,
  ``scaled_dot_product_attention``, LayerNorm row statistics, causality and
  batch independence.
* The input generator against known CPU-RNG values.
"""

from __future__ import annotations

import dataclasses
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import strict_fp32
from tiktoktechjam2026_amd import harness
from tiktoktechjam2026_amd.config import BENCHMARK_CONFIGS, TransformerConfig

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

TINY = {
    "tiny_a": TransformerConfig(2, 8, 16, 2, 32, 2, True),
    "tiny_b": TransformerConfig(1, 5, 32, 4, 24, 1, True),
}


@pytest.fixture(scope="module")
def golden_tiny():
    with np.load(os.path.join(GOLDEN, "seeded_weights_tiny.npz"), allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.fixture(scope="module")
def fingerprints():
    with open(os.path.join(GOLDEN, "seeded_weight_fingerprints.json")) as handle:
        return json.load(handle)


@pytest.mark.parametrize("name", sorted(TINY))
@pytest.mark.parametrize("factory", ["oracle", "harness"])
def test_seeded_weights_match_reference_tiny(golden_tiny, name, factory):
    config = TINY[name]
    if factory == "oracle":
        state = strict_fp32.seeded_state_dict(config, 1234)
    else:
        state = harness.seeded_reference_state_dict(config, 1234)
    keys = sorted(k.split("/", 1)[1] for k in golden_tiny if k.startswith(name + "/"))
    assert keys == sorted(state), "state-dict keys differ from the reference model"
    for key in keys:
        expected = golden_tiny[f"{name}/{key}"]
        assert np.array_equal(state[key].numpy(), expected), key


@pytest.mark.parametrize("name", sorted(BENCHMARK_CONFIGS))
def test_seeded_weights_match_reference_fingerprints(fingerprints, name):
    config = BENCHMARK_CONFIGS[name]
    entry = fingerprints["configs"][name]
    assert entry["fields"]["d_model"] == config.d_model and entry["fields"]["num_layers"] == config.num_layers
    state = harness.seeded_reference_state_dict(config, fingerprints["seed"])
    assert sorted(state) == sorted(entry["tensors"])
    for key, fp in entry["tensors"].items():
        flat = state[key].double().reshape(-1)
        assert list(state[key].shape) == fp["shape"], key
        assert [float(v) for v in flat[:4]] == fp["head"], key
        assert [float(v) for v in flat[-4:]] == fp["tail"], key
        assert math.isclose(float(flat.sum()), fp["sum"], rel_tol=1e-9, abs_tol=1e-9), key
        assert math.isclose(float((flat * flat).sum()), fp["sumsq"], rel_tol=1e-9), key


def _brute_force_forward(x, state, config, mask=None):
    """Float64 per-query restatement with explicit loops over heads and queries.

    ``mask`` (bool ``[B, S]``, True = valid) removes padded keys from every
    query's softmax; padded rows of the attention output, of every layer's
    residual stream and of the final output are zero."""
    x = x.double()
    st = {k: v.double() for k, v in state.items()}
    d, h = config.d_model, config.num_heads
    hd = d // h

    def ln(t, name):
        mu = t.mean(-1, keepdim=True)
        var = ((t - mu) ** 2).mean(-1, keepdim=True)
        return (t - mu) / torch.sqrt(var + 1e-5) * st[name + ".weight"] + st[name + ".bias"]

    def lin(t, name):
        return t @ st[name + ".weight"].t() + st[name + ".bias"]

    for layer in range(config.num_layers):
        p = f"layers.{layer}."
        n1 = ln(x, p + "norm1")
        q, k, v = (lin(n1, p + f"attention.{c}_proj") for c in "qkv")
        ctx = torch.zeros_like(q)
        for b in range(x.shape[0]):
            for head in range(h):
                sl = slice(head * hd, (head + 1) * hd)
                for t in range(x.shape[1]):
                    keys = range(t + 1) if config.causal else range(x.shape[1])
                    if mask is not None:
                        keys = [j for j in keys if bool(mask[b, j])]
                        if not keys or not bool(mask[b, t]):
                            continue  # padded query: its row is zeroed below
                    s = torch.stack([q[b, t, sl] @ k[b, j, sl] for j in keys]) / math.sqrt(hd)
                    w = torch.exp(s - s.max())
                    w = w / w.sum()
                    ctx[b, t, sl] = sum(w[i] * v[b, j, sl] for i, j in enumerate(keys))
        attn = lin(ctx, p + "attention.out_proj")
        if mask is not None:
            attn = attn * mask[..., None]
        x = x + attn
        hid = lin(ln(x, p + "norm2"), p + "ffn_in")
        hid = 0.5 * hid * (1 + torch.erf(hid / math.sqrt(2)))
        x = x + lin(hid, p + "ffn_out")
        if mask is not None:
            x = x * mask[..., None]
    out = ln(x, "final_norm")
    return out if mask is None else out * mask[..., None]


@pytest.mark.parametrize("name", sorted(TINY))
def test_oracle_forward_matches_float64_brute_force(name):
    config = TINY[name]
    state = strict_fp32.seeded_state_dict(config, 1234)
    x, _ = harness.generate_random_case(config, torch.device("cpu"), torch.float32, 1234, 0.0, 1.0)
    got = strict_fp32.forward(x, state, config)
    ref = _brute_force_forward(x, state, config)
    assert torch.allclose(got.double(), ref, atol=2e-5, rtol=0), float((got.double() - ref).abs().max())


def test_oracle_attention_matches_sdpa():
    config = TransformerConfig(3, 40, 64, 4, 64, 1, True)
    state = strict_fp32.seeded_state_dict(config, 3)
    x = torch.randn(3, 40, 64)
    got = strict_fp32.self_attention(x, state, "layers.0.attention.", 4, None, True)
    q, k, v = (F.linear(x, state[f"layers.0.attention.{c}_proj.weight"], state[f"layers.0.attention.{c}_proj.bias"])
               for c in "qkv")
    split = lambda t: t.view(3, 40, 4, 16).transpose(1, 2)
    ctx = F.scaled_dot_product_attention(split(q), split(k), split(v), is_causal=True)
    ref = F.linear(ctx.transpose(1, 2).reshape(3, 40, 64), state["layers.0.attention.out_proj.weight"],
                   state["layers.0.attention.out_proj.bias"])
    assert torch.allclose(got, ref, atol=1e-5)


def test_oracle_properties():
    config = TransformerConfig(3, 24, 32, 2, 48, 2, True)
    state = strict_fp32.seeded_state_dict(config, 11)
    x = torch.randn(3, 24, 32)
    out = strict_fp32.forward(x, state, config)
    # final LayerNorm with gamma=1, beta=0: zero mean, unit (biased) variance per row
    assert torch.allclose(out.mean(-1), torch.zeros(3, 24), atol=1e-5)
    assert torch.allclose(out.var(-1, unbiased=False), torch.ones(3, 24), atol=1e-3)
    # causality: outputs up to t ignore inputs after t
    x2 = x.clone()
    x2[:, 10:] = torch.randn(3, 14, 32)
    out2 = strict_fp32.forward(x2, state, config)
    assert torch.allclose(out[:, :10], out2[:, :10], atol=1e-6)
    assert not torch.allclose(out[:, 10:], out2[:, 10:])
    # batch independence and slice evaluation
    sliced = strict_fp32.forward_in_slices(x, state, config, slice_size=1, rows=[2, 0])
    assert torch.allclose(sliced, out[[2, 0]], atol=1e-6)


def test_oracle_padding_mask_zeroes_rows():
    config = TransformerConfig(2, 16, 32, 2, 32, 1, True)
    state = strict_fp32.seeded_state_dict(config, 2)
    x, mask = harness.generate_random_case(config, torch.device("cpu"), torch.float32, 4, 0.4, 1.0)
    out = strict_fp32.forward(x, state, config, mask)
    assert torch.count_nonzero(out[~mask]) == 0
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_padded_prefix_equals_truncated_sequence(causal):
    """With prefix masks, a padded sequence's valid prefix is the forward of the truncated
    sequence.  The padded positions hold large non-zero inputs, so a key mask applied on the
    wrong side (queries instead of keys) or not at all changes the non-causal result."""
    config = TransformerConfig(3, 20, 32, 4, 48, 2, causal)
    state = strict_fp32.seeded_state_dict(config, 21)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 20, 32, generator=g)
    lengths = [20, 13, 6]
    mask = torch.arange(20)[None, :] < torch.tensor(lengths)[:, None]
    x = torch.where(mask[..., None], x, 25.0 * torch.randn(3, 20, 32, generator=g))
    out = strict_fp32.forward(x, state, config, mask)
    for b, n in enumerate(lengths):
        alone = strict_fp32.forward(x[b:b + 1, :n], state, dataclasses.replace(config, batch_size=1, seq_len=n))
        assert torch.allclose(out[b, :n], alone[0], atol=2e-5), (b, n)
        assert torch.count_nonzero(out[b, n:]) == 0
    if not causal:
        # the same forward without the mask lets valid queries see the padded keys
        unmasked = strict_fp32.forward(x, state, config)
        assert not torch.allclose(unmasked[1, :13], out[1, :13], atol=1e-3)


def test_oracle_arbitrary_key_mask_matches_brute_force():
    """A non-prefix key mask (holes inside the sequence) against the float64 per-query loop."""
    config = TransformerConfig(2, 12, 16, 2, 24, 2, False)
    state = strict_fp32.seeded_state_dict(config, 8)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 12, 16, generator=g)
    mask = torch.ones(2, 12, dtype=torch.bool)
    mask[0, [2, 3, 7]] = False
    mask[1, [0, 11]] = False
    got = strict_fp32.forward(x, state, config, mask)
    ref = _brute_force_forward(x, state, config, mask)
    assert torch.allclose(got.double(), ref, atol=2e-5, rtol=0), float((got.double() - ref).abs().max())


def test_input_generator_pins_cpu_rng():
    config = TransformerConfig(1, 1, 4, 1, 4, 1, True)
    x, mask = harness.generate_random_case(config, torch.device("cpu"), torch.float32, 1234, 0.0, 1.0)
    expected = [0.04613046, 0.40240282, -1.01152909, 0.21673824]
    assert np.allclose(x.reshape(-1).numpy(), expected, atol=1e-7)
    assert bool(mask.all())
