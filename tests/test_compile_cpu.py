"""The module traces into ONE graph of the library's custom operators (CPU, fake tensors).

The reference CLI compiles the candidate with ``torch.compile(mode="reduce-overhead")``
by default (``mixed_precision_benchmark.py:86-90``).  ``torch._dynamo.export`` fails on any
graph break, so exporting the forward with fake CUDA tensors (no device needed) shows that
Dynamo sees every launch as an opaque ``mpk::`` operator and nothing else computes."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from tiktoktechjam2026_amd.config import TransformerConfig
from tiktoktechjam2026_amd.mixed_precision import MixedPrecisionTransformer

ROUTES = {
    "layer_tail_d128": (TransformerConfig(2, 64, 128, 4, 128, 2, True),
                        {"mpk.layer_norm_qkv.default": 1, "mpk.attention.default": 2, "mpk.layer_tail.default": 2}),
    # d_model 64, head dim 32, 64 positions: attention runs inside the layer-tail kernel (1 + L launches)
    "layer_tail_d64_attention": (TransformerConfig(2, 64, 64, 2, 128, 2, True),
                                 {"mpk.layer_norm_qkv.default": 1, "mpk.attention_layer_tail.default": 2,
                                  "mpk.attention.default": 0, "mpk.layer_tail.default": 0}),
    # 80 positions are not whole 64-row tiles: separate attention + layer tail (1 + 2L launches)
    "layer_tail_d64_ragged": (TransformerConfig(2, 80, 64, 2, 128, 2, True),
                              {"mpk.layer_norm_qkv.default": 1, "mpk.attention.default": 2,
                               "mpk.layer_tail.default": 2}),
    "gemm_ln_epilogue_d256": (TransformerConfig(2, 64, 256, 8, 1024, 2, True),
                              {"mpk.layer_norm.default": 1, "mpk.attention.default": 2}),
    "gemm_d512": (TransformerConfig(2, 64, 512, 8, 2048, 2, True), {"mpk.attention.default": 2}),
    # head dim 32 from 256 positions: q leaves the projection pre-scaled, the attention skips the scale
    # d_model 128, head dim 32, 256 positions: the layer-tail route's QKV producers scale q
    "layer_tail_prescaled_d128": (TransformerConfig(1, 256, 128, 4, 128, 2, True),
                                  {"mpk.layer_norm_qkv.default": 1, "mpk.attention_prescaled.default": 2,
                                   "mpk.attention.default": 0, "mpk.layer_tail.default": 2}),
    "gemm_prescaled_d256": (TransformerConfig(1, 256, 256, 8, 1024, 2, True),
                            {"mpk.linear_qscaled.default": 2, "mpk.attention_prescaled.default": 2,
                             "mpk.attention.default": 0}),
    "row_fused_d96": (TransformerConfig(2, 64, 96, 3, 192, 2, True), {"mpk.attention.default": 2}),
}

ALLOWED = ("mpk.", "aten.sym_size", "<built-in function getitem>")
# metadata-only tensor methods (views of the packed QKV; contiguous() of a contiguous input)
VIEWS = {"view", "permute", "unbind", "contiguous"}


def _export(config, masked: bool, with_out: bool = False):
    model = MixedPrecisionTransformer(config).eval()
    model.convert_projections_to_fp16()
    model.assume_all_tokens_valid = not masked
    with FakeTensorMode(allow_non_fake_inputs=True):
        model = model.to("cuda")
        x = torch.empty(config.batch_size, config.seq_len, config.d_model, device="cuda")
        args = (x,)
        if masked:
            args = (x, torch.ones(config.batch_size, config.seq_len, dtype=torch.bool, device="cuda"))
        kwargs = {}
        if with_out:
            kwargs["out"] = torch.empty(config.batch_size, config.seq_len, config.d_model, device="cuda")
        graph_module, _ = torch._dynamo.export(model)(*args, **kwargs)
    return [str(n.target) for n in graph_module.graph.nodes if n.op in ("call_function", "call_method")]


@pytest.mark.parametrize("name", sorted(ROUTES))
def test_forward_exports_as_one_graph_of_library_ops(name):
    config, expected = ROUTES[name]
    targets = _export(config, masked=False)
    strays = [t for t in targets if not t.startswith(ALLOWED) and t not in VIEWS]
    assert not strays, f"non-library computation in the traced forward: {strays}"
    for op, count in expected.items():
        assert targets.count(op) == count, (op, targets)


def test_masked_forward_exports_too():
    """With a key mask the graph adds only the mask conversion and the final masked zero-fill."""
    config, _ = ROUTES["gemm_ln_epilogue_d256"]
    targets = _export(config, masked=True)
    assert targets.count("mpk.attention.default") == 2
    assert any("masked_fill" in t for t in targets)


@pytest.mark.parametrize("name", ["gemm_ln_epilogue_d256", "layer_tail_d128", "layer_tail_d64_attention"])
def test_forward_with_out_exports_as_one_graph(name):
    """``forward(x, None, out=t)`` (the microbatch harness's direct-write call) traces too."""
    config, expected = ROUTES[name]
    targets = _export(config, masked=False, with_out=True)
    strays = [t for t in targets if not t.startswith(ALLOWED) and t not in VIEWS and "copy_" not in t]
    assert not strays, f"non-library computation in the traced forward: {strays}"
    for op, count in expected.items():
        assert targets.count(op) == count, (op, targets)
