"""Shape-dispatch table (CPU): routes, support limits, and agreement with the library's tables."""

from __future__ import annotations

import pytest
import torch

from tiktoktechjam2026_amd import dispatch
from tiktoktechjam2026_amd.config import BENCHMARK_CONFIGS, TransformerConfig
from tiktoktechjam2026_amd.mixed_precision import MixedPrecisionTransformer


def test_benchmark_config_routes():
    fused = {name: dispatch.plan(cfg).fuse_layer_tail for name, cfg in BENCHMARK_CONFIGS.items()}
    assert fused == {"cfg1": True, "cfg2": True, "cfg3": True, "cfg4": False, "cfg5": False}
    for cfg in BENCHMARK_CONFIGS.values():
        route = dispatch.plan(cfg)
        narrow = cfg.d_model < dispatch.WIDE_GEMM_FROM
        assert route.supported and route.fuse_attention_output_norm == narrow
        assert route.fuse_full_ffn == (narrow or cfg.d_model == dispatch.WIDE_FFN_WIDTH)
        assert route.normalized_dtype == torch.float16


def test_wide_layernorm_epilogue_route():
    """d_model 256 (cfg5) and 512 (cfg4): the residual GEMMs carry the next LayerNorm; other
    widths and disabled fusions keep the separate LayerNorm launches."""
    flags = {name: dispatch.plan(cfg).wide_ln_epilogue for name, cfg in BENCHMARK_CONFIGS.items()}
    assert flags == {"cfg1": False, "cfg2": False, "cfg3": False, "cfg4": True, "cfg5": True}
    from tiktoktechjam2026_amd import profiling

    cfg4 = BENCHMARK_CONFIGS["cfg4"]
    costs4 = profiling.forward_costs(cfg4, 2, dispatch.plan(cfg4))
    # d 512: the out-projection carries LN2; the FFN output keeps its LayerNorm (1 + L launches)
    assert dispatch.plan(cfg4).wide_ln_ffn_out is False and dispatch.plan(BENCHMARK_CONFIGS["cfg5"]).wide_ln_ffn_out
    assert costs4["layernorm"].launches_per_forward == 1 + cfg4.num_layers
    assert {"out_proj_ln", "ffn_in", "ffn_out_residual"} <= set(costs4)
    assert not {"out_proj_residual", "ffn_out_ln"} & set(costs4)
    assert not dispatch.plan(TransformerConfig(2, 8, 384, 8, 64, 1, True)).wide_ln_epilogue
    cfg5 = BENCHMARK_CONFIGS["cfg5"]
    assert not dispatch.plan(cfg5, enable_attention_output_norm_fusion=False).wide_ln_epilogue
    assert not dispatch.plan(cfg5, enable_full_ffn_fusion=False).wide_ln_epilogue
    costs = profiling.forward_costs(cfg5, 2, dispatch.plan(cfg5))
    assert costs["layernorm"].launches_per_forward == 1
    assert {"out_proj_ln", "ffn_ln"} <= set(costs)
    assert not {"ffn_in", "ffn_out_ln", "ffn_out_residual", "out_proj_residual"} & set(costs)
    # without the FFN fusion the FFN runs as two GEMMs, the second with the LayerNorm epilogue
    unfused = dispatch.plan(cfg5, enable_full_ffn_fusion=False)
    assert not unfused.fuse_full_ffn and not unfused.wide_ln_epilogue
    # widths above the wide FFN kernel's hidden limit keep the GEMM route
    assert not dispatch.plan(TransformerConfig(2, 8, 256, 8, dispatch.WIDE_FFN_MAX_F + 32, 1, True)).fuse_full_ffn


def test_enable_flags_change_the_route():
    cfg = BENCHMARK_CONFIGS["cfg2"]
    assert not dispatch.plan(cfg, enable_full_ffn_fusion=False).fuse_layer_tail
    r = dispatch.plan(cfg, enable_fp16_custom_attention=False)
    assert not r.fp16_attention and not r.fuse_layer_tail
    r = dispatch.plan(cfg, enable_fp16_normalized_stream=False)
    assert r.normalized_dtype == torch.float32 and not r.fuse_layer_tail


@pytest.mark.parametrize(
    "d,h,ok",
    [(128, 4, True), (96, 3, True), (128, 16, True), (24, 3, True), (1024, 4, True), (96, 2, False), (36, 3, False),
     (512, 1, False)],
)
def test_support_limits(d, h, ok):
    route = dispatch.plan(TransformerConfig(2, 8, d, h, 64, 1, True))
    assert route.supported == ok
    if not ok:
        with pytest.raises(ValueError):
            MixedPrecisionTransformer(TransformerConfig(2, 8, d, h, 64, 1, True))


def test_python_tables_match_library(built_library):
    lib = built_library
    for d in (16, 32, 64, 96, 128, 256, 512):
        assert bool(lib.mpk_layernorm_qkv_supported(d)) == (d in dispatch.LAYERNORM_QKV_WIDTHS)
        for f in (32, 64, 96, 128, 256, 512, 1024, 2048):
            assert bool(lib.mpk_layer_tail_supported(d, f)) == ((d, f) in dispatch.LAYER_TAIL_SHAPES)
    # attention inside the layer tail: head dim 32 on the tail shapes, 16 at d_model 32 / 64
    assert lib.mpk_attention_layer_tail_rows() == dispatch.ATTENTION_TAIL_ROWS
    for d in (16, 32, 64, 96, 128, 256):
        for f in (32, 64, 96, 128, 256, 512):
            for heads in (1, 2, 3, 4, 8):
                expected = dispatch.attention_tail_supported(d, f, heads)
                assert bool(lib.mpk_attention_layer_tail_supported(d, f, heads)) == expected, (d, f, heads)
    assert dispatch.attention_tail_supported(32, 64, 2) and dispatch.attention_tail_supported(128, 128, 4)
    assert not dispatch.attention_tail_supported(128, 128, 8) and not dispatch.attention_tail_supported(64, 64, 1)
    # the wide fused FFN (variant 4, the role-split kernel) is the library's choice exactly
    # where the route fuses it
    for d in (128, 256, 512):
        for f in (32, 96, 1024, dispatch.WIDE_FFN_MAX_F, dispatch.WIDE_FFN_MAX_F + 32):
            wide = d == dispatch.WIDE_FFN_WIDTH and f <= dispatch.WIDE_FFN_MAX_F
            assert (lib.mpk_ffn_residual_layernorm_auto_variant(65536, d, f) == 4) == wide, (d, f)


def test_model_interface_mirrors_reference():
    cfg = BENCHMARK_CONFIGS["cfg1"]
    model = MixedPrecisionTransformer(
        cfg, enable_case11_schedule=True, enable_attention_output_norm_fusion=True, enable_full_ffn_fusion=True,
        enable_fp16_custom_attention=True, enable_fp16_normalized_stream=True,
    )
    for attr in ("use_case8_triton", "use_d128_triton", "use_d128_custom_attention", "use_fp16_custom_attention",
                 "use_case11_schedule", "fuse_attention_output_norm", "fuse_full_ffn", "use_fp16_normalized_stream",
                 "use_d32_triton", "assume_all_tokens_valid"):
        assert hasattr(model, attr)
    keys = list(model.state_dict())
    assert keys[:6] == ["layers.0.norm1.weight", "layers.0.norm1.bias", "layers.0.attention.qkv_proj.weight",
                        "layers.0.attention.qkv_proj.bias", "layers.0.attention.out_proj.weight",
                        "layers.0.attention.out_proj.bias"]
    assert model.state_dict()["layers.0.attention.qkv_proj.weight"].shape == (384, 128)
    model.convert_projections_to_fp16()
    sd = model.state_dict()
    assert sd["layers.0.attention.qkv_proj.weight"].dtype == torch.float16
    assert sd["layers.0.ffn_out.bias"].dtype == torch.float16
    assert sd["layers.0.norm2.weight"].dtype == torch.float32
    with pytest.raises(ValueError):
        model(torch.zeros(1, 2, 128, dtype=torch.float16))


def test_copy_weights_packs_qkv():
    from oracle import strict_fp32
    from tiktoktechjam2026_amd.mixed_precision import copy_mixed_model_weights

    cfg = TransformerConfig(1, 4, 32, 2, 64, 2, True)
    state = strict_fp32.seeded_state_dict(cfg, 9)
    model = MixedPrecisionTransformer(cfg)
    copy_mixed_model_weights(state, model)
    packed = model.state_dict()["layers.1.attention.qkv_proj.weight"]
    assert torch.equal(packed[:32], state["layers.1.attention.q_proj.weight"])
    assert torch.equal(packed[32:64], state["layers.1.attention.k_proj.weight"])
    assert torch.equal(packed[64:], state["layers.1.attention.v_proj.weight"])
    assert torch.equal(model.state_dict()["layers.1.attention.qkv_proj.bias"][64:],
                       state["layers.1.attention.v_proj.bias"])


def test_attention_in_layer_tail_route():
    """The layer-tail route runs attention inside the tail for unmasked sequences of whole
    64-row tiles up to the measured length of its (d_model, head dim) (d_model 32 and 64, head
    dim 32 or 16); d_model 128 (measured slower fused), other head dims, masked forwards,
    ragged or longer sequences keep the separate attention kernel."""
    from tiktoktechjam2026_amd.config import TransformerConfig

    d64 = dispatch.plan(TransformerConfig(2, 128, 64, 2, 128, 2, True))  # hd 32
    assert d64.fuse_layer_tail and d64.fuse_attention_tail
    assert dispatch.attention_tail_for(d64, 128, masked=False)
    assert dispatch.attention_tail_for(d64, 256, masked=False)
    assert not dispatch.attention_tail_for(d64, 128, masked=True)
    assert not dispatch.attention_tail_for(d64, 100, masked=False)   # ragged tiles
    assert not dispatch.attention_tail_for(d64, 512, masked=False)   # long: the attention kernel
    assert dispatch.plan(TransformerConfig(2, 64, 32, 1, 64, 2, True)).fuse_attention_tail  # D32 H1
    cfg3 = dispatch.plan(BENCHMARK_CONFIGS["cfg3"])  # D32 H2: hd 16
    assert cfg3.fuse_attention_tail and dispatch.attention_tail_for(cfg3, 256, masked=False)
    assert dispatch.attention_tail_for(cfg3, 512, masked=False) and not dispatch.attention_tail_for(cfg3, 1024, False)
    d64h16 = dispatch.plan(TransformerConfig(2, 128, 64, 4, 128, 2, True))  # hd 16
    assert dispatch.attention_tail_for(d64h16, 128, False) and not dispatch.attention_tail_for(d64h16, 256, False)
    cfg1 = dispatch.plan(BENCHMARK_CONFIGS["cfg1"])  # D128 H4: hd 32, but d_model 128
    assert cfg1.fuse_layer_tail and not cfg1.fuse_attention_tail
    assert not dispatch.plan(TransformerConfig(2, 64, 64, 1, 64, 2, True)).fuse_attention_tail  # hd 64
    for (d, hd) in dispatch.ATTENTION_TAIL_ROUTE_MAX_SEQ:
        assert any(dispatch.attention_tail_supported(d, f, d // hd) for (dd, f) in dispatch.LAYER_TAIL_SHAPES if dd == d)


def test_prescaled_q_route():
    """Head dim 32 from 256 keys runs the pre-scaled attention wherever the attention is a launch of
    its own (its producers scale q): cfg2 (layer-tail route) and cfg5 (GEMM route); cfg1 (128 keys:
    the 16x16 kernel), cfg3 (attention inside the layer tail), cfg4 (head dim 64) and forced
    16x16 variants keep the scaling kernel."""
    from dataclasses import replace

    routes = {name: dispatch.plan(cfg) for name, cfg in BENCHMARK_CONFIGS.items()}
    chosen = {}
    for name, cfg in BENCHMARK_CONFIGS.items():
        route = routes[name]
        in_tail = route.fuse_layer_tail and dispatch.attention_tail_for(route, cfg.seq_len, masked=False)
        chosen[name] = not in_tail and dispatch.prescaled_attention_for(route, cfg.seq_len)
    assert chosen == {"cfg1": False, "cfg2": True, "cfg3": False, "cfg4": False, "cfg5": True}
    cfg5 = routes["cfg5"]
    assert not dispatch.prescaled_attention_for(cfg5, dispatch.PRESCALED_ATTENTION_MIN_SEQ - 1)
    assert not dispatch.prescaled_attention_for(replace(cfg5, attention_variant=1), 4096)
    assert dispatch.prescaled_attention_for(replace(cfg5, attention_variant=7), 4096)
    assert not dispatch.prescaled_attention_for(replace(cfg5, prescale_q=False), 4096)
