"""``torch.compile(model, mode="reduce-overhead")`` - the reference CLI's default treatment of the
candidate (``mixed_precision_benchmark.py:86-90`` -> ``torch_transformer_benchmark.py:800-805``) -
runs the HIP forward and matches the strict-FP32 oracle with zero failed elements on every call
(the first calls record, later ones replay the captured graph)."""

from __future__ import annotations

import pytest
import torch

from oracle import strict_fp32
from tiktoktechjam2026_amd import harness
from tiktoktechjam2026_amd.config import BENCHMARK_CONFIGS, TransformerConfig
from tiktoktechjam2026_amd.mixed_precision import MixedPrecisionTransformer, copy_mixed_model_weights

pytestmark = pytest.mark.gpu

CASES = {
    "cfg1": BENCHMARK_CONFIGS["cfg1"],                   # layer-tail route
    "d256": TransformerConfig(4, 256, 256, 8, 1024, 2, True),  # GEMM route with LayerNorm epilogues, q pre-scaled
    "d128_s512": TransformerConfig(2, 512, 128, 4, 128, 2, True),  # layer-tail route, q pre-scaled by the tail
}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", sorted(CASES))
def test_reduce_overhead_compile_matches_oracle(hip_device, name):
    config = CASES[name]
    print(f"\n[compile {name}] config={config}", flush=True)
    state = strict_fp32.seeded_state_dict(config, 1234)
    model = MixedPrecisionTransformer(config)
    copy_mixed_model_weights(state, model)
    model = model.to(hip_device).eval()
    model.convert_projections_to_fp16()
    model.assume_all_tokens_valid = True
    torch._dynamo.reset()
    compiled = torch.compile(model, mode="reduce-overhead")
    for call in range(4):
        x, _ = harness.generate_random_case(config, torch.device("cpu"), torch.float32, 1234 + call, 0.0, 1.0)
        with torch.inference_mode():
            out = compiled(x.to(hip_device)).clone()
            eager = model(x.to(hip_device))
        torch.cuda.synchronize()
        ref = strict_fp32.forward(x, state, config)
        result = harness.compare_outputs(ref, out.cpu(), rtol=0.02, atol=0.002)
        print(f"[compile {name}] call {call}: max_abs={result.max_abs_error:.6g} failed={result.failed_elements}",
              flush=True)
        assert result.failed_elements == 0
        assert torch.equal(out, eager), "compiled forward differs from the eager forward"
