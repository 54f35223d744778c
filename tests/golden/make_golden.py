"""Write the seeded-weight golden fixtures from the reference's own model class.

Run once in the build container (never on the GPU box, which has no copy of the
reference tree):

    python tests/golden/make_golden.py /root/reference

What it pins.  The strict-FP32 model's parameters come from
``torch.manual_seed(seed)`` followed by PyTorch default init, in the order the
reference constructs its modules (``torch_transformer_benchmark.py:136-249``:
per layer q/k/v/out projections, then ffn_in, ffn_out; LayerNorms draw
nothing).  No closed form fixes that order, so the reference's
``BaselineTransformer.__init__`` is executed here and only its *parameters*
are recorded:

* ``seeded_weights_tiny.npz`` - every tensor of two tiny configurations;
* ``seeded_weight_fingerprints.json`` - per tensor shape, float64 sum, float64
  sum of squares, and the first/last four values, for the five benchmark
  configurations.

The forward pass is not executed here: its arithmetic is pinned by closed-form
checks in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

SEED = 1234

TINY = {
    "tiny_a": dict(batch_size=2, seq_len=8, d_model=16, num_heads=2, ffn_dim=32, num_layers=2, causal=True),
    "tiny_b": dict(batch_size=1, seq_len=5, d_model=32, num_heads=4, ffn_dim=24, num_layers=1, causal=True),
}

BENCH = {
    "cfg1": dict(batch_size=64, seq_len=128, d_model=128, num_heads=4, ffn_dim=128, num_layers=4, causal=True),
    "cfg2": dict(batch_size=64, seq_len=1024, d_model=128, num_heads=4, ffn_dim=128, num_layers=4, causal=True),
    "cfg3": dict(batch_size=128, seq_len=256, d_model=32, num_heads=2, ffn_dim=64, num_layers=2, causal=True),
    "cfg4": dict(batch_size=16, seq_len=2048, d_model=512, num_heads=8, ffn_dim=2048, num_layers=6, causal=True),
    "cfg5": dict(batch_size=512, seq_len=4096, d_model=256, num_heads=8, ffn_dim=1024, num_layers=4, causal=True),
}


def _build(ref, fields):
    torch.manual_seed(SEED)
    return ref.BaselineTransformer(ref.TransformerConfig(**fields))


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    import torch_transformer_benchmark as ref  # noqa: E402  (reference module)

    arrays = {}
    for name, fields in TINY.items():
        model = _build(ref, fields)
        for key, value in model.state_dict().items():
            arrays[f"{name}/{key}"] = value.detach().cpu().numpy().astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "seeded_weights_tiny.npz"), **arrays)

    prints = {"seed": SEED, "configs": {}}
    for name, fields in BENCH.items():
        model = _build(ref, fields)
        entry = {"fields": fields, "tensors": {}}
        for key, value in model.state_dict().items():
            flat = value.detach().double().reshape(-1)
            entry["tensors"][key] = {
                "shape": list(value.shape),
                "sum": float(flat.sum()),
                "sumsq": float((flat * flat).sum()),
                "head": [float(v) for v in flat[:4]],
                "tail": [float(v) for v in flat[-4:]],
            }
        prints["configs"][name] = entry
    with open(os.path.join(HERE, "seeded_weight_fingerprints.json"), "w") as handle:
        json.dump(prints, handle, indent=1, sort_keys=True)
    print(f"wrote {len(arrays)} tiny tensors and {len(BENCH)} fingerprint sets")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
