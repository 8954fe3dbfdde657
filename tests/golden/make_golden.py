"""Writes reference_vectors.json: the known answers the reference's own tests assert.

Each case is data only (inputs and expected outputs) transcribed from the
reference test or docstring named in its "source" field (paths relative to
the reference's packages/).  Nothing here imports or runs reference code.
Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import os

ENG_T = "opaque-engine/tests/clipping"

CASES = [
    {
        "name": "per_group_independent",
        "source": f"{ENG_T}/test_per_group_clipping.py:42-61",
        "kind": "clip",
        "tree": {"attn.q": [3.0], "attn.k": [4.0], "mlp.w": [3.0]},
        "groups": {"attn.q": "attn", "attn.k": "attn", "mlp.w": "mlp"},
        "values": {"attn": 1.0, "mlp": 6.0},
        "expected": {"attn.q": [0.6], "attn.k": [0.8], "mlp.w": [3.0]},
        "rtol": 1.3e-6,
    },
    {
        "name": "per_group_large_bounds_passthrough",
        "source": f"{ENG_T}/test_per_group_clipping.py:26-40",
        "kind": "clip",
        "tree": {"attn.q": [1.0, 0.0], "attn.k": [0.0, 1.0], "mlp.w": [0.5, 0.0]},
        "groups": {"attn.q": "attn", "attn.k": "attn", "mlp.w": "mlp"},
        "values": {"attn": 10.0, "mlp": 10.0},
        "expected": {"attn.q": [1.0, 0.0], "attn.k": [0.0, 1.0], "mlp.w": [0.5, 0.0]},
        "rtol": 0.0,
    },
    {
        "name": "per_group_global_norm_aux",
        "source": f"{ENG_T}/test_per_group_clipping.py:63-73",
        "kind": "clip",
        "tree": {"a": [3.0], "b": [4.0]},
        "groups": {"a": "g1", "b": "g2"},
        "values": {"g1": 10.0, "g2": 10.0},
        "expected_norm": 5.0,
    },
    {
        "name": "per_group_zero_norm_group",
        "source": f"{ENG_T}/test_per_group_clipping.py:100-112",
        "kind": "clip",
        "tree": {"a": [0.0, 0.0], "b": [1.0]},
        "groups": {"a": "g1", "b": "g2"},
        "values": {"g1": 1.0, "g2": 10.0},
        "expected": {"a": [0.0, 0.0], "b": [1.0]},
        "rtol": 0.0,
    },
    {
        "name": "per_group_nested",
        "source": f"{ENG_T}/test_per_group_clipping.py:114-145",
        "kind": "clip",
        "tree": {"layer1": {"attn": [3.0, 4.0], "mlp": [30.0]}, "layer2": {"attn": [5.0, 12.0], "mlp": [40.0]}},
        "patterns": {"attn": 1.0, "mlp": 1.0},
        "expected": {
            "layer1": {"attn": [3.0 / math.sqrt(194.0), 4.0 / math.sqrt(194.0)], "mlp": [30.0 / 50.0]},
            "layer2": {"attn": [5.0 / math.sqrt(194.0), 12.0 / math.sqrt(194.0)], "mlp": [40.0 / 50.0]},
        },
        "expected_group_norms": {"attn": math.sqrt(194.0), "mlp": 50.0},
        "rtol": 1.3e-6,
    },
    {
        "name": "auto_formula_scalar",
        "source": f"{ENG_T}/test_auto.py:23-30",
        "kind": "auto",
        "tree": {"a": [3.0, 4.0]},
        "R": 1.0,
        "gamma": 0.01,
        "expected": {"a": [3.0 / 5.01, 4.0 / 5.01]},
        "expected_norm": 5.0,
        "rtol": 1.3e-6,
    },
    {
        "name": "auto_large_norm_unit_projection",
        "source": f"{ENG_T}/test_auto.py:47-53",
        "kind": "auto",
        "tree": {"a": [300.0, 400.0]},
        "R": 1.0,
        "gamma": 0.01,
        "expected_output_norm": 1.0,
        "rtol": 1e-4,
    },
    {
        "name": "auto_zero_gradient",
        "source": f"{ENG_T}/test_auto.py:55-60",
        "kind": "auto",
        "tree": {"a": [0.0, 0.0, 0.0, 0.0]},
        "R": 1.0,
        "gamma": 0.01,
        "expected": {"a": [0.0, 0.0, 0.0, 0.0]},
        "expected_norm": 0.0,
        "rtol": 0.0,
    },
    {
        "name": "auto_per_group",
        "source": f"{ENG_T}/test_auto.py:74-98",
        "kind": "auto",
        "tree": {"attn.q": [3.0], "attn.k": [4.0], "mlp.w": [6.0]},
        "groups": {"attn.q": "attn", "attn.k": "attn", "mlp.w": "mlp"},
        "values": {"attn": 2.0, "mlp": 3.0},
        "gamma": 0.01,
        "expected": {"attn.q": [3.0 * 2.0 / 5.01], "attn.k": [4.0 * 2.0 / 5.01], "mlp.w": [6.0 * 3.0 / 6.01]},
        "expected_group_norms": {"attn": 5.0, "mlp": 6.0},
        "rtol": 1.3e-6,
    },
    {
        "name": "auto_nested",
        "source": f"{ENG_T}/test_auto.py:117-138",
        "kind": "auto",
        "tree": {"layer1": {"attn": [3.0, 4.0], "mlp": [6.0]}, "layer2": {"attn": [0.0, 0.0], "mlp": [8.0]}},
        "patterns": {"attn": 2.0, "mlp": 1.0},
        "gamma": 0.01,
        "expected": {
            "layer1": {"attn": [3.0 * 2.0 / 5.01, 4.0 * 2.0 / 5.01], "mlp": [6.0 / 10.01]},
            "layer2": {"attn": [0.0, 0.0], "mlp": [8.0 / 10.01]},
        },
        "expected_group_norms": {"attn": 5.0, "mlp": 10.0},
        "rtol": 1.3e-6,
    },
    {
        "name": "global_norm_13",
        "source": "opaque-engine/src/opaque/api/engine/pytree.py:359-363",
        "kind": "global_norm",
        "tree": {"w": [3.0, 4.0], "b": [0.0, 12.0]},
        "expected_norm": 13.0,
    },
    {
        "name": "clipped_grad_docstring",
        "source": "opaque-engine/src/opaque/api/engine/clipping/_clipped_grad.py:112-129",
        "kind": "clipped_grad_mean_sq",
        "theta": 3.0,
        "data": [0.0, 7.0, -2.0],
        "expected_loss_values": [4.5, 8.0, 12.5],
        "expected_grad_norms": [3.0, 4.0, 5.0],
        "expected_sum": 4.0,
        "note": "the docstring prints 1.3333, which is the mean 4/3 (normalize_by=3)",
    },
    {
        "name": "noise_per_group_sigma",
        "source": "opaque-dpsgd/tests/noise/test_noise.py:179-198",
        "kind": "per_group_sigma",
        "noise_multiplier": 2.0,
        "values": {"small": 1.0, "large": 3.0},
        "expected": {"small": 4.0, "large": 6.928203230275509},
    },
    {
        "name": "noise_stddev_for_scalar",
        "source": "opaque-engine/tests/types/test_clipped_pytree_noise_stddev.py:24-33",
        "kind": "noise_stddev_for",
        "max_norm": 2.0,
        "noise_multiplier": 0.8,
        "expected": 1.6,
    },
    {
        "name": "per_group_bound_arithmetic",
        "source": f"{ENG_T}/test_per_group_clipping.py:306-323",
        "kind": "bound_arithmetic",
        "patterns": {"a": 1.0, "b": 2.0},
        "noise_multiplier": 1.1,
        "expected": {"a": 1.1, "b": 2.2},
    },
]


def main() -> None:
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.json")
    with open(out, "w") as f:
        json.dump({"cases": CASES}, f, indent=1, sort_keys=False)
        f.write("\n")
    print(f"wrote {len(CASES)} cases to {out}")


if __name__ == "__main__":
    main()
