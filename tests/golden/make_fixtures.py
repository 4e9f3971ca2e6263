"""Writes the committed golden vectors of this directory from the CPU oracle.

Run from the repository root:  python tests/golden/make_fixtures.py

``moe_small.npz`` -- one small routed-MoE layer (T=3, d=256, E=8, top-2,
I=128, bf16 shared expert I=128, group routing 2/1) with its inputs and the
oracle's outputs and intermediates.  The tests check that the oracle still
reproduces it bit for bit (a regression pin of the oracle itself) and compare
the HIP layer against it.  Arrays only (np.savez, no pickles).
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import moe_oracle as O  # noqa: E402

SHAPE = dict(T=3, d=256, E=8, k=2, I=128, Is=128, n_group=2, topk_group=1,
             routed_scaling_factor=2.5, swiglu_limit=10.0)


def small_layer(seed: int = 20260):
    rng = np.random.default_rng(seed)
    T, d, E, I, Is = (SHAPE[k] for k in ("T", "d", "E", "I", "Is"))
    return {
        "x": O.f32_to_bf16_bits(rng.standard_normal((T, d), dtype=np.float32)),
        "router_weight": rng.normal(0.0, 0.05, (E, d)).astype(np.float32),
        "router_bias": rng.normal(0.0, 0.1, E).astype(np.float32),
        "gate_proj.weight_packed": rng.integers(0, 256, (E, I, d // 2), dtype=np.uint8),
        "gate_proj.weight_scale": rng.integers(119, 128, (E, I, d // 32), dtype=np.uint8),
        "up_proj.weight_packed": rng.integers(0, 256, (E, I, d // 2), dtype=np.uint8),
        "up_proj.weight_scale": rng.integers(119, 128, (E, I, d // 32), dtype=np.uint8),
        "down_proj.weight_packed": rng.integers(0, 256, (E, d, I // 2), dtype=np.uint8),
        "down_proj.weight_scale": rng.integers(119, 128, (E, d, I // 32), dtype=np.uint8),
        "shared.gate": O.f32_to_bf16_bits(rng.normal(0.0, 0.05, (Is, d)).astype(np.float32)),
        "shared.up": O.f32_to_bf16_bits(rng.normal(0.0, 0.05, (Is, d)).astype(np.float32)),
        "shared.down": O.f32_to_bf16_bits(rng.normal(0.0, 0.05, (d, Is)).astype(np.float32)),
    }


def expected(layer):
    keys = ("gate_proj.weight_packed", "gate_proj.weight_scale", "up_proj.weight_packed",
            "up_proj.weight_scale", "down_proj.weight_packed", "down_proj.weight_scale")
    x = O.bf16_bits_to_f32(layer["x"])
    sw = tuple(O.bf16_bits_to_f32(layer[k]) for k in ("shared.gate", "shared.up", "shared.down"))
    out, inter = O.moe_layer(x, layer["router_weight"], layer["router_bias"],
                             O.Bank(*(layer[k] for k in keys)), sw, top_k=SHAPE["k"],
                             n_group=SHAPE["n_group"], topk_group=SHAPE["topk_group"],
                             norm_topk_prob=True,
                             routed_scaling_factor=SHAPE["routed_scaling_factor"],
                             swiglu_limit=SHAPE["swiglu_limit"], return_intermediates=True)
    return {"expected.out": out, "expected.indices": inter["indices"],
            "expected.weights": inter["weights"],
            "expected.h": O.f32_to_bf16_bits(inter["h"]),
            "expected.y": O.f32_to_bf16_bits(inter["route_outputs"])}


def main() -> None:
    layer = small_layer()
    arrays = dict(layer)
    arrays.update(expected(layer))
    np.savez(os.path.join(HERE, "moe_small.npz"), **arrays)
    print("wrote", os.path.join(HERE, "moe_small.npz"))


if __name__ == "__main__":
    main()
