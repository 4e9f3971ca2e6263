"""Synthetic routed-expert checkpoints for the loader tests.

Writes safetensors shards whose routed-expert tensors follow the reference's
names and shapes (``contract.py:47-50``, ``expert_source.py:189-204``): per
(layer, expert) ``down_proj`` / ``gate_proj`` / ``up_proj`` x
``weight_packed`` (U8 [rows, cols/2]) / ``weight_scale`` (U8 [rows, cols/32]),
plus an index ``model.safetensors.index.json`` and a ``config.json``.
"""

from __future__ import annotations

import json
import os
import struct

import numpy as np

COMPONENTS = ("down_proj", "gate_proj", "up_proj")
PARTS = ("weight_packed", "weight_scale")


def name(layer: int, expert: int, component: str, part: str) -> str:
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{component}.{part}"


def expert_arrays(rng: np.random.Generator, d: int, I: int,
                  scales: str = "uniform") -> dict[tuple[str, str], np.ndarray]:
    """``scales``: "uniform" E8M0 bytes in [119, 127]; "two_value" mostly 120
    and 121 with 1 % of other bytes in [119, 127] (the shape of the real
    checkpoint's scales, which ScaleX codes with one bit per scale)."""
    out = {}
    for comp in COMPONENTS:
        rows, cols = (d, I) if comp == "down_proj" else (I, d)
        out[(comp, "weight_packed")] = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
        shape = (rows, cols // 32)
        if scales == "uniform":
            sc = rng.integers(119, 128, shape, dtype=np.uint8)
        else:
            sc = rng.choice(np.array([120, 121], np.uint8), shape)
            odd = rng.random(shape) < 0.01
            sc[odd] = rng.integers(119, 128, int(odd.sum()), dtype=np.uint8)
        out[(comp, "weight_scale")] = sc
    return out


def write_safetensors(path: str, items: list[tuple[str, np.ndarray]]) -> None:
    """Writes the tensors in the given order: 8-byte little-endian header size,
    JSON header padded with spaces to a multiple of 8, then the raw data."""
    dtypes = {np.dtype(np.uint8): "U8", np.dtype(np.float32): "F32", np.dtype(np.int8): "I8",
              np.dtype(np.uint16): "BF16"}
    header, offset = {}, 0
    for key, arr in items:
        header[key] = {"dtype": dtypes[arr.dtype], "shape": list(arr.shape),
                       "data_offsets": [offset, offset + arr.nbytes]}
        offset += arr.nbytes
    raw = json.dumps(header).encode()
    raw += b" " * (-len(raw) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        for _, arr in items:
            f.write(np.ascontiguousarray(arr).tobytes())


def make_checkpoint(root: str, *, layers=(3, 4), E: int = 12, d: int = 64, I: int = 32,
                    seed: int = 5304, misalign: bool = False, shards_per_layer: int = 1,
                    shuffle: bool = True, extras: bool = True, scales: str = "uniform",
                    scalex: bool = False):
    """Writes a checkpoint under ``root``; returns {(layer, expert): arrays}.

    Each layer's experts go to ``shards_per_layer`` shards.  Within a shard the
    experts are written in a shuffled order (each expert's six tensors stay
    adjacent, as in the real checkpoint), with a non-expert F32 tensor between
    some of them so that not every record touches the next.  ``misalign``
    puts a 3-byte tensor first so that every expert tensor starts at an odd
    file offset.  ``scalex``: each layer's shard (one per layer, expert tensors
    only) is then rewritten as a ScaleX container."""
    rng = np.random.default_rng(seed)
    os.makedirs(root, exist_ok=True)
    weight_map, arrays = {}, {}
    for layer in layers:
        experts = list(range(E))
        if shuffle:
            rng.shuffle(experts)
        groups = np.array_split(np.array(experts), shards_per_layer)
        for s, group in enumerate(groups):
            shard = f"model-layer{layer}-{s:02d}.safetensors"
            items: list[tuple[str, np.ndarray]] = []
            if misalign:
                items.append((f"model.language_model.layers.{layer}.pad", np.zeros(3, np.uint8)))
            for n, e in enumerate(group):
                e = int(e)
                a = expert_arrays(rng, d, I, scales)
                arrays[(layer, e)] = a
                for comp in COMPONENTS:
                    for part in PARTS:
                        items.append((name(layer, e, comp, part), a[(comp, part)]))
                if extras and n % 3 == 1:
                    items.append((f"model.language_model.layers.{layer}.mlp.gate.w{e}",
                                  rng.standard_normal(5).astype(np.float32)))
            write_safetensors(os.path.join(root, shard), items)
            for key, _ in items:
                weight_map[key] = shard
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump({"text_config": {"hidden_size": d, "moe_intermediate_size": I,
                                   "n_routed_experts": E}}, f)
    if scalex:
        from livglm_amd.workloads import write_scalex_layer
        assert shards_per_layer == 1 and not extras and not misalign
        for layer in layers:
            shard = os.path.join(root, f"model-layer{layer}-00.safetensors")
            write_scalex_layer(shard, shard + ".sx", layer=layer, experts=E)
            os.replace(shard + ".sx", shard)
    return arrays
