"""Synthetic MoE-layer workloads (seeded) for tests and the benchmark.

Shapes follow the routed-MoE layer of GLM-5.3-Flash at benchmark geometry:

* ``decode_t1``    T=1,    d=1024, E=16,  k=2, I=512  (+ bf16 shared expert)
* ``verify_t2``    T=2,    d=2048, E=128, k=8, I=768  (MTP width-two verify)
* ``batch_t64``    T=64,   as verify_t2, Zipf(s=1.1)-skewed routing bias
* ``prefill_t4096`` T=4096, as verify_t2, near-uniform routing
* ``stack42_t1``   T=1, 42 layers of (2048x2048 MXFP8 resident linear + MoE
  as verify_t2), 256 decode steps, Markov routing with 70% expert reuse
* ``real_t2``      T=2 at the real GLM expert geometry: d=4096, E=288, k=8,
  I=2048 (bf16 shared expert I=2048)
* ``ffn_t2``       the decoder FFN site at verify_t2: hyper-connection of 4 f32
  residual streams (20 Sinkhorn rounds) + post-attention RMSNorm + the MoE
  layer + hyper_residual

Expert weights: uniform random E2M1 codes (uniform bytes) and E8M0 scale
bytes uniform in [119, 127].  Activations bf16 N(0, 1).  Router weight f32
N(0, 0.02), bias 0 unless stated.  Shared expert bf16 N(0, 0.02).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class MoEShape:
    name: str
    T: int
    d: int
    E: int
    k: int
    I: int
    I_shared: int
    routing: str = "uniform"  # "uniform" | "zipf" | "markov"
    n_group: int = 1
    topk_group: int = 1
    routed_scaling_factor: float = 2.5
    swiglu_limit: float = 10.0
    norm_topk_prob: bool = True
    layers: int = 1
    steps: int = 1
    hc: int = 0  # > 0: the decoder FFN site (hyper-connection of hc streams + norm) around it

    @property
    def expert_bytes(self) -> int:
        """MXFP4 bytes of one expert: 3 projections x (I*d/2 codes + I*d/32 scales)."""
        return 3 * (self.I * self.d // 2 + self.I * self.d // 32)

    @property
    def bank_bytes(self) -> int:
        return self.E * self.expert_bytes


SHAPES = {
    "decode_t1": MoEShape("decode_t1", T=1, d=1024, E=16, k=2, I=512, I_shared=512),
    "verify_t2": MoEShape("verify_t2", T=2, d=2048, E=128, k=8, I=768, I_shared=768),
    "batch_t64": MoEShape("batch_t64", T=64, d=2048, E=128, k=8, I=768, I_shared=768,
                          routing="zipf"),
    "prefill_t4096": MoEShape("prefill_t4096", T=4096, d=2048, E=128, k=8, I=768, I_shared=768),
    "stack42_t1": MoEShape("stack42_t1", T=1, d=2048, E=128, k=8, I=768, I_shared=768,
                           routing="markov", layers=42, steps=256),
    "ffn_t2": MoEShape("ffn_t2", T=2, d=2048, E=128, k=8, I=768, I_shared=768, hc=4),
    "real_t2": MoEShape("real_t2", T=2, d=4096, E=288, k=8, I=2048, I_shared=2048),
}

SCALE_LO, SCALE_HI = 119, 127  # inclusive E8M0 range of the synthetic scales


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def zipf_bias(E: int, rng: np.random.Generator, s: float = 1.1, scale: float = 1.0) -> np.ndarray:
    """Per-expert bias from a Zipf(s) rank profile over a random expert order:
    ``bias[pi[r]] = scale * (r + 1) ** -s``."""
    order = rng.permutation(E)
    bias = np.zeros(E, dtype=np.float32)
    bias[order] = (scale * np.arange(1, E + 1, dtype=np.float64) ** (-s)).astype(np.float32)
    return bias


def markov_bias_trace(E: int, k: int, layers: int, steps: int, rng: np.random.Generator,
                      keep: float = 0.7, boost: float = 10.0) -> np.ndarray:
    """Bias vectors [steps, layers, E] that force each layer's top-k to keep
    each of the previous step's experts with probability ``keep`` and draw the
    rest uniformly from the unused experts (a boost of ``boost`` on the chosen
    set dominates every sigmoid score)."""
    out = np.zeros((steps, layers, E), dtype=np.float32)
    prev = [rng.choice(E, k, replace=False) for _ in range(layers)]
    for s in range(steps):
        for layer in range(layers):
            if s == 0:
                chosen = prev[layer]
            else:
                kept = [e for e in prev[layer] if rng.random() < keep]
                pool = np.setdiff1d(np.arange(E), kept)
                fresh = rng.choice(pool, k - len(kept), replace=False)
                chosen = np.concatenate([np.array(kept, dtype=np.int64), fresh])
            out[s, layer, chosen] = boost
            prev[layer] = chosen
    return out


def concentrated_scales(rng: np.random.Generator, shape, kind: str = "one_bit") -> np.ndarray:
    """E8M0 scale bytes with the statistics of the real checkpoint's experts
    (docs/scalex-mode-b.md:36-50: 12,067 of 12,096 experts code at one bit
    with exceptions, 16.9 % of the raw bytes): two dominant exponents and
    ~1 % others ("one_bit"); four dominant values ("two_bit"); or uniform
    over 119..127 ("raw", which the codec stores as it is)."""
    n = int(np.prod(shape))
    if kind == "raw":
        return rng.integers(SCALE_LO, SCALE_HI + 1, n, dtype=np.uint8).reshape(shape)
    if kind == "one_bit":
        v = np.where(rng.random(n) < 0.56, 121, 122).astype(np.uint8)
        other = rng.random(n) < 0.01
    else:
        v = rng.choice(np.array([120, 121, 122, 123], np.uint8), n, p=[0.2, 0.35, 0.3, 0.15])
        other = rng.random(n) < 0.002
    v[other] = rng.integers(110, 128, int(other.sum()), dtype=np.uint8)
    return v.reshape(shape)


def make_layer(shape: MoEShape, seed: int, *, T: int | None = None) -> dict[str, np.ndarray]:
    """One layer's inputs and weights as numpy arrays (bf16 as uint16 bits)."""
    rng = np.random.default_rng(seed)
    T = shape.T if T is None else T
    d, E, I, Is = shape.d, shape.E, shape.I, shape.I_shared

    def codes(*s):
        return rng.integers(0, 256, s, dtype=np.uint8)

    def scales(*s):
        return rng.integers(SCALE_LO, SCALE_HI + 1, s, dtype=np.uint8)

    layer = {
        "x": f32_to_bf16_bits(rng.standard_normal((T, d), dtype=np.float32)),
        "router_weight": rng.normal(0.0, 0.02, (E, d)).astype(np.float32),
        "router_bias": np.zeros(E, dtype=np.float32),
        "gate_proj.weight_packed": codes(E, I, d // 2),
        "gate_proj.weight_scale": scales(E, I, d // 32),
        "up_proj.weight_packed": codes(E, I, d // 2),
        "up_proj.weight_scale": scales(E, I, d // 32),
        "down_proj.weight_packed": codes(E, d, I // 2),
        "down_proj.weight_scale": scales(E, d, I // 32),
        "shared.gate": f32_to_bf16_bits(rng.normal(0.0, 0.02, (Is, d)).astype(np.float32)),
        "shared.up": f32_to_bf16_bits(rng.normal(0.0, 0.02, (Is, d)).astype(np.float32)),
        "shared.down": f32_to_bf16_bits(rng.normal(0.0, 0.02, (d, Is)).astype(np.float32)),
    }
    if shape.routing == "zipf":
        layer["router_bias"] = zipf_bias(E, rng)
    return layer


BANK_KEYS = ("gate_proj.weight_packed", "gate_proj.weight_scale", "up_proj.weight_packed",
             "up_proj.weight_scale", "down_proj.weight_packed", "down_proj.weight_scale")


def write_expert_checkpoint(root: str, shape: MoEShape, layers, seed: int,
                            two_value_scales: bool = False) -> int:
    """Writes a routed-expert checkpoint for ``layers`` (one safetensors shard
    per layer, experts in id order, each expert's six U8 tensors adjacent in
    the reference's canonical order) plus ``model.safetensors.index.json`` and
    ``config.json``.  Every layer stores the same random bank (one layer's
    bytes drawn once); returns the payload bytes written.  Scales are uniform
    bytes, or with ``two_value_scales`` 120/121 with 1 % of other values in
    [119, 127] (the mix of the real checkpoint, which ScaleX codes with one bit
    per scale)."""
    import json
    import os
    import struct

    rng = np.random.default_rng(seed)
    d, I, E = shape.d, shape.I, shape.E
    parts = []
    for comp in ("down_proj", "gate_proj", "up_proj"):
        rows, cols = (d, I) if comp == "down_proj" else (I, d)
        parts.append((comp, "weight_packed", (rows, cols // 2)))
        parts.append((comp, "weight_scale", (rows, cols // 32)))
    record = sum(r * c for _, _, (r, c) in parts)
    blob = rng.integers(0, 256, E * record, dtype=np.uint8)
    if two_value_scales:
        rec = blob.reshape(E, record)
        at = 0
        for _, part, (r, c) in parts:
            if part == "weight_scale":
                sc = rng.choice(np.array([120, 121], np.uint8), (E, r * c))
                odd = rng.random((E, r * c)) < 0.01
                sc[odd] = rng.integers(119, 128, int(odd.sum()), dtype=np.uint8)
                rec[:, at:at + r * c] = sc
            at += r * c
    os.makedirs(root, exist_ok=True)
    weight_map = {}
    for layer in layers:
        header, offset = {}, 0
        for e in range(E):
            for comp, part, (r, c) in parts:
                name = f"model.language_model.layers.{layer}.mlp.experts.{e}.{comp}.{part}"
                header[name] = {"dtype": "U8", "shape": [r, c],
                                "data_offsets": [offset, offset + r * c]}
                offset += r * c
        raw = json.dumps(header).encode()
        raw += b" " * (-len(raw) % 8)
        shard = f"model-layer{layer:02d}.safetensors"
        with open(os.path.join(root, shard), "wb") as f:
            f.write(struct.pack("<Q", len(raw)))
            f.write(raw)
            blob.tofile(f)
        weight_map.update({name: shard for name in header})
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump({"text_config": {"hidden_size": d, "moe_intermediate_size": I,
                                   "n_routed_experts": E}}, f)
    return len(layers) * E * record


def write_scalex_layer(source, destination, *, layer: int, experts: int):
    """Test and benchmark fixture: writes the ScaleX container of a synthetic
    safetensors shard that holds exactly the routed-expert tensors of
    ``layer`` (experts 0 .. experts - 1) in the container format the package
    reads (``glm53flash.scalex_layer``), then reads it back and verifies the
    rebuild.  Every expert's coded scales must fit the Mode-B tile directory
    (at most 65535 exceptions), or nothing is written; the file is written
    beside ``destination`` and renamed onto it only once it verifies."""
    import hashlib
    import json
    import os
    from pathlib import Path

    from glm53flash import scalex_layer as X
    from glm53flash.checkpoint import read_safetensors_header
    from glm53flash.scale_codec import (decode_mode_a, encode_mode_a, inspect_mode_a,
                                        mode_b_tile_prefix)

    src, dst = Path(source), Path(destination)
    if X.is_scalex_file(src):
        raise X.ScaleXError(f"{src} is already a ScaleX container")
    if dst.exists():
        raise X.ScaleXError(f"{dst} exists; not overwriting it")
    base, header = read_safetensors_header(src)
    names = {X.tensor_name(layer, e, c, p) for e in range(experts) for c in X.RECORD_ORDER
             for p in ("weight_packed", "weight_scale")}
    present = set(header) - {"__metadata__"}
    if present != names:
        extra, missing = sorted(present - names)[:3], sorted(names - present)[:3]
        raise X.ScaleXError(f"{src}: not exactly layer {layer}'s {experts} experts "
                            f"(extra {extra}, missing {missing})")
    spans = X._payload_order(header)
    if base + (spans[-1][1] if spans else 0) != src.stat().st_size:
        raise X.ScaleXError(f"{src}: data area does not end at the end of the file")
    with src.open("rb") as fh:
        prefix = fh.read(base)

        def read(n: str) -> bytes:
            fh.seek(base + header[n]["data_offsets"][0])
            return fh.read(X._header_size(header, n))

        records, blobs = [], []
        at = base
        for e in range(experts):
            scale_parts = [read(X.tensor_name(layer, e, c, "weight_scale")) for c in X.RECORD_ORDER]
            weights = [read(X.tensor_name(layer, e, c, "weight_packed")) for c in X.RECORD_ORDER]
            raw = b"".join(scale_parts)
            coded = encode_mode_a(raw)
            if decode_mode_a(coded) != raw:
                raise X.ScaleXError(f"{src}: expert {e}'s scales do not survive coding")
            mode_b_tile_prefix(coded)  # raises when the exceptions overflow the directory
            records.append({
                "expert": e, "stored_offset": at, "encoded_bytes": len(coded),
                "decoded_bytes": len(raw), "codec": inspect_mode_a(coded).codec,
                "scale_names": [X.tensor_name(layer, e, c, "weight_scale") for c in X.RECORD_ORDER],
                "scale_nbytes": [len(p) for p in scale_parts],
                "weight_names": [X.tensor_name(layer, e, c, "weight_packed")
                                 for c in X.RECORD_ORDER],
                "weight_nbytes": [len(w) for w in weights]})
            blobs.append(coded + b"".join(weights))
            at += len(blobs[-1])
    digest = hashlib.sha256()
    with src.open("rb") as fh:
        while block := fh.read(16 << 20):
            digest.update(block)
    meta = {"format": X.FORMAT, "version": X.VERSION, "layer": int(layer),
            "experts": int(experts), "scale_order": list(X.RECORD_ORDER),
            "weight_order": list(X.RECORD_ORDER), "original_bytes": src.stat().st_size,
            "original_sha256": digest.hexdigest(), "original_prefix_bytes": len(prefix),
            "original_prefix_sha256": hashlib.sha256(prefix).hexdigest(), "records": records}
    meta_raw = json.dumps(meta, sort_keys=True, separators=(",", ":")).encode()
    tmp = dst.with_name(dst.name + f".partial{os.getpid()}")
    try:
        with tmp.open("xb") as out:
            out.write(X.PREFIX.pack(X.MAGIC, X.VERSION, len(meta_raw), at))
            out.write(meta_raw)
            out.write(prefix)
            for blob in blobs:
                out.write(blob)
        os.chmod(tmp, src.stat().st_mode)
        X.ScaleXLayer.read(tmp).verify()
        if dst.exists():
            raise X.ScaleXError(f"{dst} exists; not overwriting it")
        os.replace(tmp, dst)
    finally:
        if tmp.exists():
            tmp.unlink()
    return X.ScaleXLayer.read(dst)


def make_hc(T: int, hc: int, d: int, seed: int, *, bf16_streams: bool = False):
    """Hyper-connection inputs of a decoder FFN site: streams f32 [T, hc, d]
    N(0, 1) (bf16-representable when ``bf16_streams``), fn f32
    [2 hc + hc^2, hc d] N(0, 0.02), base N(0, 0.5), scale U(0.5, 1.5), and the
    post-attention norm weight (bf16-representable, around 1)."""
    rng = np.random.default_rng(seed)
    M = 2 * hc + hc * hc
    streams = rng.standard_normal((T, hc, d), dtype=np.float32)
    if bf16_streams:
        streams = (f32_to_bf16_bits(streams).astype(np.uint32) << 16).view(np.float32)
    norm = rng.normal(1.0, 0.1, d).astype(np.float32)
    return {
        "streams": np.ascontiguousarray(streams),
        "fn": rng.normal(0.0, 0.02, (M, hc * d)).astype(np.float32),
        "base": rng.normal(0.0, 0.5, M).astype(np.float32),
        "scale": rng.uniform(0.5, 1.5, 3).astype(np.float32),
        "norm_weight": (f32_to_bf16_bits(norm).astype(np.uint32) << 16).view(np.float32),
    }
