"""ScaleX Mode-A/B codec and layer containers (CPU).

The reference's own codec cases (``tests/test_scale_codec.py:13-34``), the
header layout byte by byte, round trips at the real checkpoint's scale mix,
the container written, read, verified against the original file's SHA-256,
and planned through the checkpoint contract (``tests/test_scalex_container.py``).
"""

from __future__ import annotations

import hashlib
import os
import struct

import numpy as np
import pytest

from checkpoint_util import COMPONENTS, make_checkpoint, name

from glm53flash.contract import ContractError, ModelContract
from glm53flash.expert_source import build_native_expert_source_plan
from glm53flash.model_config import GLMTextConfig
from glm53flash.scale_codec import (ScaleCodecError, decode_mode_a, encode_mode_a,
                                    encode_mode_b_row, inspect_mode_a, mode_b_indexed_nbytes,
                                    mode_b_tile_prefix, validate_mode_a)
from glm53flash.scalex_container import (ScaleXContainerError, is_scalex_layer,
                                         read_scalex_layout, read_scalex_tensor,
                                         verify_scalex_layer)


@pytest.mark.parametrize(("values", "codec"), [
    (np.resize(np.array([120, 121], np.uint8), 4096), "one_bit"),
    (np.resize(np.array([118, 119, 120, 121], np.uint8), 4096), "two_bit"),
    (np.arange(256, dtype=np.uint8).repeat(16), "raw"),
])
def test_reference_codec_cases(values, codec):
    raw = values.tobytes()
    encoded = encode_mode_a(raw)
    info = inspect_mode_a(encoded)
    assert info.codec == codec and info.raw_bytes == len(raw)
    assert decode_mode_a(encoded) == raw
    assert len(encode_mode_b_row(encoded)) == mode_b_indexed_nbytes(len(encoded), len(raw))
    with pytest.raises(ScaleCodecError, match="truncated"):
        decode_mode_a(b"LSA1")


def test_one_bit_record_layout_by_hand():
    """64 scales of 120 except a 121 at position 3 and a 125 at position 5: the
    palette is (120, 121, 125, 0) (counts, ties to the smaller byte), the one-bit
    form (8 + 5 bytes) beats the two-bit one (16 bytes), its first primary byte
    is 0b00001000 and 125 is the one exception."""
    raw = bytearray([120] * 64)
    raw[3], raw[5] = 121, 125
    raw = bytes(raw)
    enc = encode_mode_a(raw)
    assert enc[:4] == b"LSA1" and enc[4] == 1 and tuple(enc[5:9]) == (120, 121, 125, 0)
    assert enc[9:12] == b"\0\0\0"
    assert struct.unpack("<III", enc[12:24]) == (64, 8, 1)
    assert enc[24] == 0b00001000 and enc[25:32] == bytes(7)
    assert struct.unpack("<I", enc[32:36]) == (5,) and enc[36] == 125
    assert len(enc) == 37 and decode_mode_a(enc) == raw
    # the tile directory: exception 0 is the first at or after offset 0 and 1 after the end
    assert struct.unpack("<HH", mode_b_tile_prefix(enc)) == (0, 1)


def test_two_bit_packing_order():
    raw = bytes([1, 2, 3, 4] * 3 + [1])  # four values, each thrice or more
    enc = encode_mode_a(raw)
    info = validate_mode_a(enc)
    assert info.codec == "two_bit" and info.palette == (1, 2, 3, 4)
    assert enc[24] == (0 | 1 << 2 | 2 << 4 | 3 << 6)  # first code in the low bits
    assert decode_mode_a(enc) == raw


def test_round_trip_at_checkpoint_scale_mix():
    rng = np.random.default_rng(9)
    for n in (1, 7, 513, 100_000):
        v = rng.choice(np.array([120, 121], np.uint8), n)
        odd = rng.random(n) < 0.01
        v[odd] = rng.integers(119, 128, int(odd.sum()), dtype=np.uint8)
        enc = encode_mode_a(v.tobytes())
        assert decode_mode_a(enc) == v.tobytes()
        if n == 100_000:
            assert inspect_mode_a(enc).codec == "one_bit" and len(enc) < n // 5
    good = encode_mode_a(bytes([120] * 200 + [121, 7, 9]))  # one bit, exceptions at 200, 202
    assert inspect_mode_a(good).exceptions == 2
    bad = bytearray(good)
    pos_at = 24 + 26  # 203 scales -> 26 primary bytes
    assert struct.unpack("<II", bad[pos_at:pos_at + 8]) == (200, 202)
    bad[pos_at:pos_at + 8] = struct.pack("<II", 202, 200)  # descending positions
    with pytest.raises(ScaleCodecError, match="position"):
        validate_mode_a(bytes(bad))


def test_container_round_trip_and_plan(tmp_path):
    E, d, I, layers = 6, 256, 256, (3, 4)
    native = tmp_path / "native"
    coded = tmp_path / "coded"
    arrays = make_checkpoint(str(native), layers=layers, E=E, d=d, I=I, extras=False,
                             scales="two_value", shuffle=False)
    make_checkpoint(str(coded), layers=layers, E=E, d=d, I=I, extras=False, scales="two_value",
                    shuffle=False, scalex=True)
    shard = coded / "model-layer3-00.safetensors"
    original = native / "model-layer3-00.safetensors"
    assert is_scalex_layer(shard) and not is_scalex_layer(original)
    assert verify_scalex_layer(shard) == hashlib.sha256(original.read_bytes()).hexdigest()
    assert shard.stat().st_size < original.stat().st_size
    layout = read_scalex_layout(shard)
    assert layout.layer == 3 and layout.experts == E
    assert layout.records[0].codec == "one_bit"
    for e in range(E):
        for c in COMPONENTS:
            for p in ("weight_packed", "weight_scale"):
                assert read_scalex_tensor(layout, name(3, e, c, p)) == arrays[(3, e)][(c, p)].tobytes()
    cfg = GLMTextConfig(hidden_size=d, moe_intermediate_size=I, n_routed_experts=E)
    contract = ModelContract.from_model_dir(coded)
    plan = build_native_expert_source_plan(contract, cfg, first_layer=3, last_layer=4)
    assert plan.scalex_mode_b and plan.source_format == "livglm_scalex_mode_b"
    assert plan.read_bytes < plan.payload_bytes and plan.uniform_read_count == 1
    src = plan.expert(3, 2)
    rec = src.scalex_record
    (rng_,) = src.read_ranges
    assert rng_.absolute_offset == rec.absolute_offset and rng_.byte_length == rec.physical_bytes
    assert [t.source_name for t in rng_.tensors] == list(rec.weight_names)
    # the virtual tensor ranges still describe the original file
    native_plan = build_native_expert_source_plan(ModelContract.from_model_dir(native), cfg,
                                                  first_layer=3, last_layer=4)
    assert [t.absolute_offset for t in src.tensors] == [
        t.absolute_offset for t in native_plan.expert(3, 2).tensors]
    # a damaged container is refused
    raw = bytearray(shard.read_bytes())
    raw[-1] ^= 1
    broken = tmp_path / "broken.safetensors"
    broken.write_bytes(bytes(raw))
    with pytest.raises(ScaleXContainerError):
        verify_scalex_layer(broken)
    raw = bytearray(shard.read_bytes())
    raw[40] ^= 0xFF  # inside the JSON metadata
    broken.write_bytes(bytes(raw))
    with pytest.raises(ScaleXContainerError):
        read_scalex_layout(broken)
    # mixing ScaleX and native layers is refused
    os.replace(native / "model-layer4-00.safetensors", coded / "model-layer4-00.safetensors")
    with pytest.raises(ContractError, match="mix"):
        build_native_expert_source_plan(ModelContract.from_model_dir(coded), cfg,
                                        first_layer=3, last_layer=4)
