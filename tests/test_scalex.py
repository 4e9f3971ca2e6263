"""ScaleX Mode-A/B codec and layer containers (CPU).

The reference's own codec cases (``tests/test_scale_codec.py:13-34``), the
header layout byte by byte, round trips at the real checkpoint's scale mix,
the container written, read, verified against the original file's SHA-256,
and planned through the bank load plan.
"""

from __future__ import annotations

import hashlib
import os
import struct

import numpy as np
import pytest

from checkpoint_util import COMPONENTS, make_checkpoint, name

from glm53flash.bank_plan import plan_expert_banks
from glm53flash.checkpoint import ShardIndex
from glm53flash.contract import ContractError
from glm53flash.scale_codec import (ScaleCodecError, decode_mode_a, encode_mode_a,
                                    encode_mode_b_row, inspect_mode_a, mode_b_indexed_nbytes,
                                    mode_b_tile_prefix, validate_mode_a)
from glm53flash.scalex_layer import ScaleXError, ScaleXLayer, is_scalex_file


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
    with pytest.raises(ScaleCodecError, match="positions must ascend"):
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
    assert is_scalex_file(shard) and not is_scalex_file(original)
    layout = ScaleXLayer.read(shard)
    assert layout.verify() == hashlib.sha256(original.read_bytes()).hexdigest()
    assert shard.stat().st_size < original.stat().st_size
    assert layout.layer == 3 and layout.experts == E
    assert layout.records[0].codec == "one_bit"
    for e in range(E):
        for c in COMPONENTS:
            for p in ("weight_packed", "weight_scale"):
                assert layout.tensor_bytes(name(3, e, c, p)) == arrays[(3, e)][(c, p)].tobytes()
    plan = plan_expert_banks(ShardIndex.open(coded), hidden_size=d, intermediate_size=I,
                             experts=E, layers=layers)
    assert plan.scalex and plan.read_bytes < plan.bank_bytes
    x = plan.expert(3, 2)
    rec = x.coded
    (rd,) = x.reads
    assert rd.offset == rec.offset and rd.nbytes == rec.nbytes
    # weights follow the coded scales in gate, down, up order
    assert [(s.key, s.at) for s in rd.segments] == [
        ("gate_proj.weight_packed", rec.coded_bytes),
        ("down_proj.weight_packed", rec.coded_bytes + rec.weight_bytes[0]),
        ("up_proj.weight_packed", rec.coded_bytes + rec.weight_bytes[0] + rec.weight_bytes[1])]
    with open(shard, "rb") as f:
        f.seek(rd.offset + rd.segments[1].at)
        assert f.read(rd.segments[1].nbytes) == arrays[(3, 2)][("down_proj",
                                                               "weight_packed")].tobytes()
    # the tensor ranges the index gives for a container describe the original file
    coded_idx, native_idx = ShardIndex.open(coded), ShardIndex.open(native)
    for c in COMPONENTS:
        n = name(3, 2, c, "weight_scale")
        assert coded_idx.locate(n) == native_idx.locate(n)
    # a damaged container is refused
    raw = bytearray(shard.read_bytes())
    raw[-1] ^= 1
    broken = tmp_path / "broken.safetensors"
    broken.write_bytes(bytes(raw))
    with pytest.raises(ScaleXError, match="original_sha256"):
        ScaleXLayer.read(broken).verify()
    raw = bytearray(shard.read_bytes())
    raw[40] ^= 0xFF  # inside the JSON metadata
    broken.write_bytes(bytes(raw))
    with pytest.raises(ScaleXError):
        ScaleXLayer.read(broken)
    # mixing ScaleX and native layers is refused
    os.replace(native / "model-layer4-00.safetensors", coded / "model-layer4-00.safetensors")
    with pytest.raises(ContractError, match="mix"):
        plan_expert_banks(ShardIndex.open(coded), hidden_size=d, intermediate_size=I,
                          experts=E, layers=layers)


def test_fixture_writer_refuses_directory_overflow_and_leaves_no_file(tmp_path, monkeypatch):
    """An expert whose exceptions overflow the u16 Mode-B directory is refused
    before anything is written, and a failed write leaves neither the
    destination nor a partial file behind."""
    from glm53flash import scale_codec
    from livglm_amd.workloads import write_scalex_layer
    E, d, I = 2, 64, 64
    root = tmp_path / "ck"
    make_checkpoint(str(root), layers=(3,), E=E, d=d, I=I, extras=False, shuffle=False)
    src = root / "model-layer3-00.safetensors"

    def overflow(encoded):
        raise scale_codec.ScaleCodecError("70000 exceptions overflow the u16 tile directory")

    monkeypatch.setattr(scale_codec, "mode_b_tile_prefix", overflow)
    with pytest.raises(scale_codec.ScaleCodecError, match="overflow"):
        write_scalex_layer(src, tmp_path / "x.sx", layer=3, experts=E)
    monkeypatch.undo()
    assert sorted(p.name for p in tmp_path.iterdir()) == ["ck"]
    # a verification failure after the bytes are written removes the partial file
    from glm53flash import scalex_layer as X

    def bad_verify(self):
        raise X.ScaleXError("rebuilt original does not match original_sha256")

    monkeypatch.setattr(X.ScaleXLayer, "verify", bad_verify)
    with pytest.raises(X.ScaleXError, match="does not match"):
        write_scalex_layer(src, tmp_path / "y.sx", layer=3, experts=E)
    assert sorted(p.name for p in tmp_path.iterdir()) == ["ck"]


def test_container_reader_checks(tmp_path):
    """Metadata that disagrees with the stored data is refused with a reason."""
    import json
    import struct as st
    from glm53flash.scalex_layer import PREFIX
    from livglm_amd.workloads import write_scalex_layer
    E, d, I = 3, 64, 64
    root = tmp_path / "ck"
    make_checkpoint(str(root), layers=(3,), E=E, d=d, I=I, extras=False, shuffle=False)
    src = root / "model-layer3-00.safetensors"
    good = tmp_path / "good.sx"
    write_scalex_layer(src, good, layer=3, experts=E)
    with pytest.raises(ScaleXError, match="already a ScaleX"):
        write_scalex_layer(good, tmp_path / "again.sx", layer=3, experts=E)
    with pytest.raises(ScaleXError, match="not exactly layer 4"):
        write_scalex_layer(src, tmp_path / "wrong.sx", layer=4, experts=E)
    blob = good.read_bytes()
    magic, version, mlen, stored = PREFIX.unpack_from(blob)
    meta = json.loads(blob[PREFIX.size:PREFIX.size + mlen])

    def rewrite(change, label):
        m = json.loads(json.dumps(meta))
        change(m)
        raw = json.dumps(m, sort_keys=True, separators=(",", ":")).encode()
        out = tmp_path / f"{label}.sx"
        out.write_bytes(PREFIX.pack(magic, version, len(raw), stored) + raw
                        + blob[PREFIX.size + mlen:])
        return out

    cases = [
        (lambda m: m.update(format="other"), "unusable 'format'"),
        (lambda m: m["records"][1].update(stored_offset=m["records"][1]["stored_offset"] + 1),
         "expected expert 1"),
        (lambda m: m["records"][0].update(codec="three_bit"), "unusable 'codec'"),
        (lambda m: m["records"][2]["scale_nbytes"].__setitem__(0, 7), "decoded_bytes"),
        (lambda m: m.update(experts=4), "records for 4 experts"),
        (lambda m: m["records"][0]["weight_names"].reverse(), "gate, down, up"),
        (lambda m: m.pop("original_sha256"), "lacks 'original_sha256'"),
    ]
    for i, (change, text) in enumerate(cases):
        with pytest.raises(ScaleXError, match=text):
            ScaleXLayer.read(rewrite(change, f"c{i}"))
    # a stored length that disagrees with the file
    bad = tmp_path / "len.sx"
    bad.write_bytes(PREFIX.pack(magic, version, mlen, stored + 1) + blob[PREFIX.size:])
    with pytest.raises(ScaleXError, match="prefix promises"):
        ScaleXLayer.read(bad)
    assert st.calcsize("<8sIIQ") == PREFIX.size == 24


def test_mode_b_bank_rows_decode_to_the_scales():
    # glm_moe_forward_scalex's bank: one Mode-B row per expert at a common
    # 256-byte stride; the checkpoint-like mix codes at ~17 % of the raw bytes
    from glm53flash import scale_codec
    from livglm_amd.workloads import concentrated_scales
    rng = np.random.default_rng(12)
    E, I, d = 5, 256, 1024
    kinds = ["one_bit", "two_bit", "raw", "one_bit", "one_bit"]
    g = np.stack([concentrated_scales(rng, (I, d // 32), kd) for kd in kinds])
    dn = np.stack([concentrated_scales(rng, (d, I // 32), kd) for kd in kinds])
    u = np.stack([concentrated_scales(rng, (I, d // 32), kd) for kd in kinds])
    rows, stride, coded = scale_codec.mode_b_bank(g, dn, u)
    assert stride % 256 == 0 and rows.shape == (E, stride)
    for e in range(E):
        raw_n = g[e].size + dn[e].size + u[e].size
        rec = scale_codec.mode_b_record(rows[e], raw_n)
        assert scale_codec.decode_mode_a(rec) == g[e].tobytes() + dn[e].tobytes() + u[e].tobytes()
        info = scale_codec.inspect_mode_a(rec)
        # the directory of encode_mode_b_row, in front of the record
        db = scale_codec.mode_b_dir_bytes(raw_n)
        directory = scale_codec.mode_b_tile_prefix(rec)
        row = bytes(rows[e])
        assert db % 16 == 0 and row[:len(directory)] == directory and not any(row[len(directory):db])
        assert row[db:db + len(rec)] == rec and not any(row[db + len(rec):])
        assert scale_codec.encode_mode_b_row(rec).endswith(directory)
        assert info.codec == {"one_bit": "one_bit", "two_bit": "two_bit", "raw": "raw"}[kinds[e]]
    one = [e for e in range(E) if kinds[e] == "one_bit"]
    raw = 3 * I * (d // 32)
    for e in one:
        info = scale_codec.inspect_mode_a(scale_codec.mode_b_record(rows[e], raw))
        assert 0.14 < info.encoded_bytes / raw < 0.20
