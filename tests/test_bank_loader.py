"""Checkpoint contract, expert source plan and the native range reader (CPU).

The plan mirrors ``expert_source.py:270-381``; the shards are written by the
test's own writer and by the ``safetensors`` library, whose reader is the
independent check of the header parsing and byte ranges.
"""

from __future__ import annotations

import ctypes
import json
import os

import numpy as np
import pytest

from checkpoint_util import COMPONENTS, PARTS, make_checkpoint, name, write_safetensors

from glm53flash.contract import (ContractError, ModelContract, local_safetensors_header,
                                 routed_expert_parts)
from glm53flash.expert_source import build_native_expert_source_plan, coalesce
from glm53flash.model_config import GLMTextConfig

D, I, E = 64, 32, 12
RECORD = 3 * I * D * 17 // 32


def _config(E=E, d=D, I=I):
    return GLMTextConfig(hidden_size=d, moe_intermediate_size=I, n_routed_experts=E)


def _file_bytes(path, off, n):
    with open(path, "rb") as f:
        f.seek(off)
        return f.read(n)


def test_header_matches_the_safetensors_library(tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(1)
    tensors = {name(3, e, c, p): rng.integers(0, 256, (4, 8 if p == "weight_packed" else 2),
                                                 dtype=np.uint8)
               for e in range(3) for c in COMPONENTS for p in PARTS}
    path = str(tmp_path / "a.safetensors")
    st.save_file(tensors, path)
    base, header = local_safetensors_header(path)
    for key, arr in tensors.items():
        start, end = header[key]["data_offsets"]
        assert _file_bytes(path, base + start, end - start) == arr.tobytes()
    loaded = st.load_file(path)
    assert set(loaded) == set(tensors)


def test_plan_locates_every_expert_record(tmp_path):
    arrays = make_checkpoint(str(tmp_path), layers=(3, 4), E=E, d=D, I=I)
    contract = ModelContract.from_model_dir(tmp_path)
    plan = build_native_expert_source_plan(contract, _config(), first_layer=3, last_layer=4)
    assert plan.expert_count == 2 * E and plan.tensor_count == 12 * E
    assert plan.uniform_pack_bytes == RECORD == plan.slot_bytes(3)
    # each expert's six tensors are adjacent in its shard: one read per record
    assert plan.uniform_read_count == 1 and plan.read_bytes == plan.payload_bytes
    for layer in (3, 4):
        for e in range(E):
            src = plan.expert(layer, e)
            assert [t.source_name for t in src.tensors] == [
                name(layer, e, c, p) for c in COMPONENTS for p in PARTS]
            (rng,) = src.read_ranges
            for t in src.tensors:
                comp, part = t.bank_name.split(".")
                path = os.path.join(plan.model_dir, t.shard_name)
                want = arrays[(layer, e)][(comp, part)]
                assert t.byte_length == want.nbytes and t.source_shape == want.shape
                assert _file_bytes(path, t.absolute_offset, t.byte_length) == want.tobytes()
                assert 0 <= rng.relative_offset(t) < rng.byte_length
            packed = [t for t in src.tensors if t.bank_name.endswith("weight_packed")]
            assert all(t.mlx_dtype == "U32" and t.mlx_shape[-1] * 4 == t.source_shape[-1]
                       for t in packed)
    d = plan.as_dict()
    assert d["uniform_pack_bytes"] == RECORD and d["layer_count"] == 2
    assert d["source_format"] == "native_mxfp4" and not d["scalex_mode_b"]
    with pytest.raises(ContractError):
        plan.expert(5, 0)
    with pytest.raises(ContractError):
        plan.expert(3, E)


def test_coalesce_splits_at_gaps_and_shards():
    from glm53flash.expert_source import ExpertTensorSource

    def t(shard, off, n):
        return ExpertTensorSource(f"x.{off}.weight_packed", "x", shard, off, n, (n,), "U8", (n,))

    ranges = coalesce((t("b", 0, 4), t("a", 10, 5), t("a", 0, 10), t("a", 16, 2)))
    assert [(r.shard_name, r.absolute_offset, r.byte_length, len(r.tensors)) for r in ranges] == [
        ("a", 0, 15, 2), ("a", 16, 2, 1), ("b", 0, 4, 1)]


def test_plan_rejects_broken_checkpoints(tmp_path):
    def fresh(sub):
        root = str(tmp_path / sub)
        make_checkpoint(root, layers=(3,), E=4, d=D, I=I, shuffle=False)
        return root

    # wrong storage dtype
    root = fresh("dtype")
    shard = os.path.join(root, "model-layer3-00.safetensors")
    base, header = local_safetensors_header(shard)
    items = []
    for key, meta in sorted(header.items(), key=lambda kv: kv[1]["data_offsets"][0]):
        s, e = meta["data_offsets"]
        raw = np.frombuffer(_file_bytes(shard, base + s, e - s), dtype=np.uint8)
        if key == name(3, 1, "up_proj", "weight_scale"):
            raw = raw.view(np.int8)
        elif meta["dtype"] == "F32":
            raw = raw.view(np.float32)
        items.append((key, raw.reshape(meta["shape"])))
    write_safetensors(shard, items)
    with pytest.raises(ContractError, match="U8"):
        build_native_expert_source_plan(ModelContract.from_model_dir(root), _config(E=4),
                                        first_layer=3, last_layer=3)
    # config geometry differs from the stored shapes
    root = fresh("shape")
    with pytest.raises(ContractError, match="shape mismatch"):
        build_native_expert_source_plan(ModelContract.from_model_dir(root), _config(E=4, I=64),
                                        first_layer=3, last_layer=3)
    # an expert that is not in the index
    root = fresh("missing")
    with pytest.raises(ContractError, match="absent from model index"):
        build_native_expert_source_plan(ModelContract.from_model_dir(root), _config(E=5),
                                        first_layer=3, last_layer=3)
    # one expert split over two shards
    root = fresh("split")
    index_path = os.path.join(root, "model.safetensors.index.json")
    index = json.load(open(index_path))
    moved = name(3, 2, "gate_proj", "weight_scale")
    arr = np.zeros((I, D // 32), np.uint8)
    write_safetensors(os.path.join(root, "extra.safetensors"), [(moved, arr)])
    index["weight_map"][moved] = "extra.safetensors"
    json.dump(index, open(index_path, "w"))
    with pytest.raises(ContractError, match="spans multiple shards"):
        build_native_expert_source_plan(ModelContract.from_model_dir(root), _config(E=4),
                                        first_layer=3, last_layer=3)
    # a header whose byte range disagrees with dtype x shape
    root = fresh("range")
    shard = os.path.join(root, "model-layer3-00.safetensors")
    base, header = local_safetensors_header(shard)
    header[name(3, 0, "down_proj", "weight_scale")]["shape"] = [D, 2]
    raw = json.dumps(header).encode()
    raw += b" " * (base - 8 - len(raw))
    with open(shard, "r+b") as f:
        f.seek(8)
        f.write(raw)
    with pytest.raises(ContractError, match="byte range"):
        ModelContract.from_model_dir(root).tensor(name(3, 0, "down_proj", "weight_scale"))
    # metadata files
    with pytest.raises(ContractError, match="incomplete"):
        ModelContract.from_model_dir(tmp_path / "nothing")
    with pytest.raises(ContractError, match="weight_map"):
        ModelContract(tmp_path, {}, {"weight_map": {}})


def test_partition_and_name_parts():
    assert routed_expert_parts(name(7, 11, "up_proj", "weight_scale")) == (
        7, 11, "up_proj", "weight_scale")
    with pytest.raises(ContractError):
        routed_expert_parts("model.language_model.layers.7.mlp.gate.weight")
    P = ModelContract.partition
    assert P(name(3, 0, "down_proj", "weight_packed")) == "routed"
    assert P(name(45, 0, "down_proj", "weight_packed")) == "mtp"
    assert P(name(2, 0, "down_proj", "weight_packed")) == "unknown"
    assert P("model.language_model.layers.45.self_attn.q.weight") == "mtp"
    assert P("model.language_model.embed_tokens.weight") == "resident"
    assert P("lm_head.weight") == "resident"
    assert P("model.visual.blocks.0.w") == "vision"


# ---------------------------------------------------------------- native reader


def _lib():
    from livglm_amd import native

    if not os.path.exists(native.library_path()):
        pytest.skip("libglm53moe.so is not built")
    return native


def _read(native, path, offsets, lengths, threads=4, flags=0):
    bufs = [np.full(max(int(n), 1), 0xEE, dtype=np.uint8) for n in lengths]
    offs = np.array(offsets, dtype=np.int64)
    lens = np.array(lengths, dtype=np.int64)
    ptrs = (ctypes.c_void_p * len(bufs))(*[b.ctypes.data for b in bufs])
    native.call("glm_file_read_ranges", path.encode(), len(bufs), offs.ctypes.data,
                lens.ctypes.data, ptrs, threads, flags)
    return [b[:n].tobytes() for b, n in zip(bufs, lengths)]


def test_native_range_reader_reads_exact_bytes(tmp_path):
    native = _lib()
    rng = np.random.default_rng(7)
    data = rng.integers(0, 256, 20 << 20, dtype=np.uint8)  # 20 MiB: many 2 MiB pieces
    path = str(tmp_path / "blob.bin")
    data.tofile(path)
    offsets = [0, 3, (8 << 20) - 5, 12345, len(data) - 17, 100]
    lengths = [1, (9 << 20) + 7, 4096, 0, 17, 1 << 20]
    for threads, flags in ((1, 0), (7, native.GLM_READ_DROP_CACHE)):
        got = _read(native, path, offsets, lengths, threads, flags)
        for g, o, n in zip(got, offsets, lengths):
            assert g == data[o:o + n].tobytes()


def test_native_range_reader_errors(tmp_path):
    native = _lib()
    path = str(tmp_path / "small.bin")
    np.arange(100, dtype=np.uint8).tofile(path)
    with pytest.raises(native.NativeError, match="beyond the end"):
        _read(native, path, [90], [11])
    with pytest.raises(native.NativeError, match="cannot open"):
        _read(native, str(tmp_path / "absent.bin"), [0], [1])
    with pytest.raises(native.NativeError, match="threads"):
        _read(native, path, [0], [1], threads=0)
    with pytest.raises(native.NativeError, match="flags"):
        _read(native, path, [0], [1], flags=8)
    offs = np.array([-1], dtype=np.int64)
    lens = np.array([1], dtype=np.int64)
    ptrs = (ctypes.c_void_p * 1)(0)
    with pytest.raises(native.NativeError, match="offset"):
        native.call("glm_file_read_ranges", path.encode(), 1, offs.ctypes.data, lens.ctypes.data,
                    ptrs, 1, 0)


def test_loader_chunks_cover_each_record_once(tmp_path):
    _lib()
    from glm53flash.bank_loader import ExpertBankLoader

    make_checkpoint(str(tmp_path), layers=(3,), E=E, d=D, I=I, shards_per_layer=2)
    plan = build_native_expert_source_plan(ModelContract.from_model_dir(tmp_path), _config(),
                                           first_layer=3, last_layer=3)
    loader = ExpertBankLoader(plan, chunk_bytes=3 * RECORD)
    chunks = loader._chunks(3)
    units = [(src.expert, r.absolute_offset, r.shard_name) for c in chunks for src, r in c]
    assert sorted(e for e, _, _ in units) == list(range(E))
    for c in chunks:
        assert len({r.shard_name for _, r in c}) == 1
        assert sum(-(-r.byte_length // 256) * 256 for _, r in c) <= loader.chunk_bytes
        offs = [r.absolute_offset for _, r in c]
        assert offs == sorted(offs)
    # a chunk never holds less than the largest record
    assert ExpertBankLoader(plan, chunk_bytes=256).chunk_bytes >= RECORD
