"""Checkpoint index, bank load plan and the native range reader (CPU).

The shards are written by the test's own writer and by the ``safetensors``
library, whose reader is the independent check of the header parsing and
byte ranges; every planned segment is checked against the bytes the writer
put in the file.
"""

from __future__ import annotations

import ctypes
import json
import os

import numpy as np
import pytest

from checkpoint_util import COMPONENTS, PARTS, make_checkpoint, name, write_safetensors

from glm53flash.bank_plan import (REAL_RECORD_BYTES, _merge_adjacent, plan_expert_banks,
                                  slot_shape)
from glm53flash.checkpoint import ShardIndex, TensorRange, read_safetensors_header
from glm53flash.contract import ContractError

D, I, E = 64, 32, 12
RECORD = 3 * I * D * 17 // 32


def _plan(root, layers=(3,), E=E, d=D, I=I):
    return plan_expert_banks(ShardIndex.open(root), hidden_size=d, intermediate_size=I,
                             experts=E, layers=layers)


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
    base, header = read_safetensors_header(path)
    for key, arr in tensors.items():
        start, end = header[key]["data_offsets"]
        assert _file_bytes(path, base + start, end - start) == arr.tobytes()
    loaded = st.load_file(path)
    assert set(loaded) == set(tensors)


def test_plan_locates_every_expert_record(tmp_path):
    arrays = make_checkpoint(str(tmp_path), layers=(3, 4), E=E, d=D, I=I)
    plan = _plan(tmp_path, layers=(3, 4))
    assert len(plan.loads) == 2 * E and not plan.scalex
    # each expert's six tensors are adjacent in its shard: one read per record
    assert plan.read_bytes == plan.bank_bytes == 2 * E * RECORD
    for layer in (3, 4):
        for e in range(E):
            x = plan.expert(layer, e)
            assert (x.layer, x.expert) == (layer, e)
            (rd,) = x.reads
            assert rd.nbytes == RECORD
            assert sorted(seg.key for seg in rd.segments) == sorted(
                f"{c}.{p}" for c in COMPONENTS for p in PARTS)
            path = plan.shard_path(rd.shard)
            for seg in rd.segments:
                comp, part = seg.key.split(".")
                want = arrays[(layer, e)][(comp, part)]
                assert want.shape == slot_shape(seg.key, D, I)
                assert seg.nbytes == want.nbytes
                assert _file_bytes(path, rd.offset + seg.at, seg.nbytes) == want.tobytes()
    with pytest.raises(ContractError):
        plan.expert(5, 0)
    with pytest.raises(ContractError):
        plan.expert(3, E)


def test_adjacent_tensors_share_a_read_gaps_and_shards_split_them():
    def t(shard, off, n, key="gate_proj.weight_packed"):
        return TensorRange(f"x.{off}.{key}", shard, off, n, "U8", (n,))

    reads = _merge_adjacent([t("b", 0, 4), t("a", 10, 5), t("a", 0, 10), t("a", 16, 2)])
    assert [(r.shard, r.offset, r.nbytes, [(s.at, s.nbytes) for s in r.segments])
            for r in reads] == [("a", 0, 15, [(0, 10), (10, 5)]), ("a", 16, 2, [(0, 2)]),
                                ("b", 0, 4, [(0, 4)])]


def test_plan_rejects_broken_checkpoints(tmp_path):
    def fresh(sub):
        root = str(tmp_path / sub)
        make_checkpoint(root, layers=(3,), E=4, d=D, I=I, shuffle=False)
        return root

    # wrong storage dtype
    root = fresh("dtype")
    shard = os.path.join(root, "model-layer3-00.safetensors")
    base, header = read_safetensors_header(shard)
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
    with pytest.raises(ContractError, match="stored as I8"):
        _plan(root, E=4)
    # config geometry differs from the stored shapes
    root = fresh("shape")
    with pytest.raises(ContractError, match="geometry"):
        _plan(root, E=4, I=64)
    # an expert that is not in the index
    root = fresh("missing")
    with pytest.raises(ContractError, match="not in the checkpoint index"):
        _plan(root, E=5)
    # one expert split over two shards
    root = fresh("split")
    index_path = os.path.join(root, "model.safetensors.index.json")
    index = json.load(open(index_path))
    moved = name(3, 2, "gate_proj", "weight_scale")
    arr = np.zeros((I, D // 32), np.uint8)
    write_safetensors(os.path.join(root, "extra.safetensors"), [(moved, arr)])
    index["weight_map"][moved] = "extra.safetensors"
    json.dump(index, open(index_path, "w"))
    with pytest.raises(ContractError, match="split over shards"):
        _plan(root, E=4)
    # a header whose byte range disagrees with dtype x shape
    root = fresh("range")
    shard = os.path.join(root, "model-layer3-00.safetensors")
    base, header = read_safetensors_header(shard)
    header[name(3, 0, "down_proj", "weight_scale")]["shape"] = [D, 2]
    raw = json.dumps(header).encode()
    raw += b" " * (base - 8 - len(raw))
    with open(shard, "r+b") as f:
        f.seek(8)
        f.write(raw)
    with pytest.raises(ContractError, match="data_offsets"):
        ShardIndex.open(root).locate(name(3, 0, "down_proj", "weight_scale"))
    # a shard cut short: its last tensor runs past the end of the file
    root = fresh("short")
    shard = os.path.join(root, "model-layer3-00.safetensors")
    os.truncate(shard, os.path.getsize(shard) - 1)
    last = max(read_safetensors_header(shard)[1].items(),
               key=lambda kv: kv[1]["data_offsets"][1])[0]
    with pytest.raises(ContractError, match="run past"):
        ShardIndex.open(root).locate(last)
    # metadata files
    with pytest.raises(ContractError, match="index.json"):
        ShardIndex.open(tmp_path / "nothing")
    with pytest.raises(ContractError, match="maps no tensors"):
        ShardIndex(tmp_path, {})


def test_slot_shapes_and_the_real_record_size():
    # gate/up: I rows of d inputs, down the transpose; codes two per byte, scales one per 32
    assert slot_shape("gate_proj.weight_packed", 4096, 2048) == (2048, 2048)
    assert slot_shape("down_proj.weight_scale", 4096, 2048) == (4096, 64)
    real = sum(r * c for r, c in (slot_shape(f"{comp}.{part}", 4096, 2048)
                                  for comp in COMPONENTS for part in PARTS))
    assert real == REAL_RECORD_BYTES == 3 * 2048 * 4096 * 17 // 32
    with pytest.raises(ContractError, match="multiple of 32"):
        slot_shape("up_proj.weight_scale", 100, 64)


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
    plan = _plan(tmp_path)
    loader = ExpertBankLoader(plan, chunk_bytes=3 * RECORD)
    chunks = loader._chunks(3)
    units = [(x.expert, r.offset, r.shard) for c in chunks for x, r in c]
    assert sorted(e for e, _, _ in units) == list(range(E))
    for c in chunks:
        assert len({r.shard for _, r in c}) == 1
        assert sum(-(-r.nbytes // 256) * 256 for _, r in c) <= loader.chunk_bytes
        offs = [r.offset for _, r in c]
        assert offs == sorted(offs)
    # a chunk never holds less than the largest record
    assert ExpertBankLoader(plan, chunk_bytes=256).chunk_bytes >= RECORD


def test_bank_layout_host_statement():
    """native.mxfp4_tile_host, the host statement of the bank layout the GPU
    writes (glm_mxfp4_tile, glm_bank_scatter): a permutation of each matrix's
    bytes; in every 1 KB block (tile t, chunk c) the 16 bytes at 16 (r + 16 q)
    are row 16 t + r, K codes 128 c + 32 q .. +31 -- the 32 codes of one E8M0
    group, i.e. what lane (r, q) of a 16-row MFMA tile consumes; geometries
    that do not tile stay as they are."""
    from livglm_amd import native
    rng = np.random.default_rng(5320)
    for lead, rows, K in (((2,), 32, 256), ((), 48, 128), ((2, 3), 16, 384)):
        a = rng.integers(0, 256, (*lead, rows, K // 2), dtype=np.uint8)
        t = native.mxfp4_tile_host(a)
        assert t.shape == a.shape
        flat_a = a.reshape(-1, rows, K // 2)
        flat_t = t.reshape(-1, rows * K // 2)
        for m in range(flat_a.shape[0]):
            assert np.array_equal(np.sort(flat_t[m]), np.sort(flat_a[m].reshape(-1)))
            for blk in range((rows // 16) * (K // 128)):
                tt, c = divmod(blk, K // 128)
                for lane in range(64):
                    r, q = lane % 16, lane // 16
                    got = flat_t[m, blk * 1024 + 16 * lane: blk * 1024 + 16 * lane + 16]
                    want = flat_a[m, 16 * tt + r, 64 * c + 16 * q: 64 * c + 16 * q + 16]
                    assert np.array_equal(got, want), (m, tt, c, r, q)
    for rows, K in ((20, 128), (16, 96), (32, 64)):
        a = rng.integers(0, 256, (rows, K // 2), dtype=np.uint8)
        assert np.array_equal(native.mxfp4_tile_host(a), a)
