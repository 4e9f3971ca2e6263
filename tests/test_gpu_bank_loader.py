"""Checkpoint shards -> HBM bank on the GPU: every slot byte-exact, and the
loaded bank computes what a bank filled from the same arrays computes.

The expected bytes are the arrays the test wrote into the shards, the packed
codes in the bank layout (``native.mxfp4_tile_host``: tile-major where the
geometry allows); the routed-expert output is checked against the oracle's
routed experts (``expert_ssd.py:185-188``) within the bf16 gate.
"""

from __future__ import annotations

import numpy as np
import pytest

from checkpoint_util import COMPONENTS, PARTS, make_checkpoint

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gu():
    import gpu_util
    return gpu_util


def _plan(root, E, d, I, layers):
    from glm53flash.bank_plan import plan_expert_banks
    from glm53flash.checkpoint import ShardIndex
    return plan_expert_banks(ShardIndex.open(root), hidden_size=d, intermediate_size=I,
                             experts=E, layers=layers)


@pytest.mark.parametrize("misalign", [False, True])
@pytest.mark.parametrize("d,I", [(64, 32), (256, 128)])  # row-major codes; tile-major codes
def test_loader_fills_every_slot_exactly(gu, tmp_path, misalign, d, I):
    from glm53flash.bank_loader import ExpertBankLoader
    from glm53flash.expert_ssd import HBMExpertBank
    E, layers = 12, (3, 4)
    record = 3 * I * d * 17 // 32
    print(f"bank loader: misalign={misalign} E={E} d={d} I={I}", flush=True)
    arrays = make_checkpoint(str(tmp_path), layers=layers, E=E, d=d, I=I, misalign=misalign,
                             shards_per_layer=2, seed=5304 + misalign)
    plan = _plan(str(tmp_path), E, d, I, layers)
    # three records per chunk: several chunks, both buffers reused
    loader = ExpertBankLoader(plan, threads=4, chunk_bytes=3 * record + 512)
    banks = [HBMExpertBank(layer=layer, num_experts=E, hidden_size=d, intermediate_size=I,
                           swiglu_limit=10.0, device="cuda") for layer in layers]
    if misalign:
        # both layers through one pipeline
        stats = loader.load_many(banks)
        assert stats.bytes == len(layers) * E * record and stats.chunks >= 8
    else:
        for bank in banks:
            stats = loader.load(bank)
            assert stats.bytes == E * record and stats.experts == E and stats.chunks >= 4
    for layer, bank in zip(layers, banks):
        for comp in COMPONENTS:
            for part in PARTS:
                got = gu.host(bank.tensors[f"{comp}.{part}"])
                want = np.stack([arrays[(layer, e)][(comp, part)] for e in range(E)])
                if part == "weight_packed":
                    want = gu.native.mxfp4_tile_host(want)
                assert got.shape == want.shape and np.array_equal(got, want), (layer, comp, part)
    loader.close()


def test_loaded_bank_matches_a_bank_from_arrays(gu, tmp_path):
    import torch

    import oracle.moe_oracle as O
    from glm53flash.bank_loader import load_layer_bank
    from glm53flash.expert_ssd import HBMExpertBank
    from livglm_amd.workloads import BANK_KEYS
    E, d, I, T, k, layer = 16, 256, 128, 3, 4, 7
    print(f"bank loader forward: E={E} d={d} I={I} T={T} k={k}", flush=True)
    arrays = make_checkpoint(str(tmp_path), layers=(layer,), E=E, d=d, I=I, seed=5310)
    plan = _plan(str(tmp_path), E, d, I, (layer,))
    loaded = load_layer_bank(plan, layer, swiglu_limit=10.0, device="cuda")
    stacked = {f"{c}.{p}": np.stack([arrays[(layer, e)][(c, p)] for e in range(E)])
               for c in COMPONENTS for p in PARTS}
    direct = HBMExpertBank(layer=layer, num_experts=E, hidden_size=d, intermediate_size=I,
                           swiglu_limit=10.0, device="cuda")
    direct.load_bank({key: gu.to_dev(v) for key, v in stacked.items()})
    rng = np.random.default_rng(5311)
    x32 = rng.standard_normal((T, d)).astype(np.float32)
    x_bits = O.f32_to_bf16_bits(x32)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    x = gu.to_dev(x_bits)
    idx_dev = torch.from_numpy(idx.astype(np.int32)).cuda()
    y_loaded = gu.bf16_bits(loaded(x, idx_dev))
    y_direct = gu.bf16_bits(direct(x, idx_dev))
    assert np.array_equal(y_loaded, y_direct)
    want = O.routed_experts(O.bf16_bits_to_f32(x_bits), idx,
                            O.Bank(*(stacked[key] for key in BANK_KEYS)), 10.0)
    assert O.rel_l2(O.bf16_bits_to_f32(y_loaded), want) < 2e-3


def test_bank_scatter_segments_of_any_alignment(gu):
    """glm_bank_scatter on segments with odd offsets and lengths (byte path),
    aligned ones (16-byte path with a tail) and an empty one; the bytes around
    every destination stay untouched."""
    import torch
    rng = np.random.default_rng(5312)
    staging_np = rng.integers(0, 256, 300_000, dtype=np.uint8)
    staging = gu.to_dev(staging_np)
    dst_np = np.full(400_000, 0xA5, dtype=np.uint8)
    dst = gu.to_dev(dst_np)
    # (src offset, dst offset, bytes): disjoint destinations inside dst
    cases = [(0, 0, 16), (3, 40, 1), (17, 100, 70_001), (64, 80_000, 131_072 + 48),
             (1000, 250_000, 0), (299_990, 260_000, 10), (12_345, 270_001, 65_537)]
    for s, o, n in cases:
        assert s + n <= staging_np.size and o + n <= dst_np.size
    # tiled segments: whole MXFP4 matrices (rows x K codes) into the bank
    # layout, from an aligned and from an odd staging offset
    tiled = [(64_000, 340_000, 32, 256), (150_001, 360_000, 48, 128)]
    for s, o, rows, K in tiled:
        assert s + rows * K // 2 <= staging_np.size and o + rows * K // 2 <= dst_np.size
    base = dst.data_ptr()
    table = np.array([(s, base + o, n, 0) for s, o, n in cases]
                     + [(s, base + o, rows * K // 2, K) for s, o, rows, K in tiled], dtype=np.int64)
    dtab = torch.empty(table.size, dtype=torch.int64, device="cuda")
    print("bank scatter: 7 segments, odd offsets; 2 tiled", flush=True)
    gu.native.call("glm_bank_scatter", gu.stream(), staging.data_ptr(), staging_np.size,
                   table.ctypes.data, table.shape[0], dtab.data_ptr())
    want = dst_np.copy()
    for s, o, n in cases:
        want[o:o + n] = staging_np[s:s + n]
    for s, o, rows, K in tiled:
        n = rows * K // 2
        want[o:o + n] = gu.native.mxfp4_tile_host(staging_np[s:s + n].reshape(rows, K // 2)).reshape(-1)
    assert np.array_equal(gu.host(dst), want)
    # a segment reaching past the staging buffer is rejected before any launch
    bad = np.array([(299_999, base, 2, 0)], dtype=np.int64)
    with pytest.raises(gu.native.NativeError, match="outside"):
        gu.native.call("glm_bank_scatter", gu.stream(), staging.data_ptr(), staging_np.size,
                       bad.ctypes.data, 1, dtab.data_ptr())


@pytest.mark.parametrize("scales", ["two_value", "uniform"])
def test_scalex_layer_loads_the_same_bank(gu, tmp_path, scales):
    """A ScaleX layer shard (coded scales, decoded on the GPU while loading)
    fills the bank with exactly the bytes of the native checkpoint (the codes
    in the bank layout).  "uniform"
    scales make the codec keep raw records; "two_value" ones code one bit per
    scale with exceptions."""
    from glm53flash.bank_loader import ExpertBankLoader
    from glm53flash.expert_ssd import HBMExpertBank
    E, d, I, layers = 10, 512, 256, (5, 6)
    print(f"scalex loader: scales={scales} E={E} d={d} I={I}", flush=True)
    arrays = make_checkpoint(str(tmp_path), layers=layers, E=E, d=d, I=I, extras=False,
                             shuffle=False, scales=scales, scalex=True, seed=5320)
    plan = _plan(str(tmp_path), E, d, I, layers)
    assert plan.scalex
    codecs = {x.coded.codec for x in plan.loads}
    assert codecs == ({"one_bit"} if scales == "two_value" else {"raw"})
    record = plan.loads[0].coded.nbytes
    loader = ExpertBankLoader(plan, threads=4, chunk_bytes=3 * record + 4096)
    banks = [HBMExpertBank(layer=layer, num_experts=E, hidden_size=d, intermediate_size=I,
                           swiglu_limit=10.0, device="cuda") for layer in layers]
    stats = loader.load_many(banks)
    assert stats.bytes == len(layers) * E * 3 * I * d * 17 // 32
    assert stats.read_bytes < stats.bytes or scales == "uniform"
    for layer, bank in zip(layers, banks):
        for comp in COMPONENTS:
            for part in PARTS:
                got = gu.host(bank.tensors[f"{comp}.{part}"])
                want = np.stack([arrays[(layer, e)][(comp, part)] for e in range(E)])
                if part == "weight_packed":
                    want = gu.native.mxfp4_tile_host(want)
                assert np.array_equal(got, want), (layer, comp, part)
    loader.close()


def test_loader_at_the_real_record_size(gu, tmp_path):
    """d = 4096, I = 2048: one expert is the real checkpoint's 13,369,344-byte
    record (expert_source.py:370), read as one range; two records per staging chunk."""
    from glm53flash.bank_loader import ExpertBankLoader
    from glm53flash.expert_ssd import HBMExpertBank
    E, d, I, layer = 4, 4096, 2048, 3
    print(f"bank loader real record: E={E} d={d} I={I}", flush=True)
    arrays = make_checkpoint(str(tmp_path), layers=(layer,), E=E, d=d, I=I, extras=False,
                             seed=5330)
    plan = _plan(str(tmp_path), E, d, I, (layer,))
    assert all(len(x.reads) == 1 and x.read_bytes == x.bank_bytes == 13_369_344
               for x in plan.loads)
    loader = ExpertBankLoader(plan, chunk_bytes=30 << 20)
    bank = HBMExpertBank(layer=layer, num_experts=E, hidden_size=d, intermediate_size=I,
                         swiglu_limit=10.0, device="cuda")
    stats = loader.load(bank)
    assert stats.chunks == 2 and stats.bytes == E * 13_369_344
    for comp in COMPONENTS:
        for part in PARTS:
            got = gu.host(bank.tensors[f"{comp}.{part}"])
            want = np.stack([arrays[(layer, e)][(comp, part)] for e in range(E)])
            if part == "weight_packed":
                want = gu.native.mxfp4_tile_host(want)
            assert np.array_equal(got, want), (comp, part)
    loader.close()


@pytest.mark.parametrize("count,rows,K", [(3, 32, 256), (2, 48, 128), (1, 2048, 4096),
                                         (2, 20, 128), (3, 16, 96), (0, 16, 128)])
def test_mxfp4_tile_writes_the_bank_layout(gu, count, rows, K):
    """glm_mxfp4_tile against the host statement of the layout: tile-major
    where rows % 16 == 0 and K % 128 == 0, a copy otherwise."""
    import torch
    rng = np.random.default_rng(rows * 7 + K)
    src_np = rng.integers(0, 256, (count, rows, K // 2), dtype=np.uint8)
    print(f"mxfp4_tile: count={count} rows={rows} K={K}", flush=True)
    src = gu.to_dev(src_np) if count else torch.empty((0, rows, K // 2), dtype=torch.uint8,
                                                          device="cuda")
    got = gu.native.mxfp4_tile(src)
    torch.cuda.synchronize()
    assert np.array_equal(gu.host(got), gu.native.mxfp4_tile_host(src_np))
    assert gu.native.mxfp4_is_tiled(rows, K) == (rows % 16 == 0 and K % 128 == 0)
