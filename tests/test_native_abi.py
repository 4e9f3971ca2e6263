"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares with the expected version, and rejects bad arguments on the
host before touching a GPU (no compute calls here)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from livglm_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "glm53_moe.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(glm_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(native.LIB_PATH):
        pytest.fail("libglm53moe.so is not built; run `python -m livglm_amd.build`")
    return native.load()


def test_header_and_binding_agree():
    assert set(declared_functions()) == set(native.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", native.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\b(glm_[a-z0-9_]+)\b", out))
    missing = set(declared_functions()) - exported
    assert not missing, missing


def test_abi_version(lib):
    assert lib.glm_abi_version() == native.ABI_VERSION == 2


def test_workspace_size_is_host_only_and_monotone(lib):
    small = lib.glm_moe_workspace_bytes(2, 2048, 128, 8, 768, 768)
    big = lib.glm_moe_workspace_bytes(4096, 2048, 128, 8, 768, 768)
    assert 0 < small < big
    assert small % 256 == 0
    assert lib.glm_moe_workspace_bytes(-1, 2048, 128, 8, 768, 768) == 0


def _expect(code, name, *args):
    rc = getattr(native.load(), name)(*args)
    assert rc == code, (name, rc, native.load().glm_last_error())
    return native.load().glm_last_error().decode()


def test_null_pointers_are_rejected_on_host(lib):
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_router_topk", None, None, 1, 32, None,
                  None, 4, 2, 1, 1, 1, 2.5, None, None, None)
    assert "null" in msg
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_moe_dispatch", None, None, 1, 2, 4, None, None,
            None, None, None, None, None, None, None)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_moe_combine", None, None, None, None, None, 1,
            2, 32, None)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_limited_swiglu", None, None, None, 4, 10.0,
            None)


def test_unsupported_shapes_are_rejected_on_host(lib):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_mx_quantize", None, fake, 4, 48,
            native.GLM_FMT_MXFP8, 0, fake, fake)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_mx_quantize", None, fake, 4, 64, 7, 0, fake,
            fake)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_mx_quantize", None, fake, 4, 64,
            native.GLM_FMT_MXFP8, 9, fake, fake)
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_moe_dispatch", None, fake, 1, 2, 4096, fake,
            fake, fake, fake, fake, fake, fake, fake, fake)
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_router_topk", None, fake, 1, 32, fake,
                  fake, 6, 2, 4, 1, 1, 2.5, fake, fake, fake)
    assert "n_group" in msg
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_linear", None, fake, 1, 40, fake, None,
            native.GLM_FMT_BF16, 16, fake)


def test_moe_forward_rejects_small_workspace(lib):
    fake = ctypes.c_void_p(0x1000)
    args = [None, fake, 2, 2048, fake, fake, 128, 8, 1, 1, 1, 2.5, 768] + [fake] * 6
    args += [768, native.GLM_FMT_BF16, fake, None, fake, None, fake, None, None, 10.0, fake,
             1024, fake, None, None]
    msg = _expect(native.GLM_ERR_WORKSPACE, "glm_moe_forward", *args)
    assert "workspace" in msg


def _forward_args(T, d=2048, E=128, k=8, I=768, *, workspace_bytes=None, shared_fmt=None,
                  shared_scales=False, ptr=None):
    fake = ptr or ctypes.c_void_p(0x1000)  # never dereferenced: the call returns before launching
    lib = native.load()
    if workspace_bytes is None:
        workspace_bytes = lib.glm_moe_workspace_bytes(max(T, 0), d, E, k, I, 768)
    fmt = native.GLM_FMT_BF16 if shared_fmt is None else shared_fmt
    sc = fake if shared_scales else None
    args = [None, fake, T, d, fake, fake, E, k, 1, 1, 1, 2.5, I] + [fake] * 6
    args += [768, fmt, fake, sc, fake, sc, fake, sc, None, 10.0, fake, workspace_bytes, fake,
             None, None]
    return args


def test_empty_batch_is_a_no_op(lib):
    # T = 0 validates and returns without touching the device
    assert lib.glm_moe_forward(*_forward_args(0)) == native.GLM_OK
    fake = ctypes.c_void_p(0x1000)
    assert lib.glm_router_topk(None, fake, 0, 2048, fake, fake, 128, 8, 1, 1, 1, 2.5, fake, fake,
                               fake) == native.GLM_OK
    assert lib.glm_act_split_fp8(None, fake, 0, 2048, fake) == native.GLM_OK


def test_moe_forward_rejects_bad_arguments(lib):
    cases = [
        (native.GLM_ERR_INVALID_ARGUMENT, _forward_args(-1), "invalid sizes"),
        (native.GLM_ERR_UNSUPPORTED_SHAPE, _forward_args(2, d=1000), "multiples of 32"),
        (native.GLM_ERR_UNSUPPORTED_SHAPE, _forward_args(2, E=449, k=8), "exceeds 448"),
        (native.GLM_ERR_INVALID_ARGUMENT, _forward_args(2, E=4, k=8), None),
        (native.GLM_ERR_INVALID_ARGUMENT, _forward_args(2, shared_fmt=7), "shared format"),
        (native.GLM_ERR_INVALID_ARGUMENT, _forward_args(2, shared_fmt=native.GLM_FMT_MXFP8),
         "scales"),
        (native.GLM_ERR_INVALID_ARGUMENT, _forward_args(2, ptr=ctypes.c_void_p(0x1004)),
         "aligned"),
    ]
    for code, args, text in cases:
        msg = _expect(code, "glm_moe_forward", *args)
        if text:
            assert text in msg, msg


def test_prefill_entry_points_reject_bad_shapes(lib):
    fake = ctypes.c_void_p(0x1000)
    assert lib.glm_act_split_bytes(4, 33) == 0 and lib.glm_act_split_bytes(-1, 64) == 0
    assert lib.glm_act_split_bytes(4, 64) % 256 == 0
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_act_split_fp8", None, fake, 4, 48, fake)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_act_split_fp8", None, None, 4, 64, fake)
    msg = _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_expert_gate_up_grouped", None, fake, 8,
                  1024, 384, fake, fake, fake, fake, fake, fake, fake, 16, 10.0, fake)
    assert "I % 256" in msg
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_expert_down_grouped", None, fake, 64, 256,
            768, fake, fake, fake, fake, 16, fake)
    # the token-major gate/up takes at most 4 tokens and 8 experts per token
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_route_gate_up", None, fake, fake, 5, 128, 8, 1,
            1, 1, 2.5, fake, 2048, 768, fake, fake, fake, fake, 10.0, fake, fake, fake)


def test_act_format_entry_points(lib):
    import act_formats as A
    fake = ctypes.c_void_p(0x1000)
    # split sizes agree with the layout model; FP8X2 is the original split
    for rows, K in [(1, 128), (7, 2048), (300, 768)]:
        for fmt in (A.FP8X2, A.FP6X2, A.FP4, A.FP8FP6):
            assert lib.glm_act_split_bytes_fmt(rows, K, fmt) == A.split_bytes(rows, K, fmt)
        assert lib.glm_act_split_bytes_fmt(rows, K, 0) == lib.glm_act_split_bytes(rows, K)
    assert lib.glm_act_split_bytes_fmt(4, 96, native.GLM_ACT_FP6X2) == 0  # K % 128
    assert lib.glm_act_split_bytes_fmt(4, 96, native.GLM_ACT_FP8FP6) == 0
    assert lib.glm_act_split_bytes_fmt(4, 96, native.GLM_ACT_FP4) > 0
    assert lib.glm_act_split_bytes_fmt(4, 128, 4) == 0
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_act_split", None, fake, 4, 128, 7, fake)
    assert "act_format" in msg
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_act_split", None, fake, 4, 96,
            native.GLM_ACT_FP6X2, fake)
    assert lib.glm_act_split(None, fake, 0, 128, native.GLM_ACT_FP4, fake) == native.GLM_OK
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_expert_gate_up_grouped_fmt", None, -1,
                  fake, 8, 1024, 512, fake, fake, fake, fake, fake, fake, fake, 16, 10.0, fake)
    assert "act_format" in msg
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_expert_down_grouped_fmt", None,
            native.GLM_ACT_FP6X2, fake, 64, 256, 768, fake, fake, fake, fake, 16, fake)


def test_ffn_site_and_loader_entry_points_reject_bad_arguments(lib):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    assert lib.glm_hc_workspace_bytes(2, 4, 2048) == 32 * 2 * 25 * 4
    assert lib.glm_hc_workspace_bytes(2, 9, 2048) == 0
    msg = _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_hc_pre", None, fake, 2, 9, 2048, fake,
                  fake, fake, 20, 1e-6, 1e-6, None, 1e-6, 0, fake, 1 << 20, fake, fake, None, None)
    assert "hc_mult" in msg
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_hc_pre", None, fake, 2, 4, 2050, fake, fake,
            fake, 20, 1e-6, 1e-6, None, 1e-6, 0, fake, 1 << 20, fake, fake, None, None)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_hc_pre", None, fake, 2, 4, 2048, fake, fake,
            fake, 0, 1e-6, 1e-6, None, 1e-6, 0, fake, 1 << 20, fake, fake, None, None)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_hc_pre", None, fake, 2, 4, 2048, fake, fake,
            fake, 20, 1e-6, 1e-6, None, 1e-6, 4, fake, 1 << 20, fake, fake, None, None)
    _expect(native.GLM_ERR_WORKSPACE, "glm_hc_pre", None, fake, 2, 4, 2048, fake, fake, fake, 20,
            1e-6, 1e-6, None, 1e-6, 0, fake, 64, fake, fake, None, None)
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_hc_post", None, None, 2, 4, 2048, fake, fake,
            fake, 0, fake)
    _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_rms_norm", None, fake, 2, 30, None, 1e-6,
            fake, None)
    # a segment past the staging buffer, a tiled segment that is not a whole
    # tileable matrix, and a ScaleX record whose lengths disagree
    seg = (ctypes.c_int64 * 4)(100, 0x2000, 200, 0)
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_bank_scatter", None, fake, 256,
                  ctypes.cast(seg, ctypes.c_void_p), 1, fake)
    assert "outside" in msg
    for tile_k, nbytes in ((128, 64 * 8), (96, 48 * 16), (128, 64 * 16 + 16)):
        seg = (ctypes.c_int64 * 4)(0, 0x2000, nbytes, tile_k)
        msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_bank_scatter", None, fake, 4096,
                      ctypes.cast(seg, ctypes.c_void_p), 1, fake)
        assert "tileable" in msg
    # the tile transform: K not a multiple of 32, overlapping buffers
    _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_mxfp4_tile", None, 0x1000, 0x2000, 1, 16, 48)
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_mxfp4_tile", None, 0x1000, 0x1200, 1, 16,
                  128)
    assert "overlap" in msg
    rec = (ctypes.c_int64 * 13)(0, 24 + 8 + 5, 64, 1, 0, 9, 1, 0x2000, 64, 0x3000, 0, 0x4000, 0)
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_scalex_decode", None, fake, 4096,
                  ctypes.cast(rec, ctypes.c_void_p), 1, fake)
    assert "length" in msg
    rec[5] = 8
    rec[8] = 63  # destinations cover 63 of 64 bytes
    msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_scalex_decode", None, fake, 4096,
                  ctypes.cast(rec, ctypes.c_void_p), 1, fake)
    assert "cover" in msg


def _grouped_items(grid, nft, num_tiles, max_tiles, xcds=8):
    """The block-scaled grouped kernels' workgroup -> (tile, feature tile)
    mapping (grouped_f8f6f4_kernel), restated: the device-side count clamped
    to max_tiles, XCD x taking the x-th contiguous share of the items."""
    ntiles = max(0, min(num_tiles, max_tiles))
    items = ntiles * nft
    per = (items + xcds - 1) // xcds
    out = []
    for lin in range(grid):
        k_on, item = lin // xcds, (lin % xcds) * per + lin // xcds
        if k_on >= per or item >= items:
            continue
        out.append((item // nft, item % nft))
    return out


@pytest.mark.parametrize("max_tiles,nft", [(1, 6), (7, 3), (256, 6), (300, 4)])
def test_grouped_item_mapping_stays_in_the_tile_list(max_tiles, nft):
    # the launcher sizes the grid from max_tiles; whatever count the device
    # holds, every item runs once and no tile past the list is read
    grid = (max_tiles * nft + 7) // 8 * 8
    for num_tiles in (0, 1, max_tiles // 2, max_tiles, max_tiles + 1, 10 * max_tiles + 3, -5):
        got = _grouped_items(grid, nft, num_tiles, max_tiles)
        n = max(0, min(num_tiles, max_tiles))
        assert sorted(got) == [(t, f) for t in range(n) for f in range(nft)]
        assert all(t < max_tiles for t, _ in got)


def test_scalex_forward_rejects_short_stride_on_host(lib):
    # a stride shorter than a row's directory + record header would make each
    # expert's header reads land in the next row: refused before any launch
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    rows = ctypes.c_void_p(0x10000)  # 256-byte aligned
    fixed = 24 + ((2 * ((3 * 768 * 64 + 511) // 512 + 1)) + 15) // 16 * 16  # 616 at d 2048, I 768
    for stride, ok in ((256, False), (512, False), (768, True)):
        assert (stride >= fixed) == ok
        if ok:
            continue
        msg = _expect(native.GLM_ERR_INVALID_ARGUMENT, "glm_moe_forward_scalex", None, fake, 2,
                      2048, fake, fake, 128, 8, 1, 1, 1, 2.5, 768, fake, fake, fake, rows, stride,
                      0, native.GLM_FMT_BF16, None, None, None, None, None, None, None, 10.0,
                      fake, 1 << 30, fake, None, None)
        assert "directory" in msg


def test_split_beyond_32_bit_offsets_is_rejected_on_host(lib):
    # the grouped GEMMs address an activation split through 32-bit offsets: a
    # split above 4 GiB is refused instead of read as zeros past the limit
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    assert lib.glm_act_split_bytes(600000, 4096) > (1 << 32)
    msg = _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_expert_gate_up_grouped", None, fake,
                  600000, 4096, 2048, fake, fake, fake, fake, fake, fake, fake, 16, 10.0, fake)
    assert "4 GiB" in msg
    msg = _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_expert_down_grouped", None, fake,
                  1100000, 2048, 4096, fake, fake, fake, fake, 16, fake)
    assert "4 GiB" in msg
    # the layer refuses more than 2^30 (token, expert) pairs before sizing anything
    msg = _expect(native.GLM_ERR_UNSUPPORTED_SHAPE, "glm_moe_forward",
                  *_forward_args(1 << 27, workspace_bytes=1 << 40))
    assert "2^30" in msg
