"""glm_moe_forward_noalloc: the MoE layer with its workspace in the library's
static device array.  Through the C ABI, two calls in a row (the second with
a smaller input, so it runs on what the first left in the array) must equal
glm_moe_forward with a fresh caller workspace bit for bit; sizes beyond the
array are rejected on the host before any device work."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from livglm_amd import native
from livglm_amd.workloads import BANK_KEYS, SHAPES, MoEShape, make_layer


def _args(dl, shape, T, out, w, idx, ws=None, ws_bytes=0):
    import gpu_util as gu
    args = [gu.stream(), gu.p(dl["x"]), T, shape.d, gu.p(dl["router_weight"]),
            gu.p(dl["router_bias"]), shape.E, shape.k, shape.n_group, shape.topk_group,
            int(shape.norm_topk_prob), shape.routed_scaling_factor, shape.I]
    args += [gu.p(dl[key]) for key in BANK_KEYS]
    args += [shape.I_shared, native.GLM_FMT_BF16, gu.p(dl["shared.gate"]), None,
             gu.p(dl["shared.up"]), None, gu.p(dl["shared.down"]), None, None,
             shape.swiglu_limit]
    if ws is not None:
        args += [gu.p(ws), ws_bytes]
    return args + [gu.p(out), gu.p(w), gu.p(idx)]


def _both(shape, seed):
    """(noalloc result, glm_moe_forward result) for one layer, host arrays."""
    import torch

    import gpu_util as gu
    layer = make_layer(shape, seed)
    dl = gu.upload_layer(layer)
    T, d, k = shape.T, shape.d, shape.k
    res = []
    for noalloc in (True, False):
        out = torch.full((T, d), float("nan"), dtype=torch.float32, device="cuda")
        w = torch.zeros((T, k), dtype=torch.float32, device="cuda")
        idx = torch.zeros((T, k), dtype=torch.int32, device="cuda")
        if noalloc:
            gu.call("glm_moe_forward_noalloc", *_args(dl, shape, T, out, w, idx))
        else:
            ws_bytes = native.load().glm_moe_workspace_bytes(T, d, shape.E, k, shape.I,
                                                             shape.I_shared)
            ws = gu.workspace(ws_bytes)
            gu.call("glm_moe_forward", *_args(dl, shape, T, out, w, idx, ws, ws_bytes))
        res.append((gu.host(out), gu.host(w), gu.host(idx)))
    return res


# pairs of calls in a row, the second smaller: the decode path (64 tokens)
# then the few-token path (2 tokens); the grouped GEMM path (300 tokens) then
# 96 tokens on the same kernels
SEQUENCES = [
    [SHAPES["batch_t64"], SHAPES["verify_t2"]],
    [MoEShape("g300", 300, 1024, 16, 4, 256, 256), MoEShape("g96", 96, 1024, 16, 4, 256, 256)],
]


@pytest.mark.gpu
@pytest.mark.parametrize("seq", range(len(SEQUENCES)))
def test_noalloc_equals_moe_forward_on_consecutive_calls(seq):
    native.load()
    for i, shape in enumerate(SEQUENCES[seq]):
        (o_n, w_n, i_n), (o_f, w_f, i_f) = _both(shape, 8800 + 10 * seq + i)
        assert np.isfinite(o_n).all(), (shape.name, "non-finite output")
        np.testing.assert_array_equal(i_n, i_f, err_msg=shape.name)
        np.testing.assert_array_equal(w_n.view(np.uint32), w_f.view(np.uint32),
                                      err_msg=shape.name)
        np.testing.assert_array_equal(o_n.view(np.uint32), o_f.view(np.uint32),
                                      err_msg=shape.name)


def test_noalloc_rejects_sizes_beyond_the_array_on_host():
    lib = native.load()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: the call returns before launching
    s = SHAPES["prefill_t4096"]
    need = lib.glm_moe_workspace_bytes(s.T, s.d, s.E, s.k, s.I, s.I_shared)
    assert need > native.GLM_NOALLOC_SCRATCH_BYTES
    args = [None, fake, s.T, s.d, fake, fake, s.E, s.k, 1, 1, 1, 2.5, s.I] + [fake] * 6
    args += [s.I_shared, native.GLM_FMT_BF16, fake, None, fake, None, fake, None, None, 10.0,
             fake, None, None]
    rc = lib.glm_moe_forward_noalloc(*args)
    assert rc == native.GLM_ERR_WORKSPACE, lib.glm_last_error()
    assert b"scratch" in lib.glm_last_error()
    # an empty batch validates and returns without touching the device
    args[2] = 0
    assert lib.glm_moe_forward_noalloc(*args) == native.GLM_OK
    # the decode sizes fit
    c2 = SHAPES["batch_t64"]
    assert lib.glm_moe_workspace_bytes(c2.T, c2.d, c2.E, c2.k, c2.I, c2.I_shared) \
        <= native.GLM_NOALLOC_SCRATCH_BYTES
