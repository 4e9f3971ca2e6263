"""glm_moe_forward_noalloc: the MoE layer with its workspace in the library's
static device array.  Through the C ABI, two calls in a row (the second with
a smaller input, so it runs on what the first left in the array) must equal
glm_moe_forward with a fresh caller workspace bit for bit; so must the
replays of a HIP graph that captured the call, both after eager calls and
when the capture holds the entry point's first call in a fresh process (the
array's address is looked up then); sizes beyond the array are rejected on
the host before any device work."""

from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys

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


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["verify_t2", "batch_t64"])
def test_noalloc_graph_replays_equal_moe_forward(name):
    # captured after eager calls; each replay (other eager work in between,
    # the outputs cleared) must give glm_moe_forward's result bit for bit
    import torch

    import gpu_util as gu
    shape = SHAPES[name]
    native.load()
    _both(shape, 8850)  # eager calls first
    layer = make_layer(shape, 8851)
    dl = gu.upload_layer(layer)
    T, d, k = shape.T, shape.d, shape.k
    ws_bytes = native.load().glm_moe_workspace_bytes(T, d, shape.E, k, shape.I, shape.I_shared)
    ws = gu.workspace(ws_bytes)
    ref = [torch.empty((T, d), dtype=torch.float32, device="cuda"),
           torch.empty((T, k), dtype=torch.float32, device="cuda"),
           torch.empty((T, k), dtype=torch.int32, device="cuda")]
    gu.call("glm_moe_forward", *_args(dl, shape, T, *ref, ws, ws_bytes))
    want = [gu.host(t).view(np.uint32) for t in ref]
    outs = [torch.empty_like(t) for t in ref]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.call("glm_moe_forward_noalloc", *_args(dl, shape, T, *outs))
    for rep in range(3):
        _both(SHAPES["verify_t2"], 8860 + rep)  # other eager work on the same array
        for t in outs:
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, exp in zip(outs, want):
            np.testing.assert_array_equal(gu.host(got).view(np.uint32), exp, err_msg=str(rep))


FIRST_CALL_IN_CAPTURE = r"""
import json, sys
import numpy as np
import torch
import gpu_util as gu
from livglm_amd import native
from livglm_amd.workloads import SHAPES, make_layer
from test_zz_no_alloc import _args
shape = SHAPES["verify_t2"]
lib = native.load()
dl = gu.upload_layer(make_layer(shape, 8900))
T, d, k = shape.T, shape.d, shape.k
outs = [torch.empty((T, d), dtype=torch.float32, device="cuda"),
        torch.empty((T, k), dtype=torch.float32, device="cuda"),
        torch.empty((T, k), dtype=torch.int32, device="cuda")]
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    rc = lib.glm_moe_forward_noalloc(*_args(dl, shape, T, *outs))
res = {"rc": rc, "error": lib.glm_last_error().decode()}
if rc == 0:
    same = True
    ws_bytes = lib.glm_moe_workspace_bytes(T, d, shape.E, k, shape.I, shape.I_shared)
    ws = gu.workspace(ws_bytes)
    ref = [torch.empty_like(t) for t in outs]
    gu.call("glm_moe_forward", *_args(dl, shape, T, *ref, ws, ws_bytes))
    for rep in range(2):
        for t in outs:
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        same = same and all(np.array_equal(gu.host(a).view(np.uint32), gu.host(b).view(np.uint32))
                            for a, b in zip(outs, ref))
    res["equal"] = bool(same)
print(json.dumps(res))
"""


@pytest.mark.gpu
def test_noalloc_first_call_inside_graph_capture():
    # a fresh process whose first glm_moe_forward_noalloc call (the one that
    # looks up the array's address on the device) is made under capture
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(
        [root, os.path.join(root, "src"), os.path.join(root, "tests")]))
    proc = subprocess.run([sys.executable, "-c", FIRST_CALL_IN_CAPTURE], cwd=root, env=env,
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stderr[-2000:]
    res = json.loads(proc.stdout.strip().splitlines()[-1])
    assert res["rc"] == native.GLM_OK, res
    assert res["equal"], res


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
