"""ctypes binding of libglm53moe.so (declared in include/glm53_moe.h).

The library is the only compute path: if it is missing or cannot load, every
call raises.  There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libglm53moe.so")

GLM_OK = 0
GLM_ERR_INVALID_ARGUMENT = -1
GLM_ERR_UNSUPPORTED_SHAPE = -2
GLM_ERR_HIP = -3
GLM_ERR_WORKSPACE = -4

GLM_FMT_BF16 = 0
GLM_FMT_MXFP8 = 1
GLM_FMT_MXFP4 = 2

GLM_MX_RULE_NEAREST = 0
GLM_MX_RULE_OCP = 1

GLM_ACT_FP8X2 = 0
GLM_ACT_FP6X2 = 1
GLM_ACT_FP4 = 2
GLM_ACT_FP8FP6 = 3

GLM_READ_DROP_CACHE = 1
GLM_HC_BF16_STREAMS = 1
GLM_NOALLOC_SCRATCH_BYTES = 64 << 20

ABI_VERSION = 2

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_i64 = ctypes.c_int64

# name -> (restype, argtypes); mirrors include/glm53_moe.h
SIGNATURES = {
    "glm_abi_version": (_i, []),
    "glm_last_error": (ctypes.c_char_p, []),
    "glm_router_topk": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _i, _f, _p, _p, _p]),
    "glm_moe_dispatch": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "glm_expert_gate_up": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _f, _p]),
    "glm_route_gate_up": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _i, _i, _p, _p, _p, _p,
                               _f, _p, _p, _p]),
    "glm_expert_down": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p]),
    "glm_moe_tiles": (_i, [_p, _p, _i, _p, _p]),
    "glm_act_split_bytes": (_sz, [_i, _i]),
    "glm_act_split_fp8": (_i, [_p, _p, _i, _i, _p]),
    "glm_expert_gate_up_grouped": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _i, _f,
                                        _p]),
    "glm_expert_down_grouped": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _p, _i, _p]),
    "glm_act_split_bytes_fmt": (_sz, [_i, _i, _i]),
    "glm_act_split": (_i, [_p, _p, _i, _i, _i, _p]),
    "glm_expert_gate_up_grouped_fmt": (_i, [_p, _i, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p,
                                            _i, _f, _p]),
    "glm_expert_down_grouped_fmt": (_i, [_p, _i, _p, _i, _i, _i, _p, _p, _p, _p, _i, _p]),
    "glm_moe_combine": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "glm_linear": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _p]),
    "glm_linear_f32": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _p]),
    "glm_rms_norm_linear": (_i, [_p, _p, _i, _i, _p, _f, _p, _p, _i, _i, _p]),
    "glm_dense_mlp": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _f, _p, _p]),
    "glm_mx_quantize": (_i, [_p, _p, _i, _i, _i, _i, _p, _p]),
    "glm_mx_dequantize": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "glm_limited_swiglu": (_i, [_p, _p, _p, _i64, _f, _p]),
    "glm_moe_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "glm_moe_workspace_init": (_i, [_p, _p, _sz]),
    "glm_moe_forward": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _i, _f, _i,
                             _p, _p, _p, _p, _p, _p, _i, _i, _p, _p, _p, _p, _p, _p, _p,
                             _f, _p, _sz, _p, _p, _p]),
    "glm_moe_forward_scalex": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _i, _f, _i,
                                    _p, _p, _p, _p, _i64, _i, _i, _p, _p, _p, _p, _p, _p,
                                    _p, _f, _p, _sz, _p, _p, _p]),
    "glm_moe_forward_noalloc": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _i, _f, _i,
                                     _p, _p, _p, _p, _p, _p, _i, _i, _p, _p, _p, _p, _p, _p,
                                     _p, _f, _p, _p, _p]),
    "glm_moe_forward_hc": (_i, [_p, _p, _i, _i, _p, _p, _i, _i, _i, _i, _i, _f, _i,
                                _p, _p, _p, _p, _p, _p, _i, _i, _p, _p, _p, _p, _p, _p, _p,
                                _f, _p, _sz, _p, _p, _p, _p, _i, _p, _p, _i, _p]),
    "glm_hc_workspace_bytes": (_sz, [_i, _i, _i]),
    "glm_hc_pre": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _i, _f, _f, _p, _f, _i, _p, _sz, _p, _p,
                        _p, _p]),
    "glm_hc_post": (_i, [_p, _p, _i, _i, _i, _p, _p, _p, _i, _p]),
    "glm_rms_norm": (_i, [_p, _p, _i, _i, _p, _f, _p, _p]),
    "glm_file_read_ranges": (_i, [ctypes.c_char_p, _i, _p, _p, _p, _i, _i]),
    "glm_bank_scatter": (_i, [_p, _p, _i64, _p, _i, _p]),
    "glm_mxfp4_tile": (_i, [_p, _p, _p, _i64, _i, _i]),
    "glm_mxfp4_is_tiled": (_i, [_i, _i]),
    "glm_scalex_decode": (_i, [_p, _p, _i64, _p, _i, _p]),
}


class NativeError(RuntimeError):
    """A libglm53moe call returned a non-zero status."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed ({code}): {message}")
        self.code = code
        self.message = message


_lib = None
_lock = threading.Lock()


def library_path() -> str:
    return LIB_PATH


def load(path: str | None = None):
    """Load (once) and return the ctypes library with typed signatures."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = path or LIB_PATH
        if not os.path.exists(target):
            raise RuntimeError(
                f"libglm53moe.so is not built ({target}); run `python -m livglm_amd.build`")
        lib = ctypes.CDLL(target)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.glm_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"libglm53moe ABI {lib.glm_abi_version()} != expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def check(name: str, code: int) -> None:
    if code != GLM_OK:
        msg = load().glm_last_error().decode("utf-8", "replace")
        raise NativeError(name, code, msg)


def call(name: str, *args) -> None:
    """Invoke ``name`` with ``args`` and raise NativeError on a non-zero status."""
    check(name, getattr(load(), name)(*args))


def mxfp4_is_tiled(rows: int, K: int) -> bool:
    """Whether the expert bank stores a rows x K MXFP4 matrix tile-major."""
    return bool(load().glm_mxfp4_is_tiled(rows, K))


def mxfp4_tile(packed, stream=None, out=None):
    """Checkpoint MXFP4 codes -> the expert bank's layout, on the GPU.

    ``packed`` is a CUDA u8 tensor ``[..., rows, K/2]`` (a stack of row-major
    matrices); returns ``out`` (allocated like ``packed`` when not given)
    holding each matrix tile-major when ``rows % 16 == 0`` and ``K % 128 ==
    0``, else copied (glm_mxfp4_tile)."""
    import torch

    if not packed.is_cuda or packed.dtype != torch.uint8:
        raise ValueError("mxfp4_tile takes a CUDA uint8 tensor")
    src = packed.contiguous()
    rows, K = int(src.shape[-2]), int(src.shape[-1]) * 2
    count = src.numel() // (rows * (K // 2)) if src.numel() else 0
    dst = torch.empty_like(src) if out is None else out
    if dst.shape != src.shape or dst.dtype != torch.uint8 or not dst.is_contiguous():
        raise ValueError("mxfp4_tile: out must be a contiguous uint8 tensor shaped like packed")
    s = torch.cuda.current_stream(src.device).cuda_stream if stream is None else stream
    call("glm_mxfp4_tile", s, src.data_ptr(), dst.data_ptr(), count, rows, K)
    return dst


def mxfp4_tile_host(packed):
    """The bank layout of checkpoint MXFP4 codes, on the host (numpy), for
    checking what the GPU wrote: a stack ``[..., rows, K/2]`` of row-major
    matrices, each tile-major when ``rows % 16 == 0`` and ``K % 128 == 0`` --
    row 16t + r, bytes 64c + 16q .. +15 go to piece r + 16q of the 1 KB block
    (t, c) -- else unchanged."""
    import numpy as np

    a = np.ascontiguousarray(packed, dtype=np.uint8)
    rows, half = a.shape[-2], a.shape[-1]
    if rows % 16 or (2 * half) % 128:
        return a.copy()
    lead = a.shape[:-2]
    t = a.reshape(*lead, rows // 16, 16, half // 64, 4, 16)  # (t, r, c, q, byte)
    n = len(lead)
    t = t.transpose(*range(n), n, n + 2, n + 3, n + 1, n + 4)  # (t, c, q, r, byte)
    return np.ascontiguousarray(t).reshape(a.shape)
