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

GLM_READ_DROP_CACHE = 1
GLM_HC_BF16_STREAMS = 1
GLM_NOALLOC_SCRATCH_BYTES = 64 << 20

ABI_VERSION = 1

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
