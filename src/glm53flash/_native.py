"""torch <-> libglm53moe plumbing: pointers, streams and argument checks."""

from __future__ import annotations

import os
import sys

import torch

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

from livglm_amd import native  # noqa: E402

from .contract import ContractError  # noqa: E402

FMT_BF16 = native.GLM_FMT_BF16
FMT_MXFP8 = native.GLM_FMT_MXFP8
FMT_MXFP4 = native.GLM_FMT_MXFP4
MX_RULE_NEAREST = native.GLM_MX_RULE_NEAREST
MX_RULE_OCP = native.GLM_MX_RULE_OCP

FORMAT_OF_MODE = {None: FMT_BF16, "mxfp8": FMT_MXFP8, "mxfp4": FMT_MXFP4}


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(t: torch.Tensor, name: str, dtypes=None) -> torch.Tensor:
    """Checks that ``t`` is a contiguous CUDA (HIP) tensor of an allowed dtype."""
    if not isinstance(t, torch.Tensor):
        raise ContractError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ContractError(f"{name} must live on the GPU (got {t.device})")
    if dtypes is not None and t.dtype not in dtypes:
        raise ContractError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if not t.is_contiguous():
        raise ContractError(f"{name} must be contiguous")
    return t


def call(name: str, *args) -> None:
    """Calls the native entry point; maps its status to ContractError/RuntimeError."""
    try:
        native.call(name, *args)
    except native.NativeError as err:
        if err.code in (native.GLM_ERR_INVALID_ARGUMENT, native.GLM_ERR_UNSUPPORTED_SHAPE,
                        native.GLM_ERR_WORKSPACE):
            raise ContractError(str(err)) from err
        raise


def workspace_bytes(T: int, d: int, E: int, k: int, I: int, I_shared: int) -> int:
    return int(native.load().glm_moe_workspace_bytes(T, d, E, k, I, I_shared))
