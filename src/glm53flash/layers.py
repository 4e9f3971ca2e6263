"""Deferred-weight linears and the dense SwiGLU MLP (shared expert).

Mirrors ``layers.py:12-105,160-171`` of the reference on torch tensors; the
arithmetic runs in libglm53moe (``glm_linear``, ``glm_dense_mlp``,
``glm_mx_quantize``).
"""

from __future__ import annotations

import torch

from . import _native as N
from .contract import ContractError
from .expert_ssd import limited_swiglu


def require_weight(value, name: str):
    """``layers.py:12-15``: reading a weight that was never attached raises."""
    if value is None:
        raise ContractError(f"resident parameter was not loaded: {name}")
    return value


class DeferredLinear:
    """A linear layer whose storage is attached after construction.

    ``weight`` is bf16 ``[out, in]`` until ``quantize_to_mxfp`` replaces it by
    MX codes (u8 ``[out, in]`` for MXFP8, ``[out, in/2]`` for MXFP4) and
    ``scales`` (u8 ``[out, in/32]``).  Inputs are bf16 ``[..., in]``; outputs
    bf16 ``[..., out]`` (``layers.py:38-70``)."""

    def __init__(self, input_dims: int, output_dims: int, *, bias: bool = False,
                 quantize_resident: bool = True):
        self.input_dims = input_dims
        self.output_dims = output_dims
        self.weight: torch.Tensor | None = None
        self.scales: torch.Tensor | None = None
        self.quantization_mode: str | None = None
        self.quantize_resident = quantize_resident
        self.bias = None if bias else False

    @property
    def fmt(self) -> int:
        return N.FORMAT_OF_MODE[self.quantization_mode]

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        weight = require_weight(self.weight, "linear.weight")
        if self.bias is not False:
            raise ContractError("biased deferred linears are not part of the MoE path")
        N.require_device(x, "x", (torch.bfloat16,))
        if x.shape[-1] != self.input_dims:
            raise ContractError(f"linear input width {x.shape[-1]} != {self.input_dims}")
        rows = x.reshape(-1, self.input_dims)
        out = torch.empty((rows.shape[0], self.output_dims), dtype=torch.bfloat16, device=x.device)
        scales = None
        if self.quantization_mode is not None:
            scales = require_weight(self.scales, "linear.scales")
        N.call("glm_linear", N.stream_of(x), rows.data_ptr(), rows.shape[0], self.input_dims,
               weight.data_ptr(), N.ptr(scales), self.fmt, self.output_dims, out.data_ptr())
        return out.reshape(*x.shape[:-1], self.output_dims)

    def quantize_to_mxfp(self, bits: int, rule: int = N.MX_RULE_NEAREST) -> tuple[int, int]:
        """Startup conversion to group-32 MXFP8/MXFP4 (``layers.py:72-99``).
        Returns ``(source_bytes, destination_bytes)``."""
        mode = f"mxfp{bits}"
        if bits not in {4, 8}:
            raise ContractError(f"unsupported resident quantization: {mode}")
        if not self.quantize_resident:
            raise ContractError(f"this deferred linear is excluded from resident {mode.upper()}")
        if self.quantization_mode is not None:
            raise ContractError("deferred linear was already quantized")
        weight = require_weight(self.weight, "linear.weight")
        if weight.ndim != 2 or weight.shape[-1] % 32:
            raise ContractError(
                f"resident {mode.upper()} requires a group-32 matrix: {tuple(weight.shape)}")
        N.require_device(weight, "linear.weight", (torch.bfloat16,))
        rows, cols = weight.shape
        codes = torch.empty((rows, cols if bits == 8 else cols // 2), dtype=torch.uint8,
                            device=weight.device)
        scales = torch.empty((rows, cols // 32), dtype=torch.uint8, device=weight.device)
        fmt = N.FMT_MXFP8 if bits == 8 else N.FMT_MXFP4
        N.call("glm_mx_quantize", N.stream_of(weight), weight.data_ptr(), rows, cols, fmt, rule,
               codes.data_ptr(), scales.data_ptr())
        source_bytes = weight.numel() * weight.element_size()
        self.weight = codes
        self.scales = scales
        self.quantization_mode = mode
        return source_bytes, codes.numel() + scales.numel()

    def quantize_to_mxfp8(self) -> tuple[int, int]:
        return self.quantize_to_mxfp(8)

    def quantize_to_mxfp4(self) -> tuple[int, int]:
        return self.quantize_to_mxfp(4)


class DenseMLP:
    """``down(limited_swiglu(gate(x), up(x)))`` (``layers.py:160-171``)."""

    def __init__(self, hidden_size: int, intermediate_size: int, swiglu_limit: float):
        self.gate_proj = DeferredLinear(hidden_size, intermediate_size)
        self.up_proj = DeferredLinear(hidden_size, intermediate_size)
        self.down_proj = DeferredLinear(intermediate_size, hidden_size)
        self.swiglu_limit = swiglu_limit
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size

    def fused_format(self) -> int | None:
        """The shared weight format if all three projections can run fused."""
        modes = {self.gate_proj.quantization_mode, self.up_proj.quantization_mode,
                 self.down_proj.quantization_mode}
        if len(modes) != 1:
            return None
        return N.FORMAT_OF_MODE[modes.pop()]

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        fmt = self.fused_format()
        if fmt is None:
            return self.down_proj(limited_swiglu(self.gate_proj(x), self.up_proj(x),
                                                 self.swiglu_limit))
        N.require_device(x, "x", (torch.bfloat16,))
        gw = require_weight(self.gate_proj.weight, "gate_proj.weight")
        uw = require_weight(self.up_proj.weight, "up_proj.weight")
        dw = require_weight(self.down_proj.weight, "down_proj.weight")
        rows = x.reshape(-1, self.hidden_size)
        T = rows.shape[0]
        h = torch.empty((T, self.intermediate_size), dtype=torch.bfloat16, device=x.device)
        out = torch.empty((T, self.hidden_size), dtype=torch.bfloat16, device=x.device)
        N.call("glm_dense_mlp", N.stream_of(x), rows.data_ptr(), T, self.hidden_size,
               self.intermediate_size, fmt, gw.data_ptr(), N.ptr(self.gate_proj.scales),
               uw.data_ptr(), N.ptr(self.up_proj.scales), dw.data_ptr(),
               N.ptr(self.down_proj.scales), float(self.swiglu_limit), h.data_ptr(),
               out.data_ptr())
        return out.reshape(*x.shape[:-1], self.hidden_size)


def _f32_param(value, cache: dict, slot: str, name: str) -> torch.Tensor:
    """The f32 device copy of a norm-style parameter (exact for bf16; the
    tensor itself when it is f32), cached in ``cache[slot]`` until the
    parameter is replaced or modified in place."""
    value = require_weight(value, name)
    key = (id(value), value._version, value.data_ptr())
    hit = cache.get(slot)
    if hit is None or hit[0] != key:
        N.require_device(value, name, (torch.float32, torch.bfloat16))
        hit = (key, value.to(torch.float32).contiguous())
        cache[slot] = hit
    return hit[1]


class RMSNorm:
    """``mx.fast.rms_norm(x, weight, eps)`` (``layers.py:119-131``): ``x * (1 /
    sqrt(mean(x^2) + eps)) * weight`` over the last axis, computed in f32; the
    output has the input's dtype (f32 or bf16)."""

    def __init__(self, dims: int, eps: float):
        self.dims = dims
        self.eps = eps
        self.weight = None
        self._f32: dict = {}

    def weight_f32(self) -> torch.Tensor:
        return _f32_param(self.weight, self._f32, "weight", "rms_norm.weight")

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return _rms_norm(x, self.dims, self.weight_f32(), self.eps)


class UnweightedRMSNorm:
    """``layers.py:134-140``: the RMS norm of ``x`` cast to f32, no weight; f32 out."""

    def __init__(self, eps: float):
        self.eps = eps

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return _rms_norm(x.to(torch.float32), x.shape[-1], None, self.eps)


def _rms_norm(x: torch.Tensor, d: int, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    N.require_device(x, "x", (torch.float32, torch.bfloat16))
    if x.shape[-1] != d:
        raise ContractError(f"rms_norm over {d} features got rows of {x.shape[-1]}")
    rows = x.reshape(-1, d)
    xf = rows if rows.dtype == torch.float32 else rows.to(torch.float32)
    out = torch.empty(xf.shape, dtype=x.dtype, device=x.device)
    f32 = out if x.dtype == torch.float32 else None
    b16 = out if x.dtype == torch.bfloat16 else None
    N.call("glm_rms_norm", N.stream_of(x), xf.data_ptr(), xf.shape[0], d, N.ptr(weight),
           float(eps), N.ptr(f32), N.ptr(b16))
    return out.reshape(x.shape)
