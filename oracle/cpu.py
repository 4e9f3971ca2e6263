"""ctypes binding of the C restatement (oracle/libmoe_cpu.so) -- test
infrastructure only (tests and the benchmark's CPU baseline)."""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libmoe_cpu.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError("oracle/libmoe_cpu.so is not built; run `python -m oracle.build`")
        lib = ctypes.CDLL(LIB)
        lib.moe_cpu_threads.restype = _i
        lib.moe_cpu_layer.restype = _i
        lib.moe_cpu_layer.argtypes = [_p, _i, _i, _p, _p, _i, _i, _i, _i, _i, _f, _i,
                                      _p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _f, _p, _p, _p]
        lib.moe_cpu_linear_mxfp8.restype = _i
        lib.moe_cpu_linear_mxfp8.argtypes = [_p, _i, _i, _p, _p, _i, _p]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def threads() -> int:
    return int(load().moe_cpu_threads())


def moe_layer(layer: dict, shape, shared: bool = True):
    """Runs the whole layer on host arrays; returns (out f32 [T,d], weights, indices)."""
    x = np.ascontiguousarray(layer["x"])
    T = x.shape[0]
    out = np.empty((T, shape.d), np.float32)
    w = np.empty((T, shape.k), np.float32)
    idx = np.empty((T, shape.k), np.uint32)
    keys = ("gate_proj.weight_packed", "gate_proj.weight_scale", "up_proj.weight_packed",
            "up_proj.weight_scale", "down_proj.weight_packed", "down_proj.weight_scale")
    bank = [np.ascontiguousarray(layer[k_]) for k_ in keys]
    sw = [np.ascontiguousarray(layer[k_]) for k_ in ("shared.gate", "shared.up", "shared.down")] \
        if shared else [None, None, None]
    rc = load().moe_cpu_layer(
        _ptr(x), T, shape.d, _ptr(np.ascontiguousarray(layer["router_weight"])),
        _ptr(np.ascontiguousarray(layer["router_bias"])), shape.E, shape.k, shape.n_group,
        shape.topk_group, int(shape.norm_topk_prob), shape.routed_scaling_factor, shape.I,
        *(_ptr(b) for b in bank), shape.I_shared if shared else 0, *(_ptr(s) for s in sw),
        shape.swiglu_limit, _ptr(out), _ptr(w), _ptr(idx))
    if rc != 0:
        raise RuntimeError("moe_cpu_layer rejected its arguments")
    return out, w, idx


def linear_mxfp8(x: np.ndarray, codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Resident MXFP8 linear on host arrays: x bf16 bits [T, in], codes u8
    [out, in], scales u8 [out, in/32]; returns bf16 bits [T, out]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    T, n_in = x.shape
    n_out = codes.shape[0]
    if codes.shape != (n_out, n_in) or scales.shape != (n_out, n_in // 32):
        raise ValueError("MXFP8 codes/scales do not match the input width")
    y = np.empty((T, n_out), np.uint16)
    if load().moe_cpu_linear_mxfp8(_ptr(x), T, n_in, _ptr(codes), _ptr(scales), n_out,
                                    _ptr(y)) != 0:
        raise RuntimeError("moe_cpu_linear_mxfp8 rejected its arguments")
    return y
