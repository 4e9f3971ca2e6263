"""Helpers for the GPU parity tests: numpy <-> device tensors, C-ABI calls."""

from __future__ import annotations

import numpy as np
import torch

from livglm_amd import native
from livglm_amd.workloads import BANK_KEYS


def to_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    elif a.dtype == np.uint32:
        t = torch.from_numpy(a.view(np.int32))
    else:
        t = torch.from_numpy(a)
    return t.to("cuda")


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


# Tensors whose pointers were handed out by p(): kept alive until the next
# call() has synchronised, so temporaries such as p(to_dev(a)) cannot be
# freed (and their memory reused) before the kernel reads them.
_live: list[torch.Tensor] = []


def call(name: str, *args) -> None:
    try:
        native.call(name, *args)
        torch.cuda.synchronize()
    finally:
        _live.clear()


def p(t: torch.Tensor | None):
    if t is None:
        return None
    _live.append(t)
    return t.data_ptr()


PACKED_KEYS = ("gate_proj.weight_packed", "up_proj.weight_packed", "down_proj.weight_packed")


def upload_layer(layer: dict[str, np.ndarray], bank_layout: bool = True) -> dict[str, torch.Tensor]:
    """The layer's arrays on the GPU; the experts' packed codes in the bank
    layout (glm_mxfp4_tile) unless bank_layout is False (checkpoint bytes, as
    the Python mirror's load_bank takes them)."""
    dev = {k: to_dev(v) for k, v in layer.items()}
    if bank_layout:
        for k in PACKED_KEYS:
            if k in dev:
                dev[k] = native.mxfp4_tile(dev[k])
    return dev


def workspace(nbytes: int) -> torch.Tensor:
    """A layer workspace, zero-filled through the C ABI (glm_moe_forward does
    not need it cleared; a defined initial state keeps failures reproducible)."""
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    call("glm_moe_workspace_init", stream(), p(ws), nbytes)
    return ws


def run_layer(dl: dict[str, torch.Tensor], shape, T: int | None = None, shared: bool = True,
              bias: torch.Tensor | None = None, ws: torch.Tensor | None = None,
              shared_in: torch.Tensor | None = None, shared_fmt: int = native.GLM_FMT_BF16):
    """glm_moe_forward on uploaded layer tensors; returns (out, weights, indices).
    An MX shared expert takes its scales from dl["shared.gate.scales"] etc."""
    T = dl["x"].shape[0] if T is None else T
    d, E, k, I, Is = shape.d, shape.E, shape.k, shape.I, shape.I_shared
    lib = native.load()
    ws_bytes = lib.glm_moe_workspace_bytes(T, d, E, k, I, Is if shared else 0)
    if ws is None:
        ws = workspace(ws_bytes)
    out = torch.empty((T, d), dtype=torch.float32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    b = dl["router_bias"] if bias is None else bias
    args = [stream(), p(dl["x"]), T, d, p(dl["router_weight"]), p(b), E, k, shape.n_group,
            shape.topk_group, int(shape.norm_topk_prob), shape.routed_scaling_factor, I]
    args += [p(dl[key]) for key in BANK_KEYS]
    if shared:
        sc = {key: (p(dl[key + ".scales"]) if shared_fmt != native.GLM_FMT_BF16 else None)
              for key in ("shared.gate", "shared.up", "shared.down")}
        args += [Is, shared_fmt, p(dl["shared.gate"]), sc["shared.gate"], p(dl["shared.up"]),
                 sc["shared.up"], p(dl["shared.down"]), sc["shared.down"], p(shared_in)]
    else:
        args += [0, native.GLM_FMT_BF16, None, None, None, None, None, None, p(shared_in)]
    args += [shape.swiglu_limit, p(ws), ws_bytes, p(out), p(w), p(idx)]
    call("glm_moe_forward", *args)
    return out, w, idx
