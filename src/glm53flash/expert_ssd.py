"""Routed experts backed by an HBM-resident MXFP4 bank.

The reference keeps routed experts on SSD behind a bounded slot cache
(``expert_ssd.py:130-194``, ``native_expert_ssd.py:389-815``).  On MI355X every
expert of a layer fits in HBM, so the bank *is* the storage: one stacked tensor
per checkpoint part (``weight_packed`` / ``weight_scale`` of gate, up and down,
``expert_source.py:189-229``) with slot = expert id.  The backend keeps the
reference's contract -- ``prepare(indices)``, ``finish(x, plan)``,
``__call__(x, indices) -> [T, k, d]``, ``stats()``, ``capacity``,
``last_expert_ids``, ``activate()``, ``close()`` -- and routes on the device
(histogram / prefix sum / stable permute) instead of materialising routes on
the host.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

import torch

from . import _native as N
from .contract import ContractError


@dataclass(frozen=True)
class ExpertCacheStats:
    """``expert_ssd.py:16-29``.  With the whole bank resident every route is a
    hit and nothing is ever evicted."""

    layer: int
    capacity: int
    resident: int
    hits: int
    misses: int
    evictions: int
    route_sync_seconds: float = 0.0
    slot_plan_seconds: float = 0.0
    policy: str = "hbm-resident"

    def as_dict(self) -> dict[str, int | float | str]:
        return asdict(self)


def limited_swiglu(gate: torch.Tensor, up: torch.Tensor, limit: float) -> torch.Tensor:
    """``expert_ssd.py:103-107`` on bf16 GPU tensors (bf16 intermediates)."""
    N.require_device(gate, "gate", (torch.bfloat16,))
    N.require_device(up, "up", (torch.bfloat16,))
    if gate.shape != up.shape:
        raise ContractError(f"gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
    out = torch.empty_like(gate)
    N.call("glm_limited_swiglu", N.stream_of(gate), gate.data_ptr(), up.data_ptr(),
           gate.numel(), float(limit), out.data_ptr())
    return out


@dataclass
class RoutePlan:
    """Device-side route plan of one call: the dispatch of ``indices``."""

    indices: torch.Tensor      # u32-as-int32 [T, k]
    counts: torch.Tensor       # [E]
    offsets: torch.Tensor      # [E + 1]
    perm: torch.Tensor         # [T*k] sorted position -> pair
    inv: torch.Tensor          # [T*k] pair -> sorted position
    pair_token: torch.Tensor   # [T*k] sorted position -> token
    active: torch.Tensor       # [E] active expert ids, ascending (-1 padded)
    num_active: torch.Tensor   # [1]
    work: torch.Tensor         # [E, 4] per active slot: expert, first row, rows, 0
    status: torch.Tensor       # [1] 1 if an out-of-range id was seen

    def check(self, num_experts: int) -> None:
        """Host-synchronising validation (the reference's range check,
        ``native_expert_ssd.py:502-513``)."""
        if int(self.status.item()) != 0:
            bad = sorted({int(v) for v in self.indices.reshape(-1).tolist() if not 0 <= int(v) < num_experts})
            raise ContractError(f"routed expert ids are out of range: {bad}")


PARTS = ("gate_proj", "up_proj", "down_proj")


class HBMExpertBank:
    """All ``num_experts`` MXFP4 experts of one MoE layer, resident in HBM."""

    def __init__(self, *, layer: int, num_experts: int, hidden_size: int, intermediate_size: int,
                 swiglu_limit: float, device: torch.device | str | None = None,
                 defer_slots: bool = False):
        if num_experts < 1:
            raise ContractError("the expert bank needs at least one expert")
        if hidden_size % 32 or intermediate_size % 32:
            raise ContractError("MXFP4 group-32 experts need hidden/intermediate sizes % 32 == 0")
        self.layer = layer
        self.num_experts = num_experts
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.swiglu_limit = swiglu_limit
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.capacity = num_experts
        self.tensors: dict[str, torch.Tensor] = {}
        self.last_plan: RoutePlan | None = None
        self._active = False
        self._closed = False
        self._calls = 0
        if not defer_slots:
            self.activate()

    # ------------------------------------------------------------ storage

    def shapes(self) -> dict[str, tuple[int, ...]]:
        E, d, I = self.num_experts, self.hidden_size, self.intermediate_size
        return {
            "gate_proj.weight_packed": (E, I, d // 2),
            "gate_proj.weight_scale": (E, I, d // 32),
            "up_proj.weight_packed": (E, I, d // 2),
            "up_proj.weight_scale": (E, I, d // 32),
            "down_proj.weight_packed": (E, d, I // 2),
            "down_proj.weight_scale": (E, d, I // 32),
        }

    @property
    def expert_bytes(self) -> int:
        """Bytes of one expert (3 projections of packed codes + scales)."""
        return sum(int(torch.Size(s[1:]).numel()) for s in self.shapes().values())

    def activate(self) -> None:
        if self._closed:
            raise RuntimeError("HBM expert bank is closed")
        if self._active:
            return
        self.tensors = {name: torch.zeros(shape, dtype=torch.uint8, device=self.device)
                        for name, shape in self.shapes().items()}
        self._active = True

    def close(self) -> None:
        self.tensors = {}
        self._active = False
        self._closed = True

    def _require_active(self) -> None:
        if self._closed:
            raise RuntimeError("HBM expert bank is closed")
        if not self._active:
            raise RuntimeError("HBM expert bank was not activated")

    @staticmethod
    def _as_bytes(t: torch.Tensor) -> torch.Tensor:
        """Accepts the checkpoint's U8 tensors or the reference's U32 view."""
        if t.dtype == torch.uint8:
            return t
        if t.dtype in (torch.int32, torch.uint32):
            return t.contiguous().view(torch.uint8)
        raise ContractError(f"expert tensors must be U8 (or a U32 view), got {t.dtype}")

    def load_expert(self, expert: int, tensors: dict[str, torch.Tensor]) -> None:
        """Copies one expert's six checkpoint tensors into its slot.  Keys are
        the checkpoint names (``gate_proj.weight_packed``, ``...weight_scale``)
        or the reference's MLX names (``gate_proj.weight``, ``...scales``).
        Packed codes land in the bank layout (``native.mxfp4_tile``)."""
        self._require_active()
        if not 0 <= expert < self.num_experts:
            raise ContractError(f"expert id {expert} is out of range")
        for name, shape in self.shapes().items():
            comp, part = name.split(".")
            alias = f"{comp}.weight" if part == "weight_packed" else f"{comp}.scales"
            src = tensors.get(name, tensors.get(alias))
            if src is None:
                raise ContractError(f"expert {expert} is missing {name}")
            src = self._as_bytes(src)
            if tuple(src.shape[:-1]) != shape[1:-1] or src.numel() != int(torch.Size(shape[1:]).numel()):
                raise ContractError(f"{name} of expert {expert} has shape {tuple(src.shape)}, "
                                    f"expected {shape[1:]}")
            if part == "weight_packed":
                N.native.mxfp4_tile(src.reshape(shape[1:]).to(self.device),
                                  out=self.tensors[name][expert])
            else:
                self.tensors[name][expert].copy_(src.reshape(shape[1:]))

    def load_bank(self, tensors: dict[str, torch.Tensor]) -> None:
        """Replaces the whole bank with stacked ``[E, ...]`` checkpoint
        tensors: the packed codes are rewritten in the bank layout
        (``native.mxfp4_tile``), the scales kept as they are (no copy when
        already contiguous u8 on this device)."""
        self._require_active()
        for name, shape in self.shapes().items():
            src = self._as_bytes(tensors[name])
            if tuple(src.shape) != shape:
                if src.numel() != int(torch.Size(shape).numel()):
                    raise ContractError(f"{name} has shape {tuple(src.shape)}, expected {shape}")
                src = src.reshape(shape)
            if src.device != self.device:
                src = src.to(self.device)
            if name.endswith(".weight_packed"):
                src = N.native.mxfp4_tile(src)
            self.tensors[name] = src.contiguous()

    def projection(self, part: str) -> tuple[torch.Tensor, torch.Tensor]:
        return self.tensors[f"{part}.weight_packed"], self.tensors[f"{part}.weight_scale"]

    # ------------------------------------------------------------ routing

    def prepare(self, indices: torch.Tensor) -> RoutePlan:
        """On-device dispatch of ``indices`` [T, k] (no host synchronisation)."""
        self._require_active()
        if indices.ndim < 1 or indices.shape[-1] < 1:
            raise ContractError("routed expert indices must have a top-k dimension")
        k = indices.shape[-1]
        idx = indices.reshape(-1, k)
        if idx.dtype not in (torch.int32, torch.uint32):
            if idx.dtype in (torch.int64, torch.int16, torch.uint8):
                idx = idx.to(torch.int32)
            else:
                raise ContractError(f"routed indices must be integers, got {idx.dtype}")
        idx = N.require_device(idx.contiguous(), "indices")
        T = idx.shape[0]
        P = T * k
        E = self.num_experts
        dev = idx.device
        i32 = dict(dtype=torch.int32, device=dev)
        plan = RoutePlan(idx, torch.empty(E, **i32), torch.empty(E + 1, **i32),
                         torch.empty(P, **i32), torch.empty(P, **i32), torch.empty(P, **i32),
                         torch.empty(E, **i32), torch.empty(1, **i32), torch.empty((E, 4), **i32),
                         torch.empty(1, **i32))
        N.call("glm_moe_dispatch", N.stream_of(idx), idx.data_ptr(), T, k, E,
               plan.counts.data_ptr(), plan.offsets.data_ptr(), plan.perm.data_ptr(),
               plan.inv.data_ptr(), plan.pair_token.data_ptr(), plan.active.data_ptr(),
               plan.num_active.data_ptr(), plan.work.data_ptr(), plan.status.data_ptr())
        self.last_plan = plan
        self._calls += 1
        return plan

    def finish(self, x: torch.Tensor, plan: RoutePlan) -> torch.Tensor:
        """Routed SwitchGLU on the plan: returns bf16 ``[T, k, d]`` in route
        order (``expert_ssd.py:185-188``, ``native_expert_ssd.py:696-743``)."""
        self._require_active()
        N.require_device(x, "x", (torch.bfloat16,))
        d, I, E = self.hidden_size, self.intermediate_size, self.num_experts
        rows = x.reshape(-1, d)
        T, k = plan.indices.shape
        if rows.shape[0] != T:
            raise ContractError(f"token count {rows.shape[0]} differs from routed rows {T}")
        stream = N.stream_of(x)
        h = torch.empty((T * k, I), dtype=torch.bfloat16, device=x.device)
        y = torch.empty((T * k, d), dtype=torch.bfloat16, device=x.device)
        gw, gs = self.projection("gate_proj")
        uw, us = self.projection("up_proj")
        dw, ds = self.projection("down_proj")
        N.call("glm_expert_gate_up", stream, rows.data_ptr(), T, d, I, E, k, gw.data_ptr(),
               gs.data_ptr(), uw.data_ptr(), us.data_ptr(), plan.pair_token.data_ptr(),
               plan.work.data_ptr(), float(self.swiglu_limit), h.data_ptr())
        N.call("glm_expert_down", stream, h.data_ptr(), T, k, I, d, E, dw.data_ptr(),
               ds.data_ptr(), plan.work.data_ptr(), y.data_ptr())
        # un-permute: row of pair p lives at sorted position inv[p]
        return y.index_select(0, plan.inv.long()).reshape(T, k, d)

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        return self.finish(x, self.prepare(indices))

    # ------------------------------------------------------------ bookkeeping

    @property
    def last_expert_ids(self) -> tuple[int, ...]:
        """Flattened routed ids of the last call (synchronises with the device)."""
        if self.last_plan is None:
            return ()
        return tuple(int(v) for v in self.last_plan.indices.reshape(-1).tolist())

    @property
    def resident_experts(self) -> tuple[int, ...]:
        return tuple(range(self.num_experts)) if self._active else ()

    def stats(self) -> ExpertCacheStats:
        return ExpertCacheStats(layer=self.layer, capacity=self.capacity,
                                resident=self.num_experts if self._active else 0,
                                hits=0, misses=0, evictions=0)

    def clear(self) -> None:
        self.last_plan = None


# Names under which the reference's MoE accepts a routed backend.
NativeExpertSSD = HBMExpertBank
ExpertSSD = HBMExpertBank
