"""Plan of an HBM expert-bank load: for every (layer, expert), the file
ranges to read and where each byte of them goes in the layer's bank.

The bank of a layer (``HBMExpertBank``) stacks six U8 tensors over experts:
``<component>.<part>`` for components ``down_proj``, ``gate_proj``,
``up_proj`` and parts ``weight_packed`` (``[rows, cols/2]``, two E2M1 codes per
byte) and ``weight_scale`` (``[rows, cols/32]``, E8M0); gate/up have
``intermediate`` rows of ``hidden`` inputs, down the transpose.  Expert ``e``'s
slot is row ``e`` of each.

A checkpoint keeps an expert's six tensors next to each other (13,369,344
bytes at the real geometry, d 4096, I 2048), so the plan reads each expert as
one range and lists the six tensors as segments of it.  Tensors that are not
adjacent get their own ranges.  In a ScaleX layer container an expert is one
record -- coded scales, then the gate, down and up weights -- read as one
range; its scales are decoded into the bank's scale slots on the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

from .checkpoint import ShardIndex, TensorRange
from .contract import ContractError

COMPONENTS = ("down_proj", "gate_proj", "up_proj")
PARTS = ("weight_packed", "weight_scale")
BANK_KEYS = tuple(f"{c}.{p}" for c in COMPONENTS for p in PARTS)
REAL_RECORD_BYTES = 13_369_344  # one expert at d 4096, I 2048: 3 x 2048 x 4096 x 17/32


def expert_tensor_name(layer: int, expert: int, component: str, part: str) -> str:
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{component}.{part}"


def slot_shape(key: str, hidden_size: int, intermediate_size: int) -> tuple[int, int]:
    """[rows, bytes per row] of bank tensor ``key`` for one expert."""
    component, part = key.split(".")
    rows, inputs = ((hidden_size, intermediate_size) if component == "down_proj"
                    else (intermediate_size, hidden_size))
    per_byte = 2 if part == "weight_packed" else 32
    if inputs % per_byte:
        raise ContractError(f"{key}: {inputs} inputs per row is not a multiple of {per_byte}")
    return rows, inputs // per_byte


@dataclass(frozen=True)
class Segment:
    """``nbytes`` at ``at`` inside a read go to bank tensor ``key``, expert slot."""

    key: str
    at: int
    nbytes: int


@dataclass(frozen=True)
class Read:
    shard: str
    offset: int
    nbytes: int
    segments: tuple[Segment, ...]


@dataclass(frozen=True)
class ExpertLoad:
    """Everything to fill one expert slot.  ``coded`` (ScaleX only): the
    record, whose first ``coded.coded_bytes`` bytes in ``reads[0]`` are the
    Mode-A scales of gate, down and up, decoded into the scale slots."""

    layer: int
    expert: int
    reads: tuple[Read, ...]
    coded: object = None

    @property
    def read_bytes(self) -> int:
        return sum(r.nbytes for r in self.reads)

    @property
    def bank_bytes(self) -> int:
        """Bytes placed in the bank (scales decoded)."""
        weights = sum(s.nbytes for r in self.reads for s in r.segments)
        return weights + (self.coded.decoded_bytes if self.coded is not None else 0)


@dataclass(frozen=True)
class BankPlan:
    root: Path
    layers: tuple[int, ...]
    experts: int
    hidden_size: int
    intermediate_size: int
    loads: tuple[ExpertLoad, ...]  # layer-major, expert order

    def expert(self, layer: int, expert: int) -> ExpertLoad:
        if layer not in self.layers:
            raise ContractError(f"layer {layer} is not planned ({self.layers[0]}.."
                                f"{self.layers[-1]})")
        if not 0 <= expert < self.experts:
            raise ContractError(f"expert {expert} is outside 0..{self.experts - 1}")
        return self.loads[self.layers.index(layer) * self.experts + expert]

    def layer_loads(self, layer: int) -> tuple[ExpertLoad, ...]:
        i = self.layers.index(layer) if layer in self.layers else -1
        if i < 0:
            raise ContractError(f"layer {layer} is not planned")
        return self.loads[i * self.experts:(i + 1) * self.experts]

    @property
    def read_bytes(self) -> int:
        return sum(x.read_bytes for x in self.loads)

    @property
    def bank_bytes(self) -> int:
        return sum(x.bank_bytes for x in self.loads)

    @property
    def scalex(self) -> bool:
        return bool(self.loads) and self.loads[0].coded is not None

    @property
    def shards(self) -> tuple[str, ...]:
        return tuple(sorted({r.shard for x in self.loads for r in x.reads}))

    def shard_path(self, shard: str) -> Path:
        return self.root / shard


def _merge_adjacent(ranges: list[TensorRange]) -> tuple[Read, ...]:
    """Tensors that touch end to end in one shard share a read."""
    reads: list[tuple[str, int, int, list[Segment]]] = []
    for t in sorted(ranges, key=lambda t: (t.shard, t.offset)):
        key = ".".join(t.name.rsplit(".", 2)[-2:])
        if reads and reads[-1][0] == t.shard and reads[-1][1] + reads[-1][2] == t.offset:
            shard, off, n, segs = reads[-1]
            segs.append(Segment(key, n, t.nbytes))
            reads[-1] = (shard, off, n + t.nbytes, segs)
        else:
            reads.append((t.shard, t.offset, t.nbytes, [Segment(key, 0, t.nbytes)]))
    return tuple(Read(s, o, n, tuple(g)) for s, o, n, g in reads)


def _scalex_load(layer: int, expert: int, scalex, ranges: list[TensorRange]) -> ExpertLoad:
    """One read per ScaleX record: coded scales, then gate, down and up weights."""
    from .scalex_layer import RECORD_ORDER, ScaleXError
    if scalex.layer != layer:
        raise ContractError(f"{scalex.path} is layer {scalex.layer}'s container, not {layer}'s")
    try:
        rec = scalex.record(expert)
    except ScaleXError as exc:
        raise ContractError(str(exc)) from exc
    sizes = {".".join(t.name.rsplit(".", 2)[-2:]): t.nbytes for t in ranges}
    segs = []
    for i, comp in enumerate(RECORD_ORDER):
        key = f"{comp}.weight_packed"
        if sizes[key] != rec.weight_bytes[i] or \
                sizes[f"{comp}.weight_scale"] != rec.scale_bytes[i]:
            raise ContractError(f"{scalex.path} expert {expert}: {comp} sizes disagree with "
                                "its embedded header")
        segs.append(Segment(key, rec.weight_offset(i), rec.weight_bytes[i]))
    read = Read(ranges[0].shard, rec.offset, rec.nbytes, tuple(segs))
    return ExpertLoad(layer, expert, (read,), coded=rec)


def plan_expert_banks(index: ShardIndex, *, hidden_size: int, intermediate_size: int,
                      experts: int, layers) -> BankPlan:
    """The load plan of ``layers`` x ``experts`` routed experts of a checkpoint
    with this geometry.  Every tensor must be a 2-D U8 tensor of the slot's
    shape, an expert's six tensors must share a shard, and all shards of the
    plan must be ScaleX containers or none."""
    layers = tuple(int(v) for v in layers)
    if not layers or experts < 1:
        raise ContractError("nothing to plan: give at least one layer and one expert")
    want = {key: slot_shape(key, hidden_size, intermediate_size) for key in BANK_KEYS}
    loads = []
    for layer in layers:
        for e in range(experts):
            ranges = []
            for key in BANK_KEYS:
                comp, part = key.split(".")
                t = index.locate(expert_tensor_name(layer, e, comp, part))
                if t.dtype != "U8":
                    raise ContractError(f"{t.name}: stored as {t.dtype}; MXFP4 bytes are U8")
                if t.shape != want[key]:
                    raise ContractError(f"{t.name}: shape {list(t.shape)}, the geometry "
                                        f"(d {hidden_size}, I {intermediate_size}) needs "
                                        f"{list(want[key])}")
                ranges.append(t)
            shards = {t.shard for t in ranges}
            if len(shards) > 1:
                raise ContractError(f"layer {layer} expert {e} is split over shards "
                                    f"{sorted(shards)}")
            scalex = index.scalex(ranges[0].shard)
            loads.append(_merge_adjacent(ranges) if scalex is None
                         else _scalex_load(layer, e, scalex, ranges))
            if scalex is None:
                loads[-1] = ExpertLoad(layer, e, loads[-1])
    if len({x.coded is not None for x in loads}) > 1:
        raise ContractError("the planned layers mix ScaleX containers and plain shards")
    plan = BankPlan(root=index.root, layers=layers, experts=experts, hidden_size=hidden_size,
                    intermediate_size=intermediate_size, loads=tuple(loads))
    if hidden_size == 4096 and intermediate_size == 2048:
        # the real geometry: each expert is one contiguous record
        for x in plan.loads:
            if x.coded is None and (len(x.reads) != 1 or x.read_bytes != REAL_RECORD_BYTES):
                raise ContractError(f"layer {x.layer} expert {x.expert}: {len(x.reads)} reads "
                                    f"of {x.read_bytes} B, expected one {REAL_RECORD_BYTES}-B "
                                    "record")
    return plan
