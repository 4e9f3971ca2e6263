"""Checkpoint shards -> HBM expert banks.

The reference refills a bounded per-layer slot cache from SSD, one expert at a
time, on a route miss (``native_expert_ssd.py:280-387``: one direct reader per
shard, ``load_into(expert, slot, destinations)``).  Every expert of a layer is
resident in HBM here, so a layer is loaded once, in bulk:

1. the layer's per-expert read ranges (one contiguous record per expert in a
   native checkpoint) are sorted by shard offset and packed into staging
   chunks; ranges that follow each other in the file become one read;
2. ``glm_file_read_ranges`` preads a chunk into pinned host memory with a pool
   of native threads;
3. one host-to-device copy moves the chunk to device staging, and
   ``glm_bank_scatter`` moves every tensor of every record to its expert's
   slot in the stacked bank tensors.  Records of a ScaleX layer shard carry
   their scales coded (``scale_codec.py``): their weights are scattered the
   same way and ``glm_scalex_decode`` writes the decoded scales into the
   bank, once, at load time (the reference decodes them in every GEMV).

Three chunk buffers rotate, so the threads read chunks c + 1 and c + 2 while
the GPU copies and scatters chunk c; ``load_many`` streams several layers through one
pipeline, so it drains once, at the end.
"""

from __future__ import annotations

from dataclasses import dataclass
import os
import time

import numpy as np
import torch

from . import _native as N
from .contract import ContractError
from .bank_plan import BankPlan, slot_shape
from .expert_ssd import HBMExpertBank
from .scale_codec import A_ONE_BIT, A_RAW, A_TWO_BIT, ScaleCodecError, validate_mode_a
from .scalex_layer import RECORD_ORDER

_CODECS = {"raw": A_RAW, "one_bit": A_ONE_BIT, "two_bit": A_TWO_BIT}

_ALIGN = 256  # staging offset of every read: keeps 16-byte tensors 16-byte aligned


@dataclass(frozen=True)
class BankLoadStats:
    layers: tuple[int, ...]
    experts: int        # expert slots filled
    bytes: int          # payload bytes placed in the banks
    read_bytes: int     # bytes read from the shards
    reads: int          # pread ranges (after merging adjacent records)
    chunks: int
    seconds: float

    @property
    def gb_per_s(self) -> float:
        return self.bytes / self.seconds / 1e9 if self.seconds > 0 else float("inf")


@dataclass
class _Read:
    shard: str
    offset: int
    length: int
    staging: int


class ExpertBankLoader:
    """Loads whole layers of a :class:`BankPlan` into
    :class:`HBMExpertBank` objects.  The staging buffers (``buffers`` pinned
    host and device chunks of ``chunk_bytes``) are allocated on first use and kept
    for later layers; ``close()`` releases them."""

    def __init__(self, plan: BankPlan, *, threads: int = 16,
                 chunk_bytes: int = 64 << 20, drop_cache: bool = False, buffers: int = 3):
        if threads < 1:
            raise ContractError("the loader needs at least one read thread")
        if chunk_bytes < _ALIGN:
            raise ContractError(f"chunk_bytes must be at least {_ALIGN}")
        if buffers < 2:
            raise ContractError("the loader needs at least two staging buffers")
        self.nbuf = int(buffers)
        self.plan = plan
        self.threads = int(threads)
        largest = max((r.nbytes for x in plan.loads for r in x.reads), default=0)
        # a chunk holds at least the largest single read
        self.chunk_bytes = max(int(chunk_bytes), _round_up(largest, _ALIGN))
        self.flags = N.native.GLM_READ_DROP_CACHE if drop_cache else 0
        self._host: list[torch.Tensor] = []
        self._dev: list[torch.Tensor] = []
        self._tables: list[torch.Tensor] = []
        self._dtables: list[torch.Tensor] = []
        self._events: list[torch.cuda.Event | None] = []
        self._keep: list[object] = [None] * self.nbuf  # host tables in flight per buffer

    def _buffers(self, device: torch.device, segments: int) -> None:
        if not self._host or self._dev[0].device != device:
            self._host = [torch.empty(self.chunk_bytes, dtype=torch.uint8, pin_memory=True)
                          for _ in range(self.nbuf)]
            self._dev = [torch.empty(self.chunk_bytes, dtype=torch.uint8, device=device)
                         for _ in range(self.nbuf)]
            self._tables = []
            self._dtables = []
            self._events = [None] * self.nbuf
        if not self._tables or self._tables[0].numel() < 4 * segments:
            self._tables = [torch.empty(4 * max(segments, 64), dtype=torch.int64, device=device)
                            for _ in range(self.nbuf)]
        if not self._dtables or self._dtables[0].numel() < 13 * segments:
            self._dtables = [torch.empty(13 * max(segments, 64), dtype=torch.int64, device=device)
                             for _ in range(self.nbuf)]

    def close(self) -> None:
        for ev in self._events:
            if ev is not None:
                ev.synchronize()
        self._host, self._dev, self._tables, self._dtables, self._events = [], [], [], [], []
        self._keep = [None] * self.nbuf

    def _chunks(self, layer: int) -> list[list[tuple[object, object]]]:
        """The layer's (expert load, read) units in shard-offset order,
        packed into chunks of at most chunk_bytes staged bytes (one shard per
        chunk)."""
        units = [(x, rd) for x in self.plan.layer_loads(layer) for rd in x.reads]
        units.sort(key=lambda u: (u[1].shard, u[1].offset))
        chunks: list[list[tuple[object, object]]] = []
        used = 0
        for unit in units:
            rd = unit[1]
            size = _round_up(rd.nbytes, _ALIGN)
            if (not chunks or used + size > self.chunk_bytes
                    or chunks[-1][-1][1].shard != rd.shard):
                chunks.append([])
                used = 0
            chunks[-1].append(unit)
            used += size
        return chunks

    def _check(self, bank: HBMExpertBank, layer: int) -> None:
        plan = self.plan
        if bank.num_experts != plan.experts:
            raise ContractError(f"bank holds {bank.num_experts} experts, the plan {plan.experts}")
        if (bank.hidden_size, bank.intermediate_size) != (plan.hidden_size,
                                                          plan.intermediate_size):
            raise ContractError(f"bank geometry d {bank.hidden_size} I {bank.intermediate_size} "
                                f"differs from the plan's d {plan.hidden_size} "
                                f"I {plan.intermediate_size}")
        bank._require_active()
        for name, shape in bank.shapes().items():
            want = slot_shape(name, plan.hidden_size, plan.intermediate_size)
            if tuple(shape[1:]) != want:
                raise ContractError(f"bank tensor {name} has rows {shape[1:]}, expected {want}")
        plan.layer_loads(layer)  # the layer must be planned

    def load(self, bank: HBMExpertBank, layer: int | None = None) -> BankLoadStats:
        """Fills every expert slot of ``bank`` from layer ``layer`` (default:
        ``bank.layer``) of the plan; returns once the bank is complete."""
        return self.load_many([bank], None if layer is None else [layer])

    def load_many(self, banks, layers=None) -> BankLoadStats:
        """Fills each bank from its layer (default: each bank's ``layer``), all
        layers through one pipeline; returns once every bank is complete."""
        banks = list(banks)
        layers = [b.layer for b in banks] if layers is None else list(layers)
        if len(layers) != len(banks):
            raise ContractError("one layer per bank")
        if not banks:
            return BankLoadStats((), 0, 0, 0, 0, 0, 0.0)
        for bank, layer in zip(banks, layers):
            self._check(bank, layer)
        devices = {b.tensors[next(iter(b.shapes()))].device for b in banks}
        if len(devices) != 1:
            raise ContractError("the banks of one load_many call must share a device")
        (device,) = devices
        work = []  # (bank base pointers, slot bytes, chunk, tile_k per tensor)
        for bank, layer in zip(banks, layers):
            shapes = bank.shapes()
            slot_bytes = {name: int(np.prod(shape[1:])) for name, shape in shapes.items()}
            base = {name: bank.tensors[name].data_ptr() for name in shapes}
            # packed codes land in the bank layout: tile-major where the
            # geometry allows (glm_bank_scatter's tile_k = codes per row)
            tile_k = {name: (2 * shape[2] if name.endswith(".weight_packed")
                             and N.native.mxfp4_is_tiled(shape[1], 2 * shape[2]) else 0)
                      for name, shape in shapes.items()}
            work.extend((base, slot_bytes, chunk, tile_k) for chunk in self._chunks(layer))
        self._buffers(device, max(sum(len(r.segments) for _, r in c) for _, _, c, _ in work))
        stream = torch.cuda.current_stream(device)
        t0 = time.perf_counter()
        total = reads_total = 0
        for c, (base, slot_bytes, chunk, tile_k) in enumerate(work):
            slot = c % self.nbuf
            if self._events[slot] is not None:
                self._events[slot].synchronize()  # the buffers of chunk c - nbuf are free again
            # merge records that follow each other in the file into one read
            reads: list[_Read] = []
            segments: list[tuple[int, int, int, int]] = []
            coded: list[tuple[int, object]] = []  # (staging offset, ScaleX record)
            staged = 0
            for x, rd in chunk:
                expert = x.expert
                if reads and reads[-1].offset + reads[-1].length == rd.offset:
                    at = reads[-1].staging + reads[-1].length
                    reads[-1].length += rd.nbytes
                    staged = at + rd.nbytes
                else:
                    at = _round_up(staged, _ALIGN)
                    reads.append(_Read(rd.shard, rd.offset, rd.nbytes, at))
                    staged = at + rd.nbytes
                for seg in rd.segments:
                    if tile_k[seg.key] and seg.nbytes != slot_bytes[seg.key]:
                        raise AssertionError(f"{seg.key}: a tiled segment must be a whole matrix")
                    segments.append((at + seg.at, base[seg.key] + expert * slot_bytes[seg.key],
                                     seg.nbytes, tile_k[seg.key]))
                    total += seg.nbytes
                if x.coded is not None:
                    # a ScaleX record: its coded scales open the read
                    coded.append((at, x.coded, expert))
                    total += x.coded.decoded_bytes
            if staged > self.chunk_bytes:
                raise AssertionError("staging chunk overflow")
            host = self._host[slot]
            offsets = np.array([r.offset for r in reads], dtype=np.int64)
            lengths = np.array([r.length for r in reads], dtype=np.int64)
            dsts = (np.array([r.staging for r in reads], dtype=np.int64)
                    + host.data_ptr()).astype(np.uint64)
            path = os.fspath(self.plan.shard_path(reads[0].shard))
            N.call("glm_file_read_ranges", path.encode(), len(reads), offsets.ctypes.data,
                   lengths.ctypes.data, dsts.ctypes.data, self.threads, self.flags)
            reads_total += len(reads)
            decode = self._decode_rows(host, coded, base, slot_bytes)
            dev = self._dev[slot]
            dev[:staged].copy_(host[:staged], non_blocking=True)
            table = np.ascontiguousarray(np.array(segments, dtype=np.int64).reshape(-1, 4))
            N.call("glm_bank_scatter", stream.cuda_stream, dev.data_ptr(), staged,
                   table.ctypes.data, table.shape[0], self._tables[slot].data_ptr())
            if decode is not None:
                N.call("glm_scalex_decode", stream.cuda_stream, dev.data_ptr(), staged,
                       decode.ctypes.data, decode.shape[0], self._dtables[slot].data_ptr())
            ev = torch.cuda.Event()
            ev.record(stream)
            self._events[slot] = ev
            self._keep[slot] = (table, decode)
        for ev in self._events:
            if ev is not None:
                ev.synchronize()
        seconds = time.perf_counter() - t0
        read_bytes = sum(x.read_bytes for layer in layers for x in self.plan.layer_loads(layer))
        return BankLoadStats(layers=tuple(layers), experts=len(layers) * self.plan.experts,
                             bytes=total, read_bytes=read_bytes, reads=reads_total,
                             chunks=len(work), seconds=seconds)


    def _decode_rows(self, host: torch.Tensor, coded, base, slot_bytes):
        """The glm_scalex_decode table of a chunk's ScaleX records, each record
        checked on the host copy first (header, codec, primary length, ascending
        exception positions)."""
        if not coded:
            return None
        buf = host.numpy()
        rows = []
        for at, rec, expert in coded:
            try:
                info = validate_mode_a(buf[at:at + rec.coded_bytes])
            except ScaleCodecError as exc:
                raise ContractError(f"ScaleX record of expert {expert}: {exc}") from exc
            if info.raw_bytes != rec.decoded_bytes or info.codec != rec.codec:
                raise ContractError(f"expert {expert}'s coded scales are {info.codec} of "
                                    f"{info.raw_bytes} B, its record says {rec.codec} of "
                                    f"{rec.decoded_bytes} B")
            p = info.palette
            row = [at, rec.coded_bytes, rec.decoded_bytes, _CODECS[info.codec],
                   p[0] | (p[1] << 8) | (p[2] << 16) | (p[3] << 24), info.primary_bytes,
                   info.exceptions]
            for comp, n in zip(RECORD_ORDER, rec.scale_bytes):
                key = f"{comp}.weight_scale"
                if n != slot_bytes[key]:
                    raise ContractError(f"expert {expert}'s {key} holds {n} bytes, the bank "
                                        f"slot {slot_bytes[key]}")
                row += [base[key] + expert * slot_bytes[key], n]
            rows.append(row)
        return np.ascontiguousarray(np.array(rows, dtype=np.int64))


def _round_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


def load_layer_bank(plan: BankPlan, layer: int, *, swiglu_limit: float,
                    device: torch.device | str | None = None,
                    loader: ExpertBankLoader | None = None) -> HBMExpertBank:
    """A new :class:`HBMExpertBank` for ``layer`` filled from the checkpoint."""
    bank = HBMExpertBank(layer=layer, num_experts=plan.experts,
                         hidden_size=plan.hidden_size, intermediate_size=plan.intermediate_size,
                         swiglu_limit=swiglu_limit, device=device)
    own = loader is None
    loader = loader or ExpertBankLoader(plan)
    try:
        loader.load(bank)
    finally:
        if own:
            loader.close()
    return bank
