"""Benchmark of the MI355X routed-MoE layer (one GPU).

A step is one MoE layer forward over one batch of synthetic tokens whose
weights are already resident in HBM: router -> top-k -> MXFP4 gate/up + SwiGLU
-> down -> bf16 shared expert -> weighted combine (with T <= 4 tokens the layer
runs token-major in three kernels; larger batches add the dispatch).  Steps
rotate over several independent layer banks (>= 4 GB in total) and token
batches so that expert reads come from HBM rather than the 256 MB Infinity
Cache.  The timed steps run as one HIP graph, bracketed by synchronisation and
HIP events.

Prints one JSON line.  With the default workload (T=2, d=2048, E=128, top-8,
I=768) it carries the metric's three parts:
  * ``value``: the layer's tokens/s;
  * ``decode_expert_hbm_gbps``: the distinct selected experts' MXFP4 bytes of
    a step over the layer step's device time (its fraction of 8 TB/s beside
    it), and ``roofline``: the dominant kernel (the routed MXFP4 gate/up kernel,
    timed live with HIP events over a graph of back-to-back launches; its HBM
    traffic from two rocprofv3 counter passes, FETCH_SIZE then WRITE_SIZE,
    scaled by the same counters over a copy of known size);
  * ``mxfp4_mfma_util`` and ``prefill``: the 4096-token layer's grouped gate/up
    GEMM, algorithmic FLOPs per second over the 10.1 PFLOP/s dense MXFP4 peak,
    with the MFMA operations the rocprofv3 MOPS counters report beside it;
  * ``stack``: the 42-layer decode stack (MXFP8 resident linear + MoE layer per
    layer, one token per step, Markov routing) per step;
  * ``decode_t1`` and ``batch_t64``: the other decode configurations (one token
    of the small layer; 64 tokens with Zipf-skewed routing), each with its
    dominant kernel against the HBM roofline, the layer-level selected-expert
    GB/s and its own CPU baseline;
and the CPU baseline (the C restatement in oracle/, OpenMP, on this host) on a
bounded sample of the default workload, with the single-threaded numpy
oracle's rate beside it.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import shutil
import signal
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "src")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE layer tokens/s; decode expert HBM GB/s; MXFP4 MFMA util at T=4096"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "fp8": 5000.0, "fp4": 10100.0}  # MI355X dense
COPY_BYTES = 256 << 20  # counter calibration: one device copy of this size
ACT_NAMES = {0: "fp8x2", 1: "fp6x2", 2: "fp4", 3: "fp8fp6"}


def design_ceiling(act_format: int) -> float:
    """Algorithmic TFLOP/s the grouped GEMM's MFMAs allow in an activation
    format: FP8 x FP4 twice per product (hi, lo) at the FP8 rate, FP6 x FP4
    twice at the FP6 rate, FP4 x FP4 once, FP8 x FP4 (hi) + FP6 x FP4 (lo)."""
    fp8, fp4 = MFMA_PEAK_TFLOPS["fp8"], MFMA_PEAK_TFLOPS["fp4"]
    return {0: fp8 / 2, 1: fp4 / 2, 2: fp4, 3: 1.0 / (1.0 / fp8 + 1.0 / fp4)}[act_format]


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--workload", default="verify_t2",
                    help="decode_t1 | verify_t2 | batch_t64 | prefill_t4096 | stack42_t1 | "
                         "bank_load | dispatch_t4096")
    ap.add_argument("--min-rotation-gb", type=float, default=4.0,
                    help="total size of the distinct layer banks the steps rotate over")
    ap.add_argument("--kernel-launches", type=int, default=128)
    ap.add_argument("--legs", default="auto", choices=["auto", "none"],
                    help="auto: with the verify_t2 workload, also measure the 4096-token "
                         "prefill (MXFP4 MFMA utilisation) and the 42-layer decode stack")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="budget of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--traffic", type=int, default=1,
                    help="1: measure the dominant kernel's HBM traffic with rocprofv3 counters")
    ap.add_argument("--seed", type=int, default=5301)
    ap.add_argument("--act-format", default="fp8x2",
                    choices=["fp8x2", "fp6x2", "fp4", "fp8fp6"],
                    help="prefill: activation format of the timed grouped gate/up GEMM "
                         "(fp8x2: the exact split the layer uses; fp6x2, fp4, fp8fp6: the "
                         "lower-precision variants)")
    ap.add_argument("--load-layers", type=int, default=8,
                    help="bank_load: layers of the synthetic checkpoint (320 MB each)")
    ap.add_argument("--load-threads", type=int, default=16,
                    help="bank_load: native read threads")
    ap.add_argument("--scalex", type=int, default=0,
                    help="bank_load: 1 = ScaleX layer shards (coded scales, decoded on the GPU); "
                         "few-token workloads (T <= 4): 1 = the routed scales kept ScaleX "
                         "Mode-B coded in HBM with the checkpoint's statistics and decoded "
                         "inside the kernels (glm_moe_forward_scalex)")
    # internal: the child runs of the counter passes
    ap.add_argument("--mode", default="full", choices=["full", "kernel", "copy"],
                    help=argparse.SUPPRESS)
    return ap.parse_args()


class Setup:
    """Resident layer banks, token batches and per-launch routes of one workload."""

    def __init__(self, args, torch, np, workload: str, steps: int, warmup: int,
                 min_rotation_gb: float):
        from livglm_amd import native
        from livglm_amd.workloads import BANK_KEYS, SHAPES

        self.torch, self.np, self.native, self.keys = torch, np, native, BANK_KEYS
        self.lib = native.load()
        self.workload = workload
        self.shape = shape = SHAPES[workload]
        T, d, E, k, I, Is = shape.T, shape.d, shape.E, shape.k, shape.I, shape.I_shared
        self.T, self.d, self.E, self.k, self.I, self.Is = T, d, E, k, I, Is
        self.dev = dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        gen = torch.Generator(device=dev)
        gen.manual_seed(args.seed)
        self.layers = shape.layers
        self.layer_bytes = shape.bank_bytes + 3 * Is * d * 2 + E * d * 4
        if self.layers > 1:
            self.layer_bytes += d * d + d * d // 32  # the resident MXFP8 linear
        self.hc = hc = shape.hc
        if hc:
            self.layer_bytes += (2 * hc + hc * hc) * hc * d * 4 + d * 4  # fn + norm weight
        self.n_banks = max(2, self.layers, math.ceil(min_rotation_gb * 1e9 / self.layer_bytes))
        self.n_inputs = 64

        def randbytes(*s):
            return torch.randint(0, 256, s, dtype=torch.uint8, device=dev, generator=gen)

        def randscales(*s):
            return torch.randint(119, 128, s, dtype=torch.uint8, device=dev, generator=gen)

        def bf16(*s):
            return (torch.randn(s, device=dev, generator=gen) * 0.02).to(torch.bfloat16)

        self.banks = []
        for _ in range(self.n_banks):
            b = {
                "gate_proj.weight_packed": randbytes(E, I, d // 2),
                "gate_proj.weight_scale": randscales(E, I, d // 32),
                "up_proj.weight_packed": randbytes(E, I, d // 2),
                "up_proj.weight_scale": randscales(E, I, d // 32),
                "down_proj.weight_packed": randbytes(E, d, I // 2),
                "down_proj.weight_scale": randscales(E, d, I // 32),
                "router_weight": torch.randn((E, d), device=dev, generator=gen) * 0.02,
                "router_bias": torch.zeros(E, device=dev),
                "shared.gate": bf16(Is, d),
                "shared.up": bf16(Is, d),
                "shared.down": bf16(d, Is),
            }
            if shape.routing == "zipf":
                from livglm_amd.workloads import zipf_bias
                b["router_bias"] = torch.from_numpy(
                    zipf_bias(E, np.random.default_rng(args.seed + len(self.banks)))).to(dev)
            if hc:
                # the FFN site's hyper-connection weights and post-attention norm
                M = 2 * hc + hc * hc
                b["hc.fn"] = torch.randn((M, hc * d), device=dev, generator=gen) * 0.02
                b["hc.base"] = torch.randn(M, device=dev, generator=gen) * 0.5
                b["hc.scale"] = torch.rand(3, device=dev, generator=gen) + 0.5
                b["norm.weight"] = (1.0 + 0.1 * torch.randn(d, device=dev, generator=gen)).to(
                    torch.bfloat16).to(torch.float32)
            if self.layers > 1:
                # the resident linear as the reference builds it at start-up:
                # bf16 N(0, 0.02) quantised to MXFP8 (layers.py:72-99)
                w = bf16(d, d)
                b["linear.codes"] = torch.empty((d, d), dtype=torch.uint8, device=dev)
                b["linear.scales"] = torch.empty((d, d // 32), dtype=torch.uint8, device=dev)
                native.call("glm_mx_quantize", self.stream, w.data_ptr(), d, d,
                            native.GLM_FMT_MXFP8, native.GLM_MX_RULE_NEAREST,
                            b["linear.codes"].data_ptr(), b["linear.scales"].data_ptr())
                del w
                # the RMSNorm in front of it (bf16-representable weights around 1)
                b["linear.norm"] = (1.0 + 0.1 * torch.randn(d, device=dev, generator=gen)).to(
                    torch.bfloat16).to(torch.float32)
            self.banks.append(b)
        self.scalex = None
        if getattr(args, "scalex", 0) and T <= 4 and self.layers == 1 and not hc:
            self.scalex = self._code_scales(args, np)
        self.trace = None
        if shape.routing == "markov":
            # per (step, layer) bias rows that keep each expert of the previous
            # step with probability 0.7
            from livglm_amd.workloads import markov_bias_trace
            n = max(1, warmup + steps)
            self.trace = torch.from_numpy(markov_bias_trace(
                E, k, self.n_banks, n, np.random.default_rng(args.seed))).to(dev)
        self.xs = torch.randn((self.n_inputs, T, d), device=dev, generator=gen).to(torch.bfloat16)
        if hc:
            self.streams = torch.randn((self.n_inputs, T, hc, d), device=dev, generator=gen)
        # the layer's routed gate/up kernel: token-major for a few tokens, tiled
        # GEMV up to 64 tokens, grouped MFMA GEMMs beyond
        # the token-major and decode kernels cover d / 512 in {2, 4, 6, 8} and
        # I / 128 in {1, 2, 4, 6, 8, 16} chunks; other shapes run on the general
        # GEMV kernels
        self.decode_kernels = (d % 512 == 0 and d // 512 in (2, 4, 6, 8) and I % 128 == 0
                               and I // 128 in (1, 2, 4, 6, 8, 16))
        self.few_token = T <= 4 and k <= 8 and self.decode_kernels
        self.grouped = T > 64
        self.act_format = {"fp8x2": native.GLM_ACT_FP8X2, "fp6x2": native.GLM_ACT_FP6X2,
                           "fp4": native.GLM_ACT_FP4, "fp8fp6": native.GLM_ACT_FP8FP6}[
                               getattr(args, "act_format", "fp8x2")]

    def _code_scales(self, args, np) -> dict:
        """Replaces every bank's routed scales by ones with the real
        checkpoint's statistics and adds their ScaleX Mode-B rows
        (bank["scalex.rows"], one stride); returns the byte counts."""
        from glm53flash.scale_codec import mode_b_bank
        from livglm_amd.workloads import concentrated_scales
        torch, E, d, I = self.torch, self.E, self.d, self.I
        rng = np.random.default_rng(args.seed + 17)
        coded = stride = 0
        for b in self.banks:
            g = concentrated_scales(rng, (E, I, d // 32))
            dn = concentrated_scales(rng, (E, d, I // 32))
            u = concentrated_scales(rng, (E, I, d // 32))
            rows, st, c = mode_b_bank(g, dn, u)
            stride = max(stride, st)
            coded += c
            b["gate_proj.weight_scale"] = torch.from_numpy(g).to(self.dev)
            b["down_proj.weight_scale"] = torch.from_numpy(dn).to(self.dev)
            b["up_proj.weight_scale"] = torch.from_numpy(u).to(self.dev)
            b["scalex.rows"] = torch.from_numpy(rows).to(self.dev)
        for b in self.banks:  # one stride for every bank
            if b["scalex.rows"].shape[1] < stride:
                pad = torch.zeros((E, stride), dtype=torch.uint8, device=self.dev)
                pad[:, :b["scalex.rows"].shape[1]] = b["scalex.rows"]
                b["scalex.rows"] = pad
        raw = 3 * I * (d // 32)
        return {"stride": stride, "coded_bytes_per_expert": coded / len(self.banks) / E,
                "raw_scale_bytes_per_expert": raw,
                "expert_bytes_decoded": 3 * I * d // 2 + raw}

    def bias(self, step: int, layer: int):
        """The router bias of one layer at one step."""
        if self.trace is None:
            return self.banks[layer]["router_bias"]
        return self.trace[step % self.trace.shape[0], layer]

    @property
    def stream(self) -> int:
        """The current stream at call time (graph capture switches it)."""
        return self.torch.cuda.current_stream().cuda_stream

    # ------------------------------------------------------------ dominant kernel
    def kernel_plans(self, R: int) -> None:
        """Routes launch r's batch once (router, plus the dispatch where the
        kernel needs it)."""
        torch, native = self.torch, self.native
        T, d, E, k, P = self.T, self.d, self.E, self.k, self.T * self.k
        i32 = dict(dtype=torch.int32, device=self.dev)
        self.max_tiles = (P + 127) // 128 + E
        self.plans = []
        self.x_splits = {}
        for r in range(R):
            b, x = self.banks[r % self.n_banks], self.xs[r % self.n_inputs]
            pl = {"logits": torch.empty((T, E), dtype=torch.float32, device=self.dev),
                  "w": torch.empty((T, k), dtype=torch.float32, device=self.dev),
                  "ix": torch.empty((T, k), **i32),
                  "bias": self.bias(r // self.n_banks, r % self.n_banks)}
            native.call("glm_router_topk", self.stream, x.data_ptr(), T, d,
                        b["router_weight"].data_ptr(), pl["bias"].data_ptr(), E, k,
                        self.shape.n_group, self.shape.topk_group, 1,
                        self.shape.routed_scaling_factor, pl["logits"].data_ptr(),
                        pl["w"].data_ptr(), pl["ix"].data_ptr())
            if not self.few_token:
                pl.update({n: torch.empty(sz, **i32) for n, sz in
                           [("counts", E), ("offsets", E + 1), ("perm", P), ("inv", P),
                            ("tok", P), ("active", E), ("nact", 1), ("work", 4 * E),
                            ("status", 1)]})
                native.call("glm_moe_dispatch", self.stream, pl["ix"].data_ptr(), T, k, E,
                            *(pl[n].data_ptr() for n in ("counts", "offsets", "perm", "inv",
                                                          "tok", "active", "nact", "work",
                                                          "status")))
            if self.grouped:
                # the grouped GEMM reads the activations as their block-scaled
                # split (the exact FP8 split unless --act-format says otherwise)
                xi = r % self.n_inputs
                if xi not in self.x_splits:
                    buf = torch.empty(self.lib.glm_act_split_bytes_fmt(T, d, self.act_format),
                                      dtype=torch.uint8, device=self.dev)
                    native.call("glm_act_split", self.stream, x.data_ptr(), T, d,
                                self.act_format, buf.data_ptr())
                    self.x_splits[xi] = buf
                pl["tiles"] = torch.empty((self.max_tiles, 4), **i32)
                pl["ntiles"] = torch.empty(1, **i32)
                native.call("glm_moe_tiles", self.stream, pl["work"].data_ptr(), E,
                            pl["tiles"].data_ptr(), pl["ntiles"].data_ptr())
            self.plans.append(pl)
        torch.cuda.synchronize()
        self.unique = [len(self.np.unique(pl["ix"].cpu().numpy())) for pl in self.plans]
        self.h = torch.empty((P, self.I), dtype=torch.bfloat16, device=self.dev)
        self.w_k = torch.empty((T, k), dtype=torch.float32, device=self.dev)
        self.i_k = torch.empty((T, k), **i32)

    def gate_up(self, r: int) -> None:
        b, pl, x = self.banks[r % self.n_banks], self.plans[r], self.xs[r % self.n_inputs]
        sh, native = self.shape, self.native
        if self.grouped:
            native.call("glm_expert_gate_up_grouped_fmt", self.stream, self.act_format,
                        self.x_splits[r % self.n_inputs].data_ptr(), self.T, self.d, self.I,
                        *(b[key].data_ptr() for key in self.keys[:4]), pl["tok"].data_ptr(),
                        pl["tiles"].data_ptr(), pl["ntiles"].data_ptr(), self.max_tiles,
                        sh.swiglu_limit, self.h.data_ptr())
        elif self.few_token:
            native.call("glm_route_gate_up", self.stream, pl["logits"].data_ptr(),
                        pl["bias"].data_ptr(), self.T, self.E, self.k, sh.n_group,
                        sh.topk_group, 1, sh.routed_scaling_factor, x.data_ptr(), self.d, self.I,
                        *(b[key].data_ptr() for key in self.keys[:4]), sh.swiglu_limit,
                        self.w_k.data_ptr(), self.i_k.data_ptr(), self.h.data_ptr())
        else:
            native.call("glm_expert_gate_up", self.stream, x.data_ptr(), self.T, self.d, self.I,
                        self.E, self.k, *(b[key].data_ptr() for key in self.keys[:4]),
                        pl["tok"].data_ptr(), pl["work"].data_ptr(), sh.swiglu_limit,
                        self.h.data_ptr())

    def kernel_name(self) -> str:
        """The dominant kernel's instantiation, as rocprofv3 names it."""
        d, E = self.d, self.E
        if self.grouped:
            return f"grouped_f8f6f4_w8_kernel<2, {self.act_format}>"
        if self.few_token:
            epl = 2 if E <= 128 else (4 if E <= 256 else (5 if E <= 320 else 8))
            return f"select_gate_up_kernel<{epl}, {d // 512}, 1, false>"
        if not self.decode_kernels:
            return "mx_gemv_kernel"
        return f"decode_gate_up_kernel<{d // 512}>"

    def kernel_flops(self) -> int:
        """Algorithmic FLOPs of one grouped gate/up launch: two projections of
        every (token, expert) pair, 2 * d * I each."""
        return 2 * 2 * self.T * self.k * self.d * self.I

    def kernel_bytes(self, r: int) -> int:
        """Algorithmic bytes of launch r: the codes and E8M0 scales of the
        gate and up projections of every distinct routed expert, once."""
        proj = self.I * self.d // 2 + self.I * self.d // 32
        return self.unique[r] * 2 * proj


def measure(args, torch, np, workload: str, *, steps: int, warmup: int, traffic: bool,
            cpu_seconds: float, kernel_launches: int, min_rotation_gb: float) -> dict:
    """One workload: the timed layer steps (one HIP graph, or one per decode step
    for the layer stack), the dominant kernel live with HIP events, optionally
    its HBM traffic (counter passes) and the CPU baseline.  Frees its device
    memory before returning."""
    S = Setup(args, torch, np, workload, steps, warmup, min_rotation_gb)
    R = kernel_launches
    S.kernel_plans(R)
    native, keys = S.native, S.keys
    T, d, E, k, I, Is, shape = S.T, S.d, S.E, S.k, S.I, S.Is, S.shape
    ws_bytes = S.lib.glm_moe_workspace_bytes(T, d, E, k, I, Is)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=S.dev)
    native.call("glm_moe_workspace_init", S.stream, ws.data_ptr(), ws_bytes)
    out = torch.empty((T, d), dtype=torch.float32, device=S.dev)
    wts = torch.empty((T, k), dtype=torch.float32, device=S.dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=S.dev)

    def moe(x, layer: int, step: int) -> None:
        b = S.banks[layer]
        if S.scalex is not None:
            native.call(
                "glm_moe_forward_scalex", S.stream, x.data_ptr(), T, d,
                b["router_weight"].data_ptr(), S.bias(step, layer).data_ptr(), E, k,
                shape.n_group, shape.topk_group, int(shape.norm_topk_prob),
                shape.routed_scaling_factor, I, b["gate_proj.weight_packed"].data_ptr(),
                b["up_proj.weight_packed"].data_ptr(), b["down_proj.weight_packed"].data_ptr(),
                b["scalex.rows"].data_ptr(), S.scalex["stride"], Is, native.GLM_FMT_BF16,
                b["shared.gate"].data_ptr(), None, b["shared.up"].data_ptr(), None,
                b["shared.down"].data_ptr(), None, None, shape.swiglu_limit, ws.data_ptr(),
                ws_bytes, out.data_ptr(), wts.data_ptr(), idx.data_ptr())
            return
        native.call(
            "glm_moe_forward", S.stream, x.data_ptr(), T, d, b["router_weight"].data_ptr(),
            S.bias(step, layer).data_ptr(), E, k, shape.n_group, shape.topk_group,
            int(shape.norm_topk_prob), shape.routed_scaling_factor, I,
            *(b[key].data_ptr() for key in keys), Is, native.GLM_FMT_BF16,
            b["shared.gate"].data_ptr(), None, b["shared.up"].data_ptr(), None,
            b["shared.down"].data_ptr(), None, None, shape.swiglu_limit, ws.data_ptr(), ws_bytes,
            out.data_ptr(), wts.data_ptr(), idx.data_ptr())

    def layer_step(s: int) -> None:
        moe(S.xs[s % S.n_inputs], s % S.n_banks, s)

    if S.hc:
        # the decoder FFN site: hyper-connection + post-attention norm (one call,
        # bf16 output), the MoE layer on it, hyper_residual
        hc = S.hc
        hc_ws_bytes = S.lib.glm_hc_workspace_bytes(T, hc, d)
        hc_ws = torch.empty(max(hc_ws_bytes, 256), dtype=torch.uint8, device=S.dev)
        post = torch.empty((T, hc), dtype=torch.float32, device=S.dev)
        comb = torch.empty((T, hc, hc), dtype=torch.float32, device=S.dev)
        normed = torch.empty((T, d), dtype=torch.bfloat16, device=S.dev)
        site_out = torch.empty((T, hc, d), dtype=torch.float32, device=S.dev)

        def layer_step(s: int) -> None:  # noqa: F811 -- the FFN site replaces the bare layer
            b = S.banks[s % S.n_banks]
            streams = S.streams[s % S.n_inputs]
            native.call("glm_hc_pre", S.stream, streams.data_ptr(), T, hc, d,
                        b["hc.fn"].data_ptr(), b["hc.base"].data_ptr(), b["hc.scale"].data_ptr(),
                        20, 1e-6, 1e-6, b["norm.weight"].data_ptr(), 1e-6, 0, hc_ws.data_ptr(),
                        hc_ws.numel(), post.data_ptr(), comb.data_ptr(), None, normed.data_ptr())
            # the MoE layer with hyper_residual in its last kernel
            lb = s % S.n_banks
            native.call(
                "glm_moe_forward_hc", S.stream, normed.data_ptr(), T, d,
                b["router_weight"].data_ptr(), S.bias(s, lb).data_ptr(), E, k, shape.n_group,
                shape.topk_group, int(shape.norm_topk_prob), shape.routed_scaling_factor, I,
                *(b[key].data_ptr() for key in keys), Is, native.GLM_FMT_BF16,
                b["shared.gate"].data_ptr(), None, b["shared.up"].data_ptr(), None,
                b["shared.down"].data_ptr(), None, None, shape.swiglu_limit, ws.data_ptr(),
                ws_bytes, out.data_ptr(), wts.data_ptr(), idx.data_ptr(), streams.data_ptr(), hc,
                post.data_ptr(), comb.data_ptr(), 0, site_out.data_ptr())

    act = torch.empty((T, d), dtype=torch.bfloat16, device=S.dev)

    def stack_step(s: int) -> None:
        """One decode step through the layer stack: per layer the resident
        MXFP8 linear, then the MoE layer on its output.  The next layer reads
        the f32 MoE output through an RMSNorm fused into its linear (the
        decoder's norm in front of each block; the residual stream is not part
        of this path)."""
        x = S.xs[s % S.n_inputs]
        for layer in range(S.layers):
            b = S.banks[layer]
            if layer == 0:
                native.call("glm_linear", S.stream, x.data_ptr(), T, d,
                            b["linear.codes"].data_ptr(), b["linear.scales"].data_ptr(),
                            native.GLM_FMT_MXFP8, d, act.data_ptr())
            else:
                native.call("glm_rms_norm_linear", S.stream, out.data_ptr(), T, d,
                            b["linear.norm"].data_ptr(), 1e-6, b["linear.codes"].data_ptr(),
                            b["linear.scales"].data_ptr(), native.GLM_FMT_MXFP8, d,
                            act.data_ptr())
            moe(act, layer, s)

    def capture(fn, first: int, count: int):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for s in range(first, first + count):
                fn(s)
        return g

    def timed(g, count: int):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        wall0 = time.perf_counter()
        ev0.record()
        g.replay()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / count, time.perf_counter() - wall0

    # ------------------------------------------------------------ timed steps
    unique_per_step = None
    if S.layers > 1:
        stack_step(0)  # eager pass (validates the launches outside capture)
        torch.cuda.synchronize()
        # one graph per decode step (each step has its own routing biases)
        graphs = [capture(stack_step, s, 1) for s in range(warmup + steps)]
        for g in graphs[:warmup]:
            g.replay()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        wall0 = time.perf_counter()
        ev0.record()
        for g in graphs[warmup:]:
            g.replay()
        ev1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        ms_per_step = ev0.elapsed_time(ev1) / steps
        del graphs
    else:
        for s in range(S.n_banks):  # eager pass over every bank first
            layer_step(s)
        torch.cuda.synchronize()
        # the distinct experts each timed step routes to (an eager run of the
        # same steps: same banks, inputs and biases)
        unique_per_step = []
        for s in range(warmup, warmup + steps):
            layer_step(s)
            unique_per_step.append(len(np.unique(idx.cpu().numpy())))
        if warmup > 0:
            capture(layer_step, 0, warmup).replay()
        ms_per_step, wall = timed(capture(layer_step, warmup, steps), steps)
    tokens_per_s = T / (ms_per_step / 1e3)

    # ------------------------------------------------------------ dominant kernel
    gk = capture(S.gate_up, 0, R)
    gk.replay()
    k_ms, _ = timed(gk, R)
    bytes_per_launch = sum(S.kernel_bytes(r) for r in range(R)) / R
    achieved = bytes_per_launch / (k_ms / 1e3) / 1e9
    tflops = S.kernel_flops() / (k_ms / 1e3) / 1e12
    del gk
    torch.cuda.synchronize()

    traffic_v, traffic_note = None, "not measured (--traffic 0)"
    if traffic:
        traffic_v, traffic_note = measure_traffic(args, workload, S.kernel_name())

    cpu = None
    if cpu_seconds > 0:
        cpu = cpu_baseline(shape, S.banks[0], S.xs, cpu_seconds,
                           None if S.trace is None else S.trace[0, 0],
                           S.streams if S.hc else None)

    res = {
        "workload": workload, "shape": shape, "tokens_per_s": tokens_per_s,
        "ms_per_step": ms_per_step, "wall": wall, "grouped": S.grouped, "few_token": S.few_token,
        "layers": S.layers, "hc": S.hc, "n_banks": S.n_banks,
        "rotation_bytes": S.n_banks * S.layer_bytes, "kernel_name": S.kernel_name(),
        "roofline": roofline(S, achieved, tflops, bytes_per_launch, k_ms, R, traffic_v,
                             traffic_note),
        "kernel_tflops": tflops, "kernel_ms": k_ms, "kernel_flops": S.kernel_flops(),
        "act_format": S.act_format,
        "cpu": cpu,
    }
    if unique_per_step and not S.grouped:
        # the layer-level decode rate: the selected experts' bytes of a step
        # over the whole step's device time (router -> gate/up -> down ->
        # combine, shared expert included)
        u = sum(unique_per_step) / len(unique_per_step)
        res["unique_experts_per_step"] = u
        res["layer_expert_gbps"] = u * shape.expert_bytes / (ms_per_step / 1e3) / 1e9
        if S.scalex is not None:
            # the same experts with their scales read as ScaleX Mode-B rows:
            # a step moves each selected expert's codes and its coded row
            sx = S.scalex
            coded_expert = sx["expert_bytes_decoded"] - sx["raw_scale_bytes_per_expert"] + \
                sx["coded_bytes_per_expert"]
            res["scalex"] = {
                "mode": "ScaleX Mode-B rows decoded inside select_gate_up / down_combine",
                "row_stride": sx["stride"],
                "coded_scale_bytes_per_expert": round(sx["coded_bytes_per_expert"]),
                "raw_scale_bytes_per_expert": sx["raw_scale_bytes_per_expert"],
                "expert_bytes_coded": round(coded_expert),
                "expert_bytes_decoded": sx["expert_bytes_decoded"],
                "expert_bytes_saved_frac": round(1 - coded_expert / sx["expert_bytes_decoded"], 4),
                "coded_expert_gbps": round(u * coded_expert / (ms_per_step / 1e3) / 1e9, 1),
            }
    if S.layers > 1:
        # bytes one decode step reads: every layer's k experts (Markov
        # routing at T=1 picks k distinct ones), shared expert, linear, router
        expert = S.layers * k * shape.expert_bytes
        other = S.layers * (3 * Is * d * 2 + d * d + d * d // 32 + d * 4 + E * d * 4)
        sec = ms_per_step / 1e3
        res["stack"] = {"layers": S.layers,
                        "us_per_layer": round(ms_per_step * 1e3 / S.layers, 3),
                        "expert_bytes_per_step": expert, "all_bytes_per_step": expert + other,
                        "expert_hbm_gbps": round(expert / sec / 1e9, 1),
                        "expert_hbm_frac": round(expert / sec / 1e9 / HBM_PEAK_GBPS, 4),
                        "all_hbm_gbps": round((expert + other) / sec / 1e9, 1)}
    del S, ws, out, wts, idx, act
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def describe(r: dict) -> str:
    """The workload's configuration in words."""
    sh, T = r["shape"], r["shape"].T
    if r["hc"]:
        return (f"{sh.name}: decoder FFN site, hyper-connection of {r['hc']} f32 residual "
                f"streams (20 Sinkhorn rounds) + RMSNorm + MoE layer T={T} d={sh.d} E={sh.E} "
                f"top-{sh.k} I={sh.I} (MXFP4 group-32 experts, bf16 shared expert "
                f"I={sh.I_shared}) + hyper_residual")
    if r["layers"] > 1:
        return (f"{sh.name}: {r['layers']} layers x (RMSNorm + MXFP8 {sh.d}x{sh.d} resident "
                f"linear + MoE layer T={T} d={sh.d} E={sh.E} top-{sh.k} I={sh.I}, MXFP4 group-32 "
                f"experts, bf16 shared expert I={sh.I_shared}), Markov routing keeping 70% of the "
                f"previous step's experts, one token per step")
    return (f"{sh.name}: MoE layer T={T} d={sh.d} E={sh.E} top-{sh.k} I={sh.I} "
            f"(MXFP4 group-32 experts, bf16 shared expert I={sh.I_shared})")


def prefill_leg(r: dict, counters: dict | None) -> dict:
    """The metric's third part: the T=4096 grouped gate/up GEMM's MXFP4 MFMA
    utilisation -- algorithmic FLOPs (two projections x 2 d I per (token,
    expert) pair) per second over the 10.1 PFLOP/s dense FP4 peak, and the
    executed MFMA operations the counters report over the same launches."""
    peak = MFMA_PEAK_TFLOPS["fp4"]
    alg = r["kernel_tflops"]
    leg = {
        "workload": describe(r), "tokens_per_s": round(r["tokens_per_s"], 1),
        "ms_per_step": round(r["ms_per_step"], 5), "kernel": r["kernel_name"],
        "avg_launch_us": round(r["kernel_ms"] * 1e3, 3),
        "algorithmic_flops_per_launch": r["kernel_flops"],
        "algorithmic_tflops": round(alg, 1), "fp4_peak_tflops": peak,
        "mxfp4_mfma_util": round(alg / peak, 4),
        # the exact split issues two FP8 x FP4 MFMAs (x's hi and lo parts) per
        # product at the 5.0 PFLOP/s FP8 rate: 2.5 PFLOP/s of algorithmic work
        # at most (FP6 split: 5.05, FP4: 10.1)
        "act_format": ACT_NAMES[r["act_format"]],
        "design_ceiling_tflops": design_ceiling(r["act_format"]),
        "frac_of_design_ceiling": round(alg / design_ceiling(r["act_format"]), 4),
    }
    if counters:
        leg["counters"] = counters
        ex = counters.get("executed_flops_per_launch")
        if ex:
            ex_tf = ex / (r["kernel_ms"] / 1e3) / 1e12
            leg["executed_tflops"] = round(ex_tf, 1)
            leg["executed_frac_of_fp4_peak"] = round(ex_tf / peak, 4)
            leg["executed_frac_of_fp8_peak"] = round(ex_tf / MFMA_PEAK_TFLOPS["fp8"], 4)
    return leg


def decode_leg(r: dict) -> dict:
    """A decode configuration's figures: the layer's tokens/s, the dominant
    routed gate/up kernel against the HBM roofline (HIP events over a graph
    of its launches), the selected experts' bytes over the layer step's device
    time, and the C restatement on this host's cores."""
    leg = {"workload": describe(r), "tokens_per_s": round(r["tokens_per_s"], 1),
           "ms_per_step": round(r["ms_per_step"], 5), "roofline": r["roofline"]}
    if "layer_expert_gbps" in r:
        leg["decode_expert_hbm_gbps"] = round(r["layer_expert_gbps"], 1)
        leg["decode_expert_hbm_frac"] = round(r["layer_expert_gbps"] / HBM_PEAK_GBPS, 4)
        leg["decode_unique_experts_per_step"] = round(r["unique_experts_per_step"], 2)
    leg["cpu_baseline"] = r["cpu"]
    return leg


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs the MoE layer on one GPU; runs over "
                                   "several GPUs (the layer sharded by expert) are not supported",
                          "n_gpus": args.gpus}))
        return 2

    import numpy as np
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    if args.mode == "copy":
        return copy_probe(torch)
    if args.workload == "bank_load":
        return bank_load_bench(args, torch, np)
    if args.workload == "dispatch_t4096":
        return dispatch_bench(args, torch, np)
    if args.mode == "kernel":
        S = Setup(args, torch, np, args.workload, args.steps, args.warmup, args.min_rotation_gb)
        S.kernel_plans(args.kernel_launches)
        for r in range(args.kernel_launches):
            S.gate_up(r)
        torch.cuda.synchronize()
        return 0

    r = measure(args, torch, np, args.workload, steps=args.steps, warmup=args.warmup,
                traffic=bool(args.traffic), cpu_seconds=args.cpu_seconds,
                kernel_launches=args.kernel_launches, min_rotation_gb=args.min_rotation_gb)
    legs = args.legs == "auto" and args.workload == "verify_t2"
    line = {
        "metric": METRIC,
        "value": round(r["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": describe(r),
            "tokens_per_step": r["shape"].T, "weights": "mxfp4-e2m1+e8m0",
            "mfma": ("fp8 hi/lo split x mxfp4, block-scaled" if r["grouped"]
                     else "bf16 x dequantised mxfp4"), "layer_banks": r["n_banks"],
            "rotation_bytes": r["rotation_bytes"], "graph_steps": args.steps,
            "wall_s": round(r["wall"], 4),
        },
        "roofline": r["roofline"],
    }
    if "scalex" in r:
        line["scalex"] = r["scalex"]
    if "layer_expert_gbps" in r:
        # selected-expert bytes over the layer step's whole device time
        line["decode_expert_hbm_gbps"] = round(r["layer_expert_gbps"], 1)
        line["decode_expert_hbm_frac"] = round(r["layer_expert_gbps"] / HBM_PEAK_GBPS, 4)
        line["decode_unique_experts_per_step"] = round(r["unique_experts_per_step"], 2)
    if r["grouped"]:
        line["prefill"] = prefill_leg(r, mfma_counters(args, r["workload"], r["kernel_name"])
                                      if args.traffic else None)
        line["mxfp4_mfma_util"] = line["prefill"]["mxfp4_mfma_util"]
    if "stack" in r:
        line["stack"] = r["stack"]
    if legs:
        # the metric's other parts in the same run: the T=4096 prefill layer
        # (MXFP4 MFMA utilisation of its grouped GEMM) and the 42-layer decode
        # stack, each on its own banks
        pf = measure(args, torch, np, "prefill_t4096", steps=args.steps, warmup=args.warmup,
                     traffic=False, cpu_seconds=0.0, kernel_launches=32, min_rotation_gb=0.0)
        line["prefill"] = prefill_leg(pf, mfma_counters(args, "prefill_t4096", pf["kernel_name"])
                                      if args.traffic else None)
        line["mxfp4_mfma_util"] = line["prefill"]["mxfp4_mfma_util"]
        st = measure(args, torch, np, "stack42_t1", steps=args.steps, warmup=args.warmup,
                     traffic=False, cpu_seconds=0.0, kernel_launches=64, min_rotation_gb=0.0)
        line["stack"] = {"workload": describe(st), "tokens_per_s": round(st["tokens_per_s"], 1),
                         "ms_per_step": round(st["ms_per_step"], 5), **st["stack"]}
        # the other decode configurations: one token of the small layer (banks
        # of 16 MB rotating over >= 1 GB, four times the memory-side cache) and
        # 64 tokens with Zipf-skewed routing (as many banks as the default
        # workload's rotation), each on its own banks
        cpu_leg = min(3.0, args.cpu_seconds)
        for name, rot in (("decode_t1", 1.0), ("batch_t64", args.min_rotation_gb)):
            line[name] = decode_leg(measure(
                args, torch, np, name, steps=args.steps, warmup=args.warmup, traffic=False,
                cpu_seconds=cpu_leg, kernel_launches=64, min_rotation_gb=rot))
    line["cpu_baseline"] = r["cpu"]
    if legs and args.cpu_seconds > 0:
        line["cpu_baseline"]["numpy_1thread"] = cpu_baseline_numpy(
            r["shape"], args.seed, min(3.0, args.cpu_seconds))
    print(json.dumps(line))
    return 0


def roofline(S, achieved, tflops, bytes_per_launch, k_ms, R, traffic, traffic_note):
    """The dominant kernel against its bound: HBM for the decode GEMVs, the
    dense MXFP4 MFMA peak for the grouped prefill GEMM."""
    common = {"traffic": traffic, "traffic_note": traffic_note,
              "bytes_per_launch": round(bytes_per_launch), "avg_launch_us": round(k_ms * 1e3, 3),
              "launches": R, "unique_experts_per_launch": round(sum(S.unique) / R, 2)}
    if S.grouped:
        # algorithmic FLOPs over the 10.1 PFLOP/s dense MXFP4 peak; the kernel
        # runs block-scaled MFMAs on a split of the activations: two FP8 x FP4
        # per product at the 5.0 PFLOP/s FP8 rate for the exact split (a
        # ceiling of 2.5 PFLOP/s of algorithmic work, reported beside it), two
        # at the FP6 rate for the FP6 split, one at the FP4 rate for FP4
        ceiling = design_ceiling(S.act_format)
        return {"kernel": S.kernel_name() + " (grouped MXFP4 gate/up + SwiGLU GEMMs, block-scaled "
                                            f"MFMA on the {ACT_NAMES[S.act_format]} split of x)",
                "bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS["fp4"],
                "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS["fp4"], 4),
                "flops_per_launch": S.kernel_flops(),
                "design_ceiling": ceiling,
                "frac_of_design_ceiling": round(tflops / ceiling, 4),
                **common}
    return {"kernel": S.kernel_name() + (" (few-token selection + routed MXFP4 gate/up + SwiGLU)"
                                         if S.few_token else
                                         " (routed MXFP4 gate/up + SwiGLU)"),
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), **common}


def bank_load_bench(args, torch, np) -> int:
    """Checkpoint shards -> HBM banks: writes a synthetic routed-expert
    checkpoint at the verify_t2 geometry (one 320 MB shard per layer), then
    loads every layer into its own HBM bank twice -- from the page cache
    (``value``) and after the shards' pages were dropped (``cold_gbps``, the
    storage's rate).  The device side's kernel, the scatter of staged records
    into the bank tensors, is timed with HIP events on its stream."""
    from glm53flash.bank_loader import ExpertBankLoader
    from glm53flash.bank_plan import plan_expert_banks
    from glm53flash.checkpoint import ShardIndex
    from glm53flash.expert_ssd import HBMExpertBank
    from livglm_amd import native
    from livglm_amd.workloads import SHAPES, write_expert_checkpoint

    shape = SHAPES["verify_t2"]
    layers = list(range(3, 3 + max(1, args.load_layers)))
    chunk = 64 << 20
    root = tempfile.mkdtemp(prefix="glm_ckpt_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        t0 = time.perf_counter()
        payload = write_expert_checkpoint(root, shape, layers, args.seed,
                                          two_value_scales=bool(args.scalex))
        if args.scalex:
            from livglm_amd.workloads import write_scalex_layer
            for layer in layers:
                shard = os.path.join(root, f"model-layer{layer:02d}.safetensors")
                write_scalex_layer(shard, shard + ".sx", layer=layer, experts=shape.E)
                os.replace(shard + ".sx", shard)
        print(f"bank_load: wrote {payload / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s",
              file=sys.stderr, flush=True)
        plan = plan_expert_banks(ShardIndex.open(root), hidden_size=shape.d,
                                 intermediate_size=shape.I, experts=shape.E, layers=layers)
        banks = [HBMExpertBank(layer=l, num_experts=shape.E, hidden_size=shape.d,
                               intermediate_size=shape.I, swiglu_limit=shape.swiglu_limit,
                               device="cuda") for l in layers]
        loader = ExpertBankLoader(plan, threads=args.load_threads, chunk_bytes=chunk)
        loader.load(banks[0])  # staging allocation, first touch of the banks

        def load_all():
            torch.cuda.synchronize()
            t = time.perf_counter()
            stats = loader.load_many(banks)
            torch.cuda.synchronize()
            return time.perf_counter() - t, stats

        warm_s, stats = load_all()
        print(f"bank_load: page cache -> HBM {payload / warm_s / 1e9:.2f} GB/s", file=sys.stderr,
              flush=True)
        shards = list(plan.shards)

        def drop_pages():
            for shard in shards:
                fd = os.open(os.path.join(root, shard), os.O_RDONLY)
                try:
                    os.fsync(fd)
                    os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
                finally:
                    os.close(fd)

        for b in banks:  # the cold pass must refill, not find the right bytes already there
            for t in b.tensors.values():
                t.zero_()
        drop_pages()
        cold_s, _ = load_all()
        print(f"bank_load: storage -> HBM {payload / cold_s / 1e9:.2f} GB/s", file=sys.stderr,
              flush=True)
        # every slot of the first and the last layer against the shard bytes
        # (a ScaleX shard: against the tensors its reader rebuilds)
        if args.scalex:
            from glm53flash.bank_plan import BANK_KEYS, expert_tensor_name
            from glm53flash.scalex_layer import ScaleXLayer
            checked = 0
            for b in (banks[0], banks[-1]):
                layout = ScaleXLayer.read(os.path.join(root, shards[0 if b is banks[0] else -1]))
                for e in (0, shape.E // 2, shape.E - 1):
                    for key in BANK_KEYS:
                        tname = expert_tensor_name(b.layer, e, *key.split("."))
                        want = np.frombuffer(layout.tensor_bytes(tname), np.uint8)
                        if key.endswith(".weight_packed"):  # the bank layout of the codes
                            want = native.mxfp4_tile_host(
                                want.reshape(b.tensors[key].shape[1:])).reshape(-1)
                        got = b.tensors[key][e].cpu().numpy().reshape(-1)
                        if not np.array_equal(got, want):
                            raise SystemExit(f"bank_load: layer {b.layer} {tname} differs")
                        checked += want.size
        else:
            first = plan.expert(layers[0], 0).reads[0]
            blob = np.fromfile(os.path.join(root, shards[0]), dtype=np.uint8,
                               offset=first.offset)
            blob = blob[:shape.E * shape.expert_bytes].reshape(shape.E, shape.expert_bytes)
            checked = 0
            for b in (banks[0], banks[-1]):
                # every layer stores the same bank, expert records back to back
                for seg in first.segments:
                    want = blob[:, seg.at:seg.at + seg.nbytes]
                    if seg.key.endswith(".weight_packed"):  # the bank layout of the codes
                        want = native.mxfp4_tile_host(
                            want.reshape(b.tensors[seg.key].shape)).reshape(shape.E, -1)
                    got = b.tensors[seg.key].cpu().numpy().reshape(shape.E, -1)
                    if not np.array_equal(got, want):
                        raise SystemExit(f"bank_load: layer {b.layer} {seg.key} differs")
                    checked += want.size
        # host side alone: the native reader into pinned memory
        host = torch.empty(chunk, dtype=torch.uint8, pin_memory=True)
        rng0 = plan.expert(layers[0], 0).reads[0].offset
        n_read = min(chunk, shape.E * shape.expert_bytes)
        offs = np.array([rng0], dtype=np.int64)
        lens = np.array([n_read], dtype=np.int64)
        ptrs = np.array([host.data_ptr()], dtype=np.uint64)
        path = os.path.join(root, shards[0]).encode()
        native.call("glm_file_read_ranges", path, 1, offs.ctypes.data, lens.ctypes.data,
                    ptrs.ctypes.data, args.load_threads, 0)
        t = time.perf_counter()
        for _ in range(4):
            native.call("glm_file_read_ranges", path, 1, offs.ctypes.data, lens.ctypes.data,
                        ptrs.ctypes.data, args.load_threads, 0)
        read_gbps = 4 * n_read / (time.perf_counter() - t) / 1e9
        # host -> device link: pinned staging to device staging
        dev = torch.empty(chunk, dtype=torch.uint8, device="cuda")
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        dev.copy_(host, non_blocking=True)
        e0.record(stream)
        for _ in range(4):
            dev.copy_(host, non_blocking=True)
        e1.record(stream)
        e1.synchronize()
        h2d_gbps = 4 * chunk / (e0.elapsed_time(e1) / 1e3) / 1e9
        # the scatter kernel alone: the experts of one staged chunk into bank
        # 0, 8 launches between HIP events
        n_exp = min(shape.E, chunk // shape.expert_bytes)
        segs = []  # records staged back to back in the checkpoint's tensor order
        for e in range(n_exp):
            rel = e * shape.expert_bytes
            for key, bank_t in banks[0].tensors.items():
                n_slot = bank_t.numel() // shape.E
                # packed codes land tile-major (the bank layout), as the loader writes them
                tk = (2 * bank_t.shape[2] if key.endswith(".weight_packed")
                      and native.mxfp4_is_tiled(bank_t.shape[1], 2 * bank_t.shape[2]) else 0)
                segs.append((rel, bank_t.data_ptr() + e * n_slot, n_slot, tk))
                rel += n_slot
        table = np.array(segs, dtype=np.int64)
        dtab = torch.empty(table.size, dtype=torch.int64, device="cuda")
        staged = n_exp * shape.expert_bytes
        args_s = (stream.cuda_stream, dev.data_ptr(), staged, table.ctypes.data, len(segs),
                  dtab.data_ptr())
        native.call("glm_bank_scatter", *args_s)
        e0.record(stream)
        launches = 8
        for _ in range(launches):
            native.call("glm_bank_scatter", *args_s)
        e1.record(stream)
        e1.synchronize()
        k_s = e0.elapsed_time(e1) / 1e3 / launches
        moved = 2 * staged  # each byte read once and written once
        achieved = moved / k_s / 1e9
        loader.close()
    finally:
        shutil.rmtree(root, ignore_errors=True)
    line = {
        "metric": "expert bank load GB/s (checkpoint shards -> HBM-resident expert banks)",
        "value": round(payload / warm_s / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": len(layers),
        "warmup": 1,
        "ms_per_step": round(warm_s * 1e3 / len(layers), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": (f"bank_load: {len(layers)} layers x {shape.E} experts x "
                         f"{shape.expert_bytes} B (MXFP4 d={shape.d} I={shape.I}), one "
                         + ("ScaleX layer shard per layer (scales coded, decoded on the GPU)"
                            if args.scalex else "safetensors shard per layer")
                         + ", read from the page cache"),
            "read_bytes": stats.read_bytes,
            "payload_bytes": payload, "read_threads": args.load_threads, "chunk_bytes": chunk,
            "reads": stats.reads, "chunks": stats.chunks,
            "verified_bytes": checked,
        },
        "cold_gbps": round(payload / cold_s / 1e9, 3),
        "host_read_gbps": round(read_gbps, 3),
        "h2d_gbps": round(h2d_gbps, 3),
        "roofline": {"kernel": "bank_scatter_kernel (staged records -> bank slots)",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_launch": moved, "avg_launch_us": round(k_s * 1e6, 3),
                     "launches": launches},
        # what a CPU-only loader does: the native reader filling host memory
        "cpu_baseline": {"value": round(read_gbps, 3), "unit": "GB/s", "cores": args.load_threads,
                         **host_cpu(), "kind": "port",
                         "sample": f"4 reads of one {n_read} B range of a shard in the page cache "
                                   "into pinned host memory (glm_file_read_ranges)"},
    }
    print(json.dumps(line))
    return 0


def dispatch_bench(args, torch, np) -> int:
    """The public glm_moe_dispatch at T=4096, k=8, E=128 (32,768 pairs, random
    distinct top-8 of every token): 10 calls, then args.steps back-to-back
    calls timed with HIP events on the calling stream.  The CPU baseline is the
    oracle's dispatch (stable argsort) on the same indices."""
    from livglm_amd import native

    T, k, E = 4096, 8, 128
    P = T * k
    rng = np.random.default_rng(args.seed)
    idx_np = np.argsort(rng.random((T, E)), axis=1)[:, :k].astype(np.int32)
    native.load()
    dev = torch.device("cuda:0")
    idx = torch.from_numpy(idx_np).to(dev)
    i32 = dict(dtype=torch.int32, device=dev)
    names = ("counts", "offsets", "perm", "inv", "pair_token", "active", "num_active", "work",
             "status")
    sizes = (E, E + 1, P, P, P, E, 1, 4 * E, 1)
    b = {n: torch.empty(sz, **i32) for n, sz in zip(names, sizes)}
    stream = torch.cuda.current_stream().cuda_stream

    def call():
        native.call("glm_moe_dispatch", stream, idx.data_ptr(), T, k, E,
                    *(b[n].data_ptr() for n in names))

    for _ in range(10):
        call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / args.steps
    # CPU baseline: the oracle's dispatch, timed on the same indices
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import moe_oracle as O
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < max(0.2, args.cpu_seconds):
        O.dispatch(idx_np, E)
        reps += 1
    cpu_us = (time.perf_counter() - t0) * 1e6 / reps
    line = {
        "metric": "glm_moe_dispatch time per call", "value": round(us, 3), "unit": "us",
        "n_gpus": 1, "steps": args.steps, "warmup": 10, "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "int32",
        "data": "synthetic",
        "config": {"workload": f"dispatch_t4096: glm_moe_dispatch T={T} k={k} E={E} "
                               f"({P} pairs, distinct top-{k} per token)"},
        "cpu_baseline": {"value": round(cpu_us, 1), "unit": "us", "cores": 1, **host_cpu(),
                         "kind": "port", "sample": f"the oracle's dispatch on the same indices, "
                                                   f"{reps} calls"},
    }
    print(json.dumps(line))
    return 0


def copy_probe(torch) -> int:
    """Counter calibration run: four device copies of COPY_BYTES."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    return 0


def _counter_pass(counters: list[str], child_args: list[str]) -> dict[str, dict[str, list[float]]]:
    """One rocprofv3 counter pass over a child run of this script; returns
    {counter: {kernel name: per-dispatch values}}."""
    out = tempfile.mkdtemp(prefix="glm_pmc_", dir="/tmp")
    env = dict(os.environ, TMPDIR="/tmp")
    cmd = ["rocprofv3", "--pmc", *counters, "-f", "csv", "-d", out, "-o", "run", "--",
           sys.executable, os.path.abspath(__file__)] + child_args
    print(f"bench: counter pass {' '.join(counters)} over {' '.join(child_args)}",
          file=sys.stderr, flush=True)
    try:
        # own process group, so that a pass over its time limit ends with its children
        proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL,
                                stderr=subprocess.DEVNULL, start_new_session=True)
        try:
            proc.wait(timeout=120)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
            return {}
        vals: dict[str, dict[str, list[float]]] = {}
        for path in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for row in csv.DictReader(f):
                    if row.get("Counter_Name") in counters:
                        vals.setdefault(row["Counter_Name"], {}).setdefault(
                            row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return vals
    finally:
        shutil.rmtree(out, ignore_errors=True)


def _kernel_child(args, workload: str, launches: int, rotation_gb: float) -> list[str]:
    return ["--mode", "kernel", "--workload", workload, "--kernel-launches", str(launches),
            "--seed", str(args.seed), "--min-rotation-gb", str(rotation_gb),
            "--act-format", args.act_format]


def measure_traffic(args, workload: str, kernel_name: str):
    """HBM bytes per launch of the dominant kernel: FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch) in two passes over a run of its launches, each scaled by
    what the same counter reads for a device copy of COPY_BYTES."""
    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not found"
    child = _kernel_child(args, workload, 32, args.min_rotation_gb)
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        copy_vals = [v for name, vs in _counter_pass([counter], ["--mode", "copy"]).get(
            counter, {}).items() if "copy" in name.lower() for v in vs]
        kern = [v for name, vs in _counter_pass([counter], child).get(counter, {}).items()
                if kernel_name in name for v in vs]
        if not copy_vals or not kern or max(copy_vals) <= 0:
            return None, f"{counter}: no counter rows (copy {len(copy_vals)}, kernel {len(kern)})"
        scale = COPY_BYTES / (max(copy_vals) * 1024.0)
        res[counter] = (sum(kern) / len(kern) * 1024.0 * scale, scale, len(kern))
    fetch, write = res["FETCH_SIZE"], res["WRITE_SIZE"]
    note = (f"FETCH_SIZE x {fetch[1]:.3f} + WRITE_SIZE x {write[1]:.3f} (scales from a "
            f"{COPY_BYTES >> 20} MiB device copy), mean over {fetch[2]} dispatches: "
            f"read {fetch[0] / 1e6:.2f} MB, write {write[0] / 1e6:.3f} MB")
    return round(fetch[0] + write[0]), note


MFMA_COUNTERS = ["SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_INSTS_VALU_MFMA_MOPS_F6F4",
                 "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]


def mfma_counters(args, workload: str, kernel_name: str) -> dict | None:
    """MFMA work of the grouped GEMM from one counter pass: the MOPS counters
    count 512 floating-point operations each (F8 covers the FP8 x FP4 forms,
    F6F4 the FP4/FP6-only forms), so executed FLOPs per launch = 512 x (F8 +
    F6F4); SQ_VALU_MFMA_BUSY_CYCLES sums the MFMA pipes' busy cycles over all
    SIMDs."""
    if shutil.which("rocprofv3") is None:
        return None
    vals = _counter_pass(MFMA_COUNTERS, _kernel_child(args, workload, 8, 0.0))
    per = {}
    for c in MFMA_COUNTERS:
        v = [x for name, xs in vals.get(c, {}).items() if kernel_name in name for x in xs]
        if not v:
            return {"error": f"no {c} rows for {kernel_name}"}
        per[c] = sum(v) / len(v)
    executed = 512.0 * (per["SQ_INSTS_VALU_MFMA_MOPS_F8"] + per["SQ_INSTS_VALU_MFMA_MOPS_F6F4"])
    return {"mops_f8_per_launch": per["SQ_INSTS_VALU_MFMA_MOPS_F8"],
            "mops_f6f4_per_launch": per["SQ_INSTS_VALU_MFMA_MOPS_F6F4"],
            "mfma_busy_cycles_per_launch": per["SQ_VALU_MFMA_BUSY_CYCLES"],
            "executed_flops_per_launch": executed, "launches": 8,
            "note": "rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " over 8 launches"}


def host_cpu() -> dict:
    """The host the CPU baseline ran on: logical CPUs and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def cpu_baseline_numpy(shape, seed: int, budget_s: float) -> dict:
    """The numpy oracle (oracle/moe_oracle.py, f64 products) on one thread:
    layer steps of ``shape`` on one seeded layer, as many as fit in
    ``budget_s`` (at least one)."""
    from threadpoolctl import threadpool_limits

    from livglm_amd.workloads import make_layer
    from oracle import moe_oracle as O

    layer = make_layer(shape, seed)
    bank = O.Bank(*(layer[key] for key in ("gate_proj.weight_packed", "gate_proj.weight_scale",
                                           "up_proj.weight_packed", "up_proj.weight_scale",
                                           "down_proj.weight_packed", "down_proj.weight_scale")))
    sw = tuple(O.bf16_bits_to_f32(layer[k]) for k in ("shared.gate", "shared.up", "shared.down"))
    x = O.bf16_bits_to_f32(layer["x"])
    steps = 0
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        while True:
            O.moe_layer(x, layer["router_weight"], layer["router_bias"], bank, sw,
                        top_k=shape.k, n_group=shape.n_group, topk_group=shape.topk_group,
                        norm_topk_prob=shape.norm_topk_prob,
                        routed_scaling_factor=shape.routed_scaling_factor,
                        swiglu_limit=shape.swiglu_limit)
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
    return {"value": round(shape.T * steps / el, 3), "unit": "tokens/s", "cores": 1,
            "kind": "port",
            "sample": f"{steps} layer steps of {shape.name} (T={shape.T}) in {el:.2f} s; "
                      "numpy oracle (f64 products, one BLAS thread), not MLX"}


def cpu_baseline(shape, bank, xs, budget_s: float, bias=None, streams=None):
    """The C restatement (oracle/libmoe_cpu.so, OpenMP over this host's cores)
    on one resident layer: as many layer steps as fit in ``budget_s``.  For a
    layer stack, one step is the resident MXFP8 linear + the MoE layer, and
    the stack's rate is that of ``shape.layers`` such steps per token.  For the
    FFN site the hyper-connection, norm and hyper_residual run in the numpy
    oracle around the C MoE layer."""
    import numpy as np
    import torch

    from oracle import cpu as cpu_oracle

    try:
        cpu_oracle.load()
    except RuntimeError as err:
        return {"error": str(err)}
    host = {key: bank[key].cpu().numpy() for key in bank if not key.startswith("shared")}
    for key in ("shared.gate", "shared.up", "shared.down"):
        host[key] = bank[key].view(torch.int16).cpu().numpy().view(np.uint16)
    if bias is not None:
        host["router_bias"] = bias.cpu().numpy()
    xs_h = xs.view(torch.int16).cpu().numpy().view(np.uint16)
    stack = shape.layers > 1
    site = shape.hc > 0
    if site or stack:
        from oracle import mhc_oracle as H
        from oracle import moe_oracle as O
    if site:
        st_h = streams.cpu().numpy()
    y = None
    steps = 0
    t0 = time.perf_counter()
    while True:
        x = xs_h[steps % xs_h.shape[0]]
        if stack:
            if y is not None:  # the previous layer step's output through the norm
                x = O.f32_to_bf16_bits(H.rms_norm(y, host["linear.norm"], 1e-6))
            x = cpu_oracle.linear_mxfp8(x, host["linear.codes"], host["linear.scales"])
        if site:
            st = st_h[steps % st_h.shape[0]]
            post, comb, collapsed = H.hyper_connection(
                st, host["hc.fn"], host["hc.base"], host["hc.scale"], sinkhorn_iters=20,
                rms_eps=1e-6, hc_eps=1e-6)
            x = O.f32_to_bf16_bits(H.rms_norm(collapsed, host["norm.weight"], 1e-6))
        host["x"] = x
        y = cpu_oracle.moe_layer(host, shape)[0]
        if site:
            H.hyper_residual(st, y, post, comb)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 10000:
            break
    if stack:
        return {
            "value": round(steps / (el * shape.layers), 3),
            "unit": "tokens/s",
            "cores": cpu_oracle.threads(),
            **host_cpu(),
            "kind": "port",
            "sample": f"{steps} single-layer steps (RMSNorm + MXFP8 {shape.d}x{shape.d} linear + "
                      f"MoE layer, T={shape.T}) on one resident layer in {el:.2f} s; tokens/s = 1 / "
                      f"({shape.layers} x mean layer time); C restatement (not MLX), OpenMP",
        }
    return {
        "value": round(shape.T * steps / el, 2),
        "unit": "tokens/s",
        "cores": cpu_oracle.threads(),
        **host_cpu(),
        "kind": "port",
        "sample": f"{steps} layer steps of {shape.name} (T={shape.T}) on one resident layer "
                  f"in {el:.2f} s; C restatement (not MLX), OpenMP"
                  + ("; hyper-connection, norm and hyper_residual in the numpy oracle"
                     if site else ""),
    }

if __name__ == "__main__":
    sys.exit(main())
