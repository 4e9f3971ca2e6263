"""Benchmark of the MI355X routed-MoE layer (one GPU).

A step is one MoE layer forward (router -> dispatch -> MXFP4 gate/up + SwiGLU
-> down -> shared expert -> combine) over one batch of synthetic tokens whose
weights are already resident in HBM.  Steps rotate over several independent
layer banks (>= 2 GB in total) and token batches so that expert reads come from
HBM rather than the 256 MB Infinity Cache.  The timed steps run as one HIP
graph, bracketed by synchronisation and HIP events.

Prints one JSON line: the layer's tokens/s (``value``), plus the roofline of
the dominant kernel (the routed gate/up MXFP4 GEMV, timed live with HIP events
over a graph of back-to-back launches) and the CPU baseline (the C restatement
in oracle/, OpenMP, on this host) on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "src")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE layer tokens/s; decode expert HBM GB/s; MXFP4 MFMA util at T=4096"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK = {"bf16": 2500.0, "fp8": 5000.0, "fp4": 10100.0}  # TFLOP/s, dense


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--workload", default="verify_t2",
                    help="decode_t1 | verify_t2 | batch_t64 | prefill_t4096")
    ap.add_argument("--min-rotation-gb", type=float, default=4.0,
                    help="total size of the distinct layer banks the steps rotate over")
    ap.add_argument("--kernel-launches", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="budget of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--seed", type=int, default=5301)
    return ap.parse_args()


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU runs are not part of "
                                   "it (see DESIGN.md: how the layer would shard by expert)",
                          "n_gpus": args.gpus}))
        return 2

    import numpy as np
    import torch

    from livglm_amd import native
    from livglm_amd.workloads import BANK_KEYS, SHAPES

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    lib = native.load()
    shape = SHAPES[args.workload]
    T, d, E, k, I, Is = shape.T, shape.d, shape.E, shape.k, shape.I, shape.I_shared
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    # ------------------------------------------------------------ resident layer banks
    layer_bytes = shape.bank_bytes + 3 * Is * d * 2 + E * d * 4
    n_banks = max(2, math.ceil(args.min_rotation_gb * 1e9 / layer_bytes))
    n_inputs = 64

    def randbytes(*s):
        return torch.randint(0, 256, s, dtype=torch.uint8, device=dev, generator=gen)

    def randscales(*s):
        return torch.randint(119, 128, s, dtype=torch.uint8, device=dev, generator=gen)

    banks = []
    for _ in range(n_banks):
        b = {
            "gate_proj.weight_packed": randbytes(E, I, d // 2),
            "gate_proj.weight_scale": randscales(E, I, d // 32),
            "up_proj.weight_packed": randbytes(E, I, d // 2),
            "up_proj.weight_scale": randscales(E, I, d // 32),
            "down_proj.weight_packed": randbytes(E, d, I // 2),
            "down_proj.weight_scale": randscales(E, d, I // 32),
            "router_weight": torch.randn((E, d), device=dev, generator=gen) * 0.02,
            "router_bias": torch.zeros(E, device=dev),
            "shared.gate": (torch.randn((Is, d), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
            "shared.up": (torch.randn((Is, d), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
            "shared.down": (torch.randn((d, Is), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
        }
        if shape.routing == "zipf":
            from livglm_amd.workloads import zipf_bias
            b["router_bias"] = torch.from_numpy(
                zipf_bias(E, np.random.default_rng(args.seed + len(banks)))).to(dev)
        banks.append(b)
    xs = torch.randn((n_inputs, T, d), device=dev, generator=gen).to(torch.bfloat16)

    ws_bytes = lib.glm_moe_workspace_bytes(T, d, E, k, I, Is)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    native.call("glm_moe_workspace_init", torch.cuda.current_stream().cuda_stream, ws.data_ptr(),
                ws_bytes)
    out = torch.empty((T, d), dtype=torch.float32, device=dev)
    wts = torch.empty((T, k), dtype=torch.float32, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)

    def layer_step(s: int) -> None:
        b = banks[s % n_banks]
        x = xs[s % n_inputs]
        native.call(
            "glm_moe_forward", torch.cuda.current_stream().cuda_stream, x.data_ptr(), T, d,
            b["router_weight"].data_ptr(), b["router_bias"].data_ptr(), E, k, shape.n_group,
            shape.topk_group, int(shape.norm_topk_prob), shape.routed_scaling_factor, I,
            *(b[key].data_ptr() for key in BANK_KEYS), Is, native.GLM_FMT_BF16,
            b["shared.gate"].data_ptr(), None, b["shared.up"].data_ptr(), None,
            b["shared.down"].data_ptr(), None, None, shape.swiglu_limit, ws.data_ptr(), ws_bytes,
            out.data_ptr(), wts.data_ptr(), idx.data_ptr())

    def capture(first: int, count: int):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for s in range(first, first + count):
                layer_step(s)
        return g

    # eager pass over every bank first (validates the launches outside capture)
    for s in range(n_banks):
        layer_step(s)
    torch.cuda.synchronize()

    # ------------------------------------------------------------ timed layer steps
    if args.warmup > 0:
        gw = capture(0, args.warmup)
        gw.replay()
    gt = capture(args.warmup, args.steps)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    ev0.record()
    gt.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    elapsed_ms = ev0.elapsed_time(ev1)
    ms_per_step = elapsed_ms / args.steps
    tokens_per_s = T * args.steps / (elapsed_ms / 1e3)

    # ------------------------------------------------------------ dominant kernel: gate/up
    # Route each launch's batch once (router + dispatch) so the plans exist,
    # then time a graph of back-to-back gate/up launches with HIP events.
    R = args.kernel_launches
    P = T * k
    i32 = dict(dtype=torch.int32, device=dev)
    plans = []
    for r in range(R):
        b = banks[r % n_banks]
        x = xs[r % n_inputs]
        lg = torch.empty((T, E), dtype=torch.float32, device=dev)
        w_ = torch.empty((T, k), dtype=torch.float32, device=dev)
        ix = torch.empty((T, k), **i32)
        native.call("glm_router_topk", torch.cuda.current_stream().cuda_stream, x.data_ptr(), T,
                    d, b["router_weight"].data_ptr(), b["router_bias"].data_ptr(), E, k,
                    shape.n_group, shape.topk_group, 1, shape.routed_scaling_factor,
                    lg.data_ptr(), w_.data_ptr(), ix.data_ptr())
        pl = {n: torch.empty(sz, **i32) for n, sz in
              [("counts", E), ("offsets", E + 1), ("perm", P), ("inv", P), ("tok", P),
               ("active", E), ("nact", 1), ("work", 4 * E), ("status", 1)]}
        native.call("glm_moe_dispatch", torch.cuda.current_stream().cuda_stream, ix.data_ptr(),
                    T, k, E, *(pl[n].data_ptr() for n in ("counts", "offsets", "perm", "inv",
                                                           "tok", "active", "nact", "work",
                                                           "status")))
        plans.append(pl)
    torch.cuda.synchronize()
    unique = [int(pl["nact"].item()) for pl in plans]
    h = torch.empty((P, I), dtype=torch.bfloat16, device=dev)

    def gate_up(r: int) -> None:
        b, pl = banks[r % n_banks], plans[r]
        native.call("glm_expert_gate_up", torch.cuda.current_stream().cuda_stream,
                    xs[r % n_inputs].data_ptr(), T, d, I, E, k,
                    *(b[key].data_ptr() for key in BANK_KEYS[:4]), pl["tok"].data_ptr(),
                    pl["work"].data_ptr(), shape.swiglu_limit, h.data_ptr())

    gk = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gk):
        for r in range(R):
            gate_up(r)
    gk.replay()
    torch.cuda.synchronize()
    ek0, ek1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ek0.record()
    gk.replay()
    ek1.record()
    torch.cuda.synchronize()
    k_ms = ek0.elapsed_time(ek1) / R
    proj_bytes = I * d // 2 + I * d // 32  # one projection of one expert
    gateup_bytes = [u * 2 * proj_bytes for u in unique]
    bytes_per_launch = sum(gateup_bytes) / R
    achieved = bytes_per_launch / (k_ms / 1e3) / 1e9

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(shape, banks[0], xs, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{shape.name}: MoE layer T={T} d={d} E={E} top-{k} I={I} "
                        f"(MXFP4 group-32 experts, bf16 shared expert I={Is})",
            "tokens_per_step": T, "weights": "mxfp4-e2m1+e8m0", "mfma": "bf16 x dequantised mxfp4",
            "layer_banks": n_banks, "rotation_bytes": n_banks * layer_bytes,
            "graph_steps": args.steps, "wall_s": round(wall, 4),
        },
        "decode_expert_hbm_gbps": round(achieved, 1),
        "roofline": {
            "kernel": "decode_gate_up_kernel<4, false> (routed MXFP4 gate+up+SwiGLU)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "bytes_per_launch": round(bytes_per_launch),
            "avg_launch_us": round(k_ms * 1e3, 3),
            "unique_experts_per_launch": round(sum(unique) / R, 2),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


def cpu_baseline(shape, bank, xs, budget_s: float):
    """The C restatement (oracle/libmoe_cpu.so, OpenMP over this host's cores)
    on one resident layer: as many layer steps as fit in ``budget_s``."""
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
    xs_h = xs.view(torch.int16).cpu().numpy().view(np.uint16)
    steps = 0
    t0 = time.perf_counter()
    while True:
        host["x"] = xs_h[steps % xs_h.shape[0]]
        cpu_oracle.moe_layer(host, shape)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 10000:
            break
    return {
        "value": round(shape.T * steps / el, 2),
        "unit": "tokens/s",
        "cores": cpu_oracle.threads(),
        "kind": "port",
        "sample": f"{steps} layer steps of {shape.name} (T={shape.T}) on one resident layer "
                  f"in {el:.2f} s; C restatement (not MLX), OpenMP",
    }


if __name__ == "__main__":
    sys.exit(main())
