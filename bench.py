#!/usr/bin/env python3
"""Headline benchmark: fused PoPE causal attention forward + backward on one MI355X.

Workload (the configuration the metric is quoted on): B=1, H=16, S=16384, D=128, bf16 operands,
fp32 accumulation; q, k, v, dO ~ N(0, 1); theta_i = 10000^(-i/D); per-head key phase bias
delta ~ U(-2 pi, 0) of shape (H, D); gradients for q, k, v and delta.  One step = one
``pe_attention`` forward (positional transform + attention) and one backward (dQ, dK, dV, ddelta)
through the C-ABI library, inputs resident in HBM.

Throughput uses the algorithmic FLOP count of fused PoPE attention (QK contracted over 2D, V of
width D, causal factor 1/2): forward 3*B*H*S^2*D, backward 8*B*H*S^2*D, together 11*B*H*S^2*D.

Per-kernel durations come from HIP events that the library records around each kernel stage on
the launch stream (pe_attn_set_stage_events) during the timed steps; the roofline entry is the
kernel stage with the largest total time.

The CPU baseline times this repository's CPU restatement of the reference's eager PyTorch path
(oracle/pe_oracle.py, fp32) on a bounded sample of the same workload: ``--cpu-heads`` of the 16
heads at the full S=16384, forward + backward.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published)
HBM_PEAK_GBS = 8000.0

WORKLOAD = dict(B=1, H=16, S=16384, D=128)

# HBM bytes per dispatch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this workload,
# scaled by a calibration copy (python -m pe_ablations_amd.profiling traffic ...); the file records
# the commands.  A stage's kernel missing from it reports traffic null.
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "pope_fwdbwd_S16k_D128_hbm_traffic.json")
STAGE_KERNEL = {"fwd_core": "fwd_bf16_kernel", "bwd_dkdv": "dkdv_bf16_kernel", "bwd_dq": "dq_gemm_kernel"}


def measured_traffic(stage: str):
    """(bytes per launch, kernel name) of the stage's kernel from the committed PMC summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None, None
    for name, v in data.get("kernels", {}).items():
        if name.startswith(STAGE_KERNEL[stage] + "<") and v.get("fetch_bytes") is not None \
                and v.get("write_bytes") is not None:
            return v["fetch_bytes"] + v["write_bytes"], name
    return None, None


def flops(B, H, S, D):
    """Algorithmic FLOPs of fused PoPE causal attention (Dqk = 2D, Dv = D, c = 1/2)."""
    base = B * H * S * S * D
    return {
        "fwd": 3.0 * base,
        "bwd": 8.0 * base,
        "total": 11.0 * base,
        "fa_convention": 7.0 * base,
        # per kernel stage: GEMMs each kernel must perform
        "fwd_core": 3.0 * base,      # S = q~k~^T (2D) + O = PV (D)
        "bwd_dkdv": 6.0 * base,      # S (2D) + dP (D) + dV (D) + dK~ (2D)
        "bwd_dq": 2.0 * base,        # dQ~ (2D); its S/dP recompute (3*base) is not algorithmic
    }


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(heads: int, reps: int):
    """Oracle fwd+bwd (fp32, torch eager, all host threads) on `heads` heads of the workload: one
    untimed warm-up pass, then the median of `reps` timed passes."""
    import torch
    from oracle import pe_oracle as O

    B, H, S, D = WORKLOAD["B"], WORKLOAD["H"], WORKLOAD["S"], WORKLOAD["D"]
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, heads, S, D, generator=g).requires_grad_(True)
    k = torch.randn(1, heads, S, D, generator=g).requires_grad_(True)
    v = torch.randn(1, heads, S, D, generator=g).requires_grad_(True)
    dO = torch.randn(1, heads, S, D, generator=g)
    delta = (torch.rand(heads, D, generator=g) * (-2 * math.pi)).requires_grad_(True)
    freqs = O.pope_freqs(D)

    def one_pass():
        for t in (q, k, v, delta):
            t.grad = None
        t0 = time.perf_counter()
        out, _ = O.pope_attention(q, k, v, freqs, delta, scale=1.0 / math.sqrt(D), clamp=False,
                                  core_dtype=torch.float32)
        out.backward(dO.to(out.dtype))
        return time.perf_counter() - t0

    one_pass()
    times = sorted(one_pass() for _ in range(reps))
    dt = times[len(times) // 2]
    f = flops(1, heads, S, D)["total"]
    return {
        "value": f / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle/pe_oracle.py pope_attention fwd+bwd, fp32 torch eager, {heads} of {H} heads "
                  f"(B=1, S={S}, D={D}); 1 warm-up + median of {reps} passes, {dt:.2f} s per pass, "
                  f"{sum(times):.1f} s timed",
        "seconds": dt,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=2)
    ap.add_argument("--cpu-reps", type=int, default=4)
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the PE attention path has no multi-GPU leg", file=sys.stderr)
        return 2

    import torch
    from pe_ablations_amd import _lib
    from pe_ablations_amd.functional import pe_attention

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, S, D = WORKLOAD["B"], WORKLOAD["H"], WORKLOAD["S"], WORKLOAD["D"]
    F = flops(B, H, S, D)

    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    q = torch.randn(B, H, S, D, generator=g, device=dev).to(bf).requires_grad_(True)
    k = torch.randn(B, H, S, D, generator=g, device=dev).to(bf).requires_grad_(True)
    v = torch.randn(B, H, S, D, generator=g, device=dev).to(bf).requires_grad_(True)
    dO = torch.randn(B, H, S, D, generator=g, device=dev).to(bf)
    delta = (torch.rand(H, D, generator=g, device=dev) * (-2 * math.pi)).requires_grad_(True)
    freqs = (10000.0 ** (-(torch.arange(0, D, dtype=torch.float32) / D))).to(dev)
    scale = 1.0 / math.sqrt(D)

    def step():
        out = pe_attention(q, k, v, mode="pope", freqs=freqs, delta=delta, scale=scale)
        return torch.autograd.grad(out, (q, k, v, delta), dO)

    L = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    nst = len(_lib.STAGES)

    log(f"bench: warmup {args.warmup} steps (B={B} H={H} S={S} D={D} bf16)")
    for _ in range(args.warmup):
        grads = step()
    torch.cuda.synchronize()
    for gr in grads:
        if not torch.isfinite(gr.float()).all():
            raise RuntimeError("non-finite gradient in warmup")

    # events per timed step, created up front (a first record materialises the HIP event)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2 * nst)] for _ in range(args.steps)]
    for row in evs:
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    arrays = [(ctypes.c_void_p * (2 * nst))(*[e.cuda_event for e in row]) for row in evs]

    log(f"bench: timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        L.pe_attn_set_stage_events(ctypes.cast(arrays[i], ctypes.c_void_p))
        step()
    L.pe_attn_set_stage_events(None)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    log(f"bench: {ms:.3f} ms/step")

    stage_ms = {}
    for si, name in enumerate(_lib.STAGES):
        vals = [row[2 * si].elapsed_time(row[2 * si + 1]) for row in evs]
        stage_ms[name] = sum(vals) / len(vals)
    core = ["fwd_core", "bwd_dkdv", "bwd_dq"]
    dom = max(core, key=lambda n: stage_ms[n])
    achieved = F[dom] / (stage_ms[dom] * 1e-3) / 1e12
    traffic, traffic_kernel = measured_traffic(dom)
    value = F["total"] / (ms * 1e-3) / 1e12

    props = torch.cuda.get_device_properties(dev)
    res = {
        "metric": "fused PoPE attn fwd+bwd TFLOP/s @S=16k,D=128; % of bf16 MFMA peak",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO, delta ~ U(-2pi,0) per head)",
        "config": {"workload": "PoPE causal attention fwd+bwd", "B": B, "H": H, "S": S, "D": D,
                   "delta": "per-head (H, D)", "grads": "q,k,v,delta", "parallelism": "single GPU"},
        "frac_of_peak": round(value / PEAK_BF16_TFLOPS, 4),
        "fa_convention_tflops": round(F["fa_convention"] / (ms * 1e-3) / 1e12, 2),
        "stage_ms": {k2: round(v2, 4) for k2, v2 in stage_ms.items()},
        "roofline": {
            "kernel": dom,
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": None if traffic is None else int(traffic),
            "traffic_unit": "bytes per launch (HBM read + write)",
            "traffic_source": None if traffic is None else f"profiles/{os.path.basename(TRAFFIC_FILE)}: {traffic_kernel}",
        },
        "device": {"name": props.name, "cus": props.multi_processor_count},
    }
    if not args.no_cpu_baseline:
        log(f"bench: CPU baseline ({args.cpu_heads} heads)")
        cb = cpu_baseline(args.cpu_heads, args.cpu_reps)
        res["cpu_baseline"] = {k2: v2 for k2, v2 in cb.items() if k2 != "seconds"}
        res["cpu_baseline"]["value"] = round(cb["value"], 5)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
