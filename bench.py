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

More workloads, selected with ``--workload`` (the default is the headline above):

* ``fwd``: the long-context evaluation forward (the same shape, forward only, under
  ``torch.inference_mode``; 3*B*H*S^2*D FLOPs per step); ``fwd32`` the same in fp32, the
  precision of the reference's 16k evaluation, against the fp32 MFMA peak.
* ``c2``: PoPE fwd+bwd at B=8, H=12, S=2048, D=64 (~125M GPT shape).
* ``c3``: FoPE fwd+bwd at B=4, H=16, S=4096, D=128, M=4 frequencies per dim; the FoPE collapse
  (FoPEPoPEEmbedding) runs in each step and the Fourier coefficients get gradients.
* ``masked``: PoPE fwd+bwd at B=2, H=16, S=4096, D=128 with an explicit bool key-padding mask
  (GroupedQueryAttention's attn_mask) and no causal mask: every query-key pair is computed.
* ``split``: the reference's training module shape, split form [content 64 | PoPE 2x32], V 64,
  8 query heads on 4 kv heads, B=8, S=512, one shared (Dr,) phase bias.

Every attention line carries a ``prologue`` entry: the algorithmic bytes of the q / k transform
stage (read raw rows, write transformed rows), its time from the stage events, GB/s against the
8 TB/s HBM peak and, for the headline, the PMC-measured bytes of its kernels.
* ``decoder``: the whole ~1B decoder forward of the long-context configuration: 24 layers,
  d_model 2048, 16 fused-PoPE heads of D=128, SwiGLU 5632, RMSNorm, vocab 32000, bf16 weights
  ~ N(0, 0.02^2), one sequence of 16384 uniform token ids, with the next-token cross entropy
  (which must come out near ln 32000 + 0.02^2 * 2048 / 2 = 10.78 at this init: the tied head's
  logits have variance 0.02^2 * d_model).  Reported as tokens/s; the roofline entry is
  the attention kernel of the last layer.

* ``decode``: one decoded token per step at the same attention shape (16 heads of D=128) against
  a cache of 16384 transformed key rows: the new key row is appended to the cache and the new
  query attends to every cached row (split-key decode kernel).  Reported as cache GB/s against
  the 8 TB/s HBM peak, the bound of decode.

``--graph`` (attention workloads) also captures the step once in a HIP graph and times its
replays: the small shapes, such as ``split``, are bound by host time per launch when run eagerly.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--graph]
                       [--workload fwdbwd|fwd|fwd32|c2|c3|masked|split|decoder|decode]
"""

from __future__ import annotations

import argparse
import ctypes
import functools
import json
import math
import os
import sys
import time

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published)
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA (published)
HBM_PEAK_GBS = 8000.0

WORKLOAD = dict(B=1, H=16, S=16384, D=128)

# Attention workloads.  Hq / Hkv heads, S queries and keys (causal), content width Dc (passed
# through), positional width Dr (PoPE: 2*Dr after the transform), value width Dv.  delta: "head" =
# per-head (Hkv, Dr) phase bias, "shared" = one (Dr,) bias (the reference module's parameter).
# fope: (M, coefficient sigma, training length) of a FoPE collapse computed per step by the
# FoPEPoPEEmbedding module (base frequency plus M - 1 extra frequencies ~ U(0, theta_0)).
ATTN_WORKLOADS = {
    "fwdbwd": dict(B=1, Hq=16, Hkv=16, S=16384, Dc=0, Dr=128, Dv=128, dtype="bf16", backward=True, delta="head",
                   name="PoPE causal attention fwd+bwd",
                   metric="fused PoPE attn fwd+bwd TFLOP/s @S=16k,D=128; % of bf16 MFMA peak"),
    "fwd": dict(B=1, Hq=16, Hkv=16, S=16384, Dc=0, Dr=128, Dv=128, dtype="bf16", backward=False, delta="head",
                name="PoPE causal attention forward (long-context eval)",
                metric="fused PoPE attn fwd TFLOP/s @S=16k,D=128 (long-context eval forward); % of bf16 MFMA peak"),
    "fwd32": dict(B=1, Hq=16, Hkv=16, S=16384, Dc=0, Dr=128, Dv=128, dtype="fp32", backward=False, delta="head",
                  name="PoPE causal attention forward in fp32 (the reference's 16k evaluation precision)",
                  metric="fused PoPE attn fwd TFLOP/s @S=16k,D=128, fp32; % of fp32 MFMA peak"),
    "c2": dict(B=8, Hq=12, Hkv=12, S=2048, Dc=0, Dr=64, Dv=64, dtype="bf16", backward=True, delta="head",
               name="PoPE causal attention fwd+bwd, ~125M GPT shape",
               metric="fused PoPE attn fwd+bwd TFLOP/s @B=8,H=12,S=2048,D=64; % of bf16 MFMA peak"),
    "c3": dict(B=4, Hq=16, Hkv=16, S=4096, Dc=0, Dr=128, Dv=128, dtype="bf16", backward=True, delta="head",
               fope=(4, 0.1, 2048), name="FoPE causal attention fwd+bwd (M=4 frequencies per dim)",
               metric="fused FoPE attn fwd+bwd TFLOP/s @B=4,H=16,S=4096,D=128; % of bf16 MFMA peak"),
    # explicit mask (GroupedQueryAttention's attn_mask, src/model/attention.py:91-96): a bool key-padding
    # mask (B, 1, 1, S), batch entry b keeping its first S - 100 b keys, and no causal mask, so every
    # query-key pair is computed
    "masked": dict(B=2, Hq=16, Hkv=16, S=4096, Dc=0, Dr=128, Dv=128, dtype="bf16", backward=True, delta="head",
                   causal=False, mask="keypad",
                   name="PoPE attention fwd+bwd with an explicit key-padding mask (not causal)",
                   metric="masked PoPE attn fwd+bwd TFLOP/s @B=2,H=16,S=4096,D=128, key-padding mask; "
                          "% of bf16 MFMA peak"),
    # the ablation's RoPE arm: the reference's GroupedQueryAttention (interleaved RoPE, theta 10000, then
    # QKNorm, src/model/attention.py:69-96) at the ~125M GPT shape; operands of width Dr, no phase bias
    "rope": dict(B=8, Hq=12, Hkv=12, S=2048, Dc=0, Dr=64, Dv=64, dtype="bf16", backward=True, delta=None,
                 mode="rope", qk_norm=True,
                 name="RoPE + QKNorm causal attention fwd+bwd (GroupedQueryAttention), ~125M GPT shape",
                 metric="fused RoPE+QKNorm attn fwd+bwd TFLOP/s @B=8,H=12,S=2048,D=64; % of bf16 MFMA peak"),
    "split": dict(B=8, Hq=8, Hkv=4, S=512, Dc=64, Dr=32, Dv=64, dtype="bf16", backward=True, delta="shared",
                  name="split-form PoPE attention fwd+bwd at the reference's training shape "
                       "([content 64 | PoPE 2x32], V 64, GQA 8 -> 4)",
                  metric="split-form PoPE attn fwd+bwd TFLOP/s @B=8,S=512,Hq=8,Hkv=4,Dc=64,Dr=32; "
                         "% of bf16 MFMA peak"),
}

# HBM bytes per dispatch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this workload,
# scaled by a calibration copy (python -m pe_ablations_amd.profiling traffic ...); the file records
# the commands.  A stage's kernel missing from it reports traffic null.
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "pope_fwdbwd_S16k_D128_hbm_traffic.json")
STAGE_KERNEL = {"fwd_core": ("fwd_bf16_kernel",), "bwd_dkdv": ("dkdv_pair_kernel", "dkdv_bf16_kernel"),
                "bwd_dq": ("dq_gemm_kernel",)}


def measured_traffic(stage: str):
    """(bytes per launch, kernel name) of the stage's kernel from the committed PMC summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None, None
    for name, v in data.get("kernels", {}).items():
        if any(name.startswith(k + "<") for k in STAGE_KERNEL[stage]) and v.get("fetch_bytes") is not None \
                and v.get("write_bytes") is not None:
            return v["fetch_bytes"] + v["write_bytes"], name
    return None, None


def flops(B, H, S, D):
    """Algorithmic FLOPs of fused PoPE causal attention (Dqk = 2D, Dv = D, c = 1/2)."""
    return attn_flops(dict(B=B, Hq=H, S=S, Dc=0, Dr=D, Dv=D))


def qk_width(w: dict) -> int:
    """Width of the transformed q / k rows: content plus 2*Dr for PoPE, plus Dr for RoPE."""
    return w["Dc"] + (w["Dr"] if w.get("mode", "pope") == "rope" else 2 * w["Dr"])


def attn_flops(w: dict) -> dict:
    """Algorithmic FLOPs of causal attention over transformed operands of width Wqk (qk_width: Dc + 2*Dr
    for PoPE, Dr for RoPE) and values of width Dv, with B*Hq*S^2/2 query-key pairs (B*Hq*S^2 without the causal mask): forward
    S~ (Wqk) + PV (Dv); backward S~
    recompute (Wqk), dP (Dv), dV (Dv), dK~ (Wqk) and dQ~ (Wqk).  At Dc = 0, Dr = Dv = D this is
    3, 8 and 11 * B*H*S^2*D."""
    pairs = w["B"] * w["Hq"] * w["S"] * w["S"] * (0.5 if w.get("causal", True) else 1.0)
    wqk, dv = qk_width(w), w["Dv"]
    return {
        "fwd": 2.0 * pairs * (wqk + dv),
        "bwd": 2.0 * pairs * (3 * wqk + 2 * dv),
        "total": 2.0 * pairs * (4 * wqk + 3 * dv),
        # flash-attention convention at head width Dv: forward 4*B*H*S^2*Dv/2, backward 2.5 times that
        "fa_convention": 2.0 * pairs * 7 * dv,
        # per kernel stage: GEMMs each kernel must perform
        "fwd_core": 2.0 * pairs * (wqk + dv),
        "bwd_dkdv": 2.0 * pairs * (2 * wqk + 2 * dv),
        "bwd_dq": 2.0 * pairs * wqk,   # its S/dP recompute is not algorithmic
    }


def prologue_bytes(w: dict) -> int:
    """Algorithmic HBM bytes of the forward's PE prologue: read the raw q and k rows (content and
    positional parts), write the transformed rows of width qk_width (Dc + 2*Dr for PoPE, Dr for RoPE)."""
    es = 4 if w["dtype"] == "fp32" else 2
    rows = w["B"] * (w["Hq"] + w["Hkv"]) * w["S"]
    return rows * (w["Dc"] + w["Dr"]) * es + rows * qk_width(w) * es


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it (what lscpu prints as the model name), with the family
    and model numbers, which identify the generation where a virtual machine shortens the name."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = (x.strip() for x in line.split(":", 1))
                    if k in ("model name", "cpu family", "model") and k not in info:
                        info[k] = v
                if not line.strip() and info:
                    break
    except OSError:
        pass
    name = info.get("model name", "unknown")
    if "cpu family" in info and "model" in info:
        name += f" (family {info['cpu family']}, model {info['model']}, {os.cpu_count()} logical CPUs)"
    return name


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def fope_module(torch, w: dict, D: int, seed: int = 33):
    """FoPEPoPEEmbedding with the workload's frequency table (base theta_c plus M - 1 frequencies
    ~ U(0, theta_0)) and coefficients ~ N(0, sigma^2)."""
    from pe_ablations_amd.fpope import FoPEPoPEEmbedding
    M, sigma, tl = w["fope"]
    g = torch.Generator().manual_seed(seed)
    base = 10000.0 ** (-(torch.arange(0, D, dtype=torch.float32) / D))
    table = torch.cat([base.unsqueeze(1), torch.rand(D, M - 1, generator=g) * float(base[0])], 1)
    m = FoPEPoPEEmbedding(D, max_seq_len=w["S"], num_fourier_terms=M, fourier_sigma=sigma, training_length=tl,
                          freq_table=table)
    with torch.no_grad():
        m.fourier_coeffs.copy_(torch.randn(D, M, generator=g) * sigma)
    return m


def keypad_mask(torch, B: int, S: int, device=None):
    """The masked workload's bool key-padding mask (B, 1, 1, S): batch entry b keeps its first S - 100 b
    keys."""
    keep = torch.tensor([S - 100 * b for b in range(B)], device=device)
    return (torch.arange(S, device=device).view(1, S) < keep.view(B, 1)).view(B, 1, 1, S)


def cpu_baseline(w: dict, heads: int, reps: int):
    """The oracle's eager path (fp32, torch eager, all host threads) forward (+ backward) on `heads`
    query heads of one batch entry of the workload at its full S: one untimed warm-up pass, then
    the median of `reps` timed passes."""
    import torch
    from oracle import pe_oracle as O

    backward = w["backward"]
    S, Dc, Dr, Dv = w["S"], w["Dc"], w["Dr"], w["Dv"]
    hkv = max(1, heads * w["Hkv"] // w["Hq"])
    g = torch.Generator().manual_seed(0)
    qr = torch.randn(1, heads, S, Dr, generator=g).requires_grad_(backward)
    kr = torch.randn(1, hkv, S, Dr, generator=g).requires_grad_(backward)
    v = torch.randn(1, hkv, S, Dv, generator=g).requires_grad_(backward)
    qc = torch.randn(1, heads, S, Dc, generator=g).requires_grad_(backward) if Dc else None
    kc = torch.randn(1, hkv, S, Dc, generator=g).requires_grad_(backward) if Dc else None
    dO = torch.randn(1, heads, S, Dv, generator=g)
    rope = w.get("mode", "pope") == "rope"
    dshape = (hkv, Dr) if w["delta"] == "head" else (Dr,)
    delta = None if rope else (torch.rand(*dshape, generator=g) * (-2 * math.pi)).requires_grad_(backward)
    fm = fope_module(torch, w, Dr) if w.get("fope") else None
    freqs = O.rope_inv_freq(Dr) if rope else (None if fm else O.pope_freqs(Dr))
    scale = 1.0 / math.sqrt(Dc + 2 * Dr) if Dc else 1.0 / math.sqrt(Dr)
    leaves = [t for t in (qr, kr, v, qc, kc, delta) if t is not None]
    if fm is not None:
        leaves.append(fm.fourier_coeffs)
    causal = w.get("causal", True)
    # the masked workload's first batch entry (its mask keeps every key)
    core = functools.partial(O.attention, dtype=torch.float32, mask=keypad_mask(torch, 1, S)) if w.get("mask") else None

    def one_pass():
        for t in leaves:
            t.grad = None
        t0 = time.perf_counter()
        with torch.set_grad_enabled(backward):
            f = freqs if fm is None else O.fope_effective_freqs(
                fm.base_freqs, fm.fourier_coeffs, freq_table=fm.freq_table, training_length=fm.training_length)
            if rope:
                out, _ = O.rope_attention(qr, kr, v, f, qk_norm=w.get("qk_norm", False), causal=causal, scale=scale,
                                          core=functools.partial(O.attention, dtype=torch.float32))
            elif Dc:
                out, _ = O.split_pope_attention(qc, kc, qr, kr, v, f, delta, scale=scale, causal=causal,
                                                core_dtype=torch.float32, core=core)
            else:
                out, _ = O.pope_attention(qr, kr, v, f, delta, scale=scale, causal=causal, clamp=False,
                                          core_dtype=torch.float32, core=core)
            if backward:
                out.backward(dO.to(out.dtype))
        return time.perf_counter() - t0

    one_pass()
    times = sorted(one_pass() for _ in range(reps))
    dt = times[len(times) // 2]
    f = attn_flops(dict(w, B=1, Hq=heads))["total" if backward else "fwd"]
    what = "fwd+bwd" if backward else "fwd"
    fn = "rope_attention" if rope else ("split_pope_attention" if Dc else "pope_attention")
    return {
        "value": f / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"oracle/pe_oracle.py {fn} {what}" + (" with the key-padding mask" if core else "")
                  + f", fp32 torch eager, {heads} of {w['Hq']} query heads "
                  f"of one batch entry (S={S}, Dc={Dc}, Dr={Dr}, Dv={Dv}); 1 warm-up + median of {reps} "
                  f"passes, {dt:.2f} s per pass, {sum(times):.1f} s timed",
        "seconds": dt,
    }


def stage_events(torch, steps: int, stream):
    """Stage events for the timed steps: a ctypes array of 2 events per library stage (start, end)
    for every `every`-th step (at most about 50 sampled steps), None for the others.  Each event is
    recorded once up front so the HIP event exists before the library records into it.  Sampling
    keeps the event records (12 per step) from adding host time to short, host-bound steps."""
    from pe_ablations_amd import _lib
    nst = len(_lib.STAGES)
    every = max(1, steps // 50)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2 * nst)] for _ in range(0, steps, every)]
    for row in evs:
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    arrays = [None] * steps
    for j, row in enumerate(evs):
        arrays[j * every] = (ctypes.c_void_p * (2 * nst))(*[e.cuda_event for e in row])
    return evs, arrays


def stage_times(evs, names):
    """Average ms of each named stage over the sampled timed steps."""
    from pe_ablations_amd import _lib
    out = {}
    for si, name in enumerate(_lib.STAGES):
        if name in names:
            vals = [row[2 * si].elapsed_time(row[2 * si + 1]) for row in evs]
            out[name] = sum(vals) / len(vals)
    return out


def timed_loop(torch, L, step, arrays, steps):
    """Run `steps` steps between two device synchronisations, handing the library the step's event
    array (or none); returns ms per step."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        a = arrays[i]
        L.pe_attn_set_stage_events(None if a is None else ctypes.cast(a, ctypes.c_void_p))
        step()
    L.pe_attn_set_stage_events(None)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def graph_loop(torch, step, warmup: int, steps: int) -> float:
    """ms per step of `step` captured in a HIP graph (torch's recipe: side-stream warm-up, one
    captured step) and replayed `steps` times after `warmup` untimed replays.  Every replay runs
    every kernel of the step on the same static inputs; the library records no stage events inside
    the graph (stage times come from the eager steps)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def roofline(stage: str, flop: float, ms: float, peak: float = PEAK_BF16_TFLOPS, headline: bool = True) -> dict:
    """Roofline entry of a kernel stage.  The measured HBM traffic comes from the committed PMC
    summary of the headline workload, so other workloads report it as null."""
    traffic, traffic_kernel = measured_traffic(stage) if headline else (None, None)
    achieved = flop / (ms * 1e-3) / 1e12
    return {
        "kernel": stage,
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "traffic": None if traffic is None else int(traffic),
        "traffic_unit": "bytes per launch (HBM read + write)",
        "traffic_source": None if traffic is None else f"profiles/{os.path.basename(TRAFFIC_FILE)}: {traffic_kernel}",
    }


def prologue_entry(w: dict, ms: float, headline: bool) -> dict:
    """The forward's PE prologue stage (q / k transforms, plus the query phase table where the
    backward uses one) against the HBM peak: algorithmic bytes / stage time, and, for the headline
    workload, the PMC-measured bytes of its kernels."""
    nbytes = prologue_bytes(w)
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"stage": "fwd_prep", "bytes": nbytes, "ms": round(ms, 4), "achieved": round(gbs, 1),
           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
    if headline:
        try:
            with open(TRAFFIC_FILE) as f:
                kern = json.load(f).get("kernels", {})
            # per step: both transforms and the query phase table in one dispatch (older summaries:
            # the key transform with the table, then the query transform; or one dispatch each)
            if "prep_k_qheads_kernel" in kern:
                parts = (("prep_k_qheads_kernel", 1),)
            elif "prep_vec_and_table_kernel" in kern:
                parts = (("prep_vec_and_table_kernel", 1), ("prep_pope_vec_kernel", 1))
            else:
                parts = (("prep_pope_vec_kernel", 2), ("phase_table_kernel", 1))
            t = 0.0
            for name, per in parts:
                v = kern[name]
                t += per * (v["fetch_bytes"] + v["write_bytes"])
            out["traffic"] = int(t)
            out["traffic_source"] = (f"profiles/{os.path.basename(TRAFFIC_FILE)}: "
                                     + " + ".join(f"{n} x{k}" for n, k in parts))
        except (OSError, ValueError, KeyError, TypeError):
            pass
    return out


def run_attention(args, torch, dev, wname: str) -> dict:
    """One step of an attention workload: forward (+ backward) through pe_attention and the C-ABI."""
    from pe_ablations_amd import _lib
    from pe_ablations_amd.functional import pe_attention

    w = ATTN_WORKLOADS[wname]
    backward = w["backward"]
    B, Hq, Hkv, S, Dc, Dr, Dv = (w[k] for k in ("B", "Hq", "Hkv", "S", "Dc", "Dr", "Dv"))
    F = attn_flops(w)
    g = torch.Generator(device=dev).manual_seed(0)
    dt = torch.float32 if w["dtype"] == "fp32" else torch.bfloat16

    def rnd(h, d):
        return torch.randn(B, h, S, d, generator=g, device=dev).to(dt).requires_grad_(backward)

    q, k, v = rnd(Hq, Dr), rnd(Hkv, Dr), rnd(Hkv, Dv)
    qc, kc = (rnd(Hq, Dc), rnd(Hkv, Dc)) if Dc else (None, None)
    dO = torch.randn(B, Hq, S, Dv, generator=g, device=dev).to(dt)
    mode = w.get("mode", "pope")
    dshape = (Hkv, Dr) if w["delta"] == "head" else (Dr,)
    delta = None if mode == "rope" else (torch.rand(*dshape, generator=g, device=dev) * (-2 * math.pi)).requires_grad_(backward)
    fm = fope_module(torch, w, Dr).to(dev) if w.get("fope") else None
    # PoPE: one frequency per dim; RoPE: one inverse frequency per interleaved pair
    freqs = (10000.0 ** (-(torch.arange(0, Dr, 2 if mode == "rope" else 1, dtype=torch.float32) / Dr))).to(dev)
    scale = 1.0 / math.sqrt(Dc + 2 * Dr) if Dc else 1.0 / math.sqrt(Dr)
    leaves = [t for t in (q, k, v, qc, kc, delta) if t is not None]
    if fm is not None:
        leaves.append(fm.fourier_coeffs)

    mask = keypad_mask(torch, B, S, dev) if w.get("mask") else None
    causal = w.get("causal", True)

    def attn():
        f = freqs if fm is None else fm.kernel_freqs()
        return pe_attention(q, k, v, mode=mode, q_c=qc, k_c=kc, freqs=f, delta=delta, scale=scale,
                            causal=causal, mask=mask, qk_norm=w.get("qk_norm", False))

    if backward:
        def step():
            return torch.autograd.grad(attn(), leaves, dO)
    else:
        def step():
            with torch.inference_mode():
                return (attn(),)

    L = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    what = "fwd+bwd" if backward else "fwd"
    log(f"bench: warmup {args.warmup} steps ({wname}: {what}, B={B} Hq={Hq} Hkv={Hkv} S={S} Dc={Dc} Dr={Dr} "
        f"Dv={Dv} {w['dtype']})")
    for _ in range(args.warmup):
        res = step()
    torch.cuda.synchronize()
    for t in res:
        if not torch.isfinite(t.float()).all():
            raise RuntimeError("non-finite result in warmup")
    evs, arrays = stage_events(torch, args.steps, stream)
    log(f"bench: timing {args.steps} steps")
    ms = timed_loop(torch, L, step, arrays, args.steps)
    log(f"bench: {ms:.3f} ms/step")
    eager_ms = ms
    if getattr(args, "graph", False):
        ms = graph_loop(torch, step, args.warmup, args.steps)
        log(f"bench: {ms:.3f} ms/step as graph replays")

    core = ["fwd_core", "bwd_dkdv", "bwd_dq"] if backward else ["fwd_core"]
    names = _lib.STAGES if backward else ["fwd_prep", "fwd_core"]
    stage_ms = stage_times(evs, names)
    dom = max(core, key=lambda n: stage_ms[n])
    total = F["total"] if backward else F["fwd"]
    value = total / (ms * 1e-3) / 1e12
    peak = PEAK_FP32_TFLOPS if w["dtype"] == "fp32" else PEAK_BF16_TFLOPS
    headline = wname == "fwdbwd"
    config = {"workload": w["name"], "B": B, "S": S}
    if Dc or Hq != Hkv:
        config.update(Hq=Hq, Hkv=Hkv, Dc=Dc, Dr=Dr, Dv=Dv)
    else:
        config.update(H=Hq, D=Dr)
    if mask is not None:
        config.update(mask="bool key padding (B, 1, 1, S), batch entry b keeps its first S - 100 b keys",
                      causal=False)
    if mode == "rope":
        config.update(pe="RoPE (interleaved pairs, theta 10000) + QKNorm" if w.get("qk_norm") else "RoPE",
                      grads="q,k,v" if backward else "none", parallelism="single GPU")
    else:
        config.update(delta="per-head (Hkv, Dr)" if w["delta"] == "head" else "shared (Dr,)",
                      grads=("q,k,v,delta" + (",q_c,k_c" if Dc else "") + (",fourier_coeffs" if fm else ""))
                      if backward else "none", parallelism="single GPU")
    if fm is not None:
        config["fope"] = {"M": w["fope"][0], "coeff_sigma": w["fope"][1], "training_length": w["fope"][2]}
    if getattr(args, "graph", False):
        config["graph"] = "the step captured once in a HIP graph (torch.cuda.CUDAGraph) and replayed"
    res = {
        "metric": w["metric"],
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": "synthetic (seeded N(0,1) q/k/v/dO" + (")" if mode == "rope" else ", delta ~ U(-2pi,0))"),
        "config": config,
        "frac_of_peak": round(value / peak, 4),
        "fa_convention_tflops": round((F["fa_convention"] if backward else 2.0 * F["fa_convention"] / 7.0)
                                      / (ms * 1e-3) / 1e12, 2),
        "stage_ms": {k2: round(v2, 4) for k2, v2 in stage_ms.items()},
        "roofline": roofline(dom, F[dom], stage_ms[dom], peak, headline),
        "prologue": prologue_entry(w, stage_ms["fwd_prep"], headline),
    }
    if getattr(args, "graph", False):
        res["eager_ms_per_step"] = round(eager_ms, 4)
    return res


DECODER = dict(vocab_size=32000, hidden_dim=2048, num_layers=24, num_heads=16, num_kv_heads=16, head_dim=128,
               ffn_dim=5632, S=16384)


def decoder_flops(c: dict) -> dict:
    """Algorithmic FLOPs of one decoder forward over S tokens: projections + SwiGLU + LM head
    GEMMs (2*S*K*N each) and the fused PoPE attention (3*H*S^2*D per layer)."""
    S, d, L = c["S"], c["hidden_dim"], c["num_layers"]
    hd = c["num_heads"] * c["head_dim"]
    gemm = L * 2 * S * (d * hd * 2 + d * c["num_kv_heads"] * c["head_dim"] * 2 + 3 * d * c["ffn_dim"])
    head = 2 * S * d * c["vocab_size"]
    attn = L * 3.0 * c["num_heads"] * S * S * c["head_dim"]
    return {"gemm": gemm, "lm_head": head, "attention": attn, "total": gemm + head + attn}


def init_loss(cfg) -> float:
    """Expected next-token CE at the N(0, 0.02^2) init: the tied LM head sees a unit-RMS input, so
    the logits are ~ N(0, 0.02^2 d) and E[logsumexp] ~ ln V + 0.02^2 d / 2 (10.78 at V=32000,
    d=2048)."""
    return math.log(cfg.vocab_size) + 0.02 ** 2 * cfg.hidden_dim / 2


def _decoder_config(torch):
    from pe_ablations_amd.transformer import TransformerConfig
    c = {k: v for k, v in DECODER.items() if k != "S"}
    return TransformerConfig(pe_mode="pope", pope_fused=True, max_seq_len=DECODER["S"], pope_delta_init="uniform",
                             **c)


def _bf16_weights(torch, model):
    """Every parameter to bf16 except the shared PoPE module's (its fp32 frequency and angle
    tables are buffers and stay fp32; its phase bias stays fp32 too)."""
    for name, p in model.named_parameters():
        if not name.startswith("pope.") and ".fpope." not in name:
            p.data = p.data.to(torch.bfloat16)
    return model


def decoder_cpu_baseline(torch, model, ids, tokens: int):
    """Oracle decoder forward (oracle.decoder_forward: fp32 weights, fp64 attention core, all host
    threads) over the first `tokens` token ids: one warm-up on 128 tokens, one timed pass."""
    from oracle import pe_oracle as O
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    x = ids[:, :tokens].cpu()
    with torch.no_grad():
        O.decoder_forward(sd, model.config, x[:, :128], labels=x[:, :128])
        t0 = time.perf_counter()
        loss = O.decoder_forward(sd, model.config, x, labels=x)["loss"].item()
        dt = time.perf_counter() - t0
    return {
        "value": tokens / dt,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"oracle/pe_oracle.py decoder_forward (fp32 weights, fp64 attention), all 24 layers, "
                  f"first {tokens} of the {DECODER['S']} tokens, one pass of {dt:.1f} s (loss {loss:.3f}); "
                  f"attention per token at {tokens} tokens is {tokens}/{DECODER['S']} of that at the full length",
        "seconds": dt,
    }


def run_decoder(args, torch, dev) -> dict:
    from pe_ablations_amd import _lib
    from pe_ablations_amd.gemm_select import use_tuned_gemms
    from pe_ablations_amd.transformer import Transformer

    # the projection GEMMs take the committed hipBLASLt selections (torch TunableOp, tuning off)
    gemm_selection = use_tuned_gemms()
    log(f"bench: decoder GEMMs: {gemm_selection}")
    cfg = _decoder_config(torch)
    S = DECODER["S"]
    torch.manual_seed(0)
    with torch.device(dev):
        model = Transformer(cfg)
    model = _bf16_weights(torch, model).eval()
    g = torch.Generator(device=dev).manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (1, S), generator=g, device=dev)
    nparam = sum(p.numel() for p in model.parameters())

    def step():
        with torch.inference_mode():
            return model(ids, labels=ids)["loss"]

    L = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    log(f"bench: decoder {nparam / 1e9:.2f}B params, warmup {args.warmup} forwards over {S} tokens")
    for _ in range(args.warmup):
        loss = step()
    torch.cuda.synchronize()
    loss = float(loss.float().item())
    expected = init_loss(cfg)
    if not abs(loss - expected) < 0.25:
        raise RuntimeError(f"decoder loss {loss:.4f} is not near ln(V) + 0.02^2 d / 2 = {expected:.4f}")
    evs, arrays = stage_events(torch, args.steps, stream)
    log(f"bench: timing {args.steps} forwards")
    ms = timed_loop(torch, L, step, arrays, args.steps)
    log(f"bench: {ms:.3f} ms/forward")
    stage_ms = stage_times(evs, ["fwd_prep", "fwd_core"])  # the last layer's attention call of each step
    Fd = decoder_flops(DECODER)
    H, D = DECODER["num_heads"], DECODER["head_dim"]
    attn_ms = stage_ms["fwd_prep"] + stage_ms["fwd_core"]
    return {
        "metric": "~1B PoPE decoder forward tokens/s @16k tokens (CE loss at init ~ ln 32000 + 0.02^2*2048/2)",
        "value": round(S / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (16384 uniform token ids; random-init weights N(0, 0.02^2))",
        "config": {"workload": "decoder forward with next-token CE loss", "layers": DECODER["num_layers"],
                   "d_model": DECODER["hidden_dim"], "heads": H, "head_dim": D, "ffn": DECODER["ffn_dim"],
                   "vocab": DECODER["vocab_size"], "tokens": S, "attention": "fused PoPE (all head dims)",
                   "params": nparam, "parallelism": "single GPU", "gemm_selection": gemm_selection},
        "loss": round(loss, 4),
        "expected_loss_at_init": round(expected, 4),
        "model_tflops": round(Fd["total"] / (ms * 1e-3) / 1e12, 2),
        "flops_per_forward": {k2: float(f"{v2:.4g}") for k2, v2 in Fd.items()},
        "attention_ms_per_layer": round(attn_ms, 4),
        "attention_share": round(attn_ms * DECODER["num_layers"] / ms, 4),
        "stage_ms": {k2: round(v2, 4) for k2, v2 in stage_ms.items()},
        "roofline": roofline("fwd_core", 3.0 * H * S * S * D, stage_ms["fwd_core"]),
        "_model": model,
        "_ids": ids,
    }


DECODE = dict(B=1, H=16, D=128, L=16384)


def run_decode(args, torch, dev) -> dict:
    """One decoded token per step at the 1B attention shape: the new key row is transformed into the
    cache (pe_attn_cache_append) and the new query attends to all L cached rows (pe_attn_decode,
    split-key kernel + merge).  Decode is bound by reading the cache, so the roofline entry is HBM
    bandwidth over the cache bytes one step must read: L rows of transformed keys (2D bf16) and
    values (D bf16) per head."""
    from pe_ablations_amd.functional import cache_widths, pe_attention_decode, pe_cache_append

    B, H, D, L = DECODE["B"], DECODE["H"], DECODE["D"], DECODE["L"]
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    k = torch.randn(B, H, L, D, generator=g, device=dev).to(bf)
    v = torch.randn(B, H, L, D, generator=g, device=dev).to(bf)
    q = torch.randn(B, H, 1, D, generator=g, device=dev).to(bf)
    delta = torch.rand(H, D, generator=g, device=dev) * (-2 * math.pi)
    freqs = (10000.0 ** (-(torch.arange(0, D, dtype=torch.float32) / D))).to(dev)
    wk, wv = cache_widths(mode="pope", d_pe=D, d_v=D)
    kc = torch.zeros(B, H, L, wk, dtype=bf, device=dev)
    vc = torch.zeros(B, H, L, wv, dtype=bf, device=dev)
    with torch.inference_mode():
        pe_cache_append(k[:, :, :L - 1], v[:, :, :L - 1], kc, vc, start_pos=0, freqs=freqs, delta=delta)

        def step():
            pe_cache_append(k[:, :, L - 1:], v[:, :, L - 1:], kc, vc, start_pos=L - 1, freqs=freqs, delta=delta)
            return pe_attention_decode(q, kc, vc, L, d_v=D, freqs=freqs, scale=1.0 / math.sqrt(D))

        log(f"bench: decode warmup {args.warmup} steps (B={B} H={H} D={D}, {L} cached rows)")
        for _ in range(args.warmup):
            out = step()
        torch.cuda.synchronize()
        if not torch.isfinite(out.float()).all():
            raise RuntimeError("non-finite decode output")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = B * H * L * (wk + wv) * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "fused PoPE KV-cache decode: cache GB/s per decoded token @16k cached rows, D=128; % of HBM peak",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "host_ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) keys / values / query, delta ~ U(-2pi,0) per head)",
        "config": {"workload": "one decoded token: cache append + split-key decode attention", "B": B, "H": H,
                   "D": D, "cached_rows": L, "parallelism": "single GPU"},
        "roofline": {"kernel": "decode_split_kernel + decode_merge_kernel + cache append", "bound": "hbm",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": nbytes},
    }


def decode_cpu_baseline(torch) -> dict:
    """The oracle's attention of one query against L cached rows (fp32 CPU, all host threads), one
    pass per head: the same arithmetic the decode step performs."""
    from oracle import pe_oracle as O
    B, H, D, L = DECODE["B"], DECODE["H"], DECODE["D"], DECODE["L"]
    g = torch.Generator().manual_seed(0)
    k, v, q = torch.randn(L, D, generator=g), torch.randn(L, D, generator=g), torch.randn(1, D, generator=g)
    delta = torch.rand(D, generator=g) * (-2 * math.pi)
    freqs = O.pope_freqs(D)
    O.pope_attention_chunked(q, k, v, freqs, delta, scale=1.0 / math.sqrt(D), start_q=L - 1)
    t0 = time.perf_counter()
    for _ in range(H):
        O.pope_attention_chunked(q, k, v, freqs, delta, scale=1.0 / math.sqrt(D), start_q=L - 1)
    dt = time.perf_counter() - t0
    wk = 2 * D
    return {"value": B * H * L * (wk + D) * 2 / dt / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(), "cpu": cpu_model(),
            "kind": "port",
            "sample": f"oracle pope_attention_chunked of 1 query against {L} keys, fp32, {H} heads one after "
                      f"another ({dt:.3f} s); bytes counted as the GPU cache bytes of the same step",
            "seconds": dt}


# (timed steps, warm-up steps) per workload: about half a second of untimed work, and timed work
# well under a minute
# query heads of one batch entry in the CPU baseline's sample (about 10-30 s of CPU work)
CPU_HEADS = {"fwdbwd": 2, "fwd": 2, "fwd32": 2, "c2": 12, "c3": 16, "split": 8, "masked": 4, "rope": 12}
CPU_REPS = {"c2": 40, "c3": 10, "fwd32": 12, "split": 1000, "masked": 4, "rope": 40}
DEFAULT_STEPS = {"fwdbwd": (50, 100), "fwd": (100, 400), "fwd32": (10, 40), "c2": (200, 600), "c3": (100, 250),
                 "split": (500, 2000), "masked": (50, 150), "rope": (200, 600), "decoder": (5, 4), "decode": (200, 200)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default per workload, DEFAULT_STEPS)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps (default per workload: about 0.5 s of work or more)")
    ap.add_argument("--workload", choices=list(ATTN_WORKLOADS) + ["decoder", "decode"], default="fwdbwd")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=None, help="CPU baseline sample: query heads at full S")
    ap.add_argument("--cpu-reps", type=int, default=None, help="CPU baseline: timed passes (default per workload)")
    ap.add_argument("--cpu-tokens", type=int, default=2048, help="decoder CPU baseline: tokens of the sample")
    ap.add_argument("--graph", action="store_true",
                    help="attention workloads: also time the step captured in a HIP graph and replayed "
                         "(ms_per_step then reports the replays; the eager figure stays in eager_ms_per_step)")
    args = ap.parse_args()
    dec = args.workload == "decoder"
    # Defaults: about half a second of untimed work before the timed steps.  Under this load the
    # chip runs at its socket power limit; after an idle host phase its clock and power state need
    # a few hundred milliseconds to settle, and timing from a 3-step warm-up measured the forward
    # 7-9 % and the fwd+bwd step 1.7 % slower than the settled state.
    args.steps = args.steps if args.steps is not None else DEFAULT_STEPS[args.workload][0]
    args.warmup = args.warmup if args.warmup is not None else DEFAULT_STEPS[args.workload][1]

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the PE attention path has no multi-GPU leg", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if dec:
        res = run_decoder(args, torch, dev)
    elif args.workload == "decode":
        res = run_decode(args, torch, dev)
    else:
        res = run_attention(args, torch, dev, args.workload)
    props = torch.cuda.get_device_properties(dev)
    res["device"] = {"name": props.name, "cus": props.multi_processor_count}
    model, ids = res.pop("_model", None), res.pop("_ids", None)
    if not args.no_cpu_baseline:
        if dec:
            log(f"bench: CPU baseline (decoder, {args.cpu_tokens} tokens)")
            cb = decoder_cpu_baseline(torch, model, ids, args.cpu_tokens)
        elif args.workload == "decode":
            log("bench: CPU baseline (decode)")
            cb = decode_cpu_baseline(torch)
        else:
            w = ATTN_WORKLOADS[args.workload]
            heads = args.cpu_heads if args.cpu_heads is not None else CPU_HEADS[args.workload]
            log(f"bench: CPU baseline ({heads} heads)")
            cb = cpu_baseline(w, min(heads, w["Hq"]), args.cpu_reps or CPU_REPS.get(args.workload, 4))
        res["cpu_baseline"] = {k2: v2 for k2, v2 in cb.items() if k2 != "seconds"}
        res["cpu_baseline"]["value"] = round(cb["value"], 5)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
