"""CPU checks of the measurement plumbing: rocprofv3 kernel-name normalisation and the committed
HBM-traffic summary that bench.py reports as roofline.traffic."""

import importlib.util
import json
import os

from pe_ablations_amd.profiling import _kernel_key

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_kernel_key():
    assert _kernel_key("void pe::dkdv_bf16_kernel<256, 128, 4>(pe::CoreArgs)") == "dkdv_bf16_kernel<256, 128, 4>"
    assert _kernel_key("pe::prep_pope_vec_kernel(pe::PrepArgs)") == "prep_pope_vec_kernel"
    assert _kernel_key("void pe::fwd_bf16_kernel<256, 128, 64, 8>(pe::CoreArgs, int)") == \
        "fwd_bf16_kernel<256, 128, 64, 8>"


def test_committed_traffic_covers_the_attention_kernels():
    bench = _bench()
    with open(bench.TRAFFIC_FILE) as f:
        data = json.load(f)
    cal = data["calibration"]
    # the calibration copy moves 1 GiB each way: the factors turn its own counts back into 1 GiB
    assert abs(cal["fetch_kib_counted"] * 1024 * cal["fetch_factor"] - (1 << 30)) < 1e-3 * (1 << 30)
    assert abs(cal["write_kib_counted"] * 1024 * cal["write_factor"] - (1 << 30)) < 1e-3 * (1 << 30)
    for stage in ("fwd_core", "bwd_dkdv", "bwd_dq"):
        traffic, name = bench.measured_traffic(stage)
        assert traffic is not None and traffic > 0, stage
        assert name.startswith(bench.STAGE_KERNEL[stage])
    # the dK/dV kernel writes the bf16 dS of the causal triangle, B*H*S^2/2 * 2 bytes at S = 16384
    dk = next(v for k, v in data["kernels"].items() if k.startswith(("dkdv_pair_kernel<", "dkdv_bf16_kernel<")))
    assert dk["write_bytes"] > 16 * 16384 * 16384 // 2 * 2 * 0.95


def test_workload_flops_and_prologue_bytes():
    """The general FLOP count reduces to 3 / 8 / 11 * B*H*S^2*D in the fused form, counts the split
    form's content width once and its positional width twice, and the prologue moves raw rows in
    and transformed rows out."""
    bench = _bench()
    w = bench.ATTN_WORKLOADS["fwdbwd"]
    F = bench.attn_flops(w)
    base = 1 * 16 * 16384 ** 2 * 128
    assert (F["fwd"], F["bwd"], F["total"], F["fa_convention"]) == (3 * base, 8 * base, 11 * base, 7 * base)
    assert F["fwd_core"] + F["bwd_dkdv"] + F["bwd_dq"] == F["total"]
    assert bench.flops(1, 16, 16384, 128) == F
    # q and k: 16 heads x 16384 rows of 128 bf16 in, 256 bf16 out
    assert bench.prologue_bytes(w) == 2 * 16 * 16384 * (128 + 256) * 2
    sp = bench.ATTN_WORKLOADS["split"]
    Fs = bench.attn_flops(sp)
    pairs = 8 * 8 * 512 * 512 / 2
    assert Fs["fwd"] == 2 * pairs * ((64 + 64) + 64)          # S~ over [content | cos | sin], PV over 64
    assert Fs["bwd"] == 2 * pairs * (3 * 128 + 2 * 64)
    assert bench.prologue_bytes(sp) == 8 * (8 + 4) * 512 * ((64 + 32) + (64 + 64)) * 2
    assert bench.prologue_bytes(bench.ATTN_WORKLOADS["fwd32"]) == 2 * bench.prologue_bytes(w)
    # RoPE: operands keep their width (64), so the C2-shape RoPE step is 7 * B*H*S^2*D / 2 per causal pair
    rw = bench.ATTN_WORKLOADS["rope"]
    Fr = bench.attn_flops(rw)
    rbase = 8 * 12 * 2048 ** 2 * 64
    assert (Fr["fwd"], Fr["total"]) == (2 * rbase, 7 * rbase)
    assert bench.prologue_bytes(rw) == 8 * 24 * 2048 * (64 + 64) * 2


def test_cpu_baseline_runs_every_form():
    """The cpu_baseline leg on tiny copies of the workloads (fused, FoPE, split form with GQA)."""
    bench = _bench()
    for name in ("fwdbwd", "c3", "split", "fwd", "rope"):
        w = dict(bench.ATTN_WORKLOADS[name], S=64)
        cb = bench.cpu_baseline(w, heads=2, reps=1)
        assert cb["value"] > 0 and cb["kind"] == "port" and cb["cores"] >= 1 and cb["cpu"]
