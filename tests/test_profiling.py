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
