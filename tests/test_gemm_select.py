"""The committed hipBLASLt selections for the decoder's GEMMs (pe_ablations_amd/gemm_select.py): the
TunableOp results file covers the four bf16 GEMM shapes of a 16384-token forward of the ~1B
decoder (src/model/transformer.py: q / k / v / o projections, SwiGLU w1 / w3 and w2, the tied LM
head) and carries the validators that pin it to this stack."""

import os

import torch

from pe_ablations_amd import gemm_select


def test_tuned_file_covers_the_decoder_shapes():
    rows = gemm_select.tuned_shapes()
    shapes = {r[1] for r in rows}
    tokens, d, ffn, vocab = 16384, 2048, 5632, 32000
    want = {f"tn_{d}_{tokens}_{d}_ld_{d}_{d}_{d}",              # q / k / v / o projections
            f"tn_{ffn}_{tokens}_{d}_ld_{d}_{d}_{ffn}",          # w1, w3
            f"tn_{d}_{tokens}_{ffn}_ld_{ffn}_{ffn}_{d}",        # w2
            f"tn_{vocab}_{tokens}_{d}_ld_{d}_{d}_{vocab}"}      # LM head
    assert want <= shapes
    assert all(r[0] == "GemmTunableOp_BFloat16_TN" and r[2].startswith("Gemm_Hipblaslt_") and r[3] > 0 for r in rows)


def test_tuned_file_validators_name_this_gpu():
    with open(gemm_select.TUNED_FILE) as f:
        val = dict(line.strip().split(",")[1:3] for line in f if line.startswith("Validator"))
    assert val["GCN_ARCH_NAME"].startswith("gfx950")
    assert {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION"} <= set(val)


def test_use_tuned_gemms_reports_what_it_did():
    """use_tuned_gemms switches TunableOp on for the whole process; the test puts torch's TunableOp
    state back afterwards so that later tests' GEMMs do not depend on whether this one ran."""
    from torch.cuda import tunable
    gpu = torch.cuda.is_available()  # the TunableOp calls need a device
    state = (tunable.is_enabled(), tunable.tuning_is_enabled(), tunable.get_filename()) if gpu else None
    try:
        msg = gemm_select.use_tuned_gemms()
        if not torch.cuda.is_available():
            assert msg == "hipBLASLt default heuristic (no GPU)"
        else:
            assert "TunableOp" in msg or "default heuristic" in msg
        assert not any(n.startswith("pe_tunableop_") for n in os.listdir(os.path.dirname(gemm_select.TUNED_FILE)))
    finally:
        if gpu:
            tunable.enable(state[0])
            tunable.tuning_enable(state[1])
            tunable.set_filename(state[2])
