"""The library's modules on the GPU against vectors of the reference's own modules (tests/golden).

PoPEEmbedding / FoPEPoPEEmbedding.forward_query / forward_key and the RoPE family's forward run the
HIP transform kernels (fp32 in, fp32 out) with the stored parameters; the stored outputs are what
torch-CPU gave for the reference's modules (tests/golden/make_pe_golden.py).  The kernels evaluate
sin / cos with their own routine (max abs error 9.2e-8 against float64) and softplus within a few
float32 roundings of torch's, so each output element is held to 2e-6 times max(1, its magnitude
factor): mu = softplus(x) for PoPE and FoPE, the largest |x| of the row for RoPE."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from pe_ablations_amd.fpope import FoPEPoPEEmbedding
from pe_ablations_amd.pope import PoPEEmbedding
from pe_ablations_amd.rope import NTKAwareRotaryEmbedding, RotaryEmbedding, YaRNRotaryEmbedding
from tests.test_golden import GOLD

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: torch.from_numpy(f[k].copy()) for k in f.files}


def check_pope(y, x, ref, tag, phase_err=None):
    """phase_err (S, D): a bound on how far the phases the kernel was given sit from the
    reference's, which moves mu cos / mu sin by up to mu times that much."""
    mu = F.softplus(x).repeat(1, 1, 1, 2)          # [mu | mu] beside [mu cos | mu sin]
    err = (y.cpu() - ref).abs()
    bar = 2e-6 * torch.clamp(mu, min=1.0)
    if phase_err is not None:
        bar = bar + mu * phase_err.repeat(1, 2).view(1, x.shape[1], 1, 2 * x.shape[3])
    assert (err <= bar).all(), (tag, err.max().item(), (err / bar).max().item())


@pytest.mark.parametrize("floor", [False, True])
def test_pope_module_matches_reference_vectors(cuda, g, floor):
    t = "pope_floor" if floor else "pope"
    m = PoPEEmbedding(16, max_seq_len=64, training_length=64, use_floor=floor, delta_init="uniform")
    with torch.no_grad():
        m.phase_bias.copy_(g[t + "_phase_bias"])
    m = m.to(cuda)
    assert torch.equal(m.effective_freqs.cpu(), g[t + "_eff_freqs"])
    with torch.no_grad():
        for start in (0, 40, 70):
            xq, xk = g[f"{t}_{start}_xq"], g[f"{t}_{start}_xk"]
            check_pope(m.forward_query(xq.to(cuda), start), xq, g[f"{t}_{start}_q"], (t, start, "q"))
            check_pope(m.forward_key(xk.to(cuda), start), xk, g[f"{t}_{start}_k"], (t, start, "k"))


def test_fope_module_matches_reference_vectors(cuda, g):
    """The collapse to one frequency per dim runs as torch ops on the device, as in the reference,
    and torch's device reduction over the Fourier terms may round a frequency differently from its
    CPU one (by an ulp).  The CPU collapse here is the oracle's, bitwise the reference's own
    (tests/test_golden.py); each output is held to the kernel bar plus what the frequency
    difference moves its phase by (position times the difference, plus one rounding of the phase)."""
    import oracle.pe_oracle as O
    m = FoPEPoPEEmbedding(16, max_seq_len=64, num_fourier_terms=4, training_length=64, delta_init="uniform")
    with torch.no_grad():
        m.fourier_coeffs.copy_(g["fope_coeffs"])
        m.phase_bias.copy_(g["fope_phase_bias"])
    m = m.to(cuda)
    w_cpu = O.fope_effective_freqs(g["fope_base_freqs"], g["fope_coeffs"], g["fope_indices"], training_length=64)
    with torch.no_grad():
        w_dev = m.kernel_freqs().cpu()
        dw = (w_dev - w_cpu).abs()
        assert (dw <= 2 * torch.finfo(torch.float32).eps * w_cpu.abs()).all(), dw.max()
        for start in (0, 37):
            xq, xk = g[f"fope_{start}_xq"], g[f"fope_{start}_xk"]
            pos = torch.arange(start, start + xq.shape[1], dtype=torch.float32)
            # both phases are rounded products: where the frequencies differ, add one rounding of the phase
            perr = torch.outer(pos, dw) + (dw > 0) * torch.finfo(torch.float32).eps * torch.outer(pos, w_cpu).abs()
            check_pope(m.forward_query(xq.to(cuda), start), xq, g[f"fope_{start}_q"], ("fope", start, "q"), perr)
            check_pope(m.forward_key(xk.to(cuda), start), xk, g[f"fope_{start}_k"], ("fope", start, "k"), perr)


@pytest.mark.parametrize("t", ["rope", "ntk", "yarn"])
def test_rope_modules_match_reference_vectors(cuda, g, t):
    m = {"rope": lambda: RotaryEmbedding(16, max_seq_len=64),
         "ntk": lambda: NTKAwareRotaryEmbedding(16, max_seq_len=64, scale=4.0),
         "yarn": lambda: YaRNRotaryEmbedding(16, max_seq_len=64, scale=4.0, original_max_seq_len=16)}[t]().to(cuda)
    with torch.no_grad():
        for start in (0, 29):
            xq, xk = g[f"{t}_{start}_xq"], g[f"{t}_{start}_xk"]
            yq, yk = m(xq.to(cuda), xk.to(cuda), start)
            for y, x, side in ((yq, xq, "q"), (yk, xk, "k")):
                ref = g[f"{t}_{start}_{side}"]
                err = (y.cpu() - ref).abs()
                bar = 2e-6 * torch.clamp(x.abs().amax(dim=-1, keepdim=True), min=1.0)
                assert (err <= bar).all(), (t, start, side, err.max().item())
