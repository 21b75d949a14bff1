"""Host-side behaviour of the drop-in modules (no GPU): reference state-dict names (so reference
checkpoints load), constructor semantics, the frequency tables they hand to the kernel, the
YaRN-after-extend quirk, and that the hot path refuses CPU tensors instead of falling back."""

import math

import pytest
import torch

from oracle import pe_oracle as O
from pe_ablations_amd.attention import GroupedQueryAttention
from pe_ablations_amd.fpope import FoPEPoPEEmbedding
from pe_ablations_amd.fpope_attention import FPoPEGroupedQueryAttention, FPoPEGroupedQueryAttentionWithCache
from pe_ablations_amd.functional import pe_attention
from pe_ablations_amd.kernels import fpope_attention_forward
from pe_ablations_amd.pope import PoPEEmbedding
from pe_ablations_amd.rope import NTKAwareRotaryEmbedding, RotaryEmbedding, YaRNRotaryEmbedding


def test_pope_state_and_tables():
    """src/model/pope.py:71-97: buffers freqs / effective_freqs / base_angles, parameter phase_bias."""
    p = PoPEEmbedding(32, 512, use_floor=True, training_length=512)
    assert sorted(p.state_dict()) == ["base_angles", "effective_freqs", "freqs", "phase_bias"]
    assert torch.equal(p.freqs, O.pope_freqs(32))
    assert torch.equal(p.effective_freqs, O.floor_clip(O.pope_freqs(32), 512))
    assert torch.equal(p.base_angles, torch.outer(torch.arange(512, dtype=torch.float32), p.effective_freqs))
    assert torch.equal(p.phase_bias, torch.zeros(32))
    u = PoPEEmbedding(16, 64, delta_init="uniform")
    assert (u.phase_bias <= 0).all() and (u.phase_bias >= -2 * math.pi).all()
    d = torch.tensor([-9.0, -1.0, 2.0] + [0.0] * 13)
    u.phase_bias.data.copy_(d)
    assert torch.equal(u.kernel_delta(), O.clamp_delta(d))
    p.extend_seq_len(2048)
    assert p.base_angles.shape == (2048, 32) and p.max_seq_len == 2048
    assert "base_angles" not in p.state_dict()  # re-registered non-persistent, as the reference does


def test_fope_state_and_effective_freqs():
    """src/model/fpope.py:81-146: buffers / parameters and the frequency collapse."""
    torch.manual_seed(0)
    f = FoPEPoPEEmbedding(32, 512, num_fourier_terms=8, training_length=512, use_ceiling=True)
    assert sorted(f.state_dict()) == ["base_freqs", "fourier_coeffs", "fourier_indices", "phase_bias", "positions"]
    assert f.fourier_coeffs.shape == (32, 8) and f.positions.shape == (512,)
    ref = O.fope_effective_freqs(f.base_freqs, f.fourier_coeffs.detach(), f.fourier_indices,
                                 training_length=512, use_ceiling=True)
    assert torch.equal(f.kernel_freqs().detach(), ref)
    frozen = FoPEPoPEEmbedding(8, 64, num_fourier_terms=4, freeze_coeffs=True)
    assert not frozen.fourier_coeffs.requires_grad
    u = FoPEPoPEEmbedding(8, 64, num_fourier_terms=4, delta_init="uniform")
    assert (u.phase_bias.abs() <= math.pi).all()       # U(-pi, pi) for FoPE (src/model/fpope.py:100)
    ph = f.compute_attention_phases(5, 5)
    assert ph.shape == (5, 5, 32)
    assert torch.allclose(ph[2, 2], f.phase_bias.detach())
    f.extend_seq_len(4096)
    assert f.positions.shape == (4096,)


def test_rope_tables_and_yarn_extend_quirk():
    r = RotaryEmbedding(64, 128)
    assert torch.equal(r.inv_freq, O.rope_inv_freq(64))
    assert r.freqs_cis.shape == (128, 32) and r.freqs_cis.dtype == torch.complex64
    assert "freqs_cis" not in r.state_dict()
    n = NTKAwareRotaryEmbedding(64, 128, scale=4.0)
    assert abs(n.theta - O.ntk_theta(64, 10000.0, 4.0)) < 1e-6
    y = YaRNRotaryEmbedding(64, 128, scale=4.0)
    inv, ms, low, high = O.yarn_inv_freq(64, 10000.0, 4.0)
    assert (y.low, y.high) == (low, high) == (6, 31)
    assert torch.allclose(y.inv_freq, inv) and abs(y.kernel_mscale() - ms) < 1e-6
    y.extend_seq_len(1024)     # reference quirk: standard frequencies after extending, mscale kept
    assert torch.equal(y.inv_freq, O.rope_inv_freq(64))
    assert abs(y.kernel_mscale() - ms) < 1e-6


def test_attention_module_state_dict_names():
    pe = PoPEEmbedding(32, 512)
    m = FPoPEGroupedQueryAttention(512, 8, 4, 64, 32, fpope=pe, use_triton=False)
    assert sorted(k for k in m.state_dict() if not k.startswith("fpope.")) == sorted(
        ["wq_c.weight", "wk_c.weight", "wq_r.weight", "wk_r.weight", "qr_norm.weight", "kr_norm.weight",
         "wv.weight", "wo.weight"])
    assert abs(m.scale - (64 + 64) ** -0.5) < 1e-12
    c = FPoPEGroupedQueryAttentionWithCache(256, 4, 2, 64, 32, fpope=pe, max_cache_len=128)
    assert c.k_cache is None and c.cache_len == 0
    g = GroupedQueryAttention(512, 8, 4, 64, use_qk_norm=True, rope=RotaryEmbedding(64, 512))
    assert sorted(g.state_dict()) == ["wk.weight", "wo.weight", "wq.weight", "wv.weight"]


def test_hot_path_refuses_cpu_tensors():
    """No CPU fallback: the fused path raises on CPU tensors."""
    q = torch.randn(1, 2, 8, 16)
    with pytest.raises(RuntimeError, match="GPU only"):
        pe_attention(q, q, q, freqs=O.pope_freqs(16), delta=torch.zeros(16))
    with pytest.raises(RuntimeError, match="GPU only"):
        fpope_attention_forward(q, q, q, O.pope_freqs(16), torch.zeros(16))
    m = FPoPEGroupedQueryAttention(64, 2, 2, 16, 8, fpope=PoPEEmbedding(8, 64))
    with pytest.raises(RuntimeError, match="GPU only"):
        m(torch.randn(1, 4, 64))
    with pytest.raises(RuntimeError, match="GPU only"):
        PoPEEmbedding(8, 64).forward_query(torch.randn(1, 4, 2, 8))
