"""The oracle's PE transforms against vectors of the reference's own modules (tests/golden).

tests/golden/make_pe_golden.py evaluated PoPEEmbedding, FoPEPoPEEmbedding and the RoPE family
(src/model/pope.py, fpope.py, rope.py) with torch on the CPU and stored inputs, parameters and
outputs.  The oracle restates those modules from their source; here it must reproduce the stored
outputs: bit for bit where it issues the same torch operations on the same shapes (the PoPE and
FoPE transforms, frequency tables and clips), and within one float32 rounding where the reference
reaches the same values through another route (its precomputed complex table for RoPE, and YaRN's
mscale, formed in float32 by the reference and in float64 by the oracle).  Plausible mistakes in
the restatement (delta on queries, no key clamp, a rotate-half pairing) change the outputs far
beyond these bars, which the last tests show."""

import os

import numpy as np
import pytest
import torch

import oracle.pe_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pe_transforms.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: torch.from_numpy(f[k].copy()) for k in f.files}


def bshd(fn, x, *args, **kw):
    """Apply a (B, H, S, D) oracle transform to a reference-layout (B, S, H, D) tensor."""
    return fn(x.permute(0, 2, 1, 3), *args, **kw).permute(0, 2, 1, 3)


def ulps(a, b):
    """Largest distance in float32 units of the last place."""
    ia = a.contiguous().view(torch.int32).long()
    ib = b.contiguous().view(torch.int32).long()
    ia = torch.where(ia < 0, -(ia & 0x7fffffff), ia)
    ib = torch.where(ib < 0, -(ib & 0x7fffffff), ib)
    return int((ia - ib).abs().max())


@pytest.mark.parametrize("t", ["pope", "pope_floor"])
def test_pope_tables_and_transforms_bitwise(g, t):
    freqs = O.pope_freqs(16)
    if t == "pope_floor":
        freqs = O.floor_clip(freqs, 64)
        assert int((freqs == 0).sum()) == 11   # theta_i < 2 pi / 64 for i >= 5
    assert torch.equal(freqs, g[t + "_eff_freqs"])
    delta = O.clamp_delta(g[t + "_phase_bias"])
    assert delta[0] == 0.0 and delta[1] == np.float32(-2 * np.pi)   # both clamp ends taken
    for start in (0, 40, 70):
        q = bshd(O.pope_transform, g[f"{t}_{start}_xq"], freqs, start)
        k = bshd(O.pope_transform, g[f"{t}_{start}_xk"], freqs, start, delta=delta)
        assert torch.equal(q, g[f"{t}_{start}_q"]), (t, start, (q - g[f"{t}_{start}_q"]).abs().max())
        assert torch.equal(k, g[f"{t}_{start}_k"]), (t, start, (k - g[f"{t}_{start}_k"]).abs().max())


def test_pope_restatement_mistakes_miss(g):
    """The bar is not vacuous: the oracle with delta on queries, or without the key clamp, misses."""
    freqs = O.pope_freqs(16)
    raw = g["pope_phase_bias"]
    q_wrong = bshd(O.pope_transform, g["pope_0_xq"], freqs, 0, delta=O.clamp_delta(raw))
    k_wrong = bshd(O.pope_transform, g["pope_0_xk"], freqs, 0, delta=raw)
    assert (q_wrong - g["pope_0_q"]).abs().max() > 1e-2
    assert (k_wrong - g["pope_0_k"]).abs().max() > 1e-2


def test_fope_transforms_bitwise(g):
    freqs = O.fope_effective_freqs(g["fope_base_freqs"], g["fope_coeffs"], g["fope_indices"], training_length=64)
    delta = O.clamp_delta(g["fope_phase_bias"])
    for start in (0, 37):
        q = bshd(O.pope_transform, g[f"fope_{start}_xq"], freqs, start)
        k = bshd(O.pope_transform, g[f"fope_{start}_xk"], freqs, start, delta=delta)
        assert torch.equal(q, g[f"fope_{start}_q"]), (start, (q - g[f"fope_{start}_q"]).abs().max())
        assert torch.equal(k, g[f"fope_{start}_k"]), (start, (k - g[f"fope_{start}_k"]).abs().max())


def _rope_inv(t):
    if t == "rope":
        return O.rope_inv_freq(16), 1.0
    if t == "ntk":
        return O.rope_inv_freq(16, O.ntk_theta(16, 10000.0, 4.0)), 1.0
    inv, mscale, low, high = O.yarn_inv_freq(16, 10000.0, 4.0, original_max_seq_len=16)
    assert (low, high) == (0, 2)
    return inv, mscale


@pytest.mark.parametrize("t", ["rope", "ntk", "yarn"])
def test_rope_family_within_one_rounding(g, t):
    inv, mscale = _rope_inv(t)
    if t == "yarn":
        assert ulps(torch.tensor(mscale, dtype=torch.float32), g["yarn_mscale"]) <= 1
    for start in (0, 29):
        for side in ("q", "k"):
            x = g[f"{t}_{start}_x{side}"]
            y = bshd(O.rope_rotate_complex, x, inv, start)
            if t == "yarn":
                y = y * g["yarn_mscale"]
            ref = g[f"{t}_{start}_{side}"]
            # same values by another route: a product of a rounded cos / sin with x, so within a
            # rounding of the largest term of each output element
            tol = 2 * torch.finfo(torch.float32).eps * x.abs().amax(dim=-1, keepdim=True)
            assert ((y - ref).abs() <= tol.expand_as(ref)).all(), (t, start, side, (y - ref).abs().max())
            # the real-arithmetic restatement agrees as closely
            y2 = bshd(O.rope_rotate, x, inv, start)
            if t == "yarn":
                y2 = y2 * g["yarn_mscale"]
            assert ((y2 - ref).abs() <= tol.expand_as(ref)).all(), (t, start, side, (y2 - ref).abs().max())


def test_rope_pairing_mistake_misses(g):
    """A rotate-half pairing (dims i and i + D/2) in place of interleaved pairs misses."""
    x = g["rope_29_xq"]
    inv = O.rope_inv_freq(16)
    half = torch.cat([x[..., 0::2], x[..., 1::2]], dim=-1)     # reorder so pairs become halves
    y = bshd(O.rope_rotate, half, inv, 29)
    assert (y - g["rope_29_q"]).abs().max() > 1e-1
