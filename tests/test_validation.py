"""Operand validation ahead of every launch (CPU: the shape checks are pure host logic).

The C ABI carries pointers and strides only, so a mismatch the host does not catch reaches the
kernels as an out-of-bounds access.  Each case below must raise ValueError from the checker that
pe_attention / pe_transform call before anything is enqueued; the GPU test at the end shows the
public entry raising with a CPU-resident delta and a short freqs."""

import pytest
import torch

from pe_ablations_amd import _lib
from pe_ablations_amd.functional import check_operands
from pe_ablations_amd.transform import check_transform_operands

POPE, ROPE, NONE = _lib.PE_MODE_POPE, _lib.PE_MODE_ROPE, _lib.PE_MODE_NONE


def z(*s):
    return torch.zeros(*s)


def good(**over):
    d = dict(q=z(2, 4, 8, 16), k=z(2, 2, 10, 16), v=z(2, 2, 10, 32), q_c=None, k_c=None, freqs=z(16),
             delta=z(2, 16), mode=POPE)
    d.update(over)
    return d


def call(d):
    kw = dict(d)
    q, k, v = kw.pop("q"), kw.pop("k"), kw.pop("v")
    check_operands(q, k, v, **kw)


def test_valid_operands_pass():
    call(good())
    call(good(delta=z(16)))
    call(good(delta=None))
    call(good(q_c=z(2, 4, 8, 64), k_c=z(2, 2, 10, 64)))
    call(good(mode=ROPE, freqs=z(8), delta=None))
    call(good(mode=NONE, freqs=None, delta=None))
    call(good(q_norm_weight=z(64), k_norm_weight=z(32)))


@pytest.mark.parametrize("over, what", [
    (dict(k=z(3, 2, 10, 16)), "batch"),
    (dict(k=z(2, 2, 10, 8)), "width"),
    (dict(k=z(2, 3, 10, 16), v=z(2, 3, 10, 32)), "multiple"),
    (dict(v=z(2, 2, 9, 32)), "v "),
    (dict(v=z(2, 1, 10, 32)), "v "),
    (dict(v=z(1, 2, 10, 32)), "v "),
    (dict(q=z(2, 4, 8)), "(B, H, S, D)"),
    (dict(q_c=z(2, 4, 8, 64)), "together"),
    (dict(q_c=z(2, 4, 7, 64), k_c=z(2, 2, 10, 64)), "rows"),
    (dict(q_c=z(2, 4, 8, 64), k_c=z(2, 2, 10, 32)), "widths"),
    (dict(freqs=z(8)), "freqs"),
    (dict(freqs=None), "freqs"),
    (dict(freqs=z(16, 1)), "freqs"),
    (dict(mode=ROPE, freqs=z(16), delta=None), "freqs"),
    (dict(delta=z(8)), "delta"),
    (dict(delta=z(4, 16)), "delta"),
    (dict(delta=z(1, 16)), "delta"),
    (dict(mode=ROPE, freqs=z(8)), "delta"),
    (dict(q_norm_weight=z(63)), "qr_norm_weight"),
    (dict(k_norm_weight=z(64)), "kr_norm_weight"),
])
def test_mismatch_raises(over, what):
    with pytest.raises(ValueError, match=what.replace("(", r"\(").replace(")", r"\)")):
        call(good(**over))


def test_device_mismatch_raises():
    # a meta tensor stands in for "another device" on a CPU-only host
    with pytest.raises(ValueError, match="one device"):
        call(good(delta=torch.zeros(2, 16, device="meta")))
    with pytest.raises(ValueError, match="one device"):
        call(good(freqs=torch.zeros(16, device="meta")))


def test_transform_checks():
    check_transform_operands(z(1, 8, 2, 16), z(16), z(2, 16), mode="pope", is_key=True)
    check_transform_operands(z(1, 8, 2, 16), z(8), None, mode="rope", is_key=False)
    with pytest.raises(ValueError, match="freqs"):
        check_transform_operands(z(1, 8, 2, 16), z(8), None, mode="pope", is_key=False)
    with pytest.raises(ValueError, match="delta"):
        check_transform_operands(z(1, 8, 2, 16), z(16), z(3, 16), mode="pope", is_key=True)
    with pytest.raises(ValueError, match="even"):
        check_transform_operands(z(1, 8, 2, 15), z(7), None, mode="rope", is_key=False)
    with pytest.raises(ValueError, match="x must be"):
        check_transform_operands(z(8, 2, 16), z(16), None, mode="pope", is_key=False)
    with pytest.raises(ValueError, match="freqs is on"):
        check_transform_operands(z(1, 8, 2, 16), torch.zeros(16, device="meta"), None, mode="pope", is_key=False)


@pytest.mark.gpu
def test_public_entry_raises_before_launch(cuda):
    from pe_ablations_amd.functional import pe_attention
    q = torch.randn(1, 2, 64, 16, device=cuda, dtype=torch.bfloat16)
    freqs = torch.ones(16, device=cuda)
    with pytest.raises(ValueError, match="one device"):
        pe_attention(q, q, q, mode="pope", freqs=freqs, delta=torch.zeros(16))
    with pytest.raises(ValueError, match="freqs"):
        pe_attention(q, q, q, mode="pope", freqs=freqs[:8])
    with pytest.raises(ValueError, match="v "):
        pe_attention(q, q, q[:, :, :32], mode="pope", freqs=freqs)
    torch.cuda.synchronize()
