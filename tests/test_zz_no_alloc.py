"""pe_attn_fwd_noalloc: the forward with its workspace in the library's static device scratch.

Called through the C ABI (ctypes) and compared with pe_attn_fwd on a caller workspace: both run the
same kernels on the same operands, so out and lse must agree bit for bit.  Two calls in a row, the
second on a smaller problem, check that the shared scratch carries nothing over from the last call;
a problem whose workspace exceeds the scratch must be refused with PE_ERR_SCRATCH_LIMIT before any
launch."""

import ctypes
import math

import pytest
import torch

from pe_ablations_amd import _lib
from pe_ablations_amd.functional import _params, _tensor

pytestmark = pytest.mark.gpu


def _case(cuda, B, H, S, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, S, H, D, generator=g).to(dtype).to(cuda).transpose(1, 2) for _ in range(3))
    freqs = (10000.0 ** (-(torch.arange(D, dtype=torch.float32) / D))).to(cuda)
    delta = (torch.rand(H, D, generator=g) * (-2 * math.pi)).to(cuda)
    cfg = dict(mode=_lib.PE_MODE_POPE, dtype=_lib.PE_DTYPE_BF16 if dtype == torch.bfloat16 else _lib.PE_DTYPE_FP32,
               causal=_lib.PE_CAUSAL_TOP_LEFT, start_pos_q=0, start_pos_k=0, qk_norm=False,
               scale=1.0 / math.sqrt(D), mscale=1.0, pos_round=_lib.PE_POS_EXACT)
    return q, k, v, freqs, delta, cfg


def _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc):
    p = _params(cfg, q, k, v, None, delta)
    B, H, S, D = q.shape
    out = torch.empty((B, S, H, D), dtype=q.dtype, device=cuda).transpose(1, 2)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=cuda)
    stream = torch.cuda.current_stream(cuda).cuda_stream
    args = (ctypes.byref(p), ctypes.byref(_tensor(None)), ctypes.byref(_tensor(q)), ctypes.byref(_tensor(None)),
            ctypes.byref(_tensor(k)), ctypes.byref(_tensor(v)), freqs.data_ptr(), delta.data_ptr(),
            ctypes.byref(_tensor(out)), lse.data_ptr())
    if noalloc:
        rc = L.pe_attn_fwd_noalloc(*args, stream)
    else:
        nb = L.pe_attn_fwd_workspace_bytes(ctypes.byref(p))
        ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
        rc = L.pe_attn_fwd(*args, ws.data_ptr(), nb, stream)
    torch.cuda.synchronize()
    return rc, out, lse


def test_noalloc_forward_matches_workspace_forward(cuda):
    L = _lib.lib()
    limit = L.pe_attn_noalloc_scratch_bytes()
    assert limit == 128 << 20
    for B, H, S, D, seed in ((2, 4, 1000, 64, 1), (1, 2, 300, 128, 2)):   # the second call is smaller
        q, k, v, freqs, delta, cfg = _case(cuda, B, H, S, D, seed)
        rc0, out0, lse0 = _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=False)
        rc1, out1, lse1 = _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=True)
        assert rc0 == 0 and rc1 == 0, (rc0, rc1)
        assert torch.equal(out0, out1), (B, H, S, D, (out0.float() - out1.float()).abs().max().item())
        assert torch.equal(lse0, lse1)


def test_noalloc_forward_fp32_and_limit(cuda):
    L = _lib.lib()
    q, k, v, freqs, delta, cfg = _case(cuda, 1, 3, 257, 64, 3, dtype=torch.float32)
    rc0, out0, lse0 = _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=False)
    rc1, out1, lse1 = _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=True)
    assert rc0 == 0 and rc1 == 0
    assert torch.equal(out0, out1) and torch.equal(lse0, lse1)
    # a forward workspace above the scratch (16 heads of 16384 rows: 128 MiB each of q~ and k~) is
    # refused before anything is enqueued; the tensors are real ones of that size
    q, k, v, freqs, delta, cfg = _case(cuda, 1, 16, 16384, 128, 4)
    big = _params(cfg, q, k, v, None, delta)
    assert L.pe_attn_fwd_workspace_bytes(ctypes.byref(big)) > L.pe_attn_noalloc_scratch_bytes()
    rc, _, _ = _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=True)
    assert rc == _lib.ERRORS["PE_ERR_SCRATCH_LIMIT"]
    assert "static scratch" in L.pe_attn_strerror(rc).decode()


_RESERVE_PROBE = r"""
import sys, torch
sys.path[:0] = [{root!r}, {tests!r}]
from test_zz_no_alloc import _case, _run
from pe_ablations_amd import _lib
cuda = torch.device("cuda:0")
torch.zeros(1, device=cuda)
torch.cuda.synchronize()
def outside_torch():
    return torch.cuda.mem_get_info()[0] + torch.cuda.memory_reserved()
f0 = outside_torch()
L = _lib.lib()
q, k, v, freqs, delta, cfg = _case(cuda, 1, 2, 300, 128, 2)
assert _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=False)[0] == 0
f1 = outside_torch()
assert _run(L, cuda, q, k, v, freqs, delta, cfg, noalloc=True)[0] == 0
f2 = outside_torch()
print("RESULT", f0 - f1, f1 - f2)
"""


def test_scratch_is_reserved_only_once_noalloc_runs(cuda):
    """The 128 MiB scratch lives in the code object of the translation unit that defines it, which
    the HIP runtime loads on the first use of that code object (deferred loading, its default): the
    first pe_attn_fwd_noalloc call resolves the symbol.  A fresh process that loads the library and
    runs the workspace forward therefore holds no scratch; the first no-alloc call then takes it.
    Device memory outside torch's caching allocator is compared in a child process (this one may
    already hold the scratch from the tests above)."""
    import os
    import subprocess
    import sys
    tests = os.path.dirname(os.path.abspath(__file__))
    env = {k: v for k, v in os.environ.items() if k != "HIP_ENABLE_DEFERRED_LOADING"}
    r = subprocess.run([sys.executable, "-c", _RESERVE_PROBE.format(root=os.path.dirname(tests), tests=tests)],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-2000:]
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("RESULT")][-1]
    before, at_first_noalloc = (int(x) for x in line.split()[1:])
    mib = 1 << 20
    assert before < 64 * mib, before / mib          # code objects of the kernels used, no scratch
    assert at_first_noalloc >= 128 * mib, at_first_noalloc / mib
