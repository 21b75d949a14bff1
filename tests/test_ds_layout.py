"""The packed dS layout (pe_internal.h: ds_first / ds_row_base) against a replay of the kernels.

The bf16 backward stores dS in 4 KiB blocks (32 keys x 64 queries), key-row major, packed per
(batch, head) to the blocks the causal dK/dV kernels write; the dQ GEMM reads them back.  This
replays, on the CPU, the loop bounds of the writers (32-query tiles from max(0, k0 - off) / 32:
dkdv_pair_kernel; 64-query tiles from max(0, k0 - off) / 64: dkdv_pair_kernel at QK width 128 and V
width 64, and dkdv_bf16_kernel; all per 128-key block) and of the reader (dq_gemm_kernel: 256-query blocks, key steps up to
min(Sk, q0 + 256 + off), unmasked steps below min(Sk, q0 + off + 1), masked fragments elsewhere),
and checks that

* no two written blocks share an address and every written block lies inside its (b, h) region;
* every dS element the reader uses unmasked was written (by block and 32-query half);
* every address the reader loads, masked ones included, lies inside the B * Hq regions that
  pe_attn_bwd_workspace_bytes sizes (the reads before a row's first block fall in earlier rows),
  and never past its own head's region, so that a head group indexed from its first head (the
  capped backward, PE_BWD_DS_CAP_BYTES) reads only its own regions.

The closed form of ds_row_base is also compiled from pe_internal.h on the host and compared with
the running sum of the row lengths it must equal."""

import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def first(kb, e, causal):
    return max(0, 2 * kb - e) if causal else 0


def row_base_sum(r, e, nqt, causal):
    """Brute force: the rows before r hold nqt - first(r' / 4) blocks each."""
    return sum(nqt - first(rr // 4, e, causal) for rr in range(r))


def row_base(r, e, nqt, causal):
    if not causal:
        return r * nqt
    K, m = r // 4, (e + 1) // 2
    n = max(0, K - m)
    return r * nqt - 4 * n * (K - 1 + m - e) - (r % 4) * first(K, e, causal)


def addr(r, j, e, nqt, causal):
    return row_base(r, e, nqt, causal) + j - first(r // 4, e, causal)


def geometry(Sq, Sk, causal, bottom_right):
    off = Sk - Sq if bottom_right else 0
    nqt64 = (Sq + 255) // 256 * 4
    rows = (Sk + 127) // 128 * 128
    R = rows // 128
    e = (off + 63) // 64 if causal else 0
    return off, nqt64, R, e


def written(Sq, Sk, causal, bottom_right, pair):
    """{(row, j, half)} stored by the dK/dV kernel of one (b, h): 32-query tiles (pair) or 64."""
    off, _, R, _ = geometry(Sq, Sk, causal, bottom_right)
    out = set()
    for kb in range(R):
        k0 = 128 * kb
        if pair:
            nqt = (Sq + 31) // 32
            qb0 = min(max(0, k0 - off) // 32, nqt) if causal else 0
            for qt in range(qb0, nqt):
                for pw in range(4):
                    out.add((4 * kb + pw, qt >> 1, qt & 1))
        else:
            nqb = (Sq + 63) // 64
            qb0 = min(max(0, k0 - off) // 64, nqb) if causal else 0
            for qt in range(qb0, nqb):
                for pw in range(4):
                    out.add((4 * kb + pw, qt, 0))
                    out.add((4 * kb + pw, qt, 1))
    return out


CASES = [(512, 512, True, False), (1000, 1000, True, False), (300, 300, False, False), (200, 1000, True, True),
         (64, 4100, True, True), (1, 700, True, True), (2048, 2048, True, False), (777, 777, True, False),
         (256, 1024, False, False), (100, 164, True, True)]


@pytest.mark.parametrize("Sq, Sk, causal, br", CASES)
@pytest.mark.parametrize("pair", [True, False])
def test_packed_ds_layout_covers_every_read(Sq, Sk, causal, br, pair):
    off, nqt64, R, e = geometry(Sq, Sk, causal, br)
    head = row_base(4 * R, e, nqt64, causal)
    for r in range(4 * R + 1):
        assert row_base(r, e, nqt64, causal) == row_base_sum(r, e, nqt64, causal)
    W = written(Sq, Sk, causal, br, pair)
    addrs = {}
    for (row, j, half) in W:
        assert first(row // 4, e, causal) <= j < nqt64, (row, j)
        a = addr(row, j, e, nqt64, causal)
        assert 0 <= a < head
        assert addrs.setdefault(a, (row, j)) == (row, j), "two blocks share an address"
    nheads = 3   # region h starts at h * head; reads must stay inside [0, nheads * head)
    for hh in range(nheads):
        for bk in (32, 64):   # the dQ GEMM's key step: 32 for 128/256-wide k~, 64 otherwise
            for qb in range((Sq + 255) // 256):
                q0, j0 = 256 * qb, 4 * qb
                kend = min(Sk, q0 + 256 + off) if causal else Sk
                nkb = (kend + bk - 1) // bk if kend > 0 else 0
                kfull = min(Sk, q0 + off + 1) if causal else Sk
                nfull = min(nkb, max(kfull, 0) // bk)
                for kb in range(nkb):
                    for kl in range(0, bk, 32):
                        row = (kb * bk + kl) // 32
                        for j in range(j0, j0 + 4):
                            a = hh * head + addr(row, j, e, nqt64, causal)
                            assert 0 <= a < nheads * head, (hh, qb, kb, row, j, a, head)
                            # never past the head's own region: with head 0 never before the
                            # buffer, a group of n heads (the capped backward runs the kernels over
                            # groups, indexing dS from the group's first head) reads [0, n * head)
                            assert a < (hh + 1) * head, (hh, qb, kb, row, j, a, head)
                            for half in (0, 1):
                                qlo = 64 * j + 32 * half
                                if qlo >= Sq:
                                    continue   # padding queries: their dq rows are never stored
                                qhi = min(qlo + 31, Sq - 1)
                                klo = row * 32
                                if kb < nfull:
                                    used = klo < Sk   # unmasked step: every element is used
                                else:
                                    used = klo < Sk and (not causal or klo <= qhi + off)
                                if used:
                                    assert (row, j, half) in W, ("read of an unwritten block", qb, kb, row, j, half)


def test_row_base_matches_header():
    hipcc = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else None)
    if hipcc is None:
        pytest.skip("hipcc is not available")
    src = r'''
#include "pe_internal.h"
#include <stdio.h>
int main() {
  for (int causal = 0; causal < 2; ++causal)
    for (int nqt = 4; nqt <= 12; nqt += 4)
      for (int e = 0; e <= 5; ++e)
        for (int r = 0; r <= 40; r += 3)
          printf("%d %d %d %d %lld %d\n", causal, nqt, e, r, (long long)pe::ds_row_base(r, e, nqt, causal),
                 pe::ds_first(r / 4, e, causal));
  return 0;
}
'''
    with tempfile.TemporaryDirectory() as d:
        cpp, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(cpp, "w").write(src)
        r = subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-I",
                            os.path.join(ROOT, "pe_ablations_amd", "csrc"), cpp, "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        out = subprocess.run([exe], capture_output=True, text=True, env={**os.environ, "HIP_VISIBLE_DEVICES": ""})
    lines = [l for l in out.stdout.split("\n") if l.strip()]
    assert len(lines) == 2 * 3 * 6 * 14
    for l in lines:
        causal, nqt, e, r, base, f = (int(x) for x in l.split())
        assert base == row_base_sum(r, e, nqt, causal) and f == first(r // 4, e, causal), l
