"""The one-launch PoPE prologue (pe_prep.hip: prep_k_qheads_kernel) replayed on the CPU.

The launch interleaves nkblk blocks of key rows with nqblk blocks of query rows: block i is query
block cq(i) = floor(i * nqblk / n) when cq(i + 1) > cq(i), else key block i - cq(i), n = nkblk +
nqblk.  A query thread (b, head group, s, chunk t) covers QHG = 8 heads.  This checks, for the
benchmark shapes and ragged ones (head counts that are not a multiple of 8, a batch above one,
strided views), that

* every key block and every query block is taken exactly once;
* every (b, h, s, chunk) of the queries is written exactly once, and the phase table's every
  (s, chunk) exactly once (by the threads of b = 0 and the first head group);
* every address a query thread loads or stores lies inside its tensor: the x view (its strides),
  the (B, H, S, 2 Dr) operand rows and the [S][2][Dr] table."""

import numpy as np
import pytest

QHG = 8


def block_kinds(nkblk, nqblk):
    i = np.arange(nkblk + nqblk, dtype=np.int64)
    n = nkblk + nqblk
    cq = i * nqblk // n
    cq1 = (i + 1) * nqblk // n
    is_q = cq1 > cq
    return is_q, np.where(is_q, cq, i - cq)


@pytest.mark.parametrize("B,H,S,Dr", [(1, 16, 16384, 128), (8, 12, 2048, 64), (4, 16, 4096, 128),
                                      (2, 3, 1000, 64), (3, 20, 517, 32), (1, 9, 300, 128)])
def test_blocks_each_once(B, H, S, Dr):
    tpr = Dr // 8
    nk = B * H * S * tpr
    nq = B * -(-H // QHG) * S * tpr
    nkblk, nqblk = -(-nk // 256), -(-nq // 256)
    is_q, idx = block_kinds(nkblk, nqblk)
    assert np.array_equal(np.sort(idx[is_q]), np.arange(nqblk))
    assert np.array_equal(np.sort(idx[~is_q]), np.arange(nkblk))
    # the query blocks are spread over the launch: no run of key blocks much longer than n / nqblk
    qpos = np.flatnonzero(is_q)
    assert np.diff(qpos).max() <= -(-(nkblk + nqblk) // nqblk)


@pytest.mark.parametrize("B,H,S,Dr,layout", [(2, 12, 130, 64, "bshd"), (3, 20, 67, 32, "bshd"),
                                             (1, 9, 40, 128, "bhsd"), (2, 8, 33, 64, "padded")])
def test_query_threads_cover_and_stay_in_bounds(B, H, S, Dr, layout):
    tpr = Dr // 8
    ngrp = -(-H // QHG)
    nq = B * ngrp * S * tpr
    nqblk = -(-nq // 256)
    if layout == "bshd":          # the projections' (B, S, H, D) view seen as (B, H, S, D)
        st = (S * H * Dr, Dr, H * Dr, 1)
        numel = B * S * H * Dr
    elif layout == "bhsd":
        st = (H * S * Dr, S * Dr, Dr, 1)
        numel = B * H * S * Dr
    else:                         # rows padded to 2 Dr (a wider projection sliced)
        st = (S * H * 2 * Dr, 2 * Dr, H * 2 * Dr, 1)
        numel = B * S * H * 2 * Dr
    gid = np.arange(nqblk * 256, dtype=np.int64)
    unit, t = gid // tpr, gid % tpr
    live = unit < B * ngrp * S
    unit, t = unit[live], t[live]
    s = unit % S
    bg = unit // S
    hg, b = bg % ngrp, bg // ngrp
    written = np.zeros((B, H, S, tpr), dtype=np.int64)
    for j in range(QHG):
        h = hg * QHG + j
        ok = h < H
        off = b[ok] * st[0] + h[ok] * st[1] + s[ok] * st[2] + t[ok] * 8
        assert off.min() >= 0 and (off + 8).max() <= numel
        row = (b[ok] * H + h[ok]) * S + s[ok]
        for c0 in (t[ok] * 8, Dr + t[ok] * 8):
            dst = row * 2 * Dr + c0
            assert dst.min() >= 0 and (dst + 8).max() <= B * H * S * 2 * Dr
        np.add.at(written, (b[ok], h[ok], s[ok], t[ok]), 1)
    assert (written == 1).all()
    tw = (b == 0) & (hg == 0)
    tab = np.zeros((S, tpr), dtype=np.int64)
    np.add.at(tab, (s[tw], t[tw]), 1)
    assert (tab == 1).all()
    for c0 in (t[tw] * 8, Dr + t[tw] * 8):
        off = s[tw] * 2 * Dr + c0
        assert off.min() >= 0 and (off + 8).max() <= S * 2 * Dr
