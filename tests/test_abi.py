"""C-ABI checks that need no GPU: libpe_attn.so loads, exports every function include/pe_attn.h
declares, and its host-side validation returns the documented error codes (the failure paths a
caller can hit before any kernel launch: bad shapes, unsupported widths, bad mode / dtype /
causal flags)."""

import ctypes
import os
import re

import pytest

from pe_ablations_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pe_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pe_(?:attn|rmsnorm|swiglu)_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.available():
        pytest.fail("libpe_attn.so is not built (python -m pe_ablations_amd.build)")
    return _lib.lib()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert names, "no declarations parsed from the header"
    assert sorted(_lib.EXPORTED) == names
    for n in names:
        assert hasattr(lib, n), n


def test_enums_match_header():
    text = open(HEADER).read()
    def val(name):
        m = re.search(rf"\b{name}\s*=\s*(-?\d+)", text)
        assert m, name
        return int(m.group(1))
    for name, code in _lib.ERRORS.items():
        assert val(name) == code, name
    assert val("PE_MODE_POPE") == _lib.PE_MODE_POPE
    assert val("PE_MODE_ROPE") == _lib.PE_MODE_ROPE
    assert val("PE_MODE_NONE") == _lib.PE_MODE_NONE
    assert val("PE_DTYPE_BF16") == _lib.PE_DTYPE_BF16
    assert val("PE_DTYPE_FP32") == _lib.PE_DTYPE_FP32
    assert val("PE_DTYPE_FP16") == _lib.PE_DTYPE_FP16
    assert val("PE_DTYPE_BOOL") == _lib.PE_DTYPE_BOOL
    assert val("PE_CAUSAL_BOTTOM_RIGHT") == _lib.PE_CAUSAL_BOTTOM_RIGHT
    assert (val("PE_POS_EXACT"), val("PE_POS_BF16"), val("PE_POS_FP16")) == \
        (_lib.PE_POS_EXACT, _lib.PE_POS_BF16, _lib.PE_POS_FP16)
    assert val("PE_STAGE_COUNT") == len(_lib.STAGES)


def test_params_struct_layout():
    # int32 x 14, float x 2, int64, int32 x 2: 80 bytes, int64 at offset 64
    assert ctypes.sizeof(_lib.PeParams) == 80
    assert _lib.PeParams.delta_head_stride.offset == 64
    assert _lib.PeParams.position_rounding.offset == 72
    assert ctypes.sizeof(_lib.PeTensor) == 48


def params(**kw):
    p = _lib.PeParams()
    base = dict(B=1, Hq=4, Hkv=4, Sq=512, Sk=512, Dc=0, Dr=64, Dv=64, mode=_lib.PE_MODE_POPE,
                dtype=_lib.PE_DTYPE_BF16, causal=_lib.PE_CAUSAL_TOP_LEFT, start_pos_q=0,
                start_pos_k=0, qk_l2norm=0, scale=0.125, rope_mscale=1.0, delta_head_stride=0)
    base.update(kw)
    for k, v in base.items():
        setattr(p, k, v)
    return p


def check(lib, **kw):
    return lib.pe_attn_check(ctypes.byref(params(**kw)))


def test_valid_configs(lib):
    assert check(lib) == 0
    assert check(lib, Dr=128, Dv=128) == 0                       # fused PoPE D=128 (2D = 256)
    assert check(lib, Dc=64, Dr=32, Dv=64) == 0                  # reference split module
    assert check(lib, mode=_lib.PE_MODE_ROPE, Dr=64) == 0
    assert check(lib, mode=_lib.PE_MODE_NONE, Dr=64, qk_l2norm=1) == 0
    assert check(lib, Hq=8, Hkv=2) == 0                          # GQA
    assert check(lib, Sq=1, Sk=700, causal=_lib.PE_CAUSAL_BOTTOM_RIGHT) == 0
    assert check(lib, Sq=3, Sk=5, causal=_lib.PE_CAUSAL_NONE) == 0
    assert check(lib, dtype=_lib.PE_DTYPE_FP32) == 0


@pytest.mark.parametrize("kw,code", [
    (dict(B=0), "PE_ERR_SHAPE"),
    (dict(Sq=-1), "PE_ERR_SHAPE"),
    (dict(Hq=6, Hkv=4), "PE_ERR_SHAPE"),
    (dict(Sq=4, Sk=8), "PE_ERR_SHAPE"),                          # top-left causal needs Sq == Sk
    (dict(Sq=9, Sk=8, causal=_lib.PE_CAUSAL_BOTTOM_RIGHT), "PE_ERR_SHAPE"),
    (dict(Dr=160), "PE_ERR_HEAD_DIM"),                           # 2*160 > 256
    (dict(Dv=200), "PE_ERR_HEAD_DIM"),
    (dict(mode=7), "PE_ERR_MODE"),
    (dict(dtype=3), "PE_ERR_MODE"),
    (dict(causal=5), "PE_ERR_MODE"),
    (dict(position_rounding=3), "PE_ERR_MODE"),
    (dict(mode=_lib.PE_MODE_ROPE, position_rounding=1), "PE_ERR_MODE"),   # rounding is PoPE / FoPE only
    (dict(mode=_lib.PE_MODE_ROPE, Dr=63), "PE_ERR_MODE"),        # RoPE pairs need an even width
])
def test_invalid_configs(lib, kw, code):
    assert check(lib, **kw) == _lib.ERRORS[code]


def test_null_params(lib):
    assert lib.pe_attn_check(None) == _lib.ERRORS["PE_ERR_NULL"]
    assert lib.pe_attn_fwd_workspace_bytes(None) == 0


def test_workspace_sizes(lib):
    p = params(B=2, Hq=3, Hkv=3, Sq=100, Sk=100, Dr=64, Dv=64)
    fws = lib.pe_attn_fwd_workspace_bytes(ctypes.byref(p))
    # q~ and k~ of width 128 in bf16 (v is read in place when it is aligned and unpadded, but the
    # layout always reserves its repack slot)
    rows = 2 * 3 * 100
    assert fws >= 2 * rows * 128 * 2 + rows * 64 * 2
    bws = lib.pe_attn_bwd_workspace_bytes(ctypes.byref(p))
    # bf16 fused PoPE (Dc = 0, Dr = 64): dO repack, Di and L2, and the packed causal dS (at least
    # the triangle's 100 * 101 / 2 bf16 elements per head, at most the padded 128 x 256 square);
    # no fp32 dq~ / dk~ buffers
    assert bws >= rows * 64 * 2 + 2 * rows * 4 + 6 * (100 * 101 // 2) * 2
    assert bws < rows * 64 * 2 + 2 * rows * 4 + 2 * rows * 128 * 4 + 6 * 128 * 256 * 2 + 8 * 4096
    # the fp32 path and the split form keep them
    for kw in (dict(dtype=_lib.PE_DTYPE_FP32), dict(Dc=64, Dr=32)):
        q = params(**dict(dict(B=2, Hq=3, Hkv=3, Sq=100, Sk=100, Dr=64, Dv=64), **kw))
        assert lib.pe_attn_bwd_workspace_bytes(ctypes.byref(q)) >= 2 * rows * 128 * 4, kw
    assert lib.pe_attn_fwd_workspace_bytes(ctypes.byref(params(B=0))) == 0
    assert lib.pe_attn_operand_width(ctypes.byref(p)) == 128
    assert lib.pe_attn_operand_width(ctypes.byref(params(Dc=64, Dr=32))) == 128
    assert lib.pe_attn_operand_width(ctypes.byref(params(Dr=100, Dv=128))) == 256


def test_strerror_and_version(lib):
    for name, code in _lib.ERRORS.items():
        msg = lib.pe_attn_strerror(code).decode()
        assert msg
        if code:
            assert msg.startswith("pe_attn:")
    assert lib.pe_attn_version() == 2
    with pytest.raises(_lib.PEAttnError) as ei:
        _lib.check(_lib.ERRORS["PE_ERR_WORKSPACE"])
    assert ei.value.code == _lib.ERRORS["PE_ERR_WORKSPACE"]


def test_stage_hook_toggles(lib):
    arr = (ctypes.c_void_p * (2 * len(_lib.STAGES)))()
    assert lib.pe_attn_set_stage_events(ctypes.cast(arr, ctypes.c_void_p)) == 0
    assert lib.pe_attn_set_stage_events(None) == 0


def ds_unit_bytes(Sq, grp, causal=True):
    """dS bytes of one (batch, kv head) unit at Sq = Sk: grp query heads of ds_row_base(rows / 32)
    4 KiB blocks (pe_internal.h), from the row lengths summed directly (causal top-left: row r
    holds the 64-query blocks from 2 * (r / 4) on; no mask: all of them)."""
    nqt = (Sq + 255) // 256 * 4
    rows = (Sq + 127) // 128 * 128
    blocks = sum(nqt - (max(0, 2 * (r // 4)) if causal else 0) for r in range(rows // 32))
    return grp * blocks * 4096


@pytest.mark.parametrize("S, H, Hkv, groups", [(16384, 16, 16, 1), (32768, 16, 16, 4), (32768, 16, 4, 4),
                                               (65536, 4, 4, 4), (8192, 64, 8, 1), (4096, 1, 1, 1)])
def test_bwd_workspace_caps_the_score_gradient(lib, S, H, Hkv, groups):
    """The bf16 backward's dS share of the workspace holds as many (batch, kv head) units as
    PE_BWD_DS_CAP_BYTES (4.5 GiB) allows: the whole problem at the headline shape (16 heads at
    S = 16384, 4.33 GB), one unit group in `groups` at longer lengths.  Only dS depends on the mask,
    so the causal and unmasked workspaces differ by exactly the two capped dS shares."""
    cap = 4608 << 20
    lib.pe_attn_bwd_workspace_bytes.restype = ctypes.c_size_t
    kw = dict(B=1, Hq=H, Hkv=Hkv, Sq=S, Sk=S, Dr=128, Dv=128, scale=1 / 16.0, delta_head_stride=128)
    share = {}
    for causal in (True, False):
        unit = ds_unit_bytes(S, H // Hkv, causal)
        per_group = min(Hkv, max(1, cap // unit))
        share[causal] = per_group * unit
        if causal:
            assert -(-Hkv // per_group) == groups
            assert share[causal] <= cap or per_group == 1
    tc = lib.pe_attn_bwd_workspace_bytes(ctypes.byref(params(**kw, causal=_lib.PE_CAUSAL_TOP_LEFT)))
    tn = lib.pe_attn_bwd_workspace_bytes(ctypes.byref(params(**kw, causal=_lib.PE_CAUSAL_NONE)))
    assert abs((tc - tn) - (share[True] - share[False])) < 512, (tc, tn, share)


def test_bwd_workspace_reserves_the_query_head_split_partials(lib):
    """A 16-bit GQA backward whose dK/dV grid has fewer key blocks than the MI355X's 256 CUs shares
    each key block's query heads over workgroups that leave fp32 partials: at the reference training
    shape (B=8, 8 -> 4 heads, S=512, QK width 128, V width 64, 128 key blocks) two slices of dK~ and
    dV, one more dK~ slice and two dV slices than the unsplit layout (16 MiB).  At B=64 (1024 key
    blocks) and without GQA there is no split, so the workspace per batch entry is the same up to the
    small per-block partial sums."""
    lib.pe_attn_bwd_workspace_bytes.restype = ctypes.c_size_t

    def per_batch(B, Hq, dtype=_lib.PE_DTYPE_BF16):
        p = params(B=B, Hq=Hq, Hkv=4, Sq=512, Sk=512, Dc=64, Dr=32, Dv=64, dtype=dtype)
        return lib.pe_attn_bwd_workspace_bytes(ctypes.byref(p)) / B

    rows = 4 * 512  # kv rows per batch entry
    split_extra = rows * (128 + 2 * 64) * 4
    for dt in (_lib.PE_DTYPE_BF16, _lib.PE_DTYPE_FP16):
        extra = 8 * (per_batch(8, 8, dt) - per_batch(64, 8, dt))
        assert split_extra * 8 <= extra < split_extra * 8 + (1 << 20), (dt, extra)
    assert abs(8 * (per_batch(8, 4) - per_batch(64, 4))) < 1 << 20  # no GQA: no split
    assert abs(8 * (per_batch(8, 8, _lib.PE_DTYPE_FP32) - per_batch(64, 8, _lib.PE_DTYPE_FP32))) < 1 << 20


def test_masked_bwd_workspace(lib):
    """The explicit-mask backward's workspace.  In fp32 (and at widths outside the dK/dV pair
    kernel's) it runs the generic kernels, which store no dS: dO, Di / L2 and the fp32 dq~ / dk~,
    linear in S (0.61 GB at the headline widths with 16 heads at S = 16384) and independent of the
    causal flag.  In bf16 at the pair kernel's widths it runs the tuned kernels and takes the
    unmasked backward's workspace, dS included, without the query-head split's partials."""
    lib.pe_attn_bwd_masked_workspace_bytes.restype = ctypes.c_size_t
    lib.pe_attn_bwd_workspace_bytes.restype = ctypes.c_size_t

    def ws(S, **kw):
        return lib.pe_attn_bwd_masked_workspace_bytes(ctypes.byref(params(Hq=16, Hkv=16, Sq=S, Sk=S, Dr=128, Dv=128, **kw)))

    f32 = dict(dtype=_lib.PE_DTYPE_FP32)
    for S in (1024, 16384):
        rows = 16 * S
        # dO in fp32, Di and L2, fp32 dq~ and dk~, plus the phase gradient's per-block partial sums
        assert ws(S, **f32) >= rows * 128 * 4 + 2 * rows * 4 + 2 * rows * 256 * 4
        assert ws(S, **f32) < rows * 128 * 4 + 2 * rows * 4 + 2 * rows * 256 * 4 + (4 << 20)
        assert ws(S, **f32) == ws(S, causal=_lib.PE_CAUSAL_NONE, **f32)
    assert abs(ws(32768, **f32) / ws(16384, **f32) - 2) < 0.01
    # bf16, headline: 2048 key blocks fill the chip, so the unmasked backward has no split either
    unmasked = lib.pe_attn_bwd_workspace_bytes(ctypes.byref(params(Hq=16, Hkv=16, Sq=16384, Sk=16384, Dr=128, Dv=128)))
    assert ws(16384) == unmasked
    # bf16 at QK width 64 (Dr = 32): generic kernels, no dS
    small = lib.pe_attn_bwd_masked_workspace_bytes(ctypes.byref(params(Hq=16, Hkv=16, Sq=16384, Sk=16384, Dr=32, Dv=64)))
    assert small < 16 * 16384 * (64 * 2 + 8 + 2 * 64 * 4) + (4 << 20)
    assert lib.pe_attn_bwd_masked_workspace_bytes(ctypes.byref(params(B=0))) == 0


def test_masked_entry_points_validate_the_mask(lib):
    """Host-side checks of the mask view, made before any device call: a missing mask, an element
    type that is neither bool nor a float type, a negative stride and a base that is not aligned to
    its element each return their code."""
    p = params(causal=_lib.PE_CAUSAL_NONE)
    buf = (ctypes.c_float * 16)()
    base = ctypes.addressof(buf)

    def mask(dtype=_lib.PE_DTYPE_BOOL, stride=(0, 0, 512, 1), offset=0):
        m = _lib.PeTensor()
        m.data = base + offset
        m.dtype = dtype
        for i, st in enumerate(stride):
            m.stride[i] = st
        return m

    def fwd(m):
        return lib.pe_attn_fwd_masked(ctypes.byref(p), None, None, None, None, None, None, None,
                                      None if m is None else ctypes.byref(m), None, None, None, 0, None)

    def bwd(m):
        return lib.pe_attn_bwd_masked(ctypes.byref(p), None, None, None, None, None, None, None,
                                      None if m is None else ctypes.byref(m), None, None, None, None, None, None,
                                      None, None, None, None, None, 0, None, 0, None)

    for call in (fwd, bwd):
        assert call(None) == _lib.ERRORS["PE_ERR_NULL"]
        assert call(mask(dtype=7)) == _lib.ERRORS["PE_ERR_MODE"]
        assert call(mask(stride=(0, 0, -512, 1))) == _lib.ERRORS["PE_ERR_STRIDE"]
        assert call(mask(dtype=_lib.PE_DTYPE_FP32, offset=2)) == _lib.ERRORS["PE_ERR_STRIDE"]
        assert call(mask(dtype=_lib.PE_DTYPE_BF16, offset=1)) == _lib.ERRORS["PE_ERR_STRIDE"]
        # a valid mask passes on to the operand checks (qr missing: PE_ERR_NULL from them)
        assert call(mask()) == _lib.ERRORS["PE_ERR_NULL"]
