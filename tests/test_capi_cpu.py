"""C-ABI and wrapper checks that need no GPU: the library loads, exports every
symbol include/gruscan.h declares, sizes workspaces, and rejects bad
arguments with ValueError (never AssertionError) before any device work."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from gru_qat_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "gruscan.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(gs_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert _declared_symbols() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert lib.gs_abi_version() == _lib.ABI_VERSION


def _args(T=4, B=3, H=8, **kw):
    a = _lib.GsArgs()
    a.T, a.B, a.H = T, B, H
    a.sg_t, a.sg_b = B * 3 * H, 3 * H
    a.sh0_b = H
    a.so_t, a.so_b = B * H, H
    a.q_in = _lib.make_quant(kw.pop("q_in", None), "q_in")
    a.q_out = _lib.make_quant(kw.pop("q_out", None), "q_out")
    for k, v in kw.items():
        setattr(a, k, v)
    return a


FAKE = 0x1000  # never dereferenced: validation fails before any device access


@pytest.mark.parametrize("fn", ["gs_dense_fwd", "gs_diagonal_fwd", "gs_monarch_fwd", "gs_butterfly_fwd",
                                "gs_butterfly_fwd_generic"])
def test_null_pointers_rejected(fn):
    lib = _lib.load()
    a = _args()
    rc = getattr(lib, fn)(ctypes.byref(a), None)
    assert rc == _lib.GS_ERR_INVALID
    assert b"non-NULL" in lib.gs_last_error()


@pytest.mark.parametrize("field,msg", [("T", b"T must be > 0"), ("B", b"B must be > 0"), ("H", b"H must be > 0")])
def test_empty_dims_rejected(field, msg):
    lib = _lib.load()
    a = _args(gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE)
    setattr(a, field, 0)
    assert lib.gs_dense_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert msg in lib.gs_last_error()


def test_bad_quant_rejected():
    lib = _lib.load()
    a = _args(gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE, q_in=(0.0, -127, 127))
    assert lib.gs_diagonal_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    a = _args(gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE, q_out=(0.1, 5, -5))
    assert lib.gs_diagonal_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID


def test_missing_workspace_rejected():
    lib = _lib.load()
    a = _args(gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE)
    assert lib.gs_dense_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"workspace" in lib.gs_last_error()


def test_monarch_shape_rejected():
    lib = _lib.load()
    a = _args(H=8, gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE, nblocks=3, blksz=3)
    assert lib.gs_monarch_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"tile H" in lib.gs_last_error()


def test_butterfly_shape_rejected():
    lib = _lib.load()
    a = _args(H=8, gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE, log_n=2, bfly_nblocks=1)
    assert lib.gs_butterfly_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"H_PAD" in lib.gs_last_error()


def _bwd_args(T=4, B=3, H=8, **kw):
    a = _lib.GsBwdArgs()
    a.T, a.B, a.H = T, B, H
    a.sg_t, a.sg_b = B * 3 * H, 3 * H
    a.sh0_b = H
    a.so_t, a.so_b = B * H, H
    a.q_in = _lib.make_quant(kw.pop("q_in", None), "q_in")
    a.q_out = _lib.make_quant(kw.pop("q_out", None), "q_out")
    for k, v in kw.items():
        setattr(a, k, v)
    return a


BWD_PTRS = ("gi", "h0", "w", "bh", "out", "dout", "dgi", "dh0", "dw_part", "dbh_part")


@pytest.mark.parametrize("missing", BWD_PTRS)
def test_diagonal_bwd_null_pointer_rejected(missing):
    lib = _lib.load()
    a = _bwd_args(**{k: FAKE for k in BWD_PTRS if k != missing})
    assert lib.gs_diagonal_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"non-NULL" in lib.gs_last_error()


def test_diagonal_bwd_rejects_w2_and_bad_quant():
    lib = _lib.load()
    a = _bwd_args(w2=FAKE, **{k: FAKE for k in BWD_PTRS})
    assert lib.gs_diagonal_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"w2" in lib.gs_last_error()
    a = _bwd_args(q_out=(0.1, 5, -5), **{k: FAKE for k in BWD_PTRS})
    assert lib.gs_diagonal_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    a = _bwd_args(**{k: FAKE for k in BWD_PTRS})
    a.T = 0
    assert lib.gs_diagonal_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"T must be > 0" in lib.gs_last_error()


@pytest.mark.parametrize("missing", BWD_PTRS)
def test_dense_bwd_null_pointer_rejected(missing):
    lib = _lib.load()
    a = _bwd_args(**{k: FAKE for k in BWD_PTRS if k != missing})
    assert lib.gs_dense_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"non-NULL" in lib.gs_last_error()


def test_dense_bwd_rejects_strided_out_and_missing_workspace():
    lib = _lib.load()
    a = _bwd_args(**{k: FAKE for k in BWD_PTRS})
    a.so_t = a.so_t + 8  # steps not back to back
    assert lib.gs_dense_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"so_t == B * so_b" in lib.gs_last_error()
    a = _bwd_args(**{k: FAKE for k in BWD_PTRS})
    assert lib.gs_dense_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"workspace" in lib.gs_last_error()


def _pick_split(tiles, K, cus=256):
    """The K split of gemm_pick_split: at least 2 workgroups per CU where K
    allows (>= 256 terms per split, <= 16 splits), best-filled last round."""
    smax = max(1, min(16, -(-K // 256)))
    best, best_fill = 1, -1.0
    for s in range(1, smax + 1):
        n = tiles * s
        if n < 2 * cus and s < smax:
            continue
        fill = n / (cus * -(-n // cus))
        if fill > best_fill:
            best, best_fill = s, fill
    return best


def test_gemm_split_choice():
    assert _pick_split(192, 2048) == 4  # dense backward dWh at T=64, B=32, H=512: 768 workgroups
    assert _pick_split(256, 2048) == 2
    assert _pick_split(192, 300) == 2   # K caps it
    assert _pick_split(1, 100) == 1


def test_bwd_workspace_sizes():
    """Dense: the tagged workspace holds control words, double-buffered tagged
    D rows (H words per padded row) plus pad and one XCD word per workgroup;
    the plain scratch the coefficient block [T B, 3H], five [T B, H] planes,
    per-chunk dbh sums and the K-split partials of dWh. Diagonal needs
    neither, the stage-wise butterfly path no workspace."""
    lib = _lib.load()
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    T, B, H = 64, 32, 512
    a = _bwd_args(T=T, B=B, H=H)
    kc = 32
    P = 128 // 4
    tiles = (3 * H // 64) * (H // 64)
    split = _pick_split(tiles, T * B)
    nchunks = -(-T // 8)
    ws = 256 + al(2 * B * H * 8 + 16 * kc * 8) + al((B // 4) * P * 8)
    scratch = (al(T * B * 3 * H * 4) + 5 * al(T * B * H * 4) + al(nchunks * B * 3 * H * 4)
               + (al(split * 3 * H * H * 4) if split > 1 else 0))
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(a)) == ws
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_DENSE, ctypes.byref(a)) == scratch
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_DIAGONAL, ctypes.byref(a)) == 0
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_DIAGONAL, ctypes.byref(a)) == 0
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_BUTTERFLY, ctypes.byref(a)) == _lib.GS_ERR_INVALID
    a.log_n, a.bfly_nblocks = 9, 1
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_BUTTERFLY, ctypes.byref(a)) == 0
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_BUTTERFLY, ctypes.byref(a)) > 0
    a.log_n = 11  # stage-wise kernels cover N <= 1024: the materialized path needs the dense core
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_BUTTERFLY, ctypes.byref(a)) == ws
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_BUTTERFLY, ctypes.byref(a)) > scratch
    # the batch-tiled recurrence: no workspace, the dense scratch plus Wh transposed
    a = _bwd_args(T=T, B=B, H=H)
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_DENSE_TILED, ctypes.byref(a)) == 0
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_DENSE_TILED, ctypes.byref(a)) == scratch + al(3 * H * H * 4)
    # above H = 1024 the dense entry point takes the batch-tiled recurrence itself
    T2, B2, H2 = 2, 3, 2048
    a = _bwd_args(T=T2, B=B2, H=H2)
    tiled = (al(T2 * B2 * 3 * H2 * 4) + 5 * al(T2 * B2 * H2 * 4) + al(1 * B2 * 3 * H2 * 4)
             + al(3 * H2 * H2 * 4))  # K = T B = 6 allows no dWh split
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(a)) == 0
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_DENSE, ctypes.byref(a)) == tiled
    assert lib.gs_bwd_scratch_bytes(_lib.KIND_DENSE_TILED, ctypes.byref(a)) == tiled
    a = _bwd_args(T=2, B=3, H=8193)
    assert lib.gs_bwd_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(a)) == _lib.GS_ERR_INVALID
    assert b"8192" in lib.gs_last_error()


def test_dense_bwd_rejects_missing_scratch():
    lib = _lib.load()
    T, B, H = 4, 3, 8
    a = _bwd_args(T=T, B=B, H=H, **{k: FAKE for k in BWD_PTRS})
    need = lib.gs_bwd_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(a))
    a.workspace, a.workspace_bytes = 0x10000, need  # validated before any device access
    assert lib.gs_dense_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"scratch" in lib.gs_last_error()
    a.scratch, a.scratch_bytes = 0x10010, 1 << 30  # misaligned
    assert lib.gs_dense_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"aligned" in lib.gs_last_error()


def test_workspace_sizes():
    """Control words plus double-buffered tagged exchange words (8 bytes per
    unit and row) when a batch row's step spans workgroups; two-factor Monarch
    adds 3 gates of first-factor words. A single-factor Monarch block of 16,
    32, 64 or 128 units is produced by one workgroup per batch row, which keeps
    its state in LDS; other block sizes use the dense kernel's exchange."""
    lib = _lib.load()
    a = _args(T=64, B=32, H=512)
    n = lib.gs_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(a))
    xh = 2 * 32 * 512 * 8
    # pollers read 16 * KC words per row (KC = 32 for a 512-long reduction),
    # so the exchange area is padded by as many words past its last row; one
    # XCD-id word follows per workgroup (8 row-blocks x 32 workgroups)
    assert n == 256 + xh + 16 * 32 * 8 + 8 * 32 * 8
    q = (1.0 / 127, -127, 127)
    for kw in ({"q_in": q, "q_out": q}, {"q_in": q}):
        assert lib.gs_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(_args(T=64, B=32, H=512, **kw))) == n
    a_m1 = _args(T=64, B=32, H=512, nblocks=8, blksz=64)
    assert lib.gs_workspace_bytes(_lib.KIND_MONARCH, ctypes.byref(a_m1)) == 256
    a_m1 = _args(T=64, B=32, H=512, nblocks=4, blksz=128)
    assert lib.gs_workspace_bytes(_lib.KIND_MONARCH, ctypes.byref(a_m1)) == 256
    a_m1 = _args(T=64, B=32, H=512, nblocks=2, blksz=256)
    # 2 blocks x 16 workgroups of 4 compute waves per row-block; pollers read 16 * KC (KC = 16) words per row
    assert lib.gs_workspace_bytes(_lib.KIND_MONARCH, ctypes.byref(a_m1)) == 256 + xh + 16 * 16 * 8 + 8 * 2 * 16 * 8
    a_m2 = _args(T=64, B=32, H=512, nblocks=8, blksz=64, w2=FAKE)
    # fused two-factor kernel (bs = 64, nb = 8): one exchange of q_in(h) padded
    # by 512 words, plus one XCD-id word per workgroup (8 row-blocks x 8 blocks)
    assert lib.gs_workspace_bytes(_lib.KIND_MONARCH, ctypes.byref(a_m2)) == 256 + xh + 512 * 8 + 8 * 8 * 8
    # split two-factor kernel (bs = 128 > 64): q_in(h) plus 3 gates of z words
    a_m2 = _args(T=64, B=32, H=512, nblocks=4, blksz=128, w2=FAKE)
    assert lib.gs_workspace_bytes(_lib.KIND_MONARCH, ctypes.byref(a_m2)) == 256 + 4 * xh
    # diagonal and butterfly kernels use no workspace beyond the control words
    assert lib.gs_workspace_bytes(_lib.KIND_DIAGONAL, ctypes.byref(a)) == 256
    assert lib.gs_workspace_bytes(_lib.KIND_BUTTERFLY, ctypes.byref(a)) == 256
    assert lib.gs_workspace_bytes(9, ctypes.byref(a)) == _lib.GS_ERR_INVALID


# ---- Python wrappers: CPU tensors are rejected before any device work -----------------

def _cpu_inputs(T=4, B=3, H=8):
    gi = torch.randn(T, B, 3 * H)
    h0 = torch.zeros(B, H)
    bh = torch.zeros(3 * H)
    return gi, h0, bh


def test_wrappers_reject_cpu_tensors():
    import gru_qat_amd as G

    gi, h0, bh = _cpu_inputs()
    cases = [
        (G.gru_scan_persistent, torch.zeros(24, 8)),
        (G.gru_scan, torch.zeros(24, 8)),
        (G.gru_scan_diagonal, torch.zeros(3, 8)),
        (G.gru_scan_monarch, torch.zeros(3, 2, 4, 4)),
        (G.gru_scan_butterfly_triton, torch.zeros(3, 1, 3, 4, 2, 2)),
    ]
    for fn, w in cases:
        with pytest.raises(ValueError) as ei:
            fn(gi, h0, w, bh)
        assert not isinstance(ei.value, AssertionError)
        assert "CUDA" in str(ei.value)


def test_bad_quant_tuple_rejected_on_cpu():
    from gru_qat_amd._common import check_quant

    with pytest.raises(ValueError):
        check_quant((0.1, 1), "h_in_quant")
    with pytest.raises(ValueError):
        check_quant((-1.0, -127, 127), "h_in_quant")
    assert check_quant((0.5, -127, 127), "h_in_quant") == (0.5, -127, 127)


def _proj_args(M=6, N=12, I=8, **kw):
    a = _lib.GsProjArgs()
    a.M, a.N, a.I = M, N, I
    a.sx, a.sgi = I, N
    a.q_x = _lib.make_quant(kw.pop("q_x", None), "q_x")
    a.q_w = _lib.make_quant(kw.pop("q_w", None), "q_w")
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_input_proj_validation():
    lib = _lib.load()
    a = _proj_args(x=FAKE, w=FAKE)
    assert lib.gs_input_proj(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"non-NULL" in lib.gs_last_error()
    a = _proj_args(x=FAKE, w=FAKE, gi=FAKE, M=0)
    assert lib.gs_input_proj(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    a = _proj_args(x=FAKE, w=FAKE, gi=FAKE)
    a.sx = 4  # shorter than a row of I = 8
    assert lib.gs_input_proj(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"stride" in lib.gs_last_error()
    a = _proj_args(x=FAKE, w=FAKE, gi=FAKE, q_w=(1.0, -127, 127))
    assert lib.gs_input_proj(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"w_q" in lib.gs_last_error()
    a = _proj_args(x=FAKE, w=FAKE, gi=FAKE, q_x=(0.0, -127, 127))
    assert lib.gs_input_proj(ctypes.byref(a), None) == _lib.GS_ERR_INVALID


def test_input_proj_bwd_workspace_and_validation():
    lib = _lib.load()
    a = _lib.GsProjBwdArgs()
    a.M, a.N, a.I = 2048, 1536, 512
    a.sx, a.sdgi, a.sdx = 512, 1536, 512
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    tiles = (1536 // 64) * (512 // 64)
    split = _pick_split(tiles, 2048)
    dxs = _pick_split((2048 // 64) * (512 // 64), 1536)  # dx = dgi W, K split (dx contiguous)
    want = (al(-(-2048 // 256) * 1536 * 4) + (al(split * 1536 * 512 * 4) if split > 1 else 0)
            + (al(dxs * 2048 * 512 * 4) if dxs > 1 else 0))
    assert lib.gs_input_proj_bwd_workspace_bytes(ctypes.byref(a)) == want
    a.sdx = 520  # a strided dx is written by one unsplit product
    want_strided = al(-(-2048 // 256) * 1536 * 4) + (al(split * 1536 * 512 * 4) if split > 1 else 0)
    assert lib.gs_input_proj_bwd_workspace_bytes(ctypes.byref(a)) == want_strided
    a.sdx = 512
    a.x, a.w, a.dgi, a.dx, a.dw = FAKE, FAKE, FAKE, FAKE, FAKE
    assert lib.gs_input_proj_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"workspace" in lib.gs_last_error()
    a.dw = None
    assert lib.gs_input_proj_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"non-NULL" in lib.gs_last_error()


def test_input_projection_rejects_cpu_tensors():
    import gru_qat_amd as G

    with pytest.raises(ValueError):
        G.input_projection(torch.zeros(2, 3), torch.zeros(4, 3))
    with pytest.raises(ValueError):
        G.quantize_input_weights(torch.zeros(4, 3), (-127, 127))


@pytest.mark.parametrize("fn", ["gs_diagonal_fwd", "gs_monarch_fwd", "gs_butterfly_fwd", "gs_butterfly_fwd_generic"])
def test_gh_save_only_on_the_dense_forward(fn):
    lib = _lib.load()
    a = _args(gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE, gh_save=FAKE)
    assert getattr(lib, fn)(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"gh_save" in lib.gs_last_error()
    # the dense forward accepts it and fails later, on the missing workspace
    assert lib.gs_dense_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"workspace" in lib.gs_last_error()


@pytest.mark.parametrize("fn", ["gs_diagonal_bwd", "gs_monarch_bwd", "gs_butterfly_bwd"])
def test_gh_saved_only_on_the_dense_backward(fn):
    lib = _lib.load()
    a = _bwd_args(gh_saved=FAKE, **{k: FAKE for k in BWD_PTRS})
    assert getattr(lib, fn)(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"gh_saved" in lib.gs_last_error()
    assert lib.gs_dense_bwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"gh_saved" not in lib.gs_last_error()


def test_monarch_gh_save_rules():
    """gs_monarch_fwd takes gh_save only for the single-factor block-local
    forward and gs_monarch_bwd takes gh_saved only for the block-local
    single-factor backward; monarch_saves_gh states the same shapes."""
    from gru_qat_amd.scan_monarch import monarch_saves_gh

    lib = _lib.load()
    # two factors: rejected before any launch
    a = _args(H=32, nblocks=2, blksz=16, gi=FAKE, h0=FAKE, w=FAKE, w2=FAKE, bh=FAKE, out=FAKE, gh_save=FAKE)
    assert lib.gs_monarch_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"gh_save" in lib.gs_last_error()
    # blksz 8 has no block-local kernel
    a = _args(H=32, nblocks=4, blksz=8, gi=FAKE, h0=FAKE, w=FAKE, bh=FAKE, out=FAKE, gh_save=FAKE)
    assert lib.gs_monarch_fwd(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"gh_save" in lib.gs_last_error()
    # the block-local backward accepts gh_saved and fails later, on the missing scratch
    b = _bwd_args(H=32, nblocks=2, blksz=16, gh_saved=FAKE, **{k: FAKE for k in BWD_PTRS})
    assert lib.gs_monarch_bwd(ctypes.byref(b), None) == _lib.GS_ERR_INVALID
    assert b"gh_saved" not in lib.gs_last_error() and b"scratch" in lib.gs_last_error()
    b.w2 = FAKE
    assert lib.gs_monarch_bwd(ctypes.byref(b), None) == _lib.GS_ERR_INVALID
    assert b"gh_saved" in lib.gs_last_error()
    assert monarch_saves_gh(64, 32, 8, 64, False)
    assert not monarch_saves_gh(64, 32, 8, 64, True)
    assert not monarch_saves_gh(64, 32, 4, 8, False) and not monarch_saves_gh(64, 32, 1, 256, False)
    assert monarch_saves_gh(4, 4 * 65535, 2, 16, False) and not monarch_saves_gh(4, 4 * 65535 + 1, 2, 16, False)
    assert not monarch_saves_gh(1 << 16, 1 << 14, 8, 64, False)


def test_dense_function_saves_gh_only_under_grad_mode(monkeypatch):
    """The scan Functions store gh only when a gradient will be taken and the
    switch is on: under torch.no_grad() needs_input_grad still reads True for
    leaves that require grad, so the choice is made where apply is called,
    also for the reference's six-argument form."""
    from gru_qat_amd import _common as C
    from gru_qat_amd import scan as S

    x = torch.ones(2, requires_grad=True)
    assert C.save_gh_default(x, torch.ones(2))
    with torch.no_grad():
        assert not C.save_gh_default(x)
    assert not C.save_gh_default(torch.ones(2), torch.ones(3))
    C.set_save_gh(False)
    try:
        assert not C.save_gh_default(x)
    finally:
        C.set_save_gh(True)

    seen = []

    def fake_forward(ctx, tiled, gi, h0, Wh_cat, bh_cat, hin, hout, save_gh):
        seen.append((tiled, save_gh))
        return gi.detach().clone()

    monkeypatch.setattr(S, "_function_forward", fake_forward)
    gi = torch.ones(1, 1, 3, requires_grad=True)
    args = (gi, torch.zeros(1, 1), torch.zeros(3, 1), torch.zeros(3), None, None)
    S.GRUScanPersistentFunction.apply(*args)
    with torch.no_grad():
        S.GRUScanFunction.apply(*args)
    S.GRUScanFunction.apply(*args, False)
    assert seen == [(False, True), (True, False), (True, False)]


def test_packed_args_match_the_ctypes_layout():
    """launch() packs gs_args with one struct call; the bytes must be those of
    the ctypes GsArgs (the C layout) for the same field values."""
    a = _lib.GsArgs(1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21,
                    _lib.GsQuant(1, 0.25, -7, 9), _lib.GsQuant(0, 1.0, -(2**31), 2**31 - 1), 22)
    b = _lib.GS_ARGS.pack(1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21,
                          1, 0.25, -7, 9, *_lib._QOFF, 22)
    assert _lib.GS_ARGS.size == ctypes.sizeof(_lib.GsArgs)
    assert bytes(a) == b
    assert _lib._qfields((0.25, -7, 9), "q") == (1, 0.25, -7, 9)
    with pytest.raises(ValueError, match="tuple"):
        _lib._qfields(0.5, "h_in_quant")


def test_fast_checks_fall_back_to_the_exact_errors():
    from gru_qat_amd._common import check_common, cuda_f32

    assert not cuda_f32(torch.zeros(2), torch.zeros(2))  # CPU tensors
    assert not cuda_f32(torch.zeros(2), None)
    gi, h0, bh = torch.zeros(4, 3, 6), torch.zeros(3, 2), torch.zeros(6)
    assert check_common("f", gi, h0, bh) == (4, 3, 2)
    with pytest.raises(ValueError, match="h0 shape"):
        check_common("f", gi, torch.zeros(3, 3), bh)
    with pytest.raises(ValueError, match="bh_cat shape"):
        check_common("f", gi, h0, torch.zeros(5))
    with pytest.raises(ValueError, match="T must be > 0"):
        check_common("f", torch.zeros(0, 3, 6), h0, bh)


def test_packed_bwd_args_match_the_ctypes_layout():
    vals = list(range(1, 30))
    a = _lib.GsBwdArgs(*vals[:29], _lib.GsQuant(1, 0.5, -3, 4), _lib.GsQuant(0, 1.0, -(2**31), 2**31 - 1), 99)
    b = _lib.GS_BWD_ARGS.pack(*vals[:29], 1, 0.5, -3, 4, *_lib._QOFF, 99)
    assert _lib.GS_BWD_ARGS.size == ctypes.sizeof(_lib.GsBwdArgs)
    assert bytes(a) == b
