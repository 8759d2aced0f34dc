"""Int8 weight codes on the dense forward (gs_weight_codes, gs_dense_fwd_i8w).

A frozen int8 QAT configuration (reference scan.py:1667-1685 with Wh_cat
fake-quantized per row as quantizers.py:188-199 does)
hands the scan a weight whose every element is the fp32 product of an int8 code
and its row's scale. gru_scan_forward_persistent then finds those codes once
per version of the tensor and runs the step's products on the int8 MFMA over the
exchanged h levels and the codes; gru_scan_forward (the batch-tiled kernel)
does the same on its own pipeline. Checked here: the codes reproduce the weight
bit for bit, rows that are not such products are refused, the int8 path meets
the oracle's parity bar (codes bit-exact away from rounding boundaries) in
every hidden-quant arrangement it serves, the persistent and batch-tiled int8
forwards agree bit for bit, and every launch the int8 path does not serve
returns the fp32 kernels' result bit for bit.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from parity_util import assert_quant_parity, log, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda", 0)


def _codes(w):
    from gru_qat_amd import _lib

    return _lib.weight_codes(w)


def test_weight_codes_reproduce_the_weight(dev):
    w = make_config(2, shape=(2, 2, 512))["w"].to(dev)
    got = _codes(w)
    assert got is not None
    codes, scale = got
    assert codes.dtype == torch.int8 and codes.shape == w.shape and scale.shape == (w.shape[0],)
    assert torch.equal(codes.float() * scale[:, None], w)  # one fp32 product per element
    assert int(codes.abs().max()) == 127


def test_weight_codes_zero_row_and_refusals(dev):
    w = make_config(2, shape=(2, 2, 128))["w"].to(dev)
    z = w.clone()
    z[5].zero_()
    got = _codes(z)
    assert got is not None and not got[0][5].any()
    assert torch.equal(got[0].float() * got[1][:, None], z)
    # one element moved by an ulp: no scale of its row reproduces it
    bad = w.clone()
    bad[7, 3] = torch.nextafter(bad[7, 3], torch.tensor(float("inf"), device=dev))
    assert _codes(bad) is None
    # a plain fp32 weight (configuration 1) is not a code product
    assert _codes(make_config(1, shape=(2, 2, 128))["w"].to(dev)) is None


def test_weight_codes_follow_the_tensor_version(dev):
    w = make_config(2, shape=(2, 2, 128))["w"].to(dev)
    first = _codes(w)
    assert _codes(w) is first  # cached for this version
    w.mul_(1.0)  # an in-place write, same values: found again
    again = _codes(w)
    assert again is not first and again is not None
    w[0, 0] = torch.nextafter(w[0, 0], torch.tensor(float("inf"), device=dev))
    assert _codes(w) is None


# (shape, q_in, q_out): the arrangements the int8 path serves (q_in on, its
# levels in a byte): q_in = q_out, q_in alone, q_in after a different q_out.
Q_OTHER = (0.05, -10, 10)
CASES = [
    ((64, 32, 512), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((16, 8, 128), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((9, 5, 1024), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((12, 37, 256), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((7, 3, 80), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((20, 6, 304), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((6, 5, 1536), Q_INT8_HIDDEN, Q_INT8_HIDDEN),  # H > 1024: the batch-tiled int8 kernel
    ((5, 3, 2048), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((16, 8, 512), Q_INT8_HIDDEN, None),
    ((16, 8, 512), Q_INT8_HIDDEN, Q_OTHER),
    ((10, 9, 256), Q_OTHER, Q_INT8_HIDDEN),
]


def _cfg(shape, q_in, q_out):
    cfg = make_config(2, shape=shape)
    cfg["h_in_quant"] = q_in
    cfg["h_out_quant"] = q_out
    return cfg


def _both(cfg, dev, tiled=False):
    import gru_qat_amd.scan as S

    d = to_dev(cfg, dev)
    args = (d["gi"], d["h0"], d["w"], d["bh"], cfg["h_in_quant"], cfg["h_out_quant"])
    fp32 = S._dense_forward("fp32 products", *args, int8_codes=False, tiled=tiled)
    i8 = S._dense_forward("int8 products", *args, int8_codes=True, tiled=tiled)
    return fp32, i8


@pytest.mark.parametrize("shape,q_in,q_out", CASES)
def test_int8_products_match_the_oracle(dev, shape, q_in, q_out):
    import gru_qat_amd.scan as S

    cfg = _cfg(shape, q_in, q_out)
    assert _codes(cfg["w"].to(dev)) is not None and S._int8_codes_apply(shape[2], q_in)
    fp32, i8 = _both(cfg, dev)
    n = int((fp32 != i8).sum())
    d = (fp32 - i8).abs().max().item()
    log(f"[int8w] {shape} q_in={q_in} q_out={q_out}: {n} of {i8.numel()} outputs differ from the fp32 "
        f"products (max {d:.3e})")
    if q_out is not None:
        # quantized outputs: the two differ only through rounding-boundary flips of a code
        assert n <= max(8, 2e-3 * i8.numel())
        assert_quant_parity(cfg, dev, free_bound=2.0)  # through gru_scan_forward_persistent: the int8 path
    else:
        # q_in alone: fp32 outputs, which differ by the rounding of gh (a few 1e-7) and, after a flip of a
        # q_in code at a rounding boundary, by that flip's effect on the trajectory (about 3e-4)
        from oracle import gru_oracle as O

        ref = O.scan_config(cfg)
        err = (i8.cpu() - ref).abs().max().item()
        log(f"[int8w] {shape} q_in only: max|out - oracle| = {err:.3e}")
        assert torch.isfinite(i8).all() and d <= 1e-3 and err <= 1e-3


@pytest.mark.parametrize("shape,q_in,q_out", [
    ((64, 32, 512), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((12, 37, 256), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((9, 5, 1024), Q_INT8_HIDDEN, Q_INT8_HIDDEN),
    ((16, 8, 512), Q_INT8_HIDDEN, None),
    ((16, 8, 512), Q_INT8_HIDDEN, Q_OTHER),
    ((10, 9, 256), Q_OTHER, Q_INT8_HIDDEN),
])
def test_tiled_int8_bit_identical_to_persistent(dev, shape, q_in, q_out):
    """gru_scan_forward and gru_scan_forward_persistent on int8 weights: the
    batch-tiled and persistent int8 instances form the same exact integer sums
    and the same gate arithmetic."""
    import gru_qat_amd as G

    cfg = _cfg(shape, q_in, q_out)
    d = to_dev(cfg, dev)
    kw = dict(h_in_quant=q_in, h_out_quant=q_out)
    a = G.gru_scan_forward(d["gi"], d["h0"], d["w"], d["bh"], **kw)
    b = G.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"], **kw)
    log(f"[int8w] tiled vs persistent {shape}: {int((a != b).sum())} elements differ")
    assert torch.equal(a, b)
    fp32_t, i8_t = _both(cfg, dev, tiled=True)
    assert torch.equal(i8_t, a)


@pytest.mark.parametrize("shape", [(1, 1, 80), (2, 3, 96), (5, 1, 112), (3, 5, 1040), (1, 33, 256),
                                   (4, 7, 1056), (3, 2, 128)])
def test_int8_edge_shapes(dev, shape):
    """Odd batch tiles and row blocks, T = 1, H just past a KC step or past the
    persistent limit: the two int8 forwards agree bit for bit (H <= 1024) and
    meet the quant bar."""
    import gru_qat_amd as G

    cfg = _cfg(shape, Q_INT8_HIDDEN, Q_INT8_HIDDEN)
    d = to_dev(cfg, dev)
    kw = dict(h_in_quant=Q_INT8_HIDDEN, h_out_quant=Q_INT8_HIDDEN)
    a = G.gru_scan_forward(d["gi"], d["h0"], d["w"], d["bh"], **kw)
    b = G.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"], **kw)
    assert torch.equal(a, b)
    assert_quant_parity(cfg, dev, free_bound=2.0)


@pytest.mark.parametrize("shape,q_in,q_out", [
    ((16, 8, 512), None, Q_INT8_HIDDEN),   # q_in off: h0 is not a level
    ((8, 4, 64), Q_INT8_HIDDEN, Q_INT8_HIDDEN),  # one workgroup: no exchange
    ((8, 4, 68), Q_INT8_HIDDEN, Q_INT8_HIDDEN),  # H not a multiple of 16
    ((8, 4, 512), (1.0 / 500, -500, 500), (1.0 / 500, -500, 500)),  # levels wider than a byte
])
@pytest.mark.parametrize("tiled", [False, True])
def test_launches_outside_the_int8_path_are_unchanged(dev, shape, q_in, q_out, tiled):
    cfg = _cfg(shape, q_in, q_out)
    fp32, i8 = _both(cfg, dev, tiled=tiled)
    assert torch.equal(fp32, i8)


def _entry(dev, cfg, codes, scale, name="gs_dense_fwd_i8w"):
    from gru_qat_amd import _lib

    d = to_dev(cfg, dev)
    T, B, H = d["gi"].shape[0], d["gi"].shape[1], d["h0"].shape[1]
    out = torch.zeros((T, B, H), device=dev)
    lib = _lib.load()
    need = lib.gs_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(_lib.GsArgs(
        d["gi"].data_ptr(), d["h0"].data_ptr(), d["w"].data_ptr(), None, d["bh"].data_ptr(), out.data_ptr(), None, 0,
        None, T, B, H, d["gi"].stride(0), d["gi"].stride(1), d["h0"].stride(0), out.stride(0), out.stride(1), 0, 0,
        0, 0, _lib.make_quant(cfg["h_in_quant"], "q"), _lib.make_quant(cfg["h_out_quant"], "q"), None)))
    ws = torch.zeros(max(int(need), 4096), dtype=torch.uint8, device=dev)
    a = _lib.GsArgs(d["gi"].data_ptr(), d["h0"].data_ptr(), d["w"].data_ptr(), None, d["bh"].data_ptr(),
                    out.data_ptr(), ws.data_ptr(), ws.numel(), None, T, B, H, d["gi"].stride(0), d["gi"].stride(1),
                    d["h0"].stride(0), out.stride(0), out.stride(1), 0, 0, 0, 0,
                    _lib.make_quant(cfg["h_in_quant"], "q"), _lib.make_quant(cfg["h_out_quant"], "q"), None)
    fn = lib[name]
    if name.endswith("_i8w"):
        fn.argtypes = [ctypes.POINTER(_lib.GsArgs), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        rc = fn(ctypes.byref(a), codes, scale, ctypes.c_void_p(_lib.current_stream_handle(dev)))
    else:
        fn.argtypes = [ctypes.POINTER(_lib.GsArgs), ctypes.c_void_p]
        rc = fn(ctypes.byref(a), ctypes.c_void_p(_lib.current_stream_handle(dev)))
    torch.cuda.synchronize(dev)
    return rc, out, lib


@pytest.mark.parametrize("name", ["gs_dense_fwd_i8w", "gs_dense_fwd_tiled_i8w"])
def test_entry_point_through_the_c_abi(dev, name):
    """The int8-weight entry points called directly: on a config-2 input they
    agree with the Python route; NULL codes and a code pointer that is not
    16-byte aligned are refused before any launch."""
    from gru_qat_amd import _lib

    cfg = make_config(2, shape=(16, 8, 256))
    codes, scale = _codes(cfg["w"].to(dev))
    rc, out, lib = _entry(dev, cfg, codes.data_ptr(), scale.data_ptr(), name)
    assert rc == 0
    _, i8 = _both(cfg, dev)
    assert torch.equal(out, i8)
    rc, _, _ = _entry(dev, cfg, None, scale.data_ptr(), name)
    assert rc == _lib.GS_ERR_INVALID and b"w_codes" in lib.gs_last_error()
    rc, _, _ = _entry(dev, cfg, codes.data_ptr() + 4, scale.data_ptr(), name)
    assert rc == _lib.GS_ERR_INVALID and b"aligned" in lib.gs_last_error()


def test_non_contiguous_weight(dev):
    """A non-contiguous Wh_cat (same values) finds the same codes, cached on the
    caller's tensor, and gives the contiguous weight's outputs bit for bit."""
    import gru_qat_amd as G

    cfg = make_config(2, shape=(8, 4, 256))
    d = to_dev(cfg, dev)
    w_nc = d["w"].t().contiguous().t()
    assert not w_nc.is_contiguous()
    kw = dict(h_in_quant=cfg["h_in_quant"], h_out_quant=cfg["h_out_quant"])
    a = G.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"], **kw)
    b = G.gru_scan_forward_persistent(d["gi"], d["h0"], w_nc, d["bh"], **kw)
    assert torch.equal(a, b)
    first = _codes(w_nc)
    assert first is not None and _codes(w_nc) is first
