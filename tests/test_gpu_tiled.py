"""The barrier-free batch-tiled dense kernels (gs_dense_fwd_tiled,
gs_dense_bwd_tiled) behind gru_scan / gru_scan_forward /
gru_scan_backward_triton, and every dense recurrence above H = 1024 (the
persistent entry points and the materialized-map backwards of Monarch and
butterfly take them there).

Reference kernels: gru_scan_fwd_kernel (scan.py:755-913, launched by
gru_scan_forward :1688-1765) and gru_scan_bwd_kernel (:916-1352, launched by
gru_scan_backward_triton :1355-1447). The cases follow the reference's own
tests of gru_scan: tests/test_triton_scan.py:47-78 (persistent against
non-persistent forward, here bit-identical rather than within TF32 noise),
:114-215 (gru_scan forward and backward against the PyTorch path) and
:291-380 (int8 hidden QAT through gru_scan), all against the oracle here."""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from oracle import gru_oracle as O
from parity_util import FP32_TOL, assert_fp32_parity, assert_quant_parity, log, to_dev

pytestmark = pytest.mark.gpu

COARSE = (0.05, -10, 10)


def _dense(shape, seed=0, q=None, h0_scale=None):
    cfg = make_config(1, shape=shape, seed=seed)
    if h0_scale is not None:
        cfg["h0"] = torch.randn(cfg["B"], cfg["H"], generator=torch.Generator().manual_seed(seed + 3)) * h0_scale
    cfg["h_in_quant"] = q
    cfg["h_out_quant"] = q
    return cfg


def _fwd(fn, cfg, dev):
    import gru_qat_amd as G

    d = to_dev(cfg, dev)
    out = getattr(G, fn)(d["gi"], d["h0"], d["w"], d["bh"], h_in_quant=cfg["h_in_quant"],
                         h_out_quant=cfg["h_out_quant"])
    torch.cuda.synchronize(dev)
    return out.cpu()


# (7, 4, 16) and (32, 16, 64): the reference's gru_scan shapes; H not a multiple of 4 and H = 1
# take the element-wise weight loads; (64, 32, 512) is config 1
FWD_SHAPES = [(7, 4, 16), (32, 16, 64), (64, 32, 512), (5, 3, 7), (3, 1, 1), (9, 6, 300), (4, 5, 1000)]


@pytest.mark.parametrize("shape", FWD_SHAPES)
@pytest.mark.parametrize("fn", ["gru_scan_forward", "gru_scan"])
def test_gru_scan_by_name_matches_oracle(dev, fn, shape):
    cfg = _dense(shape, h0_scale=0.3)
    log(f"[tiled] {fn} {shape}")
    out = _fwd(fn, cfg, dev)
    ref = O.scan_config(cfg)
    err = (out - ref).abs().max().item()
    log(f"[tiled]   max|out-oracle|={err:.3e}")
    assert torch.isfinite(out).all() and err <= FP32_TOL


@pytest.mark.parametrize("shape", [(8, 4, 32), (16, 8, 32), (64, 32, 512)])
def test_gru_scan_qat_matches_oracle(dev, shape):
    """Frozen int8 hidden fake-quant through gru_scan (reference
    test_triton_qat_matches_pytorch, tests/test_triton_scan.py:291-380):
    codes bit-exact away from rounding boundaries. This configuration's weights
    are int8 codes, so at H = 512 both forwards run their int8-MFMA instances
    (test_gpu_int8_weights.py), which agree bit for bit as the fp32 ones do."""
    cfg = make_config(2, shape=shape)
    d = to_dev(cfg, dev)
    import gru_qat_amd as G

    out_t = G.gru_scan_forward(d["gi"], d["h0"], d["w"], d["bh"], h_in_quant=cfg["h_in_quant"],
                               h_out_quant=cfg["h_out_quant"])
    out_p = G.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"], h_in_quant=cfg["h_in_quant"],
                                          h_out_quant=cfg["h_out_quant"])
    assert torch.equal(out_t, out_p)
    assert_quant_parity(cfg, dev, free_bound=2.0)


@pytest.mark.parametrize("shape", [(16, 8, 128), (64, 32, 512), (5, 9, 1000), (6, 3, 62), (3, 2, 1024)])
@pytest.mark.parametrize("q", [None, Q_INT8_HIDDEN, "in_only"])
def test_tiled_bit_identical_to_persistent(dev, shape, q):
    """Same K-slice products, accumulation order and gate arithmetic: the
    batch-tiled and persistent forwards agree bit for bit (the reference's
    own check of this pair allows 5e-2 relative, scan.py's TF32 paths)."""
    cfg = _dense(shape, h0_scale=0.3, q=Q_INT8_HIDDEN if q else None)
    if q == "in_only":
        cfg["h_out_quant"] = None
    a = _fwd("gru_scan_forward", cfg, dev)
    b = _fwd("gru_scan_forward_persistent", cfg, dev)
    log(f"[tiled] {shape} q={q}: {int((a != b).sum())} elements differ")
    assert torch.equal(a, b)


def _grads(fn, cfg, dev, seed=13):
    import gru_qat_amd as G

    keys = ["gi", "h0", "w", "bh"]
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
    out = getattr(G, fn)(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"], h_in_quant=cfg["h_in_quant"],
                         h_out_quant=cfg["h_out_quant"])
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed)).to(dev)
    grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
    return out.detach(), dout, dict(zip(keys, grads))


def _check_grads(cfg, out, dout, grads, tag):
    ref = O.scan_backward(cfg, out.cpu(), dout.cpu())
    for k, g in grads.items():
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        bar = 1e-4 * max(1.0, r.abs().max().item())
        log(f"[tiled] {tag} d{k}: max err {err:.3e} (bar {bar:.1e})")
        assert torch.isfinite(g).all() and err <= bar


@pytest.mark.parametrize("shape", [(7, 4, 16), (8, 4, 32), (16, 8, 32), (6, 5, 300), (5, 3, 7), (64, 32, 512)])
@pytest.mark.parametrize("q", [None, COARSE, Q_INT8_HIDDEN])
def test_gru_scan_backward_matches_oracle(dev, shape, q):
    """gru_scan's gradients (batch-tiled forward and backward) against the
    oracle's pinned backward, from the kernel's own forward output."""
    cfg = _dense(shape, h0_scale=0.3, q=q)
    out, dout, grads = _grads("gru_scan", cfg, dev)
    _check_grads(cfg, out, dout, grads, f"gru_scan {shape} q={q}")


@pytest.mark.parametrize("shape", [(8, 4, 32), (64, 32, 512), (5, 37, 1000)])
@pytest.mark.parametrize("q", [None, Q_INT8_HIDDEN])
def test_tiled_backward_bit_identical_to_persistent(dev, shape, q):
    """gru_scan_backward_triton (batch-tiled recurrence) and
    gru_scan_backward_persistent share every pass but the recurrence, whose
    products and carry arithmetic are the same: identical gradients."""
    import gru_qat_amd.scan as S

    cfg = _dense(shape, h0_scale=0.3, q=q)
    d = to_dev(cfg, dev)
    out = S.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"], h_in_quant=q, h_out_quant=q)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(dev)
    a = S.gru_scan_backward_triton(d["gi"], d["h0"], d["w"], d["bh"], out, dout, h_in_quant=q, h_out_quant=q)
    b = S.gru_scan_backward_persistent(d["gi"], d["h0"], d["w"], d["bh"], out, dout, h_in_quant=q,
                                       h_out_quant=q)
    for name, x, y in zip(("dgi", "dh0", "dWh", "dbh"), a, b):
        log(f"[tiled] {shape} q={q} {name}: {int((x != y).sum())} elements differ")
        assert torch.equal(x, y), name


# ---- hidden sizes above the persistent kernels' 1024 --------------------------------------------

LARGE = [(6, 5, 1536), (5, 3, 2048), (3, 2, 1031)]


@pytest.mark.parametrize("shape", LARGE)
def test_dense_large_h_forward(dev, shape):
    cfg = _dense(shape, h0_scale=0.3)
    assert_fp32_parity(cfg, dev)  # gru_scan_forward_persistent
    assert torch.equal(_fwd("gru_scan_forward_persistent", cfg, dev), _fwd("gru_scan_forward", cfg, dev))


@pytest.mark.parametrize("shape", [(6, 5, 1536), (5, 3, 2048)])
def test_dense_large_h_int8(dev, shape):
    cfg = make_config(2, shape=shape)
    assert_quant_parity(cfg, dev, free_bound=2.0)


@pytest.mark.parametrize("shape", LARGE)
@pytest.mark.parametrize("q", [None, Q_INT8_HIDDEN])
@pytest.mark.parametrize("fn", ["gru_scan_persistent", "gru_scan"])
def test_dense_large_h_backward(dev, shape, q, fn):
    cfg = _dense(shape, h0_scale=0.3, q=q)
    out, dout, grads = _grads(fn, cfg, dev)
    _check_grads(cfg, out, dout, grads, f"{fn} {shape} q={q}")


def test_noalloc_large_h_runs_the_tiled_kernel(dev):
    """gs_dense_fwd_noalloc above H = 1024 needs no scratch at all: the
    batch-tiled kernel, bit-identical to gs_dense_fwd there."""
    import ctypes

    from gru_qat_amd import _lib

    cfg = _dense((4, 3, 1536), h0_scale=0.3)
    d = to_dev(cfg, dev)
    lib = _lib.load()
    outs = []
    for name in ("gs_dense_fwd_noalloc", "gs_dense_fwd_tiled"):
        out = torch.empty((4, 3, 1536), device=dev)
        a = _lib.GsArgs(d["gi"].data_ptr(), d["h0"].data_ptr(), d["w"].data_ptr(), None, d["bh"].data_ptr(),
                        out.data_ptr(), None, 0, None, 4, 3, 1536, d["gi"].stride(0), d["gi"].stride(1),
                        d["h0"].stride(0), out.stride(0), out.stride(1), 0, 0, 0, 0,
                        _lib.make_quant(None, "q"), _lib.make_quant(None, "q"), None)
        stream = _lib.current_stream_handle(dev)
        rc = getattr(lib, name)(ctypes.byref(a), ctypes.c_void_p(stream))
        _lib.raise_for(rc, lib)
        outs.append(out)
    torch.cuda.synchronize(dev)
    assert torch.equal(outs[0], outs[1])
    assert (outs[0].cpu() - O.scan_config(cfg)).abs().max().item() <= FP32_TOL


def _monarch(shape, nb, two, q, seed=0):
    T, B, H = shape
    cfg = make_config(3, shape=shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    bs = H // nb
    cfg["w"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
    cfg["w2"] = ((torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5) if two else None
    cfg["h0"] = torch.randn(B, H, generator=torch.Generator().manual_seed(seed + 3)) * 0.3
    cfg["h_in_quant"] = q
    cfg["h_out_quant"] = q
    return cfg


@pytest.mark.parametrize("nb,two", [(32, True), (8, False), (16, True)])
@pytest.mark.parametrize("q", [None, COARSE])
def test_monarch_backward_large_h(dev, nb, two, q):
    """Monarch at H = 2048 on the materialized-map backward (two factors, and
    one factor of blksz 256, outside the block-local kernels), whose dense
    recurrence takes the batch-tiled kernel there."""
    import gru_qat_amd as G

    cfg = _monarch((5, 3, 2048), nb, two, q)
    keys = ["gi", "h0", "bh"] + list(O.hidden_params(cfg))
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
    out = G.gru_scan_monarch(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"], Wh_struct2=leaves.get("w2"),
                             h_in_quant=q, h_out_quant=q)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
    ref = O.scan_backward(cfg, out.detach().cpu(), dout.cpu())
    fwd_err = (out.detach().cpu() - O.scan_config(cfg)).abs().max().item()
    log(f"[tiled] monarch nb={nb} two={two} q={q} forward max err {fwd_err:.3e}")
    if q is None:
        assert fwd_err <= FP32_TOL
    for k, g in zip(keys, grads):
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        bar = 1e-4 * max(1.0, r.abs().max().item())
        log(f"[tiled] monarch nb={nb} two={two} q={q} d{k}: max err {err:.3e} (bar {bar:.1e})")
        assert torch.isfinite(g).all() and err <= bar


@pytest.mark.parametrize("shape", [(4, 3, 2048), (3, 2, 1500)])
def test_butterfly_backward_hpad_2048(dev, shape):
    """Butterfly with H_PAD = 2048 (H = H_PAD and H < H_PAD): the forward on
    the general LDS kernel, the backward on the materialized map, whose dense
    recurrence takes the batch-tiled kernel."""
    import gru_qat_amd as G

    cfg = make_config(4, shape=shape)
    cfg["h0"] = torch.randn(shape[1], shape[2], generator=torch.Generator().manual_seed(3)) * 0.3
    keys = ["gi", "h0", "bh", "w"]
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
    out = G.gru_scan_butterfly_triton(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"])
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
    fwd_err = (out.detach().cpu() - O.scan_config(cfg)).abs().max().item()
    log(f"[tiled] butterfly {shape} forward max err {fwd_err:.3e}")
    assert fwd_err <= FP32_TOL
    ref = O.scan_backward(cfg, out.detach().cpu(), dout.cpu())
    for k, g in zip(keys, grads):
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        bar = 1e-4 * max(1.0, r.abs().max().item())
        log(f"[tiled] butterfly {shape} d{k}: max err {err:.3e} (bar {bar:.1e})")
        assert torch.isfinite(g).all() and err <= bar
