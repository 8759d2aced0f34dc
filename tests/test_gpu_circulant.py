"""Circulant hidden kind (reference _CirculantLinear, structure.py:220-240) on
the GPU against the oracle: the materialized map and the gradient fold, the
scan forward (fp32 1e-5 bar; int8 codes bit-exact away from rounding
boundaries), every gradient, the observer path, the extract helper and the
layer dispatch."""

from __future__ import annotations

import pytest
import torch

import gru_qat_amd as G
from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from gru_qat_amd.observe import hidden_map_dense, hidden_map_grad
from oracle import gru_oracle as O
from parity_util import assert_fp32_parity, assert_quant_parity, log, small_cfg, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H", [1, 7, 64, 100, 512])
def test_circulant_map_and_fold(dev, H):
    g = torch.Generator().manual_seed(H)
    col = torch.randn(3, H, generator=g)
    M = hidden_map_dense("circulant", col.to(dev), H).cpu()
    want = torch.cat([O.circulant_matrix(col[k]) for k in range(3)], dim=0)
    assert torch.equal(M, want)
    dM = torch.randn(3 * H, H, generator=g)
    dcol = hidden_map_grad("circulant", dM.to(dev), col.to(dev), H).cpu()
    # the fold is the adjoint of the map: <dM, map(col)> is linear in col
    ref = torch.stack([torch.stack([sum(dM[k * H + i, (i - d) % H] for i in range(H)) for d in range(H)])
                       for k in range(3)]) if H <= 7 else None
    cr = col.clone().requires_grad_(True)
    (torch.cat([O.circulant_matrix(cr[k]) for k in range(3)], dim=0) * dM).sum().backward()
    assert (dcol - cr.grad).abs().max().item() <= 1e-5 * max(1.0, cr.grad.abs().max().item())
    if ref is not None:
        assert torch.allclose(dcol, ref, atol=1e-5)


@pytest.mark.parametrize("shape", [(8, 4, 64), (5, 3, 7), (1, 1, 1), (9, 5, 100), (4, 33, 256), (3, 2, 1024),
                                   (64, 32, 512)])
@pytest.mark.parametrize("q", [None, Q_INT8_HIDDEN, "in_only", (0.02, -500, 500)])
def test_circulant_kernel_equals_dense_on_the_map(dev, shape, q):
    """gs_circulant_fwd forms each wave's rows of the circulant map from the
    columns: the same weights in the same products as the dense scan on the
    map gs_hidden_map_dense writes, so the outputs are equal bit for bit (local
    and remote modes, fp32 and packed int8 exchange, 8-byte words for levels
    wider than a byte)."""
    from gru_qat_amd.scan import gru_scan_forward_persistent
    from gru_qat_amd.scan_circulant import gru_scan_circulant_forward

    T, B, H = shape
    g = torch.Generator().manual_seed(H + B)
    gi = (torch.randn(T, B, 3 * H, generator=g)).to(dev)
    h0 = (torch.randn(B, H, generator=g) * 0.3).to(dev)
    col = (torch.randn(3, H, generator=g) / H ** 0.5).to(dev)
    bh = (torch.randn(3 * H, generator=g) * 0.1).to(dev)
    qi, qo = (q, q) if q != "in_only" else (Q_INT8_HIDDEN, None)
    a = gru_scan_circulant_forward(gi, h0, col, bh, h_in_quant=qi, h_out_quant=qo)
    b = gru_scan_forward_persistent(gi, h0, hidden_map_dense("circulant", col, H), bh, h_in_quant=qi,
                                    h_out_quant=qo)
    assert torch.equal(a, b)


@pytest.mark.parametrize("shape", [(8, 4, 64), (5, 3, 7), (1, 1, 1), (9, 5, 100), (4, 33, 256), (3, 2, 1024),
                                   (3, 2, 1040)])  # H > 1024: the written map on the batch-tiled kernel
def test_circulant_fp32(dev, shape):
    assert_fp32_parity(small_cfg(6, shape), dev)


def test_circulant_cfg6(dev):
    assert_fp32_parity(make_config(6), dev)


@pytest.mark.parametrize("qin,qout", [(Q_INT8_HIDDEN, Q_INT8_HIDDEN), (None, Q_INT8_HIDDEN), ((0.02, -100, 100), None)])
def test_circulant_quant(dev, qin, qout):
    cfg = small_cfg(6, (16, 8, 128), h_in_quant=qin, h_out_quant=qout)
    if qout is None:
        assert_fp32_parity(cfg, dev)
    else:
        assert_quant_parity(cfg, dev)


@pytest.mark.parametrize("q", [None, (0.05, -10, 10), Q_INT8_HIDDEN])
@pytest.mark.parametrize("shape", [(6, 4, 64), (5, 3, 33)])
def test_circulant_backward(dev, shape, q):
    cfg = small_cfg(6, shape, h_in_quant=q, h_out_quant=q)
    cfg["h0"] = torch.randn(shape[1], shape[2], generator=torch.Generator().manual_seed(4)) * 0.3
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in ("gi", "h0", "w", "bh")}
    out = G.gru_scan_circulant(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"], h_in_quant=q, h_out_quant=q)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    grads = torch.autograd.grad(out, list(leaves.values()), dout.to(dev))
    ref = O.scan_backward(cfg, out.detach().cpu(), dout)
    for k, g in zip(leaves, grads):
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        log(f"[circulant] backward d{k}: max err {err:.3e}")
        assert err <= 1e-4 * max(1.0, r.abs().max().item()), k


def test_circulant_observer_path_matches_the_scan(dev):
    cfg = small_cfg(6, (12, 4, 64))
    d = to_dev(cfg, dev)
    out = G.gru_scan_observe("circulant", d["gi"], d["h0"], d["w"], d["bh"]).cpu()
    assert (out - O.scan_config(cfg)).abs().max().item() <= 1e-5


def test_extract_and_layer_dispatch(dev):
    T, B, H = 7, 3, 48
    cfg = small_cfg(6, (T, B, H))
    cell = torch.nn.Module()
    cell.hidden_size, cell._hidden_dense = H, False
    for k, gate in enumerate("rzn"):
        m = torch.nn.Module()
        m.col = torch.nn.Parameter(cfg["w"][k].clone())
        setattr(cell, f"struct_Wh_{gate}", m)
        setattr(cell, f"b_h{gate}", torch.nn.Parameter(cfg["bh"][k * H:(k + 1) * H].clone()))
    W, bh = G.extract_circulant_factors(cell)
    assert torch.equal(W, cfg["w"]) and torch.equal(bh, cfg["bh"])
    out, h_T = G.forward_fast_dispatch("circulant", cfg["gi"].to(dev), cfg["h0"].to(dev), W.detach().to(dev),
                                       bh.detach().to(dev))
    assert (out.cpu() - O.scan_config(cfg)).abs().max().item() <= 1e-5
    assert torch.equal(h_T.cpu(), out[-1].cpu())
    layer = G.ScanLayer("circulant", torch.eye(3 * H, H), None, cfg["w"], cfg["bh"]).to(dev)
    assert layer.use_triton
    out2, _ = layer(torch.randn(T, B, H).to(dev))
    assert torch.isfinite(out2).all()
