"""The reference's fast dispatch, run through this build's modules aliased under
the reference's names (reference src/gru_qat/gru_layer.py:260-293): import the
extract helper and the scan from ``gru_qat.triton_kernels.scan_<kind>``, pull
the hidden weights out of a cell-shaped module, scan, and compare the output
and every gradient that reaches the cell's parameters with the oracle."""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN
from oracle import gru_oracle as O
from parity_util import FP32_TOL, log
from test_binding_cpu import API, aliased, make_cell  # noqa: F401  (aliased is a fixture)

pytestmark = pytest.mark.gpu

CALLS = {c["module"].rsplit("_", 1)[-1]: c for c in API["fast_dispatch"]["calls"]}


def _grad_of(cell, kind, gate):
    m = getattr(cell, f"struct_Wh_{gate}")
    return m.b.twiddle.grad.squeeze(0) if kind == "butterfly" else m.weight.grad


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("kind", ["diagonal", "monarch", "butterfly"])
def test_extract_then_scan_matches_the_oracle(dev, aliased, kind, quant):  # noqa: F811
    T, B, H = 12, 6, 64
    call = CALLS[kind]
    ns: dict = {}
    exec(f"from {call['module']} import ({call['extract']}, {call['scan']})", ns)
    extract, scan = ns[call["extract"]], ns[call["scan"]]
    cell = make_cell(kind, H, nb=4).to(dev)
    g = torch.Generator().manual_seed(11)
    gi = torch.randn(T, B, 3 * H, generator=g).to(dev).requires_grad_(True)
    h0 = (torch.randn(B, H, generator=g) * 0.1).to(dev).requires_grad_(True)
    q = Q_INT8_HIDDEN if quant else None
    log(f"[binding] {call['module']}: {call['extract']} -> {call['scan']} quant={quant}")
    W, bh = extract(cell)
    out = scan(gi, h0, W, bh, h_in_quant=q, h_out_quant=q)
    cfg = {"kind": kind, "name": f"binding_{kind}", "T": T, "B": B, "H": H, "w": W.detach().cpu(), "w2": None,
           "bh": bh.detach().cpu(), "gi": gi.detach().cpu(), "h0": h0.detach().cpu(), "h_in_quant": q,
           "h_out_quant": q}
    o = out.detach().cpu()
    if q is None:
        err = (o - O.scan_config(cfg)).abs().max().item()
        log(f"[binding]   max|out-oracle|={err:.3e}")
        assert err <= FP32_TOL
    else:
        pre = O.teacher_forced_prequant(cfg, o)
        x = pre / q[0]
        near = (x - torch.floor(x) - 0.5).abs() * q[0] <= 2e-6
        assert not ((torch.round(o / q[0]) != O.quant_codes(pre, q)) & ~near).any()
    dout = torch.randn(T, B, H, generator=torch.Generator().manual_seed(12))
    (out * dout.to(dev)).sum().backward()
    ref = O.scan_backward(cfg, o, dout)

    def close(name, got, want):
        err = (got.detach().cpu() - want).abs().max().item()
        log(f"[binding]   {name}: max err {err:.3e}")
        assert err <= 1e-4 * max(1.0, want.abs().max().item()), name

    close("dgi", gi.grad, ref["dgi"])
    close("dh0", h0.grad, ref["dh0"])
    for i, gate in enumerate("rzn"):
        close(f"dWh_{gate}", _grad_of(cell, kind, gate), ref["dw"][i])
        close(f"db_h{gate}", getattr(cell, f"b_h{gate}").grad, ref["dbh"][i * H:(i + 1) * H])
