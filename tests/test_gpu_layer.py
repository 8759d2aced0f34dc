"""layer_forward (GRULayer.forward through the fast dispatch with a dense
input side, gru_layer.py:153-200 and :234-302) on the GPU against the oracle
composed the same way: input projection, then the scan. Forward within 1e-5
without hidden quant, hidden-quantized codes exact away from rounding
boundaries (teacher-forced); gradients of x, h0, the input and hidden
weights and both biases within 1e-4 x max(1, |ref|)."""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from oracle import gru_oracle as O

pytestmark = pytest.mark.gpu

CASES = [
    ("dense", (7, 5, 64), 24, None, None, None, False),
    ("dense", (6, 4, 128), 40, (0.02, -127, 127), (-127, 127), Q_INT8_HIDDEN, True),
    ("diagonal", (9, 3, 96), 32, None, (-127, 127), None, False),
    ("monarch", (6, 4, 64), 16, None, None, Q_INT8_HIDDEN, True),
    ("butterfly", (5, 3, 100), 20, (0.05, -127, 127), None, None, False),
]
IDX = {"diagonal": 0, "dense": 1, "monarch": 3, "butterfly": 4}


@pytest.mark.parametrize("kind,shape,I,xq,wq,hq,batch_first", CASES)
def test_layer_forward_matches_oracle(dev, kind, shape, I, xq, wq, hq, batch_first):
    import gru_qat_amd as G

    T, B, H = shape
    cfg = make_config(IDX[kind], shape=shape, seed=2)
    if kind == "monarch":
        g = torch.Generator().manual_seed(4)
        cfg["w"] = (torch.rand((3, 4, H // 4, H // 4), generator=g) * 2 - 1) / (H // 4) ** 0.5
        cfg["w2"] = None
    cfg["h_in_quant"] = cfg["h_out_quant"] = hq
    g = torch.Generator().manual_seed(7)
    x = torch.randn(T, B, I, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.3
    Wi = torch.randn(3 * H, I, generator=g) / I ** 0.5
    bi = torch.randn(3 * H, generator=g) * 0.1
    cpu = dict(x=x, h0=h0, Wi=Wi, bi=bi, w=cfg["w"], bh=cfg["bh"])
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in cpu.items()}
    xin = leaves["x"].transpose(0, 1) if batch_first else leaves["x"]
    out, h_T = G.layer_forward(kind, xin, leaves["h0"], leaves["Wi"], leaves["bi"], leaves["w"], leaves["bh"],
                               x_quant=xq, w_quant=wq, h_in_quant=hq, h_out_quant=hq, batch_first=batch_first)
    out_tm = out.transpose(0, 1) if batch_first else out
    assert torch.equal(h_T, out_tm[-1])

    # forward: the oracle's projection, then its scan; hidden-quantized runs are
    # checked step by step from the kernel's own h_{t-1} (teacher forcing), codes
    # exact away from rounding boundaries (the fp32 projection sums differ ~1e-6)
    pl = {k: v.clone().requires_grad_(True) for k, v in cpu.items() if k in ("x", "Wi", "bi")}
    gi_ref = O.input_projection(pl["x"], pl["Wi"], pl["bi"], x_quant=xq, w_quant=wq, ste=True)
    rcfg = dict(cfg, gi=gi_ref.detach(), h0=h0, w=cfg["w"], bh=cfg["bh"])
    outc = out_tm.detach().cpu()
    if hq is None:
        err = (outc - O.scan_config(rcfg)).abs().max().item()
        print(f"[layer] {kind} {shape} I={I}: fwd max err {err:.3e}")
        assert err <= 1e-5
    else:
        pre = O.teacher_forced_prequant(rcfg, outc)
        code_k = torch.round(outc / hq[0])
        code_o = O.quant_codes(pre, hq)
        xs = pre / hq[0]
        near = (xs - torch.floor(xs) - 0.5).abs() * hq[0] <= 1e-4
        bad = (code_k != code_o) & ~near
        print(f"[layer] {kind} {shape} I={I}: code mismatches {int((code_k != code_o).sum())}, "
              f"away from boundaries {int(bad.sum())}")
        assert not bad.any()

    # gradients: the oracle's pinned scan backward on the kernel's trajectory,
    # chained through the projection's straight-through autograd
    dout = torch.randn(out_tm.shape, generator=g)
    keys = list(cpu)
    grads = dict(zip(keys, torch.autograd.grad(out_tm, [leaves[k] for k in keys], dout.to(dev))))
    sb = O.scan_backward(rcfg, outc, dout)
    px, pW, pb = torch.autograd.grad(gi_ref, [pl["x"], pl["Wi"], pl["bi"]], sb["dgi"])
    ref = {"x": px, "Wi": pW, "bi": pb, "h0": sb["dh0"], "w": sb["dw"], "bh": sb["dbh"]}
    for k in keys:
        e = (grads[k].cpu() - ref[k]).abs().max().item()
        print(f"[layer]   d{k}: max err {e:.3e} (|ref| {ref[k].abs().max().item():.3e})")
        assert e <= 1e-4 * max(1.0, ref[k].abs().max().item()), k
