"""The input projection (gs_input_proj / gs_input_proj_bwd) against the
oracle's restatement of the reference's gi producer (gru_layer.py:249-255):
forward within 1e-4 x max(1, |gi|) (fp32 sums over I), the per-row weight
codes and scales bit-exact, and the straight-through gradients within
1e-4 x max(1, |ref|)."""

from __future__ import annotations

import pytest
import torch

from oracle import gru_oracle as O

pytestmark = pytest.mark.gpu

CASES = [
    ((64, 32), 512, 1536, (0.02, -127, 127), (-127, 127), True),   # the benchmark shape, int8 QAT
    ((64, 32), 512, 1536, None, None, True),                       # fp32
    ((7,), 13, 30, (0.05, -8, 7), (-127, 127), False),              # odd sizes: scalar loads, no bias
    ((3, 5), 64, 24, None, (-7, 7), True),
]


@pytest.mark.parametrize("lead,I,N,xq,wq,bias", CASES)
def test_input_projection_forward_and_backward(dev, lead, I, N, xq, wq, bias):
    import gru_qat_amd as G

    g = torch.Generator().manual_seed(I + N)
    x = torch.randn(*lead, I, generator=g) * 0.8
    W = torch.randn(N, I, generator=g) / I ** 0.5
    b = torch.randn(N, generator=g) if bias else None
    xd = x.to(dev).requires_grad_(True)
    Wd = W.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True) if bias else None
    gi = G.input_projection(xd, Wd, bd, x_quant=xq, w_quant=wq)
    ref = O.input_projection(x, W, b, x_quant=xq, w_quant=wq)
    err = (gi.detach().cpu() - ref).abs().max().item()
    print(f"[proj] lead={lead} I={I} N={N}: fwd max err {err:.3e} (|ref| {ref.abs().max().item():.3e})")
    assert err <= 1e-4 * max(1.0, ref.abs().max().item())
    if wq is not None:
        wq_k, sc_k = G.quantize_input_weights(Wd.detach(), wq)
        wq_o, sc_o = O.weight_fake_quant_rows(W, *wq)
        assert torch.equal(sc_k.cpu(), sc_o)
        assert torch.equal(wq_k.cpu(), wq_o)

    dgi = torch.randn(gi.shape, generator=g)
    leaves = [xd, Wd] + ([bd] if bias else [])
    grads = torch.autograd.grad(gi, leaves, dgi.to(dev))
    xr, Wr = x.clone().requires_grad_(True), W.clone().requires_grad_(True)
    br = b.clone().requires_grad_(True) if bias else None
    gref = O.input_projection(xr, Wr, br, x_quant=xq, w_quant=wq, ste=True)
    rgrads = torch.autograd.grad(gref, [xr, Wr] + ([br] if bias else []), dgi)
    for name, a, r in zip(("dx", "dW", "db"), grads, rgrads):
        e = (a.cpu() - r).abs().max().item()
        print(f"[proj]   {name}: max err {e:.3e} (|ref| {r.abs().max().item():.3e})")
        assert e <= 1e-4 * max(1.0, r.abs().max().item()), name
