"""The input projection (gs_input_proj / gs_input_proj_bwd) against the
oracle's restatement of the reference's gi producer (gru_layer.py:249-255):
forward within 1e-4 x max(1, |gi|) (fp32 sums over I, or exact int8 sums
when both quantizers are int8 and I is a multiple of 16), the per-row weight
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
    # asymmetric per-row weight range (scale max|w| / qmax): weights below -100 s clip, and the
    # clipped-STE mask zeroes their gradient and their part of the scale's gradient
    ((3, 5), 64, 24, (0.05, -127, 127), (-100, 127), True),
    # int8 x and weight with I a multiple of 16: the product on the int8 MFMA (exact integer sums),
    # at tile tails (M = 5 and 18 rows, N = 7 and 100 columns) and the full int8 level range
    ((2, 9), 1024, 100, (0.03, -128, 127), (-127, 127), True),
    ((5,), 48, 7, (0.05, -127, 127), (-100, 127), False),
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


QUOTIENT_SCALES = [1.0 / 127.0, 1.0 / 255.0, 0.02, 3.0, 1e-8, 2.0 ** -126, 2.0 ** 64, 0.0123456]


@pytest.mark.parametrize("s", QUOTIENT_SCALES)
def test_fake_quant_codes_at_rounding_boundaries(dev, s):
    """q_x(x) from the kernel's division-free quotient equals torch's
    clamp(round(x / s)) * s bit for bit, on values within a few ulps of every
    rounding boundary (k + 1/2) s and of every k s, random values over many
    binades, zeros, subnormals, infinities and NaN. The CPU restatement of the
    same steps is pinned in test_quant_quotient.py."""
    from gru_qat_amd.input_proj import _project

    f32 = torch.float32
    s32 = torch.tensor(s, dtype=f32)
    k = torch.arange(-130, 131, dtype=torch.float64)
    base = torch.cat([((k + 0.5) * float(s32)).to(f32), (k * float(s32)).to(f32)])
    vals = [base]
    up, dn = base, base
    for _ in range(3):
        up = torch.nextafter(up, torch.full_like(up, float("inf")))
        dn = torch.nextafter(dn, torch.full_like(dn, float("-inf")))
        vals += [up, dn]
    g = torch.Generator().manual_seed(5)
    vals.append((torch.randn(2000, generator=g, dtype=torch.float64) * float(s32)
                 * 10.0 ** (torch.rand(2000, generator=g, dtype=torch.float64) * 9 - 3)).to(f32))
    vals.append(torch.tensor([0.0, -0.0, 2.0 ** -149, -(2.0 ** -149), float("inf"), float("-inf"),
                              float("nan"), 3.4e38, -3.4e38], dtype=f32))
    x = torch.cat(vals)
    x = torch.cat([x, torch.zeros((-x.numel()) % 64, dtype=f32)]).view(-1, 64)
    W = torch.zeros(8, 64)
    for qmin, qmax in ((-127, 127), (-8, 7)):
        _, _, _, xq = _project(x.to(dev), W.to(dev), None, (s, qmin, qmax), None)
        ref = torch.clamp(torch.round(x / s32), qmin, qmax) * s32
        # NaN: fmaxf/fminf return the other operand, so NaN clamps to qmin, as in the
        # reference kernel's tl.minimum(tl.maximum(q, qmin), qmax) (scan.py:136-139)
        ref = torch.where(torch.isnan(x), torch.tensor(qmin * float(s32), dtype=f32), ref)
        got = xq.cpu()
        bad = ~((got == ref) | (torch.isnan(got) & torch.isnan(ref)))
        print(f"[proj] quotient s={s:.3g} range=({qmin},{qmax}): {x.numel()} values, {int(bad.sum())} differ")
        assert not bad.any(), (x[bad][:4], got[bad][:4], ref[bad][:4])
