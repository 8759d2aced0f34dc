"""Structured input projection (reference gru_cell.py:466-503) against the oracle.

Forward: gi within 1e-5 (relative to max(1, |gi|)) of the oracle, except that
where an output quantizer's pre-quant value lies within 1e-4 of a rounding
boundary (in code units) a one-step difference is allowed. Backward: dx,
dWi_struct and dbi within 1e-4 * max(1, max|oracle|) of torch's autograd
through the oracle's restatement of the reference quantizers (STE, clipped STE,
and the dynamic per-row scale's own gradient path), teacher-forced: the oracle's
output quantizers see the kernel's own pre-quant values (the same call with the
output quantizers off), so a forward boundary flip (allowed above) does not
move the gradient it is compared with. End to end: layer_forward with a
structured input side against the oracle's projection and scan.
"""

from __future__ import annotations

import math

import pytest
import torch

import gru_qat_amd as G
from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from oracle import gru_oracle as O
from parity_util import FP32_TOL, log

pytestmark = pytest.mark.gpu

FROZEN = (0.03, -127, 127)
ROWS = ("rows", -127, 127)
# an asymmetric per-row range: the scale is max|y| / 127, so codes below -100 clip
# (the clipped-STE mask then zeroes their gradient and their scale term)
ROWS_ASYM = ("rows", -100, 127)


def _weights(kind: str, H: int, gen: torch.Generator, nb: int = 4, chains: int = 1) -> torch.Tensor:
    if kind == "diagonal":
        return torch.rand(3, H, generator=gen) * 2 - 1
    if kind == "monarch":
        bs = H // nb
        return (torch.rand(3, nb, bs, bs, generator=gen) * 2 - 1) / math.sqrt(bs)
    n = 1 << max(1, (H - 1).bit_length())
    L = n.bit_length() - 1
    return torch.randn(3, chains, L, n // 2, 2, 2, generator=gen) * math.sqrt(0.5)


def _oracle_prequant(kind, x, W, x_quant):
    return O.structured_input_projection(x, kind, W, None, x_quant=x_quant)


def _scale_of(spec, yg):
    if spec is None:
        return None
    if spec[0] == "rows":
        return (yg.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8) / spec[2])
    return torch.tensor(spec[0])


def _check_forward(kind, x, W, b, x_quant, out_quant, gi):
    ref = O.structured_input_projection(x, kind, W, b, x_quant=x_quant, out_quant=out_quant)
    pre = _oracle_prequant(kind, x, W, x_quant).reshape(-1, 3 * x.shape[-1])
    H = x.shape[-1]
    got = gi.reshape(-1, 3 * H)
    want = ref.reshape(-1, 3 * H)
    diff = (got - want).abs()
    tol = FP32_TOL * torch.clamp(want.abs(), min=1.0)
    allowed = torch.zeros_like(diff, dtype=torch.bool)
    step = torch.zeros_like(diff)
    for g in range(3):
        spec = out_quant[g]
        sl = slice(g * H, (g + 1) * H)
        s = _scale_of(spec, pre[:, sl])
        if s is None:
            continue
        code = pre[:, sl] / s
        allowed[:, sl] = (code - torch.floor(code) - 0.5).abs() <= 1e-4
        step[:, sl] = s.expand_as(code) if s.dim() else s
    bad = (diff > tol) & ~(allowed & (diff <= step + tol))
    log(f"[sproj]   forward max diff {diff.max().item():.3e}; near-boundary flips "
        f"{int(((diff > tol) & allowed).sum())}")
    assert not bad.any(), f"{int(bad.sum())} elements differ beyond the bar; max {diff[bad].max().item():.3e}"


CASES = [
    ("diagonal", 64, {}), ("diagonal", 512, {}), ("diagonal", 37, {}),
    ("monarch", 64, {"nb": 4}), ("monarch", 512, {"nb": 8}), ("monarch", 96, {"nb": 4}), ("monarch", 40, {"nb": 5}),
    ("butterfly", 256, {}), ("butterfly", 100, {}), ("butterfly", 64, {"chains": 2}),
]
QUANTS = [
    ("none", None, (None, None, None)),
    ("x", (0.05, -127, 127), (None, None, None)),
    ("frozen", (0.05, -127, 127), (FROZEN, FROZEN, FROZEN)),
    ("rows", None, (ROWS, ROWS, ROWS)),
    ("mixed", (0.05, -127, 127), (None, FROZEN, ROWS)),
    ("rows_asym", None, (ROWS_ASYM, ROWS, ROWS_ASYM)),
]


@pytest.mark.parametrize("qname,x_quant,out_quant", QUANTS, ids=[q[0] for q in QUANTS])
@pytest.mark.parametrize("kind,H,kw", CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}" for c in CASES])
def test_struct_input_projection_forward_and_gradients(dev, kind, H, kw, qname, x_quant, out_quant):
    T, B = 6, 5
    gen = torch.Generator().manual_seed(H + len(qname))
    W = _weights(kind, H, gen, **kw)
    b = torch.rand(3 * H, generator=gen) * 0.2 - 0.1
    x = torch.randn(T, B, H, generator=gen) * 2.0
    log(f"[sproj] {kind} H={H} {kw} quant={qname}")
    xd = x.to(dev).requires_grad_(True)
    Wd = W.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True)
    gi = G.structured_input_projection(xd, kind, Wd, bd, x_quant=x_quant, out_quant=out_quant)
    torch.cuda.synchronize(dev)
    _check_forward(kind, x, W, b, x_quant, out_quant, gi.detach().cpu())
    dgi = torch.randn(gi.shape, generator=gen)
    (gi * dgi.to(dev)).sum().backward()
    with torch.no_grad():
        y_kernel = G.structured_input_projection(x.to(dev), kind, W.to(dev), None, x_quant=x_quant,
                                                 out_quant=(None, None, None)).cpu()
    xr, Wr, br = (t.clone().requires_grad_(True) for t in (x, W, b))
    ref = O.structured_input_projection(xr, kind, Wr, br, x_quant=x_quant, out_quant=out_quant, ste=True,
                                        y_value=y_kernel.reshape(-1, 3 * H))
    (ref * dgi).sum().backward()
    for name, got, want in (("dx", xd.grad, xr.grad), ("dW", Wd.grad, Wr.grad), ("db", bd.grad, br.grad)):
        err = (got.cpu() - want).abs().max().item()
        log(f"[sproj]   {name}: max err {err:.3e}")
        assert err <= 1e-4 * max(1.0, want.abs().max().item()), name


def test_struct_input_projection_benchmark_shape(dev):
    """T = 64, B = 32, H = 512 (the benchmark shape), Monarch nb = 8, int8 x and
    per-row dynamic outputs."""
    T, B, H = 64, 32, 512
    gen = torch.Generator().manual_seed(3)
    W = _weights("monarch", H, gen, nb=8)
    b = torch.rand(3 * H, generator=gen) * 0.2 - 0.1
    x = torch.randn(T, B, H, generator=gen)
    oq = (ROWS, ROWS, ROWS)
    gi = G.structured_input_projection(x.to(dev), "monarch", W.to(dev), b.to(dev), x_quant=(0.05, -127, 127),
                                       out_quant=oq)
    torch.cuda.synchronize(dev)
    _check_forward("monarch", x, W, b, (0.05, -127, 127), oq, gi.cpu())


@pytest.mark.parametrize("input_kind,kind", [("diagonal", "diagonal"), ("monarch", "monarch"),
                                             ("butterfly", "butterfly"), ("monarch", "dense")])
def test_layer_forward_with_a_structured_input_side(dev, input_kind, kind):
    T, B, H = 9, 4, 64
    idx = {"diagonal": 0, "monarch": 5, "butterfly": 4, "dense": 1}[kind]
    cfg = make_config(idx, shape=(T, B, H), seed=2)
    gen = torch.Generator().manual_seed(8)
    Wi = _weights(input_kind, H, gen, nb=4)
    bi = torch.rand(3 * H, generator=gen) * 0.2 - 0.1
    x = torch.randn(T, B, H, generator=gen)
    q = Q_INT8_HIDDEN
    oq = (FROZEN, ROWS, None)
    hidden = cfg["w"]
    out, h_T = G.layer_forward(kind, x.to(dev), None, Wi.to(dev), bi.to(dev), hidden.to(dev), cfg["bh"].to(dev),
                               x_quant=(0.05, -127, 127), h_in_quant=q, h_out_quant=q, input_kind=input_kind,
                               wi_out_quant=oq)
    torch.cuda.synchronize(dev)
    # the scan is checked on the kernel's own gi (teacher forcing), which is checked against the oracle's
    gi = G.structured_input_projection(x.to(dev), input_kind, Wi.to(dev), bi.to(dev), x_quant=(0.05, -127, 127),
                                       out_quant=oq).cpu()
    _check_forward(input_kind, x, Wi, bi, (0.05, -127, 127), oq, gi)
    c = dict(cfg, gi=gi, h0=torch.zeros(B, H), h_in_quant=q, h_out_quant=q)
    pre = O.teacher_forced_prequant(c, out.cpu())
    codes = O.quant_codes(pre, q)
    xr = pre / q[0]
    near = (xr - torch.floor(xr) - 0.5).abs() * q[0] <= 2e-6
    mism = torch.round(out.cpu() / q[0]) != codes
    log(f"[sproj] layer {input_kind}->{kind}: code flips {int(mism.sum())} (near boundaries {int((mism & near).sum())})")
    assert not (mism & ~near).any()
    assert torch.equal(h_T.cpu(), out[-1].cpu())
