"""Pins of the oracle's input projection (the gi producer of the reference's
GRULayer fast dispatch, gru_layer.py:249-255) and of its per-row weight
fake-quant (quantizers.py:124-134, 188-199), independent of the restatement's
own formulas."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gru_oracle as O


def _w(N=24, I=40, seed=0):
    return torch.randn(N, I, generator=torch.Generator().manual_seed(seed)) * 0.3


def test_weight_scale_is_row_absmax_over_qmax_in_fp32():
    W = _w()
    _, scale = O.weight_fake_quant_rows(W, -127, 127)
    a = W.numpy().astype(np.float32)
    want = (np.abs(a).max(axis=1).astype(np.float32) / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(scale.numpy(), want)


def test_weight_codes_follow_the_pinned_fake_quant_row_by_row():
    """Each row is fake_quant (pinned by the round-half-even and boundary
    tests of tests/test_oracle.py) with that row's scale; the row's absmax
    element lands on +-qmax, nothing clips."""
    W = _w(seed=3)
    wq, scale = O.weight_fake_quant_rows(W, -127, 127)
    for n in range(W.shape[0]):
        q = (float(scale[n]), -127, 127)
        assert torch.equal(wq[n], O.fake_quant(W[n], q))
        codes = O.quant_codes(W[n], q)
        assert codes.abs().max().item() == 127
        k = int(W[n].abs().argmax())
        assert abs(codes[k].item()) == 127


def test_zero_row_uses_the_clamped_scale():
    W = torch.zeros(2, 5)
    W[1, 2] = 1e-12
    wq, scale = O.weight_fake_quant_rows(W, -127, 127)
    assert torch.all(scale == torch.tensor(np.float32(1e-8) / np.float32(127.0)))
    assert torch.equal(wq, torch.zeros_like(W))


def test_identity_weight_gives_quantized_input_plus_bias():
    torch.manual_seed(0)
    x = torch.randn(3, 4, 16) * 0.5
    b = torch.randn(16)
    q = (0.02, -127, 127)
    gi = O.input_projection(x, torch.eye(16), b, x_quant=q)
    assert torch.equal(gi, O.fake_quant(x, q) + b)
    assert torch.equal(O.input_projection(x, torch.eye(16), b), x + b)


def test_projection_matches_float64_brute_force():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(6, 9, generator=g)
    W = torch.randn(7, 9, generator=g)
    b = torch.randn(7, generator=g)
    gi = O.input_projection(x, W, b, w_quant=(-127, 127))
    wq, _ = O.weight_fake_quant_rows(W, -127, 127)
    ref = np.zeros((6, 7))
    for m in range(6):
        for n in range(7):
            ref[m, n] = sum(float(x[m, i]) * float(wq[n, i]) for i in range(9)) + float(b[n])
    assert np.abs(gi.numpy() - ref).max() < 1e-5


@pytest.mark.parametrize("mistake", ["qmin_scale", "no_clamp_floor"])
def test_planted_mistakes_fail_the_pins(mistake):
    """A scale over qmin (sign flip) or a missing 1e-8 floor breaks the pins."""
    W = _w(seed=1)
    W[0] = 0.0
    a = W.numpy()
    absmax = np.abs(a).max(axis=1).astype(np.float32)
    if mistake == "qmin_scale":
        bad = absmax / np.float32(-127.0)
        assert not np.array_equal(bad, O.weight_fake_quant_rows(W, -127, 127)[1].numpy())
    else:
        bad = absmax / np.float32(127.0)  # row 0 -> scale 0 -> NaN codes
        assert bad[0] == 0.0 and O.weight_fake_quant_rows(W, -127, 127)[1][0].item() > 0.0


def _rows_dynamic_grad_closed_form(W: np.ndarray, G: np.ndarray, qmax: float) -> np.ndarray:
    """d/dW of sum(G * fq(W)) for the per-row dynamic symmetric fake-quant, by
    hand in float64: STE (G itself) plus dL/ds = sum_i G_i (q_i - W_i / s) per
    row, times ds/dW = (1 / qmax) d max(|max|, |min|) / dW, where the max (min)
    element gets sign(max) (sign(min)), halved when |max| == |min| and shared
    by equal maxima (minima)."""
    W = W.astype(np.float64)
    out = G.astype(np.float64).copy()
    for n in range(W.shape[0]):
        row = W[n]
        mx, mn = row.max(), row.min()
        absmax = max(abs(mx), abs(mn))
        s = max(absmax, 1e-8) / qmax
        q = np.clip(np.round(row / s), -qmax, qmax)
        dLds = float(np.sum(G[n] * (q - row / s)))
        if absmax < 1e-8:
            continue
        w_mx = 1.0 if abs(mx) > abs(mn) else (0.5 if abs(mx) == abs(mn) else 0.0)
        w_mn = 1.0 if abs(mn) > abs(mx) else (0.5 if abs(mx) == abs(mn) else 0.0)
        at_mx, at_mn = row == mx, row == mn
        out[n, at_mx] += dLds / qmax * w_mx * np.sign(mx) / at_mx.sum()
        out[n, at_mn] += dLds / qmax * w_mn * np.sign(mn) / at_mn.sum()
    return out


def test_ste_gradients_match_the_straight_through_formulas():
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(5, 8, generator=g) * 2.0).requires_grad_(True)
    W = torch.randn(6, 8, generator=g).requires_grad_(True)
    b = torch.randn(6, generator=g).requires_grad_(True)
    q = (0.02, -127, 127)
    gi = O.input_projection(x, W, b, x_quant=q, w_quant=(-127, 127), ste=True)
    dgi = torch.randn(gi.shape, generator=g)
    dx, dW, db = torch.autograd.grad(gi, [x, W, b], dgi)
    wq, _ = O.weight_fake_quant_rows(W.detach(), -127, 127)
    mask = (torch.round(x.detach() / 0.02).abs() <= 127).float()
    assert torch.allclose(dx, (dgi @ wq) * mask, atol=1e-6)
    gw = (dgi.t() @ O.fake_quant(x.detach(), q)).numpy()  # gradient reaching W_q
    want = _rows_dynamic_grad_closed_form(W.detach().numpy(), gw, 127.0)
    assert np.allclose(dW.numpy(), want, atol=1e-4, rtol=1e-5)
    # the scale path is not negligible: dropping it (a detached scale) misses the closed form
    assert not np.allclose(gw, want, atol=1e-3)
    assert torch.allclose(db, dgi.sum(0), atol=1e-6)
    assert mask.min().item() == 0.0  # some x clip at |x| > 2.55


@pytest.mark.parametrize("row", [[1.0, -1.0, 0.5, 0.25],      # |max| == |min|: halved
                                 [2.0, 2.0, -1.0, 0.5],       # two equal maxima: shared
                                 [-3.0, 0.5, -3.0, 1.0],      # two equal minima carry the scale
                                 [0.0, 0.0, 0.0, 0.0]])       # the 1e-8 floor: no scale path
def test_dynamic_rows_gradient_ties_and_floor(row):
    W = torch.tensor([row], dtype=torch.float64, requires_grad=True)
    G = torch.tensor([[0.3, -0.7, 1.1, 0.2]], dtype=torch.float64)
    (O.fake_quant_rows_dynamic(W, -127, 127) * G).sum().backward()
    want = _rows_dynamic_grad_closed_form(W.detach().numpy(), G.numpy(), 127.0)
    assert np.allclose(W.grad.numpy(), want, atol=1e-12)


def test_fake_quant_rows_dynamic_forward_is_the_pinned_rule():
    g = torch.Generator().manual_seed(4)
    W = torch.randn(7, 33, generator=g)
    W[3] = 0.0
    assert torch.equal(O.fake_quant_rows_dynamic(W, -127, 127), O.weight_fake_quant_rows(W, -127, 127)[0])
