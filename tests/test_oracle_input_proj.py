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


# ---- the structured input side ---------------------------------------------------------------
# The oracle's structured_input_projection against a composition written out
# here from gru_cell.py:466-503 with nothing shared but the pinned butterfly
# product (tests/test_golden_butterfly.py): each gate's map materialized as a
# matrix, q_x, the map, the gate's output quantizer and then its bias done by
# hand in numpy (float64), concatenated r, z, n. Planted mistakes in the
# by-hand composition (bias before the output quantizer, q_x skipped, one
# scale for the whole tensor instead of one per row, r and z swapped) must
# each move the result away from the oracle.

def _np_fake_quant(y, s, qmin, qmax):
    return np.clip(np.rint(y / s), qmin, qmax) * s


def _np_rows(y, qmin, qmax):
    s = np.maximum(np.abs(y).max(axis=1, keepdims=True), 1e-8) / qmax
    return np.clip(np.rint(y / s), qmin, qmax) * s


def _gate_matrices(kind, w, H):
    """[3] matrices A_g with y_g = x @ A_g (x a row vector of length H)."""
    mats = []
    for g in range(3):
        if kind == "diagonal":
            mats.append(np.diag(w[g].numpy()))
        elif kind == "monarch":
            nb, bs = w.shape[1], w.shape[2]
            M = np.zeros((H, H))
            for n in range(nb):
                M[n * bs:(n + 1) * bs, n * bs:(n + 1) * bs] = w[g, n].numpy()  # (out, in) block
            mats.append(M.T)
        else:
            N = 2 * w.shape[3]
            A = O.butterfly_apply(torch.eye(N, dtype=w.dtype), w[g]).numpy()
            mats.append(A[:H, :H])
    return mats


def _by_hand(x, kind, w, b, xq_param, oq, mistake=""):
    H = x.shape[-1]
    xn = x.reshape(-1, H).numpy()
    xq = xn if (xq_param is None or mistake == "no_qx") else _np_fake_quant(xn, *xq_param)
    mats = _gate_matrices(kind, w, H)
    order = (1, 0, 2) if mistake == "rz_swapped" else (0, 1, 2)
    parts = []
    for g in order:
        y = xq @ mats[g]
        bg = b[g * H:(g + 1) * H].numpy()
        if mistake == "bias_first":
            y = y + bg
        q = oq[g]
        if q is not None:
            if q[0] == "rows":
                y = _np_fake_quant(y, np.maximum(np.abs(y).max(), 1e-8) / q[2], q[1], q[2]) \
                    if mistake == "tensor_scale" else _np_rows(y, q[1], q[2])
            else:
                y = _np_fake_quant(y, *q)
        if mistake != "bias_first":
            y = y + bg
        parts.append(y)
    return np.concatenate(parts, axis=-1).reshape(*x.shape[:-1], 3 * H)


def _struct_weights(kind, H, gen):
    if kind == "diagonal":
        return torch.rand(3, H, generator=gen, dtype=torch.float64) * 2 - 1
    if kind == "monarch":
        nb = 4
        return (torch.rand(3, nb, H // nb, H // nb, generator=gen, dtype=torch.float64) * 2 - 1) / (H // nb) ** 0.5
    N = 1 << (H - 1).bit_length()
    L = N.bit_length() - 1
    return torch.randn(3, 1, L, N // 2, 2, 2, generator=gen, dtype=torch.float64) * 0.5 ** 0.5


OUT_QUANTS = [(None, None, None), ((0.03, -20, 20), ("rows", -127, 127), None),
              (("rows", -7, 7), (0.01, -127, 127), ("rows", -127, 127))]


@pytest.mark.parametrize("kind,H", [("diagonal", 40), ("monarch", 64), ("butterfly", 64), ("butterfly", 48)])
@pytest.mark.parametrize("oq", OUT_QUANTS)
def test_structured_input_projection_matches_the_composition_by_hand(kind, H, oq):
    gen = torch.Generator().manual_seed(17)
    x = torch.randn(3, 5, H, generator=gen, dtype=torch.float64) * 0.7
    w = _struct_weights(kind, H, gen)
    b = torch.randn(3 * H, generator=gen, dtype=torch.float64) * 0.2
    xq = (0.05, -127, 127)
    got = O.structured_input_projection(x, kind, w, b, x_quant=xq, out_quant=oq).numpy()
    want = _by_hand(x, kind, w, b, xq, oq)
    assert np.abs(got - want).max() <= 1e-9
    for mistake in ("bias_first", "no_qx", "rz_swapped") + (("tensor_scale",) if any(
            q is not None and q[0] == "rows" for q in oq) else ()):
        if mistake == "bias_first" and all(q is None for q in oq):
            continue  # without an output quantizer the order of the bias does not matter
        wrong = _by_hand(x, kind, w, b, xq, oq, mistake)
        assert np.abs(got - wrong).max() > 1e-6, mistake
