"""Pins of the oracle's observer restatement (quantizers.py:63-156, the per-step
path with the hidden quantizers firing) by facts that do not retype its
formulas: reductions to the pinned frozen scan, known answers of the scale
rules, the code ranges a dynamic quantizer must produce, the float64
recursion of the running statistics, and freeze by hand."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import gru_oracle as O


def _dense_case(T=5, B=3, H=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    gi = torch.randn(T, B, 3 * H, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.3
    W = (torch.rand(3 * H, H, generator=g) * 2 - 1) / math.sqrt(H)
    bh = (torch.rand(3 * H, generator=g) * 2 - 1) / math.sqrt(H)
    return gi, h0, (lambda hq: O.gh_dense(hq, W, bh))


def test_off_and_frozen_reduce_to_scan():
    gi, h0, gh = _dense_case()
    out, trace = O.observe_scan(gi, h0, gh, O.ObserverState("off"), O.ObserverState("off"))
    assert torch.equal(out, O.scan(gi, h0, gh))
    assert torch.all(trace == torch.tensor([1.0, 0.0, 1.0, 0.0]))
    s = float(torch.tensor(1.0 / 127, dtype=torch.float32))
    q = (s, -127, 127)
    out, trace = O.observe_scan(gi, h0, gh, O.ObserverState("frozen", scale=s), O.ObserverState("frozen", scale=s))
    assert torch.equal(out, O.scan(gi, h0, gh, q, q))
    assert torch.all(trace[:, 0] == s) and torch.all(trace[:, 2] == s)


def test_scale_rule_known_answers():
    sym = O.ObserverState("dynamic")
    s, zp = O.scale_zp_from_min_max(sym, torch.tensor(-0.5), torch.tensor(0.25))
    assert float(s) == pytest.approx(0.5 / 127, rel=1e-7) and float(zp) == 0.0
    s, zp = O.scale_zp_from_min_max(sym, torch.tensor(0.0), torch.tensor(0.0))  # clamp to 1e-8
    assert float(s) == pytest.approx(1e-8 / 127, rel=1e-6)
    aff = O.ObserverState("dynamic", symmetric=False)
    assert (aff.qmin, aff.qmax) == (0.0, 255.0)
    s, zp = O.scale_zp_from_min_max(aff, torch.tensor(-1.0), torch.tensor(3.0))
    assert float(s) == pytest.approx(4.0 / 255, rel=1e-7)
    assert float(zp) == 64.0  # round(0 - (-1) / (4/255)) = round(63.75)
    four = O.ObserverState("dynamic", bits=4)
    assert (four.qmin, four.qmax) == (-7, 7)


@pytest.mark.parametrize("symmetric", [True, False])
def test_dynamic_codes_span_the_range(symmetric):
    """A dynamic symmetric quantizer maps its largest |x| to code +-qmax; an
    affine one maps min and max to qmin and qmax. A wrong scale rule (qmax -
    qmin for a symmetric range, a missing abs, a wrong zero-point sign) breaks
    one of these."""
    g = torch.Generator().manual_seed(1)
    for _ in range(20):
        x = torch.randn(6, 10, generator=g) * float(torch.rand(1, generator=g) * 3 + 0.01) + float(
            torch.randn(1, generator=g))
        st = O.ObserverState("dynamic", symmetric=symmetric)
        y, (s, zp) = O.observer_forward(st, x)
        codes = torch.round(y / s + zp)
        if symmetric:
            assert float(codes.abs().max()) == st.qmax
            i = int(x.abs().argmax())
            assert abs(float(codes.flatten()[i])) == st.qmax
        else:
            assert float(codes.min()) == st.qmin and float(codes.max()) == st.qmax
        # every output is on the grid: quantizing again changes nothing
        y2 = (torch.clamp(torch.round(y / s + zp), st.qmin, st.qmax) - zp) * s
        assert torch.allclose(y2, y, atol=1e-6 * float(x.abs().max()))


def test_running_statistics_match_float64_recursion():
    g = torch.Generator().manual_seed(2)
    st = O.ObserverState("min_max")
    rmin = rmax = None
    for k in range(40):
        x = torch.randn(4, 7, generator=g) * (1 + k % 3)
        O.observer_forward(st, x)
        mn, mx = float(x.min()), float(x.max())
        if rmin is None:
            rmin, rmax = mn, mx
        else:
            rmin = 0.99 * rmin + 0.01 * mn
            rmax = 0.99 * rmax + 0.01 * mx
    assert st.initialized
    assert float(st.running_min) == pytest.approx(rmin, rel=1e-5, abs=1e-6)
    assert float(st.running_max) == pytest.approx(rmax, rel=1e-5, abs=1e-6)


def test_dynamic_mode_leaves_statistics_alone():
    st = O.ObserverState("dynamic")
    O.observer_forward(st, torch.randn(3, 3))
    assert not st.initialized and float(st.running_min) == math.inf


def test_freeze_uses_running_statistics():
    st = O.ObserverState("min_max")
    O.observer_forward(st, torch.tensor([[-0.75, 0.5]]))
    O.freeze_observer(st)
    assert st.mode == "frozen"
    assert float(st.scale) == pytest.approx(0.75 / 127, rel=1e-7)
    y, (s, zp) = O.observer_forward(st, torch.tensor([0.3]))
    assert s == float(st.scale) and zp == 0.0
    assert float(y) == pytest.approx(round(0.3 / s) * s, rel=1e-6)


def test_observe_scan_counts_and_order():
    """quant_h_in sees h0 then out[0..T-2] (T calls), quant_h_out the T pre-quant
    states; with min_max on both, their statistics equal the float64
    recursions over exactly those tensors."""
    gi, h0, gh = _dense_case(T=6)
    qi, qo = O.ObserverState("min_max"), O.ObserverState("min_max")
    out, trace = O.observe_scan(gi, h0, gh, qi, qo)
    seen_in = [h0] + [out[t] for t in range(5)]
    r = None
    for x in seen_in:
        mn, mx = float(x.min()), float(x.max())
        r = (mn, mx) if r is None else (0.99 * r[0] + 0.01 * mn, 0.99 * r[1] + 0.01 * mx)
    assert float(qi.running_min) == pytest.approx(r[0], rel=1e-5)
    assert float(qi.running_max) == pytest.approx(r[1], rel=1e-5)
    # q_in's scale at step t is that of the tensor it saw
    for t, x in enumerate(seen_in):
        assert float(trace[t, 0]) == pytest.approx(float(x.abs().max()) / 127, rel=1e-6)
    # q_out's output codes reach +-127 every step (dynamic symmetric)
    for t in range(6):
        assert float(torch.round(out[t] / trace[t, 2]).abs().max()) == 127.0
