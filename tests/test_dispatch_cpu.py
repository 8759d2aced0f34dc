"""GRULayer scan-dispatch glue (reference src/gru_qat/gru_layer.py:30-48,
:110-124, :183-192, :260-302): eligibility, the use_triton contract, hidden
quant-parameter extraction and argument errors. CPU only."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from gru_qat_amd.gru_layer import (
    _extract_h_quant_params,
    fast_dispatch_eligible,
    forward_fast_dispatch,
    resolve_use_triton,
)


@pytest.mark.parametrize("kind,layout,expected", [
    ("diagonal", "fused", True), ("monarch", "fused", True), ("butterfly", "fused", True),
    ("diagonal", "split", False), ("monarch", "split", False), (None, "fused", False),
    ("circulant", "fused", False), ("ldr", "fused", False), ("dense", "fused", False),
])
def test_eligibility(kind, layout, expected):
    assert fast_dispatch_eligible(kind, layout) is expected
    assert resolve_use_triton("auto", kind, layout) is expected
    assert resolve_use_triton(False, kind, layout) is False


@pytest.mark.parametrize("kind,layout", [(None, "fused"), ("monarch", "split"), ("circulant", "fused")])
def test_use_triton_true_on_ineligible_raises(kind, layout):
    with pytest.raises(ValueError, match="use_triton=True requires"):
        resolve_use_triton(True, kind, layout)


def test_use_triton_true_on_eligible():
    assert resolve_use_triton(True, "butterfly", "fused") is True


def _quantizer(mode="frozen", axis=None, symmetric=True, scale=1.0 / 127, bits=8):
    qmax = 2 ** (bits - 1) - 1 if symmetric else 2 ** bits - 1
    qmin = -qmax if symmetric else 0
    s = torch.tensor(scale) if axis is None else torch.full((4, 1), scale)
    return SimpleNamespace(config=SimpleNamespace(mode=mode, axis=axis, symmetric=symmetric),
                           scale=s, qmin=float(qmin), qmax=float(qmax))


def test_extract_h_quant_params():
    q = _extract_h_quant_params(_quantizer())
    assert q == (float(torch.tensor(1.0 / 127).item()), -127, 127)
    assert isinstance(q[1], int) and isinstance(q[2], int)
    assert _extract_h_quant_params(_quantizer(bits=4)) == (float(torch.tensor(1.0 / 127).item()), -7, 7)
    # not frozen, per-channel, asymmetric: no in-kernel fake-quant
    assert _extract_h_quant_params(_quantizer(mode="dynamic")) is None
    assert _extract_h_quant_params(_quantizer(mode="min_max")) is None
    assert _extract_h_quant_params(_quantizer(axis=0)) is None
    assert _extract_h_quant_params(_quantizer(symmetric=False)) is None


def test_forward_fast_dispatch_argument_errors():
    H = 8
    w = torch.zeros(3, H)
    bh = torch.zeros(3 * H)
    with pytest.raises(ValueError, match="seq length T must be > 0; got T=0"):
        forward_fast_dispatch("diagonal", torch.zeros(0, 2, 3 * H), None, w, bh)
    with pytest.raises(ValueError, match="batch size B must be > 0; got B=0"):
        forward_fast_dispatch("diagonal", torch.zeros(3, 0, 3 * H), None, w, bh)
    with pytest.raises(ValueError, match=r"gi must be \[T, B, 3H\]"):
        forward_fast_dispatch("diagonal", torch.zeros(3, 3 * H), None, w, bh)
    with pytest.raises(RuntimeError, match="unexpected dispatch kind 'circulant'"):
        forward_fast_dispatch("circulant", torch.zeros(3, 2, 3 * H), None, w, bh)
    # CPU tensors reach the scan, which rejects them before any device work
    with pytest.raises(ValueError):
        forward_fast_dispatch("diagonal", torch.zeros(3, 2, 3 * H), None, w, bh)
