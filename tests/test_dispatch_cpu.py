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
    layer_forward,
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
    with pytest.raises(RuntimeError, match="unexpected dispatch kind 'ldr'"):
        forward_fast_dispatch("ldr", torch.zeros(3, 2, 3 * H), None, w, bh)
    # CPU tensors reach the scan, which rejects them before any device work
    with pytest.raises(ValueError):
        forward_fast_dispatch("diagonal", torch.zeros(3, 2, 3 * H), None, w, bh)


def test_frozen_scale_is_read_once_per_version(monkeypatch):
    """The reference syncs on scale.item() every forward (gru_layer.py:48); a
    frozen scale is read once, and an in-place update is seen."""
    calls = {"n": 0}
    orig = torch.Tensor.item

    def counting_item(self):
        calls["n"] += 1
        return orig(self)

    q = _quantizer(scale=0.02)
    monkeypatch.setattr(torch.Tensor, "item", counting_item)
    first = _extract_h_quant_params(q)
    n1 = calls["n"]
    for _ in range(5):
        assert _extract_h_quant_params(q) == first
    assert calls["n"] == n1 == 1
    q.scale.fill_(0.5)
    assert _extract_h_quant_params(q)[0] == 0.5
    assert calls["n"] == 2
    other = _quantizer(scale=0.02)  # a different tensor with the same value: its own entry
    assert _extract_h_quant_params(other) == first


def test_layer_forward_argument_errors():
    W = torch.zeros(12, 3)
    with pytest.raises(ValueError, match="x must be"):
        layer_forward("dense", torch.zeros(2, 3), None, W, None, torch.zeros(12, 4), torch.zeros(12))
    with pytest.raises(ValueError, match="seq length T"):
        layer_forward("dense", torch.zeros(0, 2, 3), None, W, None, torch.zeros(12, 4), torch.zeros(12))
    with pytest.raises(ValueError, match="batch size B"):
        layer_forward("dense", torch.zeros(2, 0, 3), None, W, None, torch.zeros(12, 4), torch.zeros(12))
    with pytest.raises(ValueError, match="batch size B"):
        layer_forward("dense", torch.zeros(0, 2, 3), None, W, None, torch.zeros(12, 4), torch.zeros(12),
                      batch_first=True)



@pytest.mark.parametrize("kind", ["dense", "circulant"])
def test_extended_kinds_eligible_only_when_named(kind):
    """One rule: the reference's (dense and circulant not eligible) unless the
    caller names the extension, as ScanLayer does."""
    assert resolve_use_triton("auto", kind, "fused") is False
    assert resolve_use_triton("auto", kind, "fused", extended=True) is True
    assert resolve_use_triton("auto", kind, "split", extended=True) is False
    with pytest.raises(ValueError, match="use_triton=True requires"):
        resolve_use_triton(True, kind, "fused")
    assert resolve_use_triton(True, kind, "fused", extended=True) is True
    assert resolve_use_triton("auto", "ldr", "fused", extended=True) is False


def test_scan_layer_resolves_auto_with_the_shared_rule():
    from gru_qat_amd.gru_layer import ScanLayer

    H = 8
    Wi = torch.zeros(3 * H, 4)
    for kind, hidden in (("dense", torch.zeros(3 * H, H)), ("diagonal", torch.zeros(3, H))):
        assert ScanLayer(kind, Wi, None, hidden, torch.zeros(3 * H)).use_triton is True
        assert ScanLayer(kind, Wi, None, hidden, torch.zeros(3 * H), use_triton=False).use_triton is False
