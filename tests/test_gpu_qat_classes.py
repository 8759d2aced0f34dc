"""Frozen-int8 QAT forward of every kind on the reference's three input classes.

Follows the reference's strict QAT tier (tests/test_triton_scan_strict.py:
690-732 ``_adversarial_inputs``, :940-997 dense forward;
tests/test_triton_diagonal_strict.py:600-651 diagonal forward): a layer with
frozen int8 per-row weights, a frozen per-tensor int8 input quantizer
calibrated on ``randn * 0.5`` and frozen int8 hidden quantizers at ``h_scale``
(tests/test_triton_scan_strict.py:610-688); ``gi = F.linear(quant_x(x),
Wi_q, bi)`` as the reference's ``_build_qgi_from_layer``
(tests/test_triton_diagonal_strict.py:558-574); then the scan. Classes:

* ``realistic``: x, h0 ~ N(0, 0.5^2);
* ``near-saturation``: x and h0 = linspace(-0.99, 0.99) * 127 * h_scale, just
  inside the int8 range;
* ``large-magnitude``: x, h0 ~ N(0, 5^2), so q_in(h0) clips and q_out clips at
  step 0 (the raw h0 enters h' through z h).

Bar: the kernel's codes equal the oracle's wherever the pre-quant values are
more than 2e-6 from a rounding boundary (teacher forcing); the free-running
divergence is bounded (and zero when no code flipped); the clamp fires where
the class forces it. The reference asks ``torch.equal`` of its Triton kernel
against its PyTorch path on one GPU; the oracle here is torch on the CPU with
other transcendental functions, so an exact free-running match cannot be
promised for every shape (see parity_util.assert_quant_parity).
"""

from __future__ import annotations

import math

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from oracle import gru_oracle as O
from parity_util import assert_quant_parity

pytestmark = pytest.mark.gpu

CLASSES = ("realistic", "near-saturation", "large-magnitude")
H_SCALES = (0.02, Q_INT8_HIDDEN[0])
QUANT_GRID = [(T, B, H) for T in (8, 64) for B in (1, 4, 32) for H in (32, 128, 512)]
STRUCT_GRID = [(64, B, H) for B in (1, 32) for H in (128, 512)]
# Free-running divergence bound, in quantization steps. A flip moves one unit
# by one step; the map spreads it into the next step's pre-quant values, where
# it can tip other units near a boundary, and the contracting recurrence damps
# it. Measured maxima are reported per case by assert_quant_parity.
FREE_BOUND = 2.0


def adversarial_inputs(cls: str, T: int, B: int, I: int, H: int, h_scale: float, gen: torch.Generator):
    """(x [T, B, I], h0 [B, H]) of one class (reference _adversarial_inputs)."""
    x_max = h_scale * 127
    if cls == "realistic":
        x = torch.randn(T, B, I, generator=gen) * 0.5
        h0 = torch.randn(B, H, generator=gen) * 0.5
    elif cls == "near-saturation":
        x = torch.linspace(-0.99, 0.99, T * B * I).reshape(T, B, I) * x_max
        h0 = torch.linspace(-0.99, 0.99, B * H).reshape(B, H) * x_max
    elif cls == "large-magnitude":
        x = torch.randn(T, B, I, generator=gen) * 5.0
        h0 = torch.randn(B, H, generator=gen) * 5.0
    else:
        raise ValueError(cls)
    return x.float().contiguous(), h0.float().contiguous()


def qat_config(kind: str, cls: str, shape, h_scale: float, seed: int = 0, two_factor: bool = False):
    """A config dict whose gi comes from the frozen-int8 input side."""
    T, B, H = shape
    idx = {"dense": 2, "diagonal": 0, "monarch": 3 if two_factor else 5, "butterfly": 4}[kind]
    cfg = make_config(idx, shape=shape, seed=seed)
    gen = torch.Generator().manual_seed(1000 + seed)
    I = H
    k = 1.0 / math.sqrt(H)
    Wi = (torch.rand(3 * H, I, generator=gen) * 2 - 1) * k
    bi = (torch.rand(3 * H, generator=gen) * 2 - 1) * k
    # (the dense kind's Wh_cat is config 2's: per-row int8 fake-quantized)
    # quant_x: min_max observer over one calibration batch (randn * 0.5), frozen:
    # symmetric scale = max(|min|, |max|) / 127 (quantizers.py:124-134)
    cal = torch.randn(8, 4, I, generator=gen) * 0.5
    sx = float(torch.maximum(cal.amax().abs(), cal.amin().abs()).clamp(min=1e-8) / 127.0)
    x, h0 = adversarial_inputs(cls, T, B, I, H, h_scale, gen)
    gi = O.input_projection(x, Wi, bi, x_quant=(sx, -127, 127), w_quant=(-127, 127))
    q = (float(torch.tensor(h_scale, dtype=torch.float32)), -127, 127)
    cfg.update(gi=gi.contiguous(), h0=h0, h_in_quant=q, h_out_quant=q,
               name=f"{cfg['name']}_{cls}_s{h_scale:.4g}")
    if kind == "monarch" and not two_factor:
        cfg["w2"] = None
    return cfg


def _run(kind, cls, shape, h_scale, dev, two_factor=False):
    cfg = qat_config(kind, cls, shape, h_scale, two_factor=two_factor)
    if cls == "large-magnitude":
        s = cfg["h_in_quant"][0]
        assert bool((torch.round(cfg["h0"].abs() / s) > 127).any()), "q_in(h0) must clip for this class"
    # large-magnitude forces q_out to clip at step 0
    min_clipped = 1 if cls == "large-magnitude" else 0
    return assert_quant_parity(cfg, dev, free_bound=FREE_BOUND, min_clipped=min_clipped)


@pytest.mark.parametrize("h_scale", H_SCALES)
@pytest.mark.parametrize("cls", CLASSES)
@pytest.mark.parametrize("shape", QUANT_GRID)
def test_dense_qat_classes(dev, shape, cls, h_scale):
    _run("dense", cls, shape, h_scale, dev)


@pytest.mark.parametrize("h_scale", H_SCALES)
@pytest.mark.parametrize("cls", CLASSES)
@pytest.mark.parametrize("shape", QUANT_GRID)
def test_diagonal_qat_classes(dev, shape, cls, h_scale):
    _run("diagonal", cls, shape, h_scale, dev)


@pytest.mark.parametrize("cls", CLASSES)
@pytest.mark.parametrize("shape", STRUCT_GRID)
@pytest.mark.parametrize("two_factor", [False, True])
def test_monarch_qat_classes(dev, shape, cls, two_factor):
    _run("monarch", cls, shape, 0.02, dev, two_factor=two_factor)


@pytest.mark.parametrize("cls", CLASSES)
@pytest.mark.parametrize("shape", [(64, 1, 256), (64, 32, 512), (32, 4, 1024)])
def test_butterfly_qat_classes(dev, shape, cls):
    _run("butterfly", cls, shape, 0.02, dev)
