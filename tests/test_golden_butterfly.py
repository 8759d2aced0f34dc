"""Butterfly twiddle convention pinned against the reference's own kernel.

tests/golden/butterfly_reference.safetensors holds butterfly_g(h) for the
three gates of random twiddles, computed by the reference Triton kernel
(src/gru_qat/triton_kernels/scan_butterfly.py:168-366) under Triton's CPU
interpreter; tests/golden/make_butterfly_golden.py wrote it and records how.
Cases cover H = H_PAD and H < H_PAD (zero padding), one to three chains
(alternating stride direction).

CPU: the oracle's butterfly_apply reproduces every product. GPU: one scan
step of the HIP kernels on h0 with zero gi and bias equals the GRU cell
applied to the reference products.
"""

from __future__ import annotations

import os

import pytest
import torch
from safetensors.torch import load_file

from oracle import gru_oracle as O

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "butterfly_reference.safetensors")
CASES = ["h8_c1", "h6_c1", "h16_c2", "h32_c1", "h12_c3", "h64_c2"]


def _case(name):
    d = load_file(FIXTURE)
    return d[f"{name}.twiddles"], d[f"{name}.h"], d[f"{name}.products"]


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_reference_products(name):
    tw, h, prod = _case(name)
    B, H = h.shape
    n = 2 * tw.shape[3]
    x = torch.zeros(B, n)
    x[:, :H] = h
    for g in range(3):
        got = O.butterfly_apply(x, tw[g])
        assert (got - prod[g]).abs().max().item() <= 1e-5 * max(1.0, prod[g].abs().max().item())


def test_fixture_is_not_trivially_symmetric():
    # swapping the self/partner twiddle roles must break the match, so the
    # fixture really constrains the convention
    tw, h, prod = _case("h16_c2")
    B, H = h.shape
    swapped = tw.flip(-1)
    got = O.butterfly_apply(h.clone(), swapped[0])
    assert (got - prod[0]).abs().max().item() > 1e-2


def _cell_from_products(prod_g3, h):
    """One GRU step with gi = 0, bh = 0 on hidden pre-activations gh_g =
    products[g][:, :H] (the reference cell, gru_cell.py:437-464)."""
    H = h.shape[1]
    ghr, ghz, ghn = (prod_g3[g][:, :H] for g in range(3))
    r = torch.sigmoid(ghr)
    z = torch.sigmoid(ghz)
    n = torch.tanh(r * ghn)
    return (1 - z) * n + z * h


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("generic", [False, True])
def test_hip_kernel_matches_reference_products(dev, name, generic):
    import gru_qat_amd.scan_butterfly as SB

    tw, h, prod = _case(name)
    B, H = h.shape
    gi = torch.zeros(1, B, 3 * H, device=dev)
    fwd = SB.gru_scan_butterfly_forward_generic if generic else SB.gru_scan_butterfly_forward
    out = fwd(gi, h.to(dev), tw.to(dev), torch.zeros(3 * H, device=dev))
    want = _cell_from_products(prod, h)
    assert (out[0].cpu() - want).abs().max().item() <= 1e-5
