"""Pins the oracle's backward (restatement of the reference's recompute-based
_gru_scan_backward_pytorch, src/gru_qat/triton_kernels/scan.py:1450-1550)
against torch.autograd through the oracle forward with the reference's STE
gradients (ste.py:17-95), in float64, for every hidden kind. A coarse hidden
quantizer (range +-0.5) makes both clipped-STE masks zero out some entries."""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import make_config
from oracle import gru_oracle as O

COARSE = (0.05, -10, 10)


def _cfg64(idx, shape, seed=0, nb=None, two=False, q=None):
    cfg = make_config(idx, shape=shape, seed=seed)
    T, B, H = shape
    if idx == 3:
        g = torch.Generator().manual_seed(seed + 7)
        bs = H // nb
        cfg["w"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
        cfg["w2"] = ((torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5) if two else None
    cfg["h0"] = torch.randn(B, H, generator=torch.Generator().manual_seed(seed + 3)) * 0.3
    cfg["h_in_quant"] = q
    cfg["h_out_quant"] = q
    for k in ("gi", "h0", "w", "w2", "bh"):
        if cfg.get(k) is not None:
            cfg[k] = cfg[k].double()
    return cfg


CASES = [
    (1, (4, 3, 6), None, False), (0, (5, 3, 5), None, False), (3, (4, 2, 8), 2, False),
    (3, (4, 2, 8), 2, True), (4, (3, 2, 8), None, False), (4, (3, 2, 6), None, False),
    (6, (4, 3, 7), None, False),
]


@pytest.mark.parametrize("idx,shape,nb,two", CASES)
@pytest.mark.parametrize("q", [None, COARSE])
def test_backward_matches_autograd(idx, shape, nb, two, q):
    cfg = _cfg64(idx, shape, nb=nb, two=two, q=q)
    out = O.scan_config(cfg)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    got = O.scan_backward(cfg, out, dout)

    keys = ["gi", "h0", "bh"] + list(O.hidden_params(cfg))
    leaves = {k: cfg[k].detach().clone().requires_grad_(True) for k in keys}
    out2 = O.scan_ste(dict(cfg, **leaves))
    assert torch.equal(out2.detach(), out)
    grads = torch.autograd.grad(out2, [leaves[k] for k in keys], dout)
    for k, g in zip(keys, grads):
        ref = g
        mine = got["d" + k]
        assert mine.shape == ref.shape, k
        assert (mine - ref).abs().max().item() <= 1e-10 * max(1.0, ref.abs().max().item()), k


def test_clipping_masks_are_exercised():
    cfg = _cfg64(1, (4, 3, 6), q=COARSE)
    out = O.scan_config(cfg)
    assert (out.abs() >= 0.5 - 1e-12).any()  # some outputs sit on the clipped edge


@pytest.mark.parametrize("mutation", ["dgh_n_without_r", "ignore_mask_in"])
def test_pin_catches_planted_mistakes(mutation):
    cfg = _cfg64(1, (4, 3, 6), q=COARSE)
    out = O.scan_config(cfg)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    bad = O.scan_backward(cfg, out, dout, _mutation=mutation)
    keys = ["gi", "h0", "bh", "w"]
    leaves = {k: cfg[k].detach().clone().requires_grad_(True) for k in keys}
    grads = torch.autograd.grad(O.scan_ste(dict(cfg, **leaves)), [leaves[k] for k in keys], dout)
    worst = max((bad["d" + k] - g).abs().max().item() for k, g in zip(keys, grads))
    assert worst > 1e-4
