"""Long sequences on every persistent kernel (fp32, 1e-5 bar).

The reference runs its dense forward at T in {512, 1024} x B in {1, 4, 32} x
H in {32, 128, 512} (tests/test_triton_scan_strict.py:179-184) and checks
every path for drift at T in {512, 1024} (tests/test_edge_cases.py:598-615).
Here the same grid runs on each kernel family: dense, Diagonal, single-factor
Monarch on the block-local kernel (blksz 16/32/64) and on the MFMA kernel
(blksz 8, 256), two-factor Monarch on the fused kernel (nb | bs, bs / nb a
multiple of 4) and on the split kernel, and Butterfly. T >= 512 also runs the
persistent exchange through hundreds of tag values and both parities of the
double-buffered exchange rows many times over.
"""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import make_config
from parity_util import assert_fp32_parity

pytestmark = pytest.mark.gpu

LONG_GRID = [(T, B, H) for T in (512, 1024) for B in (1, 4, 32) for H in (32, 128, 512)]

# Monarch factorizations per H: kernel family -> nblocks
MONARCH_NB = {
    "block_local": {32: 2, 128: 4, 512: 8},     # blksz 16, 32, 64
    "mfma": {32: 4, 128: 16, 512: 2},           # blksz 8, 8, 256
    "two_factor_fused": {32: 2, 128: 4, 512: 8},   # bs / nb = 8, 8, 8
    "two_factor_split": {32: 4, 128: 8, 512: 16},  # bs / nb = 2
}


def _ids(shape):
    return "T{}-B{}-H{}".format(*shape)


@pytest.mark.parametrize("shape", LONG_GRID, ids=_ids)
def test_dense_long_t(dev, shape):
    assert_fp32_parity(make_config(1, shape=shape), dev)


@pytest.mark.parametrize("shape", LONG_GRID, ids=_ids)
def test_diagonal_long_t(dev, shape):
    assert_fp32_parity(make_config(0, shape=shape), dev)


@pytest.mark.parametrize("family", list(MONARCH_NB))
@pytest.mark.parametrize("shape", LONG_GRID, ids=_ids)
def test_monarch_long_t(dev, shape, family):
    T, B, H = shape
    nb = MONARCH_NB[family][H]
    bs = H // nb
    two = family.startswith("two_factor")
    cfg = make_config(3, shape=shape)
    g = torch.Generator().manual_seed(7)
    cfg["w"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
    cfg["w2"] = ((torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5) if two else None
    cfg.update(h_in_quant=None, h_out_quant=None)
    assert_fp32_parity(cfg, dev)


@pytest.mark.parametrize("shape", [(T, B, H) for T in (512, 1024) for B in (1, 4, 32) for H in (32, 512)], ids=_ids)
def test_butterfly_long_t(dev, shape):
    assert_fp32_parity(make_config(4, shape=shape), dev)
