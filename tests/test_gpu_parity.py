"""Parity of the HIP kernels (through the C ABI) with the CPU oracle.

fp32: max |out - oracle| <= 1e-5 on every element and on h_T.
Quant: integer codes bit-exact wherever the pre-quant fp32 values agree (see
parity_util.assert_quant_parity).
Shapes cover the reference tests' grids (tests/test_triton_*.py,
tests/test_edge_cases.py: T=1, B=1, H in {1, 2, 8}, partial batch tiles,
non-multiple-of-4 sizes) and the five benchmark configurations.
"""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from parity_util import assert_fp32_parity, assert_fp32_teacher_forced, assert_quant_parity, small_cfg

pytestmark = pytest.mark.gpu

Q = Q_INT8_HIDDEN
Q2 = (0.02, -100, 100)
WIDE = (0.004, -1000, 1000)  # levels beyond a byte

# ---- diagonal -----------------------------------------------------------------------------

DIAG_SHAPES = [(8, 4, 32), (16, 8, 64), (8, 32, 64), (16, 32, 256), (1, 4, 8), (5, 1, 1), (5, 1, 2),
               (3, 4, 1), (9, 3, 7), (13, 33, 100)]


@pytest.mark.parametrize("shape", DIAG_SHAPES)
def test_diagonal_fp32(dev, shape):
    assert_fp32_parity(small_cfg(0, shape), dev)


@pytest.mark.parametrize("shape", [(16, 8, 64), (1, 1, 8), (37, 3, 100)])
@pytest.mark.parametrize("qin,qout", [(Q, Q), (None, Q), (Q, None), (Q2, Q), (Q2, None)])
def test_diagonal_quant(dev, shape, qin, qout):
    cfg = small_cfg(0, shape, h_in_quant=qin, h_out_quant=qout)
    if qout is None:
        assert_fp32_parity(cfg, dev)
    else:
        assert_quant_parity(cfg, dev)


def test_diagonal_cfg0(dev):
    assert_fp32_parity(make_config(0), dev)


# ---- dense --------------------------------------------------------------------------------

DENSE_SHAPES = [(8, 16, 128), (16, 32, 256), (7, 4, 16), (16, 8, 32), (1, 4, 8), (5, 1, 1), (5, 1, 2),
                (3, 4, 1), (3, 4, 2), (9, 3, 24), (6, 5, 17), (4, 33, 64), (3, 6, 300)]


@pytest.mark.parametrize("shape", DENSE_SHAPES)
def test_dense_fp32(dev, shape):
    assert_fp32_parity(small_cfg(1, shape), dev)


@pytest.mark.parametrize("qin,qout", [(Q, Q), (None, Q), (Q, None), (Q2, Q)])
def test_dense_quant(dev, qin, qout):
    cfg = small_cfg(1, (8, 4, 64), h_in_quant=qin, h_out_quant=qout)
    if qout is None:
        assert_fp32_parity(cfg, dev)
    else:
        assert_quant_parity(cfg, dev)


# Remote mode (the group spans workgroups) with hidden quantizers: an int8 level
# published through the packed exchange, four levels per tagged word, at KC =
# 8 (H 100), 16 (H 256), 32 (H 300 and 512; 300 leaves the second poller wave
# 11 words) and 64 (H 1024, four words per lane). H 302 is not a multiple of 4
# and WIDE's levels do not fit a byte: both keep the fp32 exchange words.
@pytest.mark.parametrize("shape", [(5, 4, 100), (5, 3, 256), (5, 4, 300), (6, 5, 512), (4, 3, 1024), (4, 3, 302)])
@pytest.mark.parametrize("qin,qout", [(Q, Q), (Q2, Q), (None, Q), (Q, None), (WIDE, WIDE)])
def test_dense_remote_quant_modes(dev, shape, qin, qout):
    cfg = small_cfg(1, shape, h_in_quant=qin, h_out_quant=qout)
    if qout is None:
        assert_fp32_teacher_forced(cfg, dev)
    else:
        assert_quant_parity(cfg, dev)


def test_dense_cfg1(dev):
    assert_fp32_parity(make_config(1), dev)


def test_dense_cfg2_quant(dev):
    assert_quant_parity(make_config(2), dev)


def test_dense_h1024(dev):
    assert_fp32_parity(small_cfg(1, (4, 8, 1024)), dev)


# ---- Monarch ------------------------------------------------------------------------------

def _monarch(shape, nb, two=False, seed=0, **over):
    T, B, H = shape
    cfg = make_config(3, shape=shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    bs = H // nb
    cfg["w"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
    cfg["w2"] = ((torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5) if two else None
    cfg["h_in_quant"] = None
    cfg["h_out_quant"] = None
    cfg.update(over)
    return cfg


# blksz 16, 32, 64 and 128 run the block-local kernel (scan_monarch1.hip; (7, 5, 64) and (9, 3, 128)
# leave the last workgroup's rows partly empty), other block sizes the MFMA kernel of scan_dense.hip
MONARCH_CASES = [((8, 4, 32), 4), ((16, 8, 64), 4), ((8, 32, 64), 4), ((16, 32, 256), 4), ((6, 3, 30), 5),
                 ((5, 4, 256), 2), ((4, 5, 8), 8), ((1, 4, 8), 2), ((7, 5, 64), 4), ((9, 3, 128), 4),
                 ((3, 2, 1024), 16), ((4, 3, 192), 3), ((1, 1, 64), 4), ((2, 1, 512), 4)]


@pytest.mark.parametrize("shape,nb", MONARCH_CASES)
def test_monarch_single_fp32(dev, shape, nb):
    assert_fp32_parity(_monarch(shape, nb), dev)


# Fused kernel (bs <= 64, nb | bs, bs / nb a multiple of 4): (6, 5, 64) nb 4,
# (7, 9, 128) nb 4, (3, 2, 96) nb 2 (12 compute waves), (5, 6, 256) nb 4 (two
# quads per wave), (3, 5, 1024) nb 16 (rows polled in two chunks), (4, 33, 512)
# nb 8 (ragged batch), (4, 3, 48) nb 2 (bs 24: K chain of 32 with the last 8
# masked). bs 32 and 64 stage z with swapped quad chunks (qpa 1, 2 and 4 here).
# Split kernel: the rest.
@pytest.mark.parametrize("shape,nb", [((5, 3, 32), 8), ((6, 5, 64), 4), ((4, 4, 256), 2), ((6, 3, 30), 5),
                                      ((7, 9, 128), 4), ((3, 2, 96), 2), ((5, 6, 256), 4), ((3, 5, 1024), 16),
                                      ((4, 33, 512), 8), ((4, 3, 48), 2)])
def test_monarch_two_factor_fp32(dev, shape, nb):
    assert_fp32_parity(_monarch(shape, nb, two=True), dev)


# Fused two-factor kernel with hidden quantizers. A published q_in(h) that is
# an int8 fake-quant level goes through the packed exchange (four levels per
# tagged word): H = 64 and 512 poll one word per lane, H = 1024 two. WIDE's
# levels do not fit a byte and keep the fp32 exchange words.


@pytest.mark.parametrize("shape,nb", [((6, 4, 64), 4), ((6, 5, 512), 8), ((5, 3, 1024), 16)])
@pytest.mark.parametrize("qin,qout", [(Q, Q), (Q2, Q), (None, Q), (Q, None), (Q2, None), (WIDE, WIDE)])
def test_monarch_two_factor_quant_modes(dev, shape, nb, qin, qout):
    cfg = _monarch(shape, nb, two=True, h_in_quant=qin, h_out_quant=qout)
    if qout is None:
        assert_fp32_teacher_forced(cfg, dev)
    else:
        assert_quant_parity(cfg, dev)


@pytest.mark.parametrize("shape,nb", [((6, 8, 64), 4), ((6, 8, 192), 4)])
def test_monarch_two_factor_identity_equals_single(dev, shape, nb):
    """Identity second factor gives the single-factor map, within 1e-6: the
    two-factor kernel's phase 1 sums each dot product over 4 K slices, the
    single-factor kernels over 16 K slices (MFMA kernel, blksz 48) or in lane
    quarters (block-local kernel, blksz 16), and phase 2 through the identity
    is exact."""
    cfg = _monarch(shape, nb)
    bs = shape[2] // nb
    eye = torch.eye(bs).expand(3, nb, bs, bs).contiguous()
    from parity_util import to_dev
    from gru_qat_amd.configs import run_config

    one = run_config(to_dev(cfg, dev)).cpu()
    two = run_config(to_dev(dict(cfg, w2=eye), dev)).cpu()
    assert (one - two).abs().max().item() <= 1e-6


@pytest.mark.parametrize("two", [False, True])
def test_monarch_quant(dev, two):
    cfg = _monarch((16, 8, 64), 4, two=two, h_in_quant=Q, h_out_quant=Q)
    assert_quant_parity(cfg, dev)


# single factor: blksz 64 (block-local kernel) and 24 (MFMA kernel), each quantizer alone and both
# with different scales (q_in then re-quantizes the carried h every step)
# blksz 64, 16, 128 (block-local kernel, every quantizer-mode instantiation) and 24 (MFMA kernel)
@pytest.mark.parametrize("shape,nb", [((12, 6, 256), 4), ((12, 6, 96), 4), ((9, 5, 128), 8), ((7, 3, 512), 4)])
@pytest.mark.parametrize("qin,qout", [(None, Q), (Q, None), (Q2, Q), (Q, Q), (Q2, None)])
def test_monarch_single_quant_modes(dev, shape, nb, qin, qout):
    cfg = _monarch(shape, nb, h_in_quant=qin, h_out_quant=qout)
    if qout is None:
        assert_fp32_parity(cfg, dev)
    else:
        assert_quant_parity(cfg, dev)


def test_monarch_cfg3_single_factor_fp32(dev):
    cfg = make_config(3)
    cfg.update(w2=None, h_in_quant=None, h_out_quant=None)
    assert_fp32_parity(cfg, dev)


def test_monarch_cfg3(dev):
    assert_quant_parity(make_config(3), dev)


def test_monarch_single_factor_cfg5(dev):
    """Config 5: the reference's single-factor Monarch (nb = 8, blksz 64) with
    int8 hidden quant, on the block-local kernel."""
    assert_quant_parity(make_config(5), dev)


# ---- butterfly ----------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(8, 4, 256), (8, 5, 512), (8, 3, 1024), (6, 4, 1000), (5, 3, 12),
                                   (4, 2, 2), (3, 3, 64), (3, 2, 2048)])
def test_butterfly_fp32(dev, shape):
    assert_fp32_parity(small_cfg(4, shape), dev)


@pytest.mark.parametrize("B", [1, 3, 5, 7, 9, 17, 33])
def test_butterfly_partial_batch_sweep(dev, B):
    # Reference tests/test_edge_cases.py:521-586 sweeps these B at (T=16, H=512).
    assert_fp32_parity(small_cfg(4, (16, B, 512)), dev)


def test_butterfly_two_chains(dev):
    cfg = small_cfg(4, (6, 4, 64))
    g = torch.Generator().manual_seed(3)
    cfg["w"] = torch.randn((3, 2, 6, 32, 2, 2), generator=g) * 0.5 ** 0.5
    assert_fp32_parity(cfg, dev)


def test_butterfly_register_equals_generic(dev):
    import gru_qat_amd.scan_butterfly as SB
    from parity_util import to_dev

    for shape in [(12, 6, 1024), (12, 6, 512), (12, 6, 256)]:
        cfg = to_dev(small_cfg(4, shape), dev)
        a = SB.gru_scan_butterfly_forward(cfg["gi"], cfg["h0"], cfg["w"], cfg["bh"])
        b = SB.gru_scan_butterfly_forward_generic(cfg["gi"], cfg["h0"], cfg["w"], cfg["bh"])
        assert (a - b).abs().max().item() <= 1e-5


@pytest.mark.parametrize("qin,qout", [(Q, Q), (None, Q), (Q2, Q)])
def test_butterfly_quant(dev, qin, qout):
    assert_quant_parity(small_cfg(4, (16, 4, 1024), h_in_quant=qin, h_out_quant=qout), dev)


def test_butterfly_cfg4(dev):
    assert_fp32_parity(make_config(4), dev)
