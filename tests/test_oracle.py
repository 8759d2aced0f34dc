"""Pins of the CPU oracle (oracle/gru_oracle.py) -- CPU only.

Each check is chosen so that a plausible mistake in the oracle (a swapped
gate, a transposed block, x*(1/s) instead of x/s, round-half-away, a wrong
twiddle element or stride order) fails it, using references independent of
the oracle's own code: torch.nn.GRUCell, exact rational arithmetic, explicit
permutation matrices, hand-derived closed forms and float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from oracle import gru_oracle as O


def _gru_cell_scan(gi, h0, M, bh):
    """nn.GRUCell with weight_ih = I, bias_ih = 0, weight_hh = M, bias_hh = bh fed x_t = gi[t]."""
    T, B, threeH = gi.shape
    H = threeH // 3
    cell = torch.nn.GRUCell(threeH, H)
    with torch.no_grad():
        cell.weight_ih.copy_(torch.eye(threeH))
        cell.bias_ih.zero_()
        cell.weight_hh.copy_(M)
        cell.bias_hh.copy_(bh)
        h = h0.clone()
        outs = []
        for t in range(T):
            h = cell(gi[t], h)
            outs.append(h)
    return torch.stack(outs)


# ---- fake-quant -----------------------------------------------------------------------

def test_round_half_even_known_answer():
    # Reference tests/test_ste.py:12-17.
    x = torch.tensor([0.1, 0.6, -0.4, -0.7, 1.5, 2.5])
    out = O.fake_quant(x, (1.0, -127, 127))
    assert torch.equal(out, torch.tensor([0.0, 1.0, -0.0, -1.0, 2.0, 2.0]))


def test_grid_roundtrip_and_clipping():
    # Reference tests/test_ste.py:44-61.
    x = torch.tensor([-2.0, -1.0, 0.0, 1.0, 2.0])
    assert torch.equal(O.fake_quant(x, (0.5, -127, 127)), x)
    y = O.fake_quant(torch.tensor([-200.0, 0.0, 200.0]), (1.0, -127, 127))
    assert y.tolist() == [-127.0, 0.0, 127.0]


def _exact_codes(xs, s: float, qmin: int, qmax: int) -> np.ndarray:
    """rint(fl32(x / s)) from numpy's IEEE fp32 division and round-half-even
    rint, independent of torch."""
    quo = np.asarray(xs, dtype=np.float32) / np.float32(s)
    return np.clip(np.rint(quo), qmin, qmax).astype(np.float32)


@pytest.mark.parametrize("scale", [Q_INT8_HIDDEN[0], float(np.float32(0.02))])
def test_fake_quant_boundary_sweep_exact(scale):
    """Every value within 3 ulps of every rounding boundary (q + 1/2) * s, and
    of every grid point, for codes -130..130: the oracle's code equals the
    code of the correctly rounded quotient, rounded half to even."""
    xs = []
    for q in range(-130, 131):
        for center in ((q + 0.5) * scale, q * scale):
            c = np.float32(center)
            v = c
            for _ in range(3):
                v = np.nextafter(v, np.float32(-np.inf))
            for _ in range(7):
                xs.append(v)
                v = np.nextafter(v, np.float32(np.inf))
    x = torch.tensor(np.array(xs, dtype=np.float32))
    codes = O.quant_codes(x, (scale, -127, 127))
    expect = torch.from_numpy(_exact_codes(xs, scale, -127, 127))
    assert torch.equal(codes, expect)
    # fake_quant is code * s and is idempotent on its own grid.
    fq = O.fake_quant(x, (scale, -127, 127))
    assert torch.equal(fq, codes * torch.tensor(scale))
    assert torch.equal(O.fake_quant(fq, (scale, -127, 127)), fq)


def test_quant_idempotent_on_every_code():
    """q_in(q_out(x)) == q_out(x) bit for bit when the quantizers are equal;
    the kernels rely on this to skip q_in on the carried state."""
    s = Q_INT8_HIDDEN[0]
    codes = torch.arange(-127, 128, dtype=torch.float32)
    grid = codes * torch.tensor(s)
    assert torch.equal(O.fake_quant(grid, Q_INT8_HIDDEN), grid)
    assert torch.equal(O.quant_codes(grid, Q_INT8_HIDDEN), codes)


# ---- hidden maps vs nn.GRUCell ----------------------------------------------------------

def test_dense_scan_matches_gru_cell():
    cfg = make_config(1, shape=(6, 5, 24))
    out = O.scan_config(cfg)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], cfg["w"], cfg["bh"])
    assert (out - ref).abs().max().item() < 2e-6


def test_gate_order_is_r_z_n():
    """Swapping the r and z rows of Wh changes the oracle exactly as it changes
    nn.GRUCell (so the oracle does not silently permute gates)."""
    cfg = make_config(1, shape=(4, 3, 8))
    W = cfg["w"].clone()
    W[[*range(8), *range(8, 16)]] = W[[*range(8, 16), *range(8)]]
    cfg2 = dict(cfg, w=W)
    out = O.scan_config(cfg2)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], W, cfg["bh"])
    assert (out - ref).abs().max().item() < 2e-6
    assert (out - O.scan_config(cfg)).abs().max().item() > 1e-3


def test_diagonal_scan_matches_gru_cell():
    cfg = make_config(0, shape=(7, 4, 16))
    w = cfg["w"]
    M = torch.cat([torch.diag(w[0]), torch.diag(w[1]), torch.diag(w[2])], dim=0)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], M, cfg["bh"])
    assert (O.scan_config(cfg) - ref).abs().max().item() < 2e-6


def test_monarch_single_matches_gru_cell():
    cfg = make_config(3, shape=(5, 3, 32))
    cfg = dict(cfg, w2=None, h_in_quant=None, h_out_quant=None)
    W = cfg["w"]
    M = torch.cat([torch.block_diag(*W[g]) for g in range(3)], dim=0)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], M, cfg["bh"])
    assert (O.scan_config(cfg) - ref).abs().max().item() < 2e-6


def _perm_matrix(nb, bs):
    H = nb * bs
    P = torch.zeros(H, H)
    for a in range(nb):
        for c in range(bs):
            P[c * nb + a, a * bs + c] = 1.0  # (P z)[c*nb + a] = z[a*bs + c]
    return P


def test_monarch_two_factor_matches_permutation_matrices():
    cfg = make_config(3, shape=(5, 3, 32))  # nb = 8, bs = 4
    cfg = dict(cfg, h_in_quant=None, h_out_quant=None)
    R, L = cfg["w"], cfg["w2"]
    nb, bs = R.shape[1], R.shape[2]
    P = _perm_matrix(nb, bs)
    M = torch.cat([P.t() @ torch.block_diag(*L[g]) @ P @ torch.block_diag(*R[g]) for g in range(3)], dim=0)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], M, cfg["bh"])
    assert (O.scan_config(cfg) - ref).abs().max().item() < 3e-6


def test_monarch_two_factor_identity_reduces_to_single():
    cfg = make_config(3, shape=(5, 3, 32))
    eye = torch.eye(cfg["w"].shape[2]).expand_as(cfg["w"]).contiguous()
    two = O.scan_config(dict(cfg, w2=eye))
    one = O.scan_config(dict(cfg, w2=None))
    assert torch.equal(two, one)


# ---- butterfly ---------------------------------------------------------------------------

def _identity_twiddles(nchains, L, N):
    tw = torch.zeros(3, nchains, L, N // 2, 2, 2)
    tw[..., 0, 0] = 1.0
    tw[..., 1, 1] = 1.0
    return tw


def test_butterfly_identity_twiddles_give_identity():
    x = torch.randn(3, 16)
    tw = _identity_twiddles(2, 4, 16)
    assert torch.equal(O.butterfly_apply(x, tw[0]), x)


def test_butterfly_single_stage_closed_form():
    """N = 4, one chain: stage 0 mixes (0,1) and (2,3) with pair index 0 and 1;
    stage 1 mixes (0,2) and (1,3) with pair index 0 and 1. Element i with member
    bit m uses t[pair, m, m] on itself and t[pair, m, 1-m] on its partner."""
    N, L = 4, 2
    tw = torch.randn(1, L, N // 2, 2, 2)
    x = torch.randn(2, N)
    # stage 0 alone (stage 1 set to identity)
    tw0 = tw.clone()
    tw0[0, 1] = torch.eye(2).expand(N // 2, 2, 2)
    y = O.butterfly_apply(x, tw0)
    t = tw[0, 0]
    exp = torch.stack([
        t[0, 0, 0] * x[:, 0] + t[0, 0, 1] * x[:, 1],
        t[0, 1, 1] * x[:, 1] + t[0, 1, 0] * x[:, 0],
        t[1, 0, 0] * x[:, 2] + t[1, 0, 1] * x[:, 3],
        t[1, 1, 1] * x[:, 3] + t[1, 1, 0] * x[:, 2],
    ], dim=1)
    assert torch.allclose(y, exp, atol=1e-6)
    # stage 1 alone
    tw1 = tw.clone()
    tw1[0, 0] = torch.eye(2).expand(N // 2, 2, 2)
    y = O.butterfly_apply(x, tw1)
    t = tw[0, 1]
    exp = torch.stack([
        t[0, 0, 0] * x[:, 0] + t[0, 0, 1] * x[:, 2],
        t[1, 0, 0] * x[:, 1] + t[1, 0, 1] * x[:, 3],
        t[0, 1, 1] * x[:, 2] + t[0, 1, 0] * x[:, 0],
        t[1, 1, 1] * x[:, 3] + t[1, 1, 0] * x[:, 1],
    ], dim=1)
    assert torch.allclose(y, exp, atol=1e-6)


def test_butterfly_second_chain_reverses_stride_order():
    """With chain 1 holding the only non-identity stage at iteration s = 0,
    that stage must use the largest stride N/2 (decreasing order)."""
    N, L = 8, 3
    tw = _identity_twiddles(2, L, N)[0]
    tw[1, 0] = torch.tensor([[0.0, 1.0], [1.0, 0.0]]).expand(N // 2, 2, 2)  # swap partners
    x = torch.arange(N, dtype=torch.float32).unsqueeze(0)
    y = O.butterfly_apply(x, tw)
    assert y[0].tolist() == [(i ^ 4) for i in range(N)]


def test_butterfly_scan_matches_gru_cell_on_materialized_map():
    cfg = make_config(4, shape=(5, 3, 12))  # N = 16, zero padding 12 -> 16
    M = O.materialize_hidden(cfg)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], M, cfg["bh"])
    assert (O.scan_config(cfg) - ref).abs().max().item() < 5e-6


# ---- circulant -------------------------------------------------------------------------------

def _reference_circulant_fft(col: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """The reference's _CirculantLinear.forward (structure.py:236-240), for the pin."""
    n = col.shape[-1]
    return torch.fft.irfft(torch.fft.rfft(col) * torch.fft.rfft(x, dim=-1), n=n, dim=-1)


def test_circulant_matrix_known_answer():
    a, b, c = 2.0, 3.0, 5.0
    C = O.circulant_matrix(torch.tensor([a, b, c]))
    assert torch.equal(C, torch.tensor([[a, c, b], [b, a, c], [c, b, a]]))


@pytest.mark.parametrize("H", [1, 2, 7, 16, 100, 512])
def test_circulant_map_matches_the_reference_fft(H):
    g = torch.Generator().manual_seed(H)
    col = torch.randn(3, H, generator=g, dtype=torch.float64) / H ** 0.5
    x = torch.randn(5, H, generator=g, dtype=torch.float64)
    got = O.gh_circulant(x, col, torch.zeros(3 * H, dtype=torch.float64))
    want = torch.cat([_reference_circulant_fft(col[k], x) for k in range(3)], dim=-1)
    assert (got - want).abs().max().item() < 1e-12
    # fp32, as the reference runs it: the direct sum stays within the scan tolerance of the FFT
    got32 = O.gh_circulant(x.float(), col.float(), torch.zeros(3 * H))
    assert (got32.double() - want).abs().max().item() < 1e-5


def test_circulant_brute_force_and_transposed_mistake():
    H = 6
    g = torch.Generator().manual_seed(2)
    col = torch.randn(H, generator=g, dtype=torch.float64)
    x = torch.randn(H, generator=g, dtype=torch.float64)
    y = [sum(col[(i - j) % H] * x[j] for j in range(H)) for i in range(H)]
    assert torch.allclose(O.circulant_matrix(col) @ x, torch.stack(y), atol=1e-12)
    transposed = O.circulant_matrix(col).t()  # col[(j - i) mod H]: a plausible index slip
    assert (transposed @ x - _reference_circulant_fft(col, x)).abs().max().item() > 1e-3


def test_circulant_scan_matches_gru_cell():
    cfg = make_config(6, shape=(6, 4, 20))
    w = cfg["w"]
    M = torch.cat([O.circulant_matrix(w[k]) for k in range(3)], dim=0)
    ref = _gru_cell_scan(cfg["gi"], cfg["h0"], M, cfg["bh"])
    assert (O.scan_config(cfg) - ref).abs().max().item() < 2e-6
    assert torch.equal(O.materialize_hidden(cfg), M)


# ---- float64 brute force, invariants ------------------------------------------------------

@pytest.mark.parametrize("idx", [0, 1, 3, 4, 6])
def test_fp32_oracle_close_to_float64(idx):
    shape = (6, 3, 16) if idx != 4 else (6, 3, 16)
    cfg = make_config(idx, shape=shape)
    cfg = dict(cfg, h_in_quant=None, h_out_quant=None)
    c64 = {k: (v.double() if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}
    out32 = O.scan_config(cfg)
    out64 = O.scan_config(c64)
    assert (out32.double() - out64).abs().max().item() < 2e-6


def test_quantized_scan_stays_on_grid():
    cfg = make_config(2, shape=(6, 4, 32))
    out = O.scan_config(cfg)
    codes = out / torch.tensor(Q_INT8_HIDDEN[0])
    assert torch.equal(torch.round(codes), O.quant_codes(out, Q_INT8_HIDDEN))
    assert out.abs().max().item() <= 127 * Q_INT8_HIDDEN[0] + 1e-7


def test_batch_invariance_oracle():
    cfg = make_config(1, shape=(5, 1, 16))
    rep = dict(cfg, gi=cfg["gi"].expand(5, 4, 48).contiguous(), h0=cfg["h0"].expand(4, 16).contiguous())
    out = O.scan_config(rep)
    for b in range(4):
        assert torch.equal(out[:, b], out[:, 0])


def test_teacher_forcing_equals_free_run_on_oracle_output():
    cfg = make_config(2, shape=(5, 4, 16))
    out = O.scan_config(cfg)
    pre = O.teacher_forced_prequant(cfg, out)
    assert torch.equal(O.fake_quant(pre, cfg["h_out_quant"]), out)
