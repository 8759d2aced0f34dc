"""Backward pass of the scans, as device-side torch ops (no HIP kernel yet).

Restates the reference's recompute-based backward
(LarocheC/gru-triton src/gru_qat/triton_kernels/scan.py:1460-1550,
scan_diagonal.py:564-647, scan_monarch.py:955-1053): walk t from T-1 to 0,
recompute r, z, n from h_{t-1} = out[t-1] (or h0), push dout[t] + the carried
gradient through q_out's clip mask, the gate derivatives and the hidden map,
and carry dh_{t-1} = dh_t * z + mask_in * (d gh / d hq)^T dgh. The hidden map's
vector-Jacobian product comes from autograd on the map itself, so one routine
serves every hidden-weight kind.
"""

from __future__ import annotations

from typing import Callable, List, Optional, Sequence, Tuple

import torch

QuantTuple = Optional[Tuple[float, int, int]]


def fake_quant_with_mask(x: torch.Tensor, q: QuantTuple) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Per-tensor symmetric fake-quant and its clipped-STE mask (scan.py:1450-1457)."""
    if q is None:
        return x, None
    scale, qmin, qmax = q
    s = torch.tensor(scale, dtype=x.dtype, device=x.device)
    qu = torch.round(x / s)
    mask = (qu >= qmin) & (qu <= qmax)
    return qu.clamp(qmin, qmax) * s, mask


def scan_backward(
    gi: torch.Tensor,
    h0: torch.Tensor,
    out: torch.Tensor,
    dout: torch.Tensor,
    gh_map: Callable[..., torch.Tensor],
    params: Sequence[torch.Tensor],
    bh_cat: torch.Tensor,
    h_in_quant: QuantTuple,
    h_out_quant: QuantTuple,
) -> Tuple[torch.Tensor, torch.Tensor, List[torch.Tensor], torch.Tensor]:
    """Returns (dgi, dh0, [d param for param in params], dbh_cat).

    gh_map(hq, *params) -> [B, 3H] hidden projection without bias.
    """
    T = gi.shape[0]
    H = h0.shape[-1]
    dgi = torch.empty_like(gi)
    dparams = [torch.zeros_like(p) for p in params]
    dbh = torch.zeros_like(bh_cat)
    dh_acc = torch.zeros_like(h0)
    dout = dout.contiguous()
    for t in reversed(range(T)):
        h_prev = h0 if t == 0 else out[t - 1]
        hq, mask_in = fake_quant_with_mask(h_prev, h_in_quant)
        with torch.enable_grad():
            hq_req = hq.detach().requires_grad_(True)
            p_req = [p.detach().requires_grad_(True) for p in params]
            gh_nob = gh_map(hq_req, *p_req)
        gh = gh_nob.detach() + bh_cat
        gi_r, gi_z, gi_n = gi[t].split(H, dim=-1)
        gh_r, gh_z, gh_n = gh.split(H, dim=-1)
        r = torch.sigmoid(gi_r + gh_r)
        z = torch.sigmoid(gi_z + gh_z)
        n = torch.tanh(gi_n + r * gh_n)
        h_raw = (1.0 - z) * n + z * h_prev

        dh_t = dout[t] + dh_acc
        if h_out_quant is not None:
            _, mask_out = fake_quant_with_mask(h_raw, h_out_quant)
            dh_t = dh_t * mask_out

        dn = dh_t * (1.0 - z)
        dz = dh_t * (h_prev - n)
        dh_direct = dh_t * z
        dgn = dn * (1.0 - n * n)
        dr = dgn * gh_n
        dgh_n = dgn * r
        dgz = dz * z * (1.0 - z)
        dgr = dr * r * (1.0 - r)
        dgi[t] = torch.cat([dgr, dgz, dgn], dim=-1)
        dgh = torch.cat([dgr, dgz, dgh_n], dim=-1)

        grads = torch.autograd.grad(gh_nob, [hq_req] + p_req, dgh, allow_unused=True)
        dh_via_w = grads[0]
        if mask_in is not None:
            dh_via_w = dh_via_w * mask_in
        for acc, g in zip(dparams, grads[1:]):
            if g is not None:
                acc += g
        dbh += dgh.sum(dim=0)
        dh_acc = dh_direct + dh_via_w
    return dgi, dh_acc, dparams, dbh
