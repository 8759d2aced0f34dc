"""Circulant-hidden GRU scan.

The reference has a circulant structured kind (``_CirculantLinear``,
LarocheC/gru-triton src/gru_qat/structure.py:220-240: ``y = irfft(rfft(col)
* rfft(x))``, the circular convolution ``y[i] = sum_j col[(i - j) mod H]
x[j]``) and runs it on its per-step loop (gru_layer.py:109-113); it has no
kernel for it. Here ``gh_g = C(col_g) q_in(h) + bh_g`` runs as the dense
persistent scan on the three circulant matrices, which ``gs_hidden_map_dense``
writes on the device (``C[i][j] = col[(i - j) mod H]``): at the sizes of this
path a circulant mat-vec done directly costs what a dense one does, and the
dense kernel keeps its rows in registers for the whole scan. The backward is
the dense backward, its [3H, H] weight gradient folded back onto each col
along the circulant diagonals (``gs_hidden_map_grad``).

``Wh_circ`` is ``[3, H]``: rows r, z, n, each a gate's ``struct_Wh_g.col``.
"""

from __future__ import annotations

from typing import Any, Tuple, cast

import torch

from . import _lib
from ._common import QuantTuple, check_common, check_quant, require_cuda, require_f32
from .observe import hidden_map_dense, hidden_map_grad
from .scan import gru_scan_backward_persistent, gru_scan_forward_persistent


def extract_circulant_factors(cell: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stack a circulant cell's ``struct_Wh_{r,z,n}.col`` into [3, H] and its
    hidden biases into [3H] (zeros without bias), the layout of the other
    kinds' extract helpers."""
    if getattr(cell, "_hidden_dense", False):
        raise ValueError("cell hidden side is dense; nothing to extract")
    Wh_circ = torch.stack([cell.struct_Wh_r.col, cell.struct_Wh_z.col, cell.struct_Wh_n.col], dim=0)
    if getattr(cell, "b_hr", None) is None:
        bh_cat = torch.zeros(3 * cell.hidden_size, device=Wh_circ.device, dtype=Wh_circ.dtype)
    else:
        bh_cat = torch.cat([cell.b_hr, cell.b_hz, cell.b_hn])
    return Wh_circ, bh_cat


def _check(who: str, gi, h0, Wh_circ, bh_cat) -> int:
    require_cuda(who, gi=gi, h0=h0, Wh_circ=Wh_circ, bh_cat=bh_cat)
    require_f32(who, gi=gi, h0=h0, Wh_circ=Wh_circ, bh_cat=bh_cat)
    _, _, H = check_common(who, gi, h0, bh_cat)
    if tuple(Wh_circ.shape) != (3, H):
        raise ValueError(f"Wh_circ shape must be (3, H)=(3, {H}); got {tuple(Wh_circ.shape)}")
    return H


def gru_scan_circulant_forward(gi, h0, Wh_circ, bh_cat, *, h_in_quant: QuantTuple = None,
                               h_out_quant: QuantTuple = None) -> torch.Tensor:
    """Forward only; returns out [T, B, H]. Up to H = 1024 the persistent kernel forms the
    circulant rows itself from Wh_circ (``gs_circulant_fwd``); above, the dense scan runs on
    the materialized map. Either way the outputs equal the dense scan's on that map."""
    H = _check("gru_scan_circulant_forward", gi, h0, Wh_circ, bh_cat)
    if H <= 1024:
        h_in_quant = check_quant(h_in_quant, "h_in_quant")
        h_out_quant = check_quant(h_out_quant, "h_out_quant")
        T, B = gi.shape[0], gi.shape[1]
        gi, h0, bh_cat = gi.contiguous(), h0.contiguous(), bh_cat.contiguous()
        out = torch.empty((T, B, H), device=gi.device, dtype=gi.dtype)
        _lib.launch(_lib.KIND_CIRCULANT, "gs_circulant_fwd", gi=gi, h0=h0, w=Wh_circ.contiguous(), w2=None,
                    bh=bh_cat, out=out, h_in_quant=h_in_quant, h_out_quant=h_out_quant, contiguous=True)
        return out
    M = hidden_map_dense("circulant", Wh_circ.contiguous(), H)
    return gru_scan_forward_persistent(gi, h0, M, bh_cat, h_in_quant=h_in_quant, h_out_quant=h_out_quant)


def gru_scan_circulant_backward(gi, h0, Wh_circ, bh_cat, out, dout, *, h_in_quant=None, h_out_quant=None):
    """(dgi, dh0, dWh_circ, dbh_cat) of the circulant scan."""
    H = _check("gru_scan_circulant_backward", gi, h0, Wh_circ, bh_cat)
    M = hidden_map_dense("circulant", Wh_circ.contiguous(), H)
    dgi, dh0, dM, dbh = gru_scan_backward_persistent(gi, h0, M, bh_cat, out, dout, h_in_quant=h_in_quant,
                                                     h_out_quant=h_out_quant)
    return dgi, dh0, hidden_map_grad("circulant", dM, Wh_circ, H), dbh


class GRUScanCirculantFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, gi, h0, Wh_circ, bh_cat, h_in_quant, h_out_quant):  # type: ignore[override]
        out = gru_scan_circulant_forward(gi, h0, Wh_circ, bh_cat, h_in_quant=h_in_quant, h_out_quant=h_out_quant)
        ctx.save_for_backward(gi, h0, Wh_circ, bh_cat, out)
        ctx.h_in_quant = check_quant(h_in_quant, "h_in_quant")
        ctx.h_out_quant = check_quant(h_out_quant, "h_out_quant")
        return out

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        gi, h0, Wh_circ, bh_cat, out = ctx.saved_tensors
        grads = gru_scan_circulant_backward(gi, h0, Wh_circ, bh_cat, out, dout, h_in_quant=ctx.h_in_quant,
                                            h_out_quant=ctx.h_out_quant)
        return (*grads, None, None)


def gru_scan_circulant(gi: torch.Tensor, h0: torch.Tensor, Wh_circ: torch.Tensor, bh_cat: torch.Tensor, *,
                       h_in_quant: QuantTuple = None, h_out_quant: QuantTuple = None) -> torch.Tensor:
    """Differentiable circulant-hidden GRU scan; returns out [T, B, H]."""
    return cast(torch.Tensor, GRUScanCirculantFunction.apply(gi, h0, Wh_circ, bh_cat, h_in_quant, h_out_quant))
