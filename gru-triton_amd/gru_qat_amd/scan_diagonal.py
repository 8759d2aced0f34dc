"""Diagonal-hidden GRU scan (drop-in for gru_qat.triton_kernels.scan_diagonal).

``gh_g = Wh_diag[g] * q_in(h) + bh_g`` elementwise; signatures follow
LarocheC/gru-triton src/gru_qat/triton_kernels/scan_diagonal.py:684-715
(``gru_scan_diagonal``), :226-282 (forward launcher) and :33-63
(``extract_diagonal_factors``). The forward is ``gs_diagonal_fwd`` of
libgruscan.so.
"""

from __future__ import annotations

from typing import Any, Tuple, cast

import torch

from . import _lib
from ._common import QuantTuple, check_common, check_quant, cuda_f32, require_cuda, require_f32


def extract_diagonal_factors(cell: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stack a structured cell's ``struct_Wh_{r,z,n}.weight`` into [3, H] and
    its hidden biases into [3H] (zeros without bias)."""
    if getattr(cell, "_hidden_dense", False):
        raise ValueError("cell hidden side is dense; nothing to extract")
    Wh_diag = torch.stack([cell.struct_Wh_r.weight, cell.struct_Wh_z.weight, cell.struct_Wh_n.weight], dim=0)
    if getattr(cell, "b_hr", None) is None:
        bh_cat = torch.zeros(3 * cell.hidden_size, device=Wh_diag.device, dtype=Wh_diag.dtype)
    else:
        bh_cat = torch.cat([cell.b_hr, cell.b_hz, cell.b_hn])
    return Wh_diag, bh_cat


def gru_scan_diagonal_forward(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_diag: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
    **_ignored_tiling: Any,
) -> torch.Tensor:
    who = "gru_scan_diagonal_forward"
    if not cuda_f32(gi, h0, Wh_diag, bh_cat):
        require_cuda(who, gi=gi, h0=h0, Wh_diag=Wh_diag, bh_cat=bh_cat)
        require_f32(who, gi=gi, h0=h0, Wh_diag=Wh_diag, bh_cat=bh_cat)
    T, B, H = check_common(who, gi, h0, bh_cat)
    if Wh_diag.shape != (3, H):
        raise ValueError(f"Wh_diag shape must be (3, H)=(3, {H}); got {tuple(Wh_diag.shape)}")
    h_in_quant = check_quant(h_in_quant, "h_in_quant")
    h_out_quant = check_quant(h_out_quant, "h_out_quant")
    gi, h0, Wh_diag, bh_cat = gi.contiguous(), h0.contiguous(), Wh_diag.contiguous(), bh_cat.contiguous()
    out = torch.empty((T, B, H), device=gi.device, dtype=gi.dtype)
    _lib.launch(_lib.KIND_DIAGONAL, "gs_diagonal_fwd", gi=gi, h0=h0, w=Wh_diag, w2=None, bh=bh_cat,
                out=out, h_in_quant=h_in_quant, h_out_quant=h_out_quant, contiguous=True)
    return out


# The reference's name for the forward launcher.
gru_scan_diagonal_forward_triton = gru_scan_diagonal_forward


def gru_scan_diagonal_backward(gi, h0, Wh_diag, bh_cat, out, dout, *, h_in_quant=None, h_out_quant=None,
                               **_ignored_tiling: Any):
    """Gradients (dgi, dh0, dWh_diag, dbh_cat) of the diagonal scan.

    Mirrors the reference's backward launcher (scan_diagonal.py:285-561):
    ``gs_diagonal_bwd`` walks t in reverse per (b, j) and writes dgi, dh0 and
    per-row partials of dWh_diag [B, 3, H] and dbh [B, 3H]; the partials are
    summed over B here.
    """
    who = "gru_scan_diagonal_backward"
    require_cuda(who, gi=gi, h0=h0, Wh_diag=Wh_diag, bh_cat=bh_cat, out=out, dout=dout)
    require_f32(who, gi=gi, h0=h0, Wh_diag=Wh_diag, bh_cat=bh_cat, out=out, dout=dout)
    T, B, H = check_common(who, gi, h0, bh_cat)
    if tuple(out.shape) != (T, B, H) or tuple(dout.shape) != (T, B, H):
        raise ValueError(f"out and dout must be (T, B, H)=({T}, {B}, {H})")
    if tuple(Wh_diag.shape) != (3, H):
        raise ValueError(f"Wh_diag shape must be (3, H)=(3, {H}); got {tuple(Wh_diag.shape)}")
    gi, h0, out = gi.contiguous(), h0.contiguous(), out.contiguous()
    Wh_diag, bh_cat, dout = Wh_diag.contiguous(), bh_cat.contiguous(), dout.contiguous()
    dgi = torch.empty((T, B, 3 * H), device=gi.device, dtype=gi.dtype)
    dh0 = torch.empty((B, H), device=gi.device, dtype=gi.dtype)
    dw_part = torch.empty((B, 3, H), device=gi.device, dtype=gi.dtype)
    dbh_part = torch.empty((B, 3 * H), device=gi.device, dtype=gi.dtype)
    _lib.launch_bwd(_lib.KIND_DIAGONAL, "gs_diagonal_bwd", gi=gi, h0=h0, w=Wh_diag, w2=None, bh=bh_cat, out=out, dout=dout,
                    dgi=dgi, dh0=dh0, dw_part=dw_part, dbh_part=dbh_part,
                    h_in_quant=check_quant(h_in_quant, "h_in_quant"),
                    h_out_quant=check_quant(h_out_quant, "h_out_quant"))
    return dgi, dh0, dw_part.sum(0), dbh_part.sum(0)


# The reference's name for the backward launcher.
gru_scan_diagonal_backward_triton = gru_scan_diagonal_backward


class GRUScanDiagonalFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, gi, h0, Wh_diag, bh_cat, h_in_quant, h_out_quant):  # type: ignore[override]
        out = gru_scan_diagonal_forward(gi, h0, Wh_diag, bh_cat, h_in_quant=h_in_quant, h_out_quant=h_out_quant)
        ctx.save_for_backward(gi, h0, Wh_diag, bh_cat, out)
        ctx.h_in_quant = check_quant(h_in_quant, "h_in_quant")
        ctx.h_out_quant = check_quant(h_out_quant, "h_out_quant")
        return out

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        gi, h0, Wh_diag, bh_cat, out = ctx.saved_tensors
        grads = gru_scan_diagonal_backward(gi, h0, Wh_diag, bh_cat, out, dout, h_in_quant=ctx.h_in_quant,
                                           h_out_quant=ctx.h_out_quant)
        return (*grads, None, None)


def gru_scan_diagonal(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_diag: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Differentiable diagonal-hidden GRU scan; returns out [T, B, H]."""
    return cast(torch.Tensor, GRUScanDiagonalFunction.apply(gi, h0, Wh_diag, bh_cat, h_in_quant, h_out_quant))
