"""Butterfly-hidden GRU scan (drop-in for the persistent path of
gru_qat.triton_kernels.scan_butterfly).

Twiddles are ``[3, nblocks, log_n, 2^log_n / 2, 2, 2]`` (gates r, z, n; the
torch-structured ``Butterfly.twiddle`` with nstacks squeezed), and the hidden
map is the chain of strided 2x2 stages described in
LarocheC/gru-triton src/gru_qat/triton_kernels/scan_butterfly.py:276-317
applied to q_in(h) zero-padded to 2^log_n, truncated to H, plus bh.
Signatures: ``gru_scan_butterfly_triton`` (:1115-1139), its forward launcher
(:369-459) and ``extract_butterfly_twiddles`` (:1142-1182). The forward is
``gs_butterfly_fwd`` of libgruscan.so.
"""

from __future__ import annotations

from typing import Any, Tuple, cast

import torch

from . import _lib
from ._common import QuantTuple, check_common, check_quant, cuda_f32, require_cuda, require_f32


def extract_butterfly_twiddles(cell: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stack the three ``struct_Wh_*.b.twiddle`` tensors ([1, nblocks, log_n,
    n/2, 2, 2] each) into [3, nblocks, log_n, n/2, 2, 2]."""
    if getattr(cell, "_hidden_dense", False):
        raise ValueError("cell hidden side is dense; nothing to extract")
    tws = [layer.b.twiddle.squeeze(0) for layer in (cell.struct_Wh_r, cell.struct_Wh_z, cell.struct_Wh_n)]
    twiddles = torch.stack(tws, dim=0)
    if getattr(cell, "b_hr", None) is None:
        bh_cat = torch.zeros(3 * cell.hidden_size, device=twiddles.device, dtype=twiddles.dtype)
    else:
        bh_cat = torch.cat([cell.b_hr, cell.b_hz, cell.b_hn])
    return twiddles, bh_cat


def check_twiddles(twiddles: torch.Tensor, H: int) -> Tuple[int, int]:
    """Validates the twiddle shape (scan_butterfly.py:403-420); returns (nblocks, log_n)."""
    if twiddles.dim() != 6:
        raise ValueError(f"twiddles shape must be (3, nblocks, log_H, H//2, 2, 2); got {tuple(twiddles.shape)}")
    n_gates, nblocks, log_n, n_div_2, two1, two2 = twiddles.shape
    if not (n_gates == 3 and two1 == 2 and two2 == 2 and nblocks >= 1):
        raise ValueError(f"twiddles shape must be (3, nblocks, log_H, H//2, 2, 2); got {tuple(twiddles.shape)}")
    h_pad = 2 * n_div_2
    if not (h_pad >= H and h_pad >= 2 and (h_pad & (h_pad - 1)) == 0):
        raise ValueError(f"twiddles imply H_PAD={h_pad}, which must be >= H={H} and a power of two "
                         f"(shape {tuple(twiddles.shape)})")
    if (1 << log_n) != h_pad:
        raise ValueError(f"twiddles log_H={log_n} inconsistent with H_PAD={h_pad}: expected 1 << log_H == H_PAD "
                         f"(shape {tuple(twiddles.shape)})")
    return nblocks, log_n


def _forward(fn_name: str, who: str, gi, h0, twiddles, bh_cat, h_in_quant, h_out_quant) -> torch.Tensor:
    if not cuda_f32(gi, h0, twiddles, bh_cat):
        require_cuda(who, gi=gi, h0=h0, twiddles=twiddles, bh_cat=bh_cat)
        require_f32(who, gi=gi, h0=h0, twiddles=twiddles, bh_cat=bh_cat)
    T, B, H = check_common(who, gi, h0, bh_cat)
    nblocks, log_n = check_twiddles(twiddles, H)
    h_in_quant = check_quant(h_in_quant, "h_in_quant")
    h_out_quant = check_quant(h_out_quant, "h_out_quant")
    gi, h0, twiddles, bh_cat = gi.contiguous(), h0.contiguous(), twiddles.contiguous(), bh_cat.contiguous()
    out = torch.empty((T, B, H), device=gi.device, dtype=gi.dtype)
    _lib.launch(_lib.KIND_BUTTERFLY, fn_name, gi=gi, h0=h0, w=twiddles, w2=None, bh=bh_cat, out=out,
                h_in_quant=h_in_quant, h_out_quant=h_out_quant, log_n=log_n, bfly_nblocks=nblocks, contiguous=True)
    return out


def gru_scan_butterfly_forward(gi, h0, twiddles, bh_cat, *, h_in_quant: QuantTuple = None,
                               h_out_quant: QuantTuple = None, **_ignored_tiling: Any) -> torch.Tensor:
    return _forward("gs_butterfly_fwd", "gru_scan_butterfly_forward", gi, h0, twiddles, bh_cat,
                    h_in_quant, h_out_quant)


gru_scan_butterfly_forward_triton = gru_scan_butterfly_forward


def gru_scan_butterfly_forward_generic(gi, h0, twiddles, bh_cat, *, h_in_quant: QuantTuple = None,
                                       h_out_quant: QuantTuple = None) -> torch.Tensor:
    """Same result from the general LDS kernel (used to cross-check the register kernel)."""
    return _forward("gs_butterfly_fwd_generic", "gru_scan_butterfly_forward_generic", gi, h0, twiddles,
                    bh_cat, h_in_quant, h_out_quant)


def gru_scan_butterfly_backward(gi, h0, twiddles, bh_cat, out, dout, *, h_in_quant=None, h_out_quant=None,
                                **_ignored_tiling: Any):
    """Gradients (dgi, dh0, dtwiddles, dbh_cat) of the butterfly scan
    (reference backward: scan_butterfly.py:462-1075).

    ``gs_butterfly_bwd`` runs, for one chain of N <= 1024, the stage-wise
    kernels (coefficient pass, per-row recurrence in spans, twiddle gradient on
    a second stream of the library's beside the recurrence); for other shapes
    it materializes the map as a [3H, H] matrix, runs the dense backward with
    it and carries the matrix gradient back through the twiddle stages. dbh
    comes back as per-row partials summed here.
    """
    who = "gru_scan_butterfly_backward"
    require_cuda(who, gi=gi, h0=h0, twiddles=twiddles, bh_cat=bh_cat, out=out, dout=dout)
    require_f32(who, gi=gi, h0=h0, twiddles=twiddles, bh_cat=bh_cat, out=out, dout=dout)
    T, B, H = check_common(who, gi, h0, bh_cat)
    nblocks, log_n = check_twiddles(twiddles, H)
    if tuple(out.shape) != (T, B, H) or tuple(dout.shape) != (T, B, H):
        raise ValueError(f"out and dout must be (T, B, H)=({T}, {B}, {H})")
    gi, h0, out = gi.contiguous(), h0.contiguous(), out.contiguous()
    twiddles, bh_cat, dout = twiddles.contiguous(), bh_cat.contiguous(), dout.contiguous()
    dgi = torch.empty((T, B, 3 * H), device=gi.device, dtype=gi.dtype)
    dh0 = torch.empty((B, H), device=gi.device, dtype=gi.dtype)
    dtw = torch.empty_like(twiddles)
    dbh_part = torch.empty((B, 3 * H), device=gi.device, dtype=gi.dtype)
    _lib.launch_bwd(_lib.KIND_BUTTERFLY, "gs_butterfly_bwd", gi=gi, h0=h0, w=twiddles, w2=None, bh=bh_cat, out=out,
                    dout=dout, dgi=dgi, dh0=dh0, dw_part=dtw, dbh_part=dbh_part,
                    h_in_quant=check_quant(h_in_quant, "h_in_quant"),
                    h_out_quant=check_quant(h_out_quant, "h_out_quant"), log_n=log_n, bfly_nblocks=nblocks)
    return dgi, dh0, dtw, dbh_part.sum(0)


# The reference's name for the backward launcher.
gru_scan_butterfly_backward_triton = gru_scan_butterfly_backward


class GRUScanButterflyTritonFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, gi, h0, twiddles, bh_cat, h_in_quant, h_out_quant):  # type: ignore[override]
        out = gru_scan_butterfly_forward(gi, h0, twiddles, bh_cat, h_in_quant=h_in_quant, h_out_quant=h_out_quant)
        ctx.save_for_backward(gi, h0, twiddles, bh_cat, out)
        ctx.h_in_quant = check_quant(h_in_quant, "h_in_quant")
        ctx.h_out_quant = check_quant(h_out_quant, "h_out_quant")
        return out

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        gi, h0, twiddles, bh_cat, out = ctx.saved_tensors
        grads = gru_scan_butterfly_backward(gi, h0, twiddles, bh_cat, out, dout, h_in_quant=ctx.h_in_quant,
                                            h_out_quant=ctx.h_out_quant)
        return (*grads, None, None)


def gru_scan_butterfly_triton(
    gi: torch.Tensor,
    h0: torch.Tensor,
    twiddles: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Differentiable butterfly-hidden GRU scan; returns out [T, B, H]. The
    name is the reference's; the kernel is hand-written HIP, not Triton."""
    return cast(torch.Tensor, GRUScanButterflyTritonFunction.apply(gi, h0, twiddles, bh_cat, h_in_quant,
                                                                   h_out_quant))


gru_scan_butterfly_persistent = gru_scan_butterfly_triton
