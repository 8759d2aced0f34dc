"""Monarch (block-diagonal) hidden GRU scan (drop-in for
gru_qat.triton_kernels.scan_monarch).

Single factor, as in the reference (LarocheC/gru-triton
src/gru_qat/triton_kernels/scan_monarch.py:74-127, 927-952):
``gh[b, g, n, o] = sum_i q_in(h)[b, n*blksz + i] * Wh_struct[g, n, o, i] + bh``.

Two factors (keyword-only ``Wh_struct2``, no reference counterpart): with
R_g = Wh_struct[g], L_g = Wh_struct2[g] (both block-diagonal, blocks stored as
(out, in)) and P the stride-``nblocks`` permutation
``(P z)[c * nblocks + a] = z[a * blksz + c]``, the hidden map is
``gh_g = P^T L_g P R_g q_in(h) + bh_g``. With identity blocks in Wh_struct2
it is exactly the single-factor map.

Saved gh (no reference counterpart): in training the single-factor forward
with blksz 16, 32, 64 or 128 also stores each step's bias-free
q_in(h_{t-1}) W^T ([T, B, 3H]), and the backward reads it instead of
recomputing it with a batched product (the reference recomputes it,
scan_monarch.py:409-884).
"""

from __future__ import annotations

from typing import Any, Optional, Tuple, cast

import torch

from . import _lib
from ._common import QuantTuple, check_common, check_quant, cuda_f32, require_cuda, require_f32, save_gh_default


def extract_monarch_factors(cell: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stack ``struct_Wh_{r,z,n}.weight`` ([nblocks, out, in] each) into
    [3, nblocks, blksz, blksz] and the hidden biases into [3H]
    (scan_monarch.py:22-58)."""
    if getattr(cell, "_hidden_dense", False):
        raise ValueError("cell hidden side is dense; nothing to extract")
    Wh_struct = torch.stack([cell.struct_Wh_r.weight, cell.struct_Wh_z.weight, cell.struct_Wh_n.weight], dim=0)
    if getattr(cell, "b_hr", None) is None:
        bh_cat = torch.zeros(3 * cell.hidden_size, device=Wh_struct.device, dtype=Wh_struct.dtype)
    else:
        bh_cat = torch.cat([cell.b_hr, cell.b_hz, cell.b_hn])
    return Wh_struct, bh_cat


def _check_struct(name: str, W: torch.Tensor, H: int) -> Tuple[int, int]:
    if W.dim() != 4:
        raise ValueError(f"{name} must be [3, nblocks, blksz, blksz]; got shape {tuple(W.shape)}")
    n_gates, nblocks, out_blksz, in_blksz = W.shape
    if n_gates != 3:
        raise ValueError(f"{name} dim 0 (n_gates) must be 3; got {n_gates} (shape {tuple(W.shape)})")
    if nblocks < 1 or not (out_blksz == in_blksz == H // nblocks) or nblocks * out_blksz != H:
        raise ValueError(
            f"{name} block dims must be square and tile H: expected out_blksz == in_blksz == "
            f"H // nblocks == {H // max(nblocks, 1)}; got out_blksz={out_blksz}, in_blksz={in_blksz}, "
            f"H={H}, nblocks={nblocks}"
        )
    return nblocks, out_blksz


def monarch_saves_gh(T: int, B: int, nblocks: int, blksz: int, two_factor: bool) -> bool:
    """Whether gs_monarch_fwd / gs_monarch_bwd take gh_save / gh_saved at this
    shape: the single-factor block-local forward (blksz 16-128, launch grid
    within 65535 in y and z) whose backward runs block-local too
    (T * B <= INT32_MAX / 4)."""
    if two_factor or blksz not in (16, 32, 64, 128):
        return False
    rows = max(1, 256 // (4 * blksz))
    return nblocks <= 65535 and (B + rows - 1) // rows <= 65535 and T * B <= (2**31 - 1) // 4


def gru_scan_monarch_forward(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_struct: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
    Wh_struct2: Optional[torch.Tensor] = None,
    gh_save: Optional[torch.Tensor] = None,
    **_ignored_tiling: Any,
) -> torch.Tensor:
    """Runs gs_monarch_fwd. gh_save (keyword-only, no reference counterpart;
    where ``monarch_saves_gh`` holds): a contiguous fp32 [T, B, 3H] tensor
    the kernel fills with each step's bias-free q_in(h_{t-1}) W^T."""
    who = "gru_scan_monarch_forward"
    if not (cuda_f32(gi, h0, Wh_struct, bh_cat) if Wh_struct2 is None
            else cuda_f32(gi, h0, Wh_struct, bh_cat, Wh_struct2)):
        tensors = dict(gi=gi, h0=h0, Wh_struct=Wh_struct, bh_cat=bh_cat)
        if Wh_struct2 is not None:
            tensors["Wh_struct2"] = Wh_struct2
        require_cuda(who, **tensors)
        require_f32(who, **tensors)
    T, B, H = check_common(who, gi, h0, bh_cat)
    nblocks, blksz = _check_struct("Wh_struct", Wh_struct, H)
    if Wh_struct2 is not None:
        if tuple(Wh_struct2.shape) != tuple(Wh_struct.shape):
            raise ValueError(f"Wh_struct2 shape {tuple(Wh_struct2.shape)} must equal Wh_struct shape "
                             f"{tuple(Wh_struct.shape)}")
        Wh_struct2 = Wh_struct2.contiguous()
    h_in_quant = check_quant(h_in_quant, "h_in_quant")
    h_out_quant = check_quant(h_out_quant, "h_out_quant")
    gi, h0, Wh_struct, bh_cat = gi.contiguous(), h0.contiguous(), Wh_struct.contiguous(), bh_cat.contiguous()
    out = torch.empty((T, B, H), device=gi.device, dtype=gi.dtype)
    _lib.launch(_lib.KIND_MONARCH, "gs_monarch_fwd", gi=gi, h0=h0, w=Wh_struct, w2=Wh_struct2, bh=bh_cat,
                out=out, h_in_quant=h_in_quant, h_out_quant=h_out_quant, nblocks=nblocks, blksz=blksz,
                gh_save=gh_save, contiguous=True)
    return out


gru_scan_monarch_forward_triton = gru_scan_monarch_forward


def gru_scan_monarch_backward(gi, h0, Wh_struct, bh_cat, out, dout, *, h_in_quant=None, h_out_quant=None,
                              Wh_struct2=None, gh_saved=None, **_ignored_tiling: Any):
    """Gradients (dgi, dh0, [dWh_struct(, dWh_struct2)], dbh_cat) of the
    Monarch scan (reference backward: scan_monarch.py:409-884 and :955-1053).

    ``gs_monarch_bwd`` materializes the (one- or two-factor) map as a [3H, H]
    matrix, runs the dense backward with it and carries the matrix gradient
    onto the factors; dbh comes back as per-row partials summed here. The
    single-factor backward works on the blocks directly instead and, given
    gh_saved (what the forward stored through gh_save), skips its gh product.
    """
    who = "gru_scan_monarch_backward"
    require_cuda(who, gi=gi, h0=h0, Wh_struct=Wh_struct, bh_cat=bh_cat, out=out, dout=dout)
    require_f32(who, gi=gi, h0=h0, Wh_struct=Wh_struct, bh_cat=bh_cat, out=out, dout=dout)
    T, B, H = check_common(who, gi, h0, bh_cat)
    nblocks, blksz = _check_struct("Wh_struct", Wh_struct, H)
    if Wh_struct2 is not None:
        require_cuda(who, gi=gi, Wh_struct2=Wh_struct2)
        require_f32(who, Wh_struct2=Wh_struct2)
        if tuple(Wh_struct2.shape) != tuple(Wh_struct.shape):
            raise ValueError(f"Wh_struct2 shape must equal Wh_struct's {tuple(Wh_struct.shape)}; "
                             f"got {tuple(Wh_struct2.shape)}")
        Wh_struct2 = Wh_struct2.contiguous()
    if tuple(out.shape) != (T, B, H) or tuple(dout.shape) != (T, B, H):
        raise ValueError(f"out and dout must be (T, B, H)=({T}, {B}, {H})")
    gi, h0, out = gi.contiguous(), h0.contiguous(), out.contiguous()
    Wh_struct, bh_cat, dout = Wh_struct.contiguous(), bh_cat.contiguous(), dout.contiguous()
    dgi = torch.empty((T, B, 3 * H), device=gi.device, dtype=gi.dtype)
    dh0 = torch.empty((B, H), device=gi.device, dtype=gi.dtype)
    dW = torch.empty_like(Wh_struct)
    dW2 = torch.empty_like(Wh_struct2) if Wh_struct2 is not None else None
    dbh_part = torch.empty((B, 3 * H), device=gi.device, dtype=gi.dtype)
    _lib.launch_bwd(_lib.KIND_MONARCH, "gs_monarch_bwd", gi=gi, h0=h0, w=Wh_struct, w2=Wh_struct2, bh=bh_cat,
                    out=out, dout=dout, dgi=dgi, dh0=dh0, dw_part=dW, dw2_part=dW2, dbh_part=dbh_part,
                    h_in_quant=check_quant(h_in_quant, "h_in_quant"),
                    h_out_quant=check_quant(h_out_quant, "h_out_quant"), nblocks=nblocks, blksz=blksz,
                    gh_saved=gh_saved)
    dps = [dW] if dW2 is None else [dW, dW2]
    return dgi, dh0, dps, dbh_part.sum(0)


# The reference's name for the backward launcher.
gru_scan_monarch_backward_triton = gru_scan_monarch_backward


class GRUScanMonarchFunction(torch.autograd.Function):
    """autograd wrapper; ``save_gh`` (no reference counterpart) asks the
    forward to store gh for the backward where ``monarch_saves_gh`` allows it;
    it is decided when ``apply`` is called, where the grad mode is still
    visible (by default ``save_gh_default``)."""

    @classmethod
    def apply(cls, *args, **kwargs):  # type: ignore[override]
        if len(args) == 7:  # without save_gh
            args = (*args, save_gh_default(*args[:4], args[6]))
        return super().apply(*args, **kwargs)

    @staticmethod
    def forward(ctx: Any, gi, h0, Wh_struct, bh_cat, h_in_quant, h_out_quant, Wh_struct2,  # type: ignore[override]
                save_gh=None):
        gh = None
        save = any(ctx.needs_input_grad[:4]) if save_gh is None else bool(save_gh)
        if save and gi.dim() == 3 and Wh_struct.dim() == 4:
            T, B, G3 = gi.shape
            if monarch_saves_gh(T, B, Wh_struct.shape[1], Wh_struct.shape[3], Wh_struct2 is not None):
                gh = torch.empty((T, B, G3), device=gi.device, dtype=torch.float32)
        out = gru_scan_monarch_forward(gi, h0, Wh_struct, bh_cat, h_in_quant=h_in_quant,
                                       h_out_quant=h_out_quant, Wh_struct2=Wh_struct2, gh_save=gh)
        ctx.save_for_backward(gi, h0, Wh_struct, bh_cat, out, Wh_struct2, gh)
        ctx.h_in_quant = check_quant(h_in_quant, "h_in_quant")
        ctx.h_out_quant = check_quant(h_out_quant, "h_out_quant")
        return out

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        gi, h0, Wh_struct, bh_cat, out, Wh_struct2, gh = ctx.saved_tensors
        dgi, dh0, dps, dbh = gru_scan_monarch_backward(gi, h0, Wh_struct, bh_cat, out, dout,
                                                       h_in_quant=ctx.h_in_quant, h_out_quant=ctx.h_out_quant,
                                                       Wh_struct2=Wh_struct2, gh_saved=gh)
        dW2 = dps[1] if Wh_struct2 is not None else None
        return dgi, dh0, dps[0], dbh, None, None, dW2, None


def gru_scan_monarch(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_struct: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
    Wh_struct2: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Differentiable Monarch-hidden GRU scan; returns out [T, B, H]."""
    wants = save_gh_default(gi, h0, Wh_struct, bh_cat, Wh_struct2)
    return cast(torch.Tensor, GRUScanMonarchFunction.apply(gi, h0, Wh_struct, bh_cat, h_in_quant, h_out_quant,
                                                           Wh_struct2, wants))
