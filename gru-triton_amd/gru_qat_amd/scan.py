"""Dense-hidden persistent GRU scan (drop-in for gru_qat.triton_kernels.scan).

Entry points keep the reference signatures
(LarocheC/gru-triton src/gru_qat/triton_kernels/scan.py):

* ``gru_scan_persistent(gi, h0, Wh_cat, bh_cat, *, h_in_quant, h_out_quant)``
  (scan.py:1667-1685) and its autograd Function (scan.py:1630-1664);
* ``gru_scan(...)`` (scan.py:1607-1627), same contract;
* ``gru_scan_forward_persistent`` / ``gru_scan_forward`` (scan.py:213-293,
  1688-1765), the forward-only launchers.

``Wh_cat`` is ``[3H, H]`` with rows ordered r, z, n and ``gh = hq @ Wh_cat.T +
bh_cat``. ``h_in_quant`` / ``h_out_quant`` are optional frozen per-tensor
symmetric ``(scale, qmin, qmax)`` tuples. The forward runs the gfx950 kernel
``gs_dense_fwd`` of libgruscan.so (one persistent launch, Wh resident in
registers, fp32 MFMA); the reference's tile and warp knobs have no meaning
there and are accepted only as keywords that are ignored.
"""

from __future__ import annotations

from typing import Any, Optional, cast

import torch

from . import _lib
from ._common import QuantTuple, check_common, check_quant, require_cuda, require_f32


def _dense_forward(who: str, gi: torch.Tensor, h0: torch.Tensor, Wh_cat: torch.Tensor,
                   bh_cat: torch.Tensor, h_in_quant: QuantTuple, h_out_quant: QuantTuple,
                   gh_save: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Runs gs_dense_fwd; with gh_save ([T, B, 3H] contiguous fp32) the kernel also
    stores every step's q_in(h_{t-1}) Wh^T (gh_t without bh) there for the backward."""
    require_cuda(who, gi=gi, h0=h0, Wh_cat=Wh_cat, bh_cat=bh_cat)
    require_f32(who, gi=gi, h0=h0, Wh_cat=Wh_cat, bh_cat=bh_cat)
    T, B, H = check_common(who, gi, h0, bh_cat)
    if tuple(Wh_cat.shape) != (3 * H, H):
        raise ValueError(f"Wh_cat shape must be (3H, H)=({3 * H}, {H}); got {tuple(Wh_cat.shape)}")
    h_in_quant = check_quant(h_in_quant, "h_in_quant")
    h_out_quant = check_quant(h_out_quant, "h_out_quant")
    gi = gi.contiguous()
    h0 = h0.contiguous()
    Wh_cat = Wh_cat.contiguous()
    bh_cat = bh_cat.contiguous()
    out = torch.empty((T, B, H), device=gi.device, dtype=gi.dtype)
    _lib.launch(_lib.KIND_DENSE, "gs_dense_fwd", gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat, out=out,
                h_in_quant=h_in_quant, h_out_quant=h_out_quant, gh_save=gh_save)
    return out


def gru_scan_forward_persistent(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_cat: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
    **_ignored_tiling: Any,
) -> torch.Tensor:
    """Forward of the dense scan; returns out [T, B, H] (h_T = out[-1])."""
    return _dense_forward("gru_scan_forward_persistent", gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant)


def gru_scan_forward(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_cat: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Same contract as the reference's autotuned launcher (scan.py:1688-1765)."""
    return _dense_forward("gru_scan_forward", gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant)


def gru_scan_backward_persistent(gi, h0, Wh_cat, bh_cat, out, dout, *, h_in_quant=None, h_out_quant=None,
                                 **_ignored_tiling: Any):
    """Gradients (dgi, dh0, dWh_cat, dbh_cat) of the dense scan.

    Same contract as the reference's gru_scan_backward_persistent
    (scan.py:646-752): ``gs_dense_bwd`` recomputes gh for every step with one
    GEMM, runs the reverse recurrence as one persistent launch and forms dWh
    with a second GEMM; dbh comes back as per-row partials summed here.
    """
    return _dense_backward("gru_scan_backward_persistent", gi, h0, Wh_cat, bh_cat, out, dout, h_in_quant,
                           h_out_quant)


def _dense_backward(who: str, gi, h0, Wh_cat, bh_cat, out, dout, h_in_quant, h_out_quant,
                    gh_saved: Optional[torch.Tensor] = None):
    """Runs gs_dense_bwd; gh_saved is the gh the forward stored through gh_save
    (then the backward skips its recompute GEMM)."""
    require_cuda(who, gi=gi, h0=h0, Wh_cat=Wh_cat, bh_cat=bh_cat, out=out, dout=dout)
    require_f32(who, gi=gi, h0=h0, Wh_cat=Wh_cat, bh_cat=bh_cat, out=out, dout=dout)
    T, B, H = check_common(who, gi, h0, bh_cat)
    if tuple(Wh_cat.shape) != (3 * H, H):
        raise ValueError(f"Wh_cat shape must be (3H, H)=({3 * H}, {H}); got {tuple(Wh_cat.shape)}")
    if tuple(out.shape) != (T, B, H) or tuple(dout.shape) != (T, B, H):
        raise ValueError(f"out and dout must be (T, B, H)=({T}, {B}, {H})")
    gi, h0, out = gi.contiguous(), h0.contiguous(), out.contiguous()
    Wh_cat, bh_cat, dout = Wh_cat.contiguous(), bh_cat.contiguous(), dout.contiguous()
    dgi = torch.empty((T, B, 3 * H), device=gi.device, dtype=gi.dtype)
    dh0 = torch.empty((B, H), device=gi.device, dtype=gi.dtype)
    dW = torch.empty((3 * H, H), device=gi.device, dtype=gi.dtype)
    dbh_part = torch.empty((B, 3 * H), device=gi.device, dtype=gi.dtype)
    _lib.launch_bwd(_lib.KIND_DENSE, "gs_dense_bwd", gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat, out=out,
                    dout=dout, dgi=dgi, dh0=dh0, dw_part=dW, dbh_part=dbh_part,
                    h_in_quant=check_quant(h_in_quant, "h_in_quant"),
                    h_out_quant=check_quant(h_out_quant, "h_out_quant"), gh_saved=gh_saved)
    return dgi, dh0, dW, dbh_part.sum(0)


# The reference's names for the dense backward launchers (scan.py:1355, :646).
gru_scan_backward_triton = gru_scan_backward_persistent
gru_scan_backward = gru_scan_backward_persistent


def _wants_grad(*tensors: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


class GRUScanPersistentFunction(torch.autograd.Function):
    """autograd wrapper; saves (gi, h0, Wh_cat, bh_cat, out) like scan.py:1650.

    When a gradient is needed the forward also has the kernel store every
    step's q_in(h_{t-1}) Wh^T ([T, B, 3H], saved with the rest), so
    the backward skips the reference's recompute of gh (scan.py:388-421).
    ``save_gh`` (not in the reference signature; default: whether any input
    needs a gradient) overrides that choice: ``needs_input_grad`` does not see
    ``torch.no_grad()``, so the wrappers pass the grad mode in."""

    @staticmethod
    def forward(ctx: Any, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, save_gh=None):  # type: ignore[override]
        gh = None
        save = any(ctx.needs_input_grad[:4]) if save_gh is None else bool(save_gh)
        if save and gi.dim() == 3:
            T, B, G3 = gi.shape
            gh = torch.empty((T, B, G3), device=gi.device, dtype=torch.float32)
        out = _dense_forward("gru_scan_forward_persistent", gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant,
                             gh_save=gh)
        ctx.save_for_backward(gi, h0, Wh_cat, bh_cat, out, gh)
        ctx.h_in_quant = check_quant(h_in_quant, "h_in_quant")
        ctx.h_out_quant = check_quant(h_out_quant, "h_out_quant")
        return out

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        gi, h0, Wh_cat, bh_cat, out, gh = ctx.saved_tensors
        grads = _dense_backward("gru_scan_backward_persistent", gi, h0, Wh_cat, bh_cat, out, dout,
                                ctx.h_in_quant, ctx.h_out_quant, gh_saved=gh)
        return (*grads, None, None, None)


GRUScanFunction = GRUScanPersistentFunction


def gru_scan_persistent(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_cat: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Differentiable dense persistent GRU scan; returns out [T, B, H]."""
    return cast(torch.Tensor, GRUScanPersistentFunction.apply(gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant,
                                                              _wants_grad(gi, h0, Wh_cat, bh_cat)))


def gru_scan(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_cat: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Differentiable dense GRU scan (reference scan.py:1607-1627); same kernel
    as ``gru_scan_persistent`` on MI355X."""
    return cast(torch.Tensor, GRUScanPersistentFunction.apply(gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant,
                                                              _wants_grad(gi, h0, Wh_cat, bh_cat)))
