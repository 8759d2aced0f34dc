"""Dense-hidden GRU scans (drop-in for gru_qat.triton_kernels.scan).

Entry points keep the reference signatures
(LarocheC/gru-triton src/gru_qat/triton_kernels/scan.py):

* ``gru_scan_persistent(gi, h0, Wh_cat, bh_cat, *, h_in_quant, h_out_quant)``
  (scan.py:1667-1685) and its autograd Function (scan.py:1630-1664), on the
  persistent kernels ``gs_dense_fwd`` / ``gs_dense_bwd`` (one launch, Wh resident
  in registers, the state exchanged between workgroups every step, fp32 MFMA);
* ``gru_scan(...)`` (scan.py:1607-1627) and ``GRUScanFunction`` (scan.py:1556-1604),
  same contract, on the barrier-free batch-tiled kernels ``gs_dense_fwd_tiled`` /
  ``gs_dense_bwd_tiled`` (one workgroup per tile of batch rows, Wh read from
  memory every step, no co-residency requirement), as the reference's
  ``gru_scan`` runs its non-persistent kernels (scan.py:755-913, :916-1352);
* the forward-only launchers ``gru_scan_forward_persistent`` (scan.py:213-293,
  persistent) and ``gru_scan_forward`` (scan.py:1688-1765, batch-tiled), and the
  backward launchers ``gru_scan_backward_persistent`` (scan.py:646-752) and
  ``gru_scan_backward_triton`` (scan.py:1355-1447, batch-tiled).

Both kernel families compute the same products in the same order, so their
outputs are bit-identical up to H = 1024; above that the persistent entry
points run the batch-tiled kernels too (up to H = 8192).

``Wh_cat`` is ``[3H, H]`` with rows ordered r, z, n and ``gh = hq @ Wh_cat.T +
bh_cat``. ``h_in_quant`` / ``h_out_quant`` are optional frozen per-tensor
symmetric ``(scale, qmin, qmax)`` tuples. The reference's tile and warp knobs
have no meaning here and are accepted only as keywords that are ignored.

Training forwards store gh ([T, B, 3H] fp32) for their backward, which then
skips the reference's recompute of gh (scan.py:388-421); ``set_save_gh(False)``
(``_common``) restores the recompute and its smaller memory footprint.
"""

from __future__ import annotations

from typing import Any, Optional, cast

import torch

from . import _lib
from ._common import QuantTuple, check_common, check_quant, cuda_f32, require_cuda, require_f32, save_gh_default


def _int8_codes_apply(H: int, h_in_quant: QuantTuple) -> bool:
    """Whether the int8-weight entry points (gs_dense_fwd_i8w,
    gs_dense_fwd_tiled_i8w) run their int8-MFMA kernels for this shape and
    hidden quant (every A operand a q_in level that fits a byte, H > 64 and a
    multiple of 16), so that finding the codes is worth its device-to-host read.
    The rule is the library's dense_i8_applies."""
    return (h_in_quant is not None and H > 64 and H % 16 == 0 and int(h_in_quant[1]) >= -128
            and int(h_in_quant[2]) <= 127)


def _dense_forward(who: str, gi: torch.Tensor, h0: torch.Tensor, Wh_cat: torch.Tensor,
                   bh_cat: torch.Tensor, h_in_quant: QuantTuple, h_out_quant: QuantTuple,
                   gh_save: Optional[torch.Tensor] = None, tiled: bool = False,
                   int8_codes: bool = False) -> torch.Tensor:
    """Runs gs_dense_fwd (tiled: gs_dense_fwd_tiled); with gh_save ([T, B, 3H]
    contiguous fp32) the kernel also stores every step's q_in(h_{t-1}) Wh^T (gh_t
    without bh) there for the backward. int8_codes (forwards that need no
    gradient): when Wh_cat is a per-row int8 fake-quantized weight (its codes
    found once per version of the tensor, ``_lib.weight_codes``) and every A
    operand is a q_in level that fits a byte, gs_dense_fwd_i8w (tiled:
    gs_dense_fwd_tiled_i8w) runs the step's products on the int8 MFMA; the two
    kernels then agree bit for bit as their fp32 forms do."""
    if not cuda_f32(gi, h0, Wh_cat, bh_cat):
        require_cuda(who, gi=gi, h0=h0, Wh_cat=Wh_cat, bh_cat=bh_cat)
        require_f32(who, gi=gi, h0=h0, Wh_cat=Wh_cat, bh_cat=bh_cat)
    T, B, H = check_common(who, gi, h0, bh_cat)
    if Wh_cat.shape != (3 * H, H):
        raise ValueError(f"Wh_cat shape must be (3H, H)=({3 * H}, {H}); got {tuple(Wh_cat.shape)}")
    h_in_quant = check_quant(h_in_quant, "h_in_quant")
    h_out_quant = check_quant(h_out_quant, "h_out_quant")
    codes = None
    if int8_codes and gh_save is None and _int8_codes_apply(H, h_in_quant):
        codes = _lib.weight_codes(Wh_cat)  # keyed on the caller's tensor, contiguous or not
    gi = gi.contiguous()
    h0 = h0.contiguous()
    Wh_cat = Wh_cat.contiguous()
    bh_cat = bh_cat.contiguous()
    out = torch.empty((T, B, H), device=gi.device, dtype=gi.dtype)
    if tiled and codes is not None:
        _lib.launch(_lib.KIND_DENSE_TILED, "gs_dense_fwd_tiled_i8w", gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat,
                    out=out, h_in_quant=h_in_quant, h_out_quant=h_out_quant, contiguous=True, w_codes=codes)
    elif tiled:
        _lib.launch(_lib.KIND_DENSE_TILED, "gs_dense_fwd_tiled", gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat,
                    out=out, h_in_quant=h_in_quant, h_out_quant=h_out_quant, gh_save=gh_save, contiguous=True)
    elif codes is not None:
        _lib.launch(_lib.KIND_DENSE, "gs_dense_fwd_i8w", gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat, out=out,
                    h_in_quant=h_in_quant, h_out_quant=h_out_quant, contiguous=True, w_codes=codes)
    else:
        _lib.launch(_lib.KIND_DENSE, "gs_dense_fwd", gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat, out=out,
                    h_in_quant=h_in_quant, h_out_quant=h_out_quant, gh_save=gh_save, contiguous=True)
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
    return _dense_forward("gru_scan_forward_persistent", gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant,
                          int8_codes=True)


def gru_scan_forward(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_cat: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Same contract as the reference's barrier-free launcher (scan.py:1688-1765):
    the batch-tiled kernel, no co-residency requirement, any H up to 8192."""
    return _dense_forward("gru_scan_forward", gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, tiled=True,
                          int8_codes=True)


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


def gru_scan_backward_triton(gi, h0, Wh_cat, bh_cat, out, dout, *, h_in_quant=None, h_out_quant=None):
    """Gradients (dgi, dh0, dWh_cat, dbh_cat) of the dense scan with the
    reverse recurrence on the barrier-free batch-tiled kernel
    (``gs_dense_bwd_tiled``); same contract as the reference's
    gru_scan_backward_triton (scan.py:1355-1447)."""
    return _dense_backward("gru_scan_backward_triton", gi, h0, Wh_cat, bh_cat, out, dout, h_in_quant,
                           h_out_quant, tiled=True)


def _dense_backward(who: str, gi, h0, Wh_cat, bh_cat, out, dout, h_in_quant, h_out_quant,
                    gh_saved: Optional[torch.Tensor] = None, tiled: bool = False):
    """Runs gs_dense_bwd (tiled: gs_dense_bwd_tiled); gh_saved is the gh the
    forward stored through gh_save (then the backward skips its recompute GEMM)."""
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
    kind, fn = (_lib.KIND_DENSE_TILED, "gs_dense_bwd_tiled") if tiled else (_lib.KIND_DENSE, "gs_dense_bwd")
    _lib.launch_bwd(kind, fn, gi=gi, h0=h0, w=Wh_cat, w2=None, bh=bh_cat, out=out,
                    dout=dout, dgi=dgi, dh0=dh0, dw_part=dW, dbh_part=dbh_part,
                    h_in_quant=check_quant(h_in_quant, "h_in_quant"),
                    h_out_quant=check_quant(h_out_quant, "h_out_quant"), gh_saved=gh_saved)
    return dgi, dh0, dW, dbh_part.sum(0)


# Our alias of the persistent backward launcher (no reference counterpart).
gru_scan_backward = gru_scan_backward_persistent


def _function_forward(ctx: Any, tiled: bool, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, save_gh):
    gh = None
    save = any(ctx.needs_input_grad[:4]) if save_gh is None else bool(save_gh)
    if save and gi.dim() == 3:
        T, B, G3 = gi.shape
        gh = torch.empty((T, B, G3), device=gi.device, dtype=torch.float32)
    who = "gru_scan_forward" if tiled else "gru_scan_forward_persistent"
    out = _dense_forward(who, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, gh_save=gh, tiled=tiled,
                         int8_codes=not any(ctx.needs_input_grad[:4]))
    ctx.save_for_backward(gi, h0, Wh_cat, bh_cat, out, gh)
    ctx.h_in_quant = check_quant(h_in_quant, "h_in_quant")
    ctx.h_out_quant = check_quant(h_out_quant, "h_out_quant")
    return out


def _function_backward(ctx: Any, tiled: bool, dout: torch.Tensor):
    gi, h0, Wh_cat, bh_cat, out, gh = ctx.saved_tensors
    who = "gru_scan_backward_triton" if tiled else "gru_scan_backward_persistent"
    grads = _dense_backward(who, gi, h0, Wh_cat, bh_cat, out, dout, ctx.h_in_quant, ctx.h_out_quant,
                            gh_saved=gh, tiled=tiled)
    return (*grads, None, None, None)


class GRUScanPersistentFunction(torch.autograd.Function):
    """autograd wrapper of the persistent kernels (scan.py:1630-1664); saves
    (gi, h0, Wh_cat, bh_cat, out) like scan.py:1650-1652, plus the forward's gh
    when a gradient is needed, so the backward skips the reference's recompute
    of gh (scan.py:388-421). ``save_gh`` (a seventh argument with no reference
    counterpart) is decided when ``apply`` is called, where the grad mode is
    still visible (the forward runs under no_grad): by default whether grad
    mode is on and any tensor input requires a gradient (``save_gh_default``;
    ``set_save_gh(False)`` turns saving off)."""

    @classmethod
    def apply(cls, *args, **kwargs):  # type: ignore[override]
        if len(args) == 6:  # the reference's six-argument form
            args = (*args, save_gh_default(*args[:4]))
        return super().apply(*args, **kwargs)

    @staticmethod
    def forward(ctx: Any, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, save_gh=None):  # type: ignore[override]
        return _function_forward(ctx, False, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, save_gh)

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        return _function_backward(ctx, False, dout)


class GRUScanFunction(torch.autograd.Function):
    """The same contract on the barrier-free batch-tiled kernels
    (scan.py:1556-1604: the reference's gru_scan Function, whose forward and
    backward are its non-persistent kernels)."""

    @classmethod
    def apply(cls, *args, **kwargs):  # type: ignore[override]
        if len(args) == 6:
            args = (*args, save_gh_default(*args[:4]))
        return super().apply(*args, **kwargs)

    @staticmethod
    def forward(ctx: Any, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, save_gh=None):  # type: ignore[override]
        return _function_forward(ctx, True, gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant, save_gh)

    @staticmethod
    def backward(ctx: Any, dout: torch.Tensor):  # type: ignore[override]
        return _function_backward(ctx, True, dout)


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
                                                              save_gh_default(gi, h0, Wh_cat, bh_cat)))


def gru_scan(
    gi: torch.Tensor,
    h0: torch.Tensor,
    Wh_cat: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
) -> torch.Tensor:
    """Differentiable dense GRU scan (reference scan.py:1607-1627) on the
    barrier-free batch-tiled kernels; returns out [T, B, H]."""
    return cast(torch.Tensor, GRUScanFunction.apply(gi, h0, Wh_cat, bh_cat, h_in_quant, h_out_quant,
                                                    save_gh_default(gi, h0, Wh_cat, bh_cat)))
