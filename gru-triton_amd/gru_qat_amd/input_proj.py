"""Input projection producing the scan's gate inputs (drop-in for the gi
producer of the reference's GRULayer fast dispatch).

Reference: ``GRULayer._forward_fast_dispatch`` (LarocheC/gru-triton
src/gru_qat/gru_layer.py:249-255) computes ``xq = cell.quant_x(x)``,
``Wi_cat, bi_cat = cell.quantize_input_weights()`` (gru_cell.py:273-299, each
gate weight through its per-channel quantizer, quantizers.py:188-199) and
``gi = F.linear(xq, Wi_cat, bi_cat)``. Here the three steps are one call of
``gs_input_proj`` (libgruscan.so): the per-row weight fake-quant, then one
fp32 MFMA GEMM that fake-quantizes x as it loads it and adds the bias in its
epilogue; with both quantizers int8 (the QAT layer) the product runs instead on
the int8 MFMA over x's levels and the weight's codes (exact integer sums, within
an fp32 rounding of each product of the fp32 GEMM). The backward (``gs_input_proj_bwd``) follows torch's autograd of
fake_quant_ste (ste.py:65-95): straight through the rounding, clipped at the
clamp, x's frozen scale constant, and the per-row weight scales (computed from
the weight, not detached, in the reference's dynamic weight quantizer)
passing gradient to each row's max and min elements.
"""

from __future__ import annotations

import ctypes
from typing import Any, Optional, Tuple, cast

import torch

from . import _lib
from ._common import QuantTuple, check_quant, require_cuda, require_f32

WeightQuant = Optional[Tuple[int, int]]


def _check_wq(w_quant: WeightQuant) -> WeightQuant:
    if w_quant is None:
        return None
    try:
        qmin, qmax = (int(v) for v in w_quant)
    except (TypeError, ValueError):
        raise ValueError(f"w_quant must be None or a (qmin, qmax) tuple; got {w_quant!r}") from None
    if not (qmax > 0 and qmin <= qmax):
        raise ValueError(f"w_quant needs qmax > 0 and qmin <= qmax; got ({qmin}, {qmax})")
    return (qmin, qmax)


def _project(x2: torch.Tensor, Wi_cat: torch.Tensor, bi_cat: Optional[torch.Tensor], x_quant: QuantTuple,
             w_quant: WeightQuant) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """gi [M, N], the weight used, its per-row scales (or None) and q_x(x) (or None)."""
    lib = _lib.load()
    M, I = x2.shape
    N = Wi_cat.shape[0]
    gi = torch.empty((M, N), device=x2.device, dtype=x2.dtype)
    a = _lib.GsProjArgs()
    a.x, a.w, a.gi = x2.data_ptr(), Wi_cat.data_ptr(), gi.data_ptr()
    a.bias = bi_cat.data_ptr() if bi_cat is not None else None
    a.M, a.N, a.I = M, N, I
    a.sx, a.sgi = x2.stride(0), gi.stride(0)
    a.q_x = _lib.make_quant(x_quant, "x_quant")
    xq = None
    if x_quant is not None:
        xq = torch.empty((M, I), device=x2.device, dtype=x2.dtype)
        a.x_q = xq.data_ptr()
    w_used, scales = Wi_cat, None
    if w_quant is not None:
        w_used = torch.empty_like(Wi_cat)
        scales = torch.empty((N,), device=x2.device, dtype=x2.dtype)
        a.w_q, a.w_scale = w_used.data_ptr(), scales.data_ptr()
        a.q_w = _lib.GsQuant(1, 1.0, int(w_quant[0]), int(w_quant[1]))
    else:
        a.q_w = _lib.make_quant(None, "w_quant")
    codes = None
    if (x_quant is not None and w_quant is not None and I % 16 == 0 and int(x_quant[1]) >= -128
            and int(x_quant[2]) <= 127 and w_quant[0] >= -128 and w_quant[1] <= 127):
        # int8 scratch for x's levels and the weight's codes: the product then runs on the int8 MFMA
        codes = torch.empty((M + N) * I, device=x2.device, dtype=torch.int8)
        a.x_codes, a.w_codes = codes.data_ptr(), codes.data_ptr() + M * I
    with _lib.on_device(x2.device):
        rc = lib.gs_input_proj(ctypes.byref(a), ctypes.c_void_p(_lib.current_stream_handle(x2.device)))
    _lib.raise_for(rc, lib)
    del codes  # the caching allocator keeps it until the stream's work is done
    return gi, w_used, scales, xq


def _validate(who: str, x: torch.Tensor, Wi_cat: torch.Tensor, bi_cat: Optional[torch.Tensor]) -> None:
    tensors = dict(x=x, Wi_cat=Wi_cat) if bi_cat is None else dict(x=x, Wi_cat=Wi_cat, bi_cat=bi_cat)
    require_cuda(who, **tensors)
    require_f32(who, **tensors)
    if Wi_cat.dim() != 2 or x.shape[-1] != Wi_cat.shape[1]:
        raise ValueError(f"{who}: Wi_cat must be [N, I] with I = x.shape[-1]={x.shape[-1]}; "
                         f"got {tuple(Wi_cat.shape)}")
    if bi_cat is not None and tuple(bi_cat.shape) != (Wi_cat.shape[0],):
        raise ValueError(f"{who}: bi_cat must be [{Wi_cat.shape[0]}]; got {tuple(bi_cat.shape)}")
    if x.numel() == 0:
        raise ValueError(f"{who}: x must be non-empty; got shape {tuple(x.shape)}")


def quantize_input_weights(Wi_cat: torch.Tensor, w_quant: WeightQuant = (-127, 127)) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric fake-quant of ``Wi_cat`` [N, I]: returns (W_q, scales)
    with scale[n] = max(max_i |W[n, i]|, 1e-8) / qmax (quantizers.py:124-134,
    188-199). Runs the same kernel as the projection's weight pass."""
    w_quant = _check_wq(w_quant)
    if w_quant is None:
        raise ValueError("quantize_input_weights needs a (qmin, qmax) weight quant")
    x = Wi_cat.new_zeros((1, Wi_cat.shape[1]))
    _validate("quantize_input_weights", x, Wi_cat, None)
    _, wq, scales, _ = _project(x, Wi_cat.contiguous(), None, None, w_quant)
    return wq, cast(torch.Tensor, scales)


class InputProjectionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, x, Wi_cat, bi_cat, x_quant, w_quant):  # type: ignore[override]
        x2 = x.reshape(-1, x.shape[-1])
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        gi, w_used, scales, xq = _project(x2, Wi_cat, bi_cat, x_quant, w_quant)
        ctx.save_for_backward(x2, w_used, xq, Wi_cat if w_quant is not None else None, scales)
        ctx.x_quant = x_quant
        ctx.w_quant = w_quant
        ctx.has_bias = bi_cat is not None
        ctx.x_shape = x.shape
        return gi.view(*x.shape[:-1], Wi_cat.shape[0])

    @staticmethod
    def backward(ctx: Any, dgi: torch.Tensor):  # type: ignore[override]
        x2, w_used, xq, w_raw, scales = ctx.saved_tensors
        lib = _lib.load()
        M, I = x2.shape
        N = w_used.shape[0]
        dgi2 = dgi.reshape(M, N)
        if dgi2.stride(-1) != 1:
            dgi2 = dgi2.contiguous()
        dx = torch.empty((M, I), device=x2.device, dtype=x2.dtype)
        dw = torch.empty_like(w_used)
        dbias = torch.empty((N,), device=x2.device, dtype=x2.dtype) if ctx.has_bias else None
        a = _lib.GsProjBwdArgs()
        a.x, a.w, a.dgi, a.dx, a.dw = x2.data_ptr(), w_used.data_ptr(), dgi2.data_ptr(), dx.data_ptr(), dw.data_ptr()
        a.x_q = xq.data_ptr() if xq is not None else None
        a.dbias = dbias.data_ptr() if dbias is not None else None
        a.M, a.N, a.I = M, N, I
        a.sx, a.sdgi, a.sdx = x2.stride(0), dgi2.stride(0), dx.stride(0)
        a.q_x = _lib.make_quant(ctx.x_quant, "x_quant")
        if ctx.w_quant is not None:
            a.w_raw, a.w_scale = w_raw.data_ptr(), scales.data_ptr()
            a.q_w = _lib.GsQuant(1, 1.0, int(ctx.w_quant[0]), int(ctx.w_quant[1]))
        need = lib.gs_input_proj_bwd_workspace_bytes(ctypes.byref(a))
        if need < 0:
            _lib.raise_for(int(need), lib)
        ws = torch.empty((max(int(need), 256),), device=x2.device, dtype=torch.uint8)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        with _lib.on_device(x2.device):
            rc = lib.gs_input_proj_bwd(ctypes.byref(a),
                                       ctypes.c_void_p(_lib.current_stream_handle(x2.device)))
        _lib.raise_for(rc, lib)
        return dx.view(ctx.x_shape), dw, dbias, None, None


def input_projection(x: torch.Tensor, Wi_cat: torch.Tensor, bi_cat: Optional[torch.Tensor] = None, *,
                     x_quant: QuantTuple = None, w_quant: WeightQuant = None) -> torch.Tensor:
    """gi = q_x(x) W_q^T + bi_cat for x [..., I] (e.g. [T, B, I]); returns
    [..., N]. ``x_quant`` is a frozen per-tensor (scale, qmin, qmax);
    ``w_quant`` = (qmin, qmax) turns on the per-row symmetric weight
    fake-quant. Differentiable in x, Wi_cat and bi_cat (straight-through)."""
    who = "input_projection"
    _validate(who, x, Wi_cat, bi_cat)
    x_quant = check_quant(x_quant, "x_quant")
    w_quant = _check_wq(w_quant)
    Wi_cat = Wi_cat.contiguous()
    bi_cat = bi_cat.contiguous() if bi_cat is not None else None
    return cast(torch.Tensor, InputProjectionFunction.apply(x, Wi_cat, bi_cat, x_quant, w_quant))
