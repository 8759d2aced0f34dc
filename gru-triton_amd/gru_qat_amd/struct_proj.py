"""Structured input projection: the gate inputs of a cell whose input side is
structured (drop-in for ``GRUCellQuant.structured_input_projection``,
LarocheC/gru-triton src/gru_qat/gru_cell.py:466-503, which the layer's fast
dispatch takes at gru_layer.py:256).

Per gate g (r, z, n): ``gi_g = out_quant_g(map_g(x_quant(x))) + bi_g``, with
``map_g`` the gate's structured input weight (``struct_Wi_g``; the input size
equals the hidden size) and ``out_quant_g`` its output-side quantizer
(``quant_struct_Wi_g``, applied before the bias). The weights are stacked over
the gates as on the hidden side:

* ``"diagonal"``: ``[3, H]``, ``y = w_g * x``;
* ``"monarch"``: ``[3, nblocks, blksz, blksz]`` as (out, in), one
  block-diagonal factor;
* ``"butterfly"``: twiddles ``[3, nchains, log_n, 2^log_n / 2, 2, 2]``.

``out_quant`` is None, one spec for all three gates, or three specs, each
None, a frozen per-tensor ``(scale, qmin, qmax)`` or ``("rows", qmin,
qmax)``: the per-row dynamic symmetric quantizer, FakeQuantizePerChannel on
axis 0 in dynamic mode (the reference's default weight recipe, which its cell
uses for these quantizers). Forward and backward run ``gs_struct_input_proj``
and ``gs_struct_input_proj_bwd`` of libgruscan.so; the backward is torch's
autograd of the reference's fake_quant_ste, the dynamic scale's own gradient
path included.
"""

from __future__ import annotations

import ctypes
from typing import Any, Optional, Sequence, Tuple, cast

import torch

from . import _lib
from ._common import QuantTuple, check_quant, require_cuda, require_f32

INPUT_KINDS = {"diagonal": _lib.KIND_DIAGONAL, "monarch": _lib.KIND_MONARCH, "butterfly": _lib.KIND_BUTTERFLY}
OQ_OFF, OQ_FROZEN, OQ_ROWS = 0, 1, 2


def _oquant(spec: Any, gate: str) -> _lib.GsOQuant:
    if spec is None:
        return _lib.GsOQuant(OQ_OFF, 1.0, 0, 0)
    if isinstance(spec, (tuple, list)) and len(spec) == 3 and spec[0] == "rows":
        qmin, qmax = int(spec[1]), int(spec[2])
        if not (qmax > 0 and qmin <= qmax):
            raise ValueError(f"out_quant[{gate}] ('rows', qmin, qmax) needs qmax > 0 and qmin <= qmax; got {spec!r}")
        return _lib.GsOQuant(OQ_ROWS, 1.0, qmin, qmax)
    q = check_quant(spec, f"out_quant[{gate}]")
    assert q is not None
    return _lib.GsOQuant(OQ_FROZEN, float(q[0]), int(q[1]), int(q[2]))


def _oquants(out_quant: Any) -> Tuple[_lib.GsOQuant, _lib.GsOQuant, _lib.GsOQuant]:
    if out_quant is None:
        specs: Sequence[Any] = (None, None, None)
    elif isinstance(out_quant, (tuple, list)) and len(out_quant) == 3 and not isinstance(out_quant[0], (int, float, str)):
        specs = out_quant
    else:
        specs = (out_quant, out_quant, out_quant)
    return tuple(_oquant(s, g) for s, g in zip(specs, "rzn"))  # type: ignore[return-value]


def struct_dims(kind: str, W: torch.Tensor, H: int) -> Tuple[int, int, int, int]:
    """(nblocks, blksz, log_n, nchains) of a stacked structured weight."""
    if kind == "diagonal":
        if tuple(W.shape) != (3, H):
            raise ValueError(f"diagonal Wi_struct must be [3, H]=[3, {H}]; got {tuple(W.shape)}")
        return 0, 0, 0, 0
    if kind == "monarch":
        if W.dim() != 4 or W.shape[0] != 3 or W.shape[2] != W.shape[3] or W.shape[1] * W.shape[2] != H:
            raise ValueError(f"monarch Wi_struct must be [3, nblocks, blksz, blksz] with nblocks * blksz = H = {H}; "
                             f"got {tuple(W.shape)}")
        return int(W.shape[1]), int(W.shape[2]), 0, 0
    if kind == "butterfly":
        if W.dim() != 6 or W.shape[0] != 3 or tuple(W.shape[4:]) != (2, 2):
            raise ValueError(f"butterfly Wi_struct must be [3, nchains, log_n, 2^log_n / 2, 2, 2]; got {tuple(W.shape)}")
        L = int(W.shape[2])
        if W.shape[3] != (1 << L) // 2 or (1 << L) < H:
            raise ValueError(f"butterfly Wi_struct: 2^log_n = {1 << L} must be >= H = {H} and dim 3 = 2^log_n / 2; "
                             f"got {tuple(W.shape)}")
        return 0, 0, L, int(W.shape[1])
    raise ValueError(f"structured input kind must be one of {sorted(INPUT_KINDS)}; got {kind!r}")


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(_lib.current_stream_handle(dev))


class StructInputProjFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, x, W, bias, kind, x_quant, out_quant):  # type: ignore[override]
        lib = _lib.load()
        H = x.shape[-1]
        x2 = x.reshape(-1, H)
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        M = x2.shape[0]
        nb, bs, L, nch = struct_dims(kind, W, H)
        oq = _oquants(out_quant)
        any_oq = any(o.mode != OQ_OFF for o in oq)
        any_rows = any(o.mode == OQ_ROWS for o in oq)
        dev = x2.device
        gi = torch.empty((M, 3 * H), device=dev, dtype=x2.dtype)
        y = torch.empty((M, 3 * H), device=dev, dtype=x2.dtype) if any_oq else None
        y_scale = torch.empty((3, M), device=dev, dtype=x2.dtype) if any_rows else None
        xq = torch.empty((M, H), device=dev, dtype=x2.dtype) if x_quant is not None else None
        a = _lib.GsSProjArgs()
        a.kind = INPUT_KINDS[kind]
        a.x, a.w, a.gi = x2.data_ptr(), W.data_ptr(), gi.data_ptr()
        a.bias = bias.data_ptr() if bias is not None else None
        a.y = y.data_ptr() if y is not None else None
        a.y_scale = y_scale.data_ptr() if y_scale is not None else None
        a.x_q = xq.data_ptr() if xq is not None else None
        a.M, a.H, a.sx, a.sgi = M, H, x2.stride(0), gi.stride(0)
        a.nblocks, a.blksz, a.log_n, a.bfly_nblocks = nb, bs, L, nch
        a.q_x = _lib.make_quant(x_quant, "x_quant")
        for g in range(3):
            a.q_out[g] = oq[g]
        need = lib.gs_struct_input_proj_scratch_bytes(ctypes.byref(a))
        if need < 0:
            _lib.raise_for(int(need), lib)
        scratch = torch.empty((max(int(need), 256),), device=dev, dtype=torch.uint8)
        a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel()
        with _lib.on_device(dev):
            rc = lib.gs_struct_input_proj(ctypes.byref(a), _stream(dev))
        _lib.raise_for(rc, lib)
        ctx.save_for_backward(x2, W, xq, y, y_scale)
        ctx.kind, ctx.x_quant, ctx.oq = kind, x_quant, oq
        ctx.dims = (nb, bs, L, nch)
        ctx.has_bias = bias is not None
        ctx.x_shape = x.shape
        return gi.view(*x.shape[:-1], 3 * H)

    @staticmethod
    def backward(ctx: Any, dgi: torch.Tensor):  # type: ignore[override]
        x2, W, xq, y, y_scale = ctx.saved_tensors
        lib = _lib.load()
        M, H = x2.shape
        dgi2 = dgi.reshape(M, 3 * H)
        if dgi2.stride(-1) != 1:
            dgi2 = dgi2.contiguous()
        dev = x2.device
        dx = torch.empty((M, H), device=dev, dtype=x2.dtype)
        dW = torch.empty_like(W)
        dbias = torch.empty((3 * H,), device=dev, dtype=x2.dtype) if ctx.has_bias else None
        a = _lib.GsSProjBwdArgs()
        a.kind = INPUT_KINDS[ctx.kind]
        a.x, a.w, a.dgi, a.dx, a.dw = x2.data_ptr(), W.data_ptr(), dgi2.data_ptr(), dx.data_ptr(), dW.data_ptr()
        a.x_q = xq.data_ptr() if xq is not None else None
        a.y = y.data_ptr() if y is not None else None
        a.y_scale = y_scale.data_ptr() if y_scale is not None else None
        a.dbias = dbias.data_ptr() if dbias is not None else None
        a.M, a.H, a.sx, a.sdgi, a.sdx = M, H, x2.stride(0), dgi2.stride(0), dx.stride(0)
        a.nblocks, a.blksz, a.log_n, a.bfly_nblocks = ctx.dims
        a.q_x = _lib.make_quant(ctx.x_quant, "x_quant")
        for g in range(3):
            a.q_out[g] = ctx.oq[g]
        need = lib.gs_struct_input_proj_bwd_scratch_bytes(ctypes.byref(a))
        if need < 0:
            _lib.raise_for(int(need), lib)
        scratch = torch.empty((max(int(need), 256),), device=dev, dtype=torch.uint8)
        a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel()
        with _lib.on_device(dev):
            rc = lib.gs_struct_input_proj_bwd(ctypes.byref(a), _stream(dev))
        _lib.raise_for(rc, lib)
        return dx.view(ctx.x_shape), dW, dbias, None, None, None


def structured_input_projection(x: torch.Tensor, kind: str, Wi_struct: torch.Tensor,
                                bi_cat: Optional[torch.Tensor] = None, *, x_quant: QuantTuple = None,
                                out_quant: Any = None) -> torch.Tensor:
    """gi [..., 3H] for x [..., H] (e.g. [T, B, H]) through the structured
    input side ``kind`` with stacked weights ``Wi_struct``; differentiable in
    x, Wi_struct and bi_cat."""
    who = "structured_input_projection"
    tensors = dict(x=x, Wi_struct=Wi_struct) if bi_cat is None else dict(x=x, Wi_struct=Wi_struct, bi_cat=bi_cat)
    require_cuda(who, **tensors)
    require_f32(who, **tensors)
    if kind not in INPUT_KINDS:
        raise ValueError(f"{who}: kind must be one of {sorted(INPUT_KINDS)}; got {kind!r}")
    if x.dim() < 1 or x.numel() == 0:
        raise ValueError(f"{who}: x must be non-empty; got shape {tuple(x.shape)}")
    H = x.shape[-1]
    struct_dims(kind, Wi_struct, H)
    if bi_cat is not None and tuple(bi_cat.shape) != (3 * H,):
        raise ValueError(f"{who}: bi_cat must be [3H]=[{3 * H}]; got {tuple(bi_cat.shape)}")
    x_quant = check_quant(x_quant, "x_quant")
    _oquants(out_quant)  # validate before launching
    Wi_struct = Wi_struct.contiguous()
    bi_cat = bi_cat.contiguous() if bi_cat is not None else None
    return cast(torch.Tensor, StructInputProjFunction.apply(x, Wi_struct, bi_cat, kind, x_quant, out_quant))
