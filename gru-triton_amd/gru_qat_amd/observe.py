"""The GRU scan with its hidden quantizers as observers (``gs_observe_scan``).

This is the reference's per-step path with quant_h_in and quant_h_out firing
(LarocheC/gru-triton src/gru_qat/gru_layer.py:205-223 over step_with_gi,
gru_cell.py:437-464), the path GRULayer.calibrate forces (gru_layer.py:308-336)
so that the hidden quantizers' observers see every step: at step t, quant_h_in
sees h_{t-1} (h0 first) and quant_h_out the new pre-quant h_t; in "dynamic" and
"min_max" mode each computes its scale from that tensor's min and max, and
"min_max" also updates its running statistics. All of it runs on the device
(no host synchronisation); the hidden map of every kind is taken in its dense
form (``hidden_map_dense``).
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib
from ._common import check_common, require_cuda, require_f32
from .quantizers import FakeQuantizePerTensor

KINDS = {"dense": _lib.KIND_DENSE, "diagonal": _lib.KIND_DIAGONAL, "monarch": _lib.KIND_MONARCH,
         "butterfly": _lib.KIND_BUTTERFLY, "circulant": _lib.KIND_CIRCULANT}


def _map_dims(kind: str, hidden: torch.Tensor, hidden2: Optional[torch.Tensor], H: int) -> Tuple[int, int, int, int]:
    """(nblocks, blksz, log_n, bfly_nblocks) of a hidden weight, with the shape
    checks of the kind's scan wrapper."""
    if kind == "dense":
        if tuple(hidden.shape) != (3 * H, H):
            raise ValueError(f"Wh_cat shape must be (3H, H)=({3 * H}, {H}); got {tuple(hidden.shape)}")
        return 0, 0, 0, 0
    if kind in ("diagonal", "circulant"):
        name = "Wh_diag" if kind == "diagonal" else "Wh_circ"
        if tuple(hidden.shape) != (3, H):
            raise ValueError(f"{name} shape must be (3, H)=(3, {H}); got {tuple(hidden.shape)}")
        return 0, 0, 0, 0
    if kind == "monarch":
        from .scan_monarch import _check_struct

        nb, bs = _check_struct("Wh_struct", hidden, H)
        if hidden2 is not None and tuple(hidden2.shape) != tuple(hidden.shape):
            raise ValueError(f"Wh_struct2 shape {tuple(hidden2.shape)} must equal Wh_struct shape "
                             f"{tuple(hidden.shape)}")
        return nb, bs, 0, 0
    if kind == "butterfly":
        from .scan_butterfly import check_twiddles

        nblocks, log_n = check_twiddles(hidden, H)
        return 0, 0, log_n, nblocks
    raise ValueError(f"kind must be one of {sorted(KINDS)}; got {kind!r}")


def hidden_map_dense(kind: str, hidden: torch.Tensor, H: int, hidden2: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The hidden map of ``kind`` as the dense [3H, H] matrix M with
    gh = hq M^T + bh (``gs_hidden_map_dense``)."""
    require_cuda("hidden_map_dense", hidden=hidden)
    require_f32("hidden_map_dense", hidden=hidden)
    if hidden2 is not None and kind != "monarch":
        raise ValueError("hidden2 is only meaningful for kind 'monarch'")
    nb, bs, log_n, bfly_nb = _map_dims(kind, hidden, hidden2, H)
    lib = _lib.load()
    w = hidden.contiguous()
    w2 = hidden2.contiguous() if hidden2 is not None else None
    m = torch.empty((3 * H, H), device=hidden.device, dtype=torch.float32)
    a = _lib.GsMapArgs()
    a.kind = KINDS[kind]
    a.w, a.w2, a.m = w.data_ptr(), (w2.data_ptr() if w2 is not None else None), m.data_ptr()
    a.H, a.nblocks, a.blksz, a.log_n, a.bfly_nblocks = H, nb, bs, log_n, bfly_nb
    need = lib.gs_hidden_map_scratch_bytes(ctypes.byref(a))
    if need < 0:
        _lib.raise_for(int(need), lib)
    with _lib.on_device(hidden.device):
        handle = _lib.current_stream_handle(hidden.device)
        scratch = torch.empty((int(need),), dtype=torch.uint8, device=hidden.device) if need > 0 else None
        if scratch is not None:
            a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel()
        rc = lib.gs_hidden_map_dense(ctypes.byref(a), ctypes.c_void_p(handle))
        del scratch
    _lib.raise_for(rc, lib)
    return m


def hidden_map_grad(kind: str, dm: torch.Tensor, hidden: torch.Tensor, H: int) -> torch.Tensor:
    """Folds a gradient ``dm`` [3H, H] of the dense form onto the parameters
    of a diagonal, single-factor Monarch or circulant hidden weight (the shape
    of ``hidden``), with ``gs_hidden_map_grad``."""
    nb, bs, log_n, bfly_nb = _map_dims(kind, hidden, None, H)
    if tuple(dm.shape) != (3 * H, H):
        raise ValueError(f"dm must be [3H, H]=[{3 * H}, {H}]; got {tuple(dm.shape)}")
    lib = _lib.load()
    dm = dm.contiguous()
    dw = torch.empty(hidden.shape, device=hidden.device, dtype=torch.float32)
    a = _lib.GsMapArgs()
    a.kind = KINDS[kind]
    a.w, a.w2, a.m = hidden.data_ptr(), None, None
    a.H, a.nblocks, a.blksz, a.log_n, a.bfly_nblocks = H, nb, bs, log_n, bfly_nb
    with _lib.on_device(hidden.device):
        handle = _lib.current_stream_handle(hidden.device)
        rc = lib.gs_hidden_map_grad(ctypes.byref(a), ctypes.c_void_p(dm.data_ptr()), ctypes.c_void_p(dw.data_ptr()),
                                    ctypes.c_void_p(handle))
    _lib.raise_for(rc, lib)
    return dw


def _off() -> _lib.GsObserver:
    o = _lib.GsObserver()
    o.mode, o.symmetric, o.qmin, o.qmax, o.scale, o.zero_point = _lib.OBS_OFF, 1, 0, 1, 1.0, 0.0
    return o


def gru_scan_observe(
    kind: str,
    gi: torch.Tensor,
    h0: torch.Tensor,
    hidden: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    quant_h_in: Optional[FakeQuantizePerTensor] = None,
    quant_h_out: Optional[FakeQuantizePerTensor] = None,
    hidden2: Optional[torch.Tensor] = None,
    return_trace: bool = False,
):
    """The T-step scan of ``kind`` with ``quant_h_in``/``quant_h_out`` (None:
    no quantizer) applied and observed as the per-step path does. Returns
    ``out [T, B, H]``, and with ``return_trace`` also ``trace [T, 4]`` = the
    (scale, zero point) of quant_h_in and of quant_h_out used at each step.
    Forward only (no autograd)."""
    who = "gru_scan_observe"
    if kind not in KINDS:
        raise ValueError(f"{who}: kind must be one of {sorted(KINDS)}; got {kind!r}")
    tensors = dict(gi=gi, h0=h0, hidden=hidden, bh_cat=bh_cat)
    if hidden2 is not None:
        if kind != "monarch":
            raise ValueError(f"{who}: hidden2 is only meaningful for kind 'monarch'")
        tensors["hidden2"] = hidden2
    require_cuda(who, **tensors)
    require_f32(who, **tensors)
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors.values()):
        raise RuntimeError(f"{who} runs without autograd (calibration); call it under torch.no_grad()")
    T, B, H = check_common(who, gi, h0, bh_cat)
    nb, bs, log_n, bfly_nb = _map_dims(kind, hidden, hidden2, H)
    lib = _lib.load()
    gi, h0, bh_cat = gi.contiguous(), h0.contiguous(), bh_cat.contiguous()
    w = hidden.contiguous()
    w2 = hidden2.contiguous() if hidden2 is not None else None
    out = torch.empty((T, B, H), device=gi.device, dtype=torch.float32)
    trace = torch.empty((T, 4), device=gi.device, dtype=torch.float32) if return_trace else None
    a = _lib.GsObserveArgs()
    a.kind = KINDS[kind]
    a.gi, a.h0, a.w, a.bh, a.out = gi.data_ptr(), h0.data_ptr(), w.data_ptr(), bh_cat.data_ptr(), out.data_ptr()
    a.w2 = w2.data_ptr() if w2 is not None else None
    a.trace = trace.data_ptr() if trace is not None else None
    a.T, a.B, a.H = T, B, H
    a.sg_t, a.sg_b, a.sh0_b = gi.stride(0), gi.stride(1), h0.stride(0)
    a.so_t, a.so_b = out.stride(0), out.stride(1)
    a.nblocks, a.blksz, a.log_n, a.bfly_nblocks = nb, bs, log_n, bfly_nb
    for name, q in (("quant_h_in", quant_h_in), ("quant_h_out", quant_h_out)):
        if q is not None and q.config.mode == "min_max" and q.observer_stats.device != gi.device:
            raise ValueError(f"{who}: {name} stats on {q.observer_stats.device}, gi on {gi.device}")
    a.q_in = quant_h_in.observer() if quant_h_in is not None else _off()
    a.q_out = quant_h_out.observer() if quant_h_out is not None else _off()
    need = lib.gs_observe_scan_scratch_bytes(ctypes.byref(a))
    if need < 0:
        _lib.raise_for(int(need), lib)
    with _lib.on_device(gi.device):
        handle = _lib.current_stream_handle(gi.device)
        scratch = torch.empty((int(need),), dtype=torch.uint8, device=gi.device)
        a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel()
        rc = lib.gs_observe_scan(ctypes.byref(a), ctypes.c_void_p(handle))
        del scratch
    _lib.raise_for(rc, lib)
    return (out, trace) if return_trace else out
