"""Export of integer weight codes, scales and zero points.

The reference leaves this as a TODO on the cell (LarocheC/gru-triton
src/gru_qat/gru_cell.py:551-553: "export_int_weights() returning a dict of
int tensors, scales, and zero points in the layout expected by the Triton
kernel"). Here every weight keeps the layout the scan and projection entry
points take, and is quantized per row of its last dimension with the
per-channel symmetric rule of the reference's weight quantizer
(FakeQuantizePerChannel, quantizers.py:188-199 with :124-134), by the
``gs_quantize_rows`` kernel:

  scale[r] = max(max_c |w[r, c]|, 1e-8) / qmax,
  codes[r, c] = clamp(round_half_even(w[r, c] / scale[r]), -qmax, qmax)   (int8)

so ``codes * scale`` is bit for bit the fake-quantized weight the input
projection uses. The rows are: Wi_cat and Wh_cat, each output row; Wh_diag,
each gate; Wh_struct (and Wh_struct2), each output row of each block
([3, nb, bs] scales); twiddles, each (gate, chain, stage) ([3, nblocks,
log_n] scales). Biases stay fp32. The activation quantizers' frozen scales
and zero points are exported with them.
"""

from __future__ import annotations

import ctypes
from typing import Any, Dict, Optional, Tuple

import torch

from . import _lib


def quantize_rows(w: torch.Tensor, rows: int, bits: int = 8) -> Tuple[torch.Tensor, torch.Tensor]:
    """int8 codes (shape of ``w``) and per-row scales ([rows]) of ``w`` viewed
    as [rows, numel / rows] (``gs_quantize_rows``)."""
    if not (isinstance(w, torch.Tensor) and w.is_cuda and w.dtype == torch.float32):
        raise ValueError("quantize_rows: w must be a float32 CUDA (HIP) tensor")
    if not 2 <= bits <= 8:
        raise ValueError(f"quantize_rows: int8 codes need 2 <= bits <= 8; got {bits}")
    if rows < 1 or w.numel() % rows != 0 or w.numel() == 0:
        raise ValueError(f"quantize_rows: {w.numel()} elements do not split into {rows} rows")
    qmax = 2 ** (bits - 1) - 1
    wc = w.detach().contiguous()
    codes = torch.empty(wc.shape, dtype=torch.int8, device=w.device)
    scale = torch.empty(rows, dtype=torch.float32, device=w.device)
    a = _lib.GsRowsArgs()
    a.w, a.scale, a.codes, a.w_q = wc.data_ptr(), scale.data_ptr(), codes.data_ptr(), None
    a.rows, a.cols = rows, wc.numel() // rows
    a.qmin, a.qmax = -qmax, qmax
    lib = _lib.load()
    with _lib.on_device(w.device):
        rc = lib.gs_quantize_rows(ctypes.byref(a), ctypes.c_void_p(_lib.current_stream_handle(w.device)))
    _lib.raise_for(rc, lib)
    return codes, scale


def _rows_of(kind: str, name: str, t: torch.Tensor) -> int:
    if name in ("Wi_cat", "Wh_cat"):
        return t.shape[0]
    if kind == "diagonal":
        return t.shape[0]  # one scale per gate
    if kind == "monarch":
        return t.shape[0] * t.shape[1] * t.shape[2]  # [3, nb, bs(out)]
    if kind == "butterfly":
        return t.shape[0] * t.shape[1] * t.shape[2]  # [3, nblocks, log_n]
    raise ValueError(kind)


def _scale_shape(kind: str, name: str, t: torch.Tensor) -> Tuple[int, ...]:
    if name in ("Wi_cat", "Wh_cat") or kind == "diagonal":
        return (t.shape[0],)
    return tuple(t.shape[:3])


def _frozen(q: Any) -> Tuple[Optional[float], Optional[float], Optional[int], Optional[int]]:
    if q is None:
        return None, None, None, None
    if q.config.mode != "frozen":
        raise ValueError(f"export_int_weights: quantizer {q.config.name!r} is in mode {q.config.mode!r}; "
                         "calibrate and freeze() the layer first")
    return float(q.scale), float(q.zero_point), int(q.qmin), int(q.qmax)


def export_int_weights(layer: Any, bits: int = 8) -> Dict[str, Any]:
    """The int8 export of a ``ScanLayer``: a dict of int8 codes, fp32 scales
    and zero points (weights: symmetric, zero point 0), fp32 biases and the
    frozen activation scales."""
    kind = layer.kind
    hidden_name = {"dense": "Wh_cat", "diagonal": "Wh_diag", "monarch": "Wh_struct", "butterfly": "twiddles"}[kind]
    out: Dict[str, Any] = {"kind": kind, "bits": bits, "hidden_size": layer.hidden_size,
                           "input_size": layer.Wi_cat.shape[1], "weight_zero_point": 0}
    weights = [("Wi_cat", layer.Wi_cat), (hidden_name, layer.hidden)]
    if layer.hidden2 is not None:
        weights.append(("Wh_struct2", layer.hidden2))
    for name, w in weights:
        rows = _rows_of(kind, name, w)
        codes, scale = quantize_rows(w.detach(), rows, bits)
        out[name] = codes
        out[name + "_scale"] = scale.view(_scale_shape(kind, name, w))
    out["bi_cat"] = layer.bi_cat.detach().clone() if layer.bi_cat is not None else None
    out["bh_cat"] = layer.bh_cat.detach().clone()
    for tag, q in (("x", layer.quant_x), ("h_in", layer.quant_h_in), ("h_out", layer.quant_h_out)):
        s, zp, lo, hi = _frozen(q)
        out[f"{tag}_scale"], out[f"{tag}_zero_point"], out[f"{tag}_qrange"] = s, zp, (
            None if lo is None else (lo, hi))
    return out


def dequantize_int_weights(export: Dict[str, Any]) -> Dict[str, torch.Tensor]:
    """codes * scale for every exported weight (the fake-quantized weights)."""
    res = {}
    for name, v in export.items():
        if isinstance(v, torch.Tensor) and v.dtype == torch.int8:
            s = export[name + "_scale"]
            shape = s.shape + (1,) * (v.dim() - s.dim())
            res[name] = v.to(torch.float32) * s.view(shape)
    return res
