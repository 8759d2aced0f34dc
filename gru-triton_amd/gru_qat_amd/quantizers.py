"""Per-tensor fake-quantize with the reference's observer modes, run by the
HIP observer kernels of libgruscan.so.

Mirrors what the scan path reads from, and what calibration drives in, the
reference's quantizer module (LarocheC/gru-triton src/gru_qat/quantizers.py):

* ``QuantizerConfig`` -- quantizers.py:45-60 (bits, symmetric, axis, mode ...);
* ``FakeQuantizePerTensor`` -- FakeQuantize (:63-156) with the per-tensor
  scale rule of FakeQuantizePerTensor (:176-181): buffers ``scale``,
  ``zero_point``, ``running_min``, ``running_max``, the flag
  ``_initialized``, ``_qrange`` (:119-122), ``freeze`` (:98-107) and
  ``_scale_zp_from_min_max`` (:124-134).

``forward`` runs ``gs_observe_tensor``: in "dynamic" and "min_max" mode the
scale and zero point come from the tensor's own min and max on the device,
and "min_max" also mixes them into the running statistics
(``_update_observer``, :136-156); "frozen" uses the stored scale. The
running statistics live in one device buffer ``observer_stats`` =
(running_min, running_max, initialized) that the kernels update in place;
``running_min``/``running_max`` are views of it.

Differences from the reference, all deliberate: only per-tensor quantizers
(the only kind the fast path reads, gru_layer.py:30-48); ``forward`` runs
without autograd (calibration and inference; QAT training goes through the
frozen tuples of the differentiable scans and input projection).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib

MODES = {"frozen": _lib.OBS_FROZEN, "dynamic": _lib.OBS_DYNAMIC, "min_max": _lib.OBS_MIN_MAX}


@dataclass
class QuantizerConfig:
    """quantizers.py:45-60. Only ``axis=None`` (per-tensor) quantizers are built here."""

    bits: int = 8
    symmetric: bool = True
    axis: Optional[int] = None
    group_size: Optional[int] = None
    mode: str = "dynamic"
    learnable_scale: bool = False
    name: str = "default"


class FakeQuantizePerTensor(nn.Module):
    """One (scale, zero_point) for the whole tensor, in mode "dynamic",
    "min_max" or "frozen" (quantizers.py:63-156, 176-181)."""

    def __init__(self, config: Optional[QuantizerConfig] = None) -> None:
        super().__init__()
        self.config = config if config is not None else QuantizerConfig()
        if self.config.axis is not None or self.config.group_size is not None:
            raise ValueError("FakeQuantizePerTensor needs config.axis is None and config.group_size is None")
        if self.config.mode not in MODES:
            raise ValueError(f"mode must be one of {sorted(MODES)}; got {self.config.mode!r}")
        if self.config.bits < 2 or self.config.bits > 16:
            raise ValueError(f"bits must be in [2, 16]; got {self.config.bits}")
        self.qmin, self.qmax = self._qrange(self.config.bits, self.config.symmetric)
        self.register_buffer("scale", torch.tensor(1.0))
        self.register_buffer("zero_point", torch.tensor(0.0))
        # running_min, running_max, initialized (1.0 once the first tensor was observed)
        self.register_buffer("observer_stats", torch.tensor([float("inf"), float("-inf"), 0.0]))

    # ---- the reference's buffers and flag, as views of observer_stats ----

    @property
    def running_min(self) -> torch.Tensor:
        return self.observer_stats[0]

    @running_min.setter
    def running_min(self, value) -> None:
        with torch.no_grad():
            self.observer_stats[0] = value

    @property
    def running_max(self) -> torch.Tensor:
        return self.observer_stats[1]

    @running_max.setter
    def running_max(self, value) -> None:
        with torch.no_grad():
            self.observer_stats[1] = value

    @property
    def _initialized(self) -> bool:
        return bool(self.observer_stats[2].item() != 0.0)

    @_initialized.setter
    def _initialized(self, value: bool) -> None:
        with torch.no_grad():
            self.observer_stats[2] = 1.0 if value else 0.0

    def reset_observer(self) -> None:
        """running_min = +inf, running_max = -inf, not initialized
        (calibration.py:90-94)."""
        with torch.no_grad():
            self.observer_stats.copy_(torch.tensor([float("inf"), float("-inf"), 0.0]))

    # ---- public API ----

    @staticmethod
    def _qrange(bits: int, symmetric: bool) -> Tuple[int, int]:
        if symmetric:
            return -(2 ** (bits - 1)) + 1, 2 ** (bits - 1) - 1
        return 0, 2**bits - 1

    def _scale_zp_from_min_max(self, x_min: torch.Tensor, x_max: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """quantizers.py:124-134, on the 0-dim statistics."""
        if self.config.symmetric:
            absmax = torch.maximum(x_max.abs(), x_min.abs()).clamp(min=1e-8)
            scale = absmax / self.qmax
            zp = torch.zeros_like(scale)
        else:
            scale = (x_max - x_min).clamp(min=1e-8) / float(self.qmax - self.qmin)
            zp = torch.round(float(self.qmin) - x_min / scale)
        return scale, zp

    def freeze(self) -> None:
        """quantizers.py:98-107: in min_max mode the scale and zero point
        become those of the running statistics; the mode becomes frozen."""
        if self.config.mode == "min_max":
            scale, zp = self._scale_zp_from_min_max(self.running_min, self.running_max)
            self.scale = scale.detach().clone()
            self.zero_point = zp.detach().clone()
        self.config.mode = "frozen"

    def observer(self) -> _lib.GsObserver:
        """The quantizer as the C ABI's gs_observer (stats pointer for min_max)."""
        from .gru_layer import _scale_value

        o = _lib.GsObserver()
        o.mode = MODES[self.config.mode]
        o.symmetric = 1 if self.config.symmetric else 0
        o.qmin, o.qmax = int(self.qmin), int(self.qmax)
        if self.config.mode == "frozen":
            o.scale = _scale_value(self.scale)
            o.zero_point = _scale_value(self.zero_point)
        else:
            o.scale, o.zero_point = 1.0, 0.0
        if self.config.mode == "min_max":
            st = self.observer_stats
            if not (st.is_cuda and st.dtype == torch.float32 and st.is_contiguous()):
                raise ValueError("observer_stats must be a contiguous float32 device tensor; move the "
                                 "quantizer to the GPU (module.to(device))")
            o.stats = st.data_ptr()
        return o

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled() and x.requires_grad:
            raise RuntimeError(
                "FakeQuantizePerTensor.forward runs without autograd (calibration and inference); "
                "differentiable QAT uses the frozen (scale, qmin, qmax) tuples of the scans and the input projection"
            )
        return observe_tensor(x, self)

    def extra_repr(self) -> str:
        return f"mode={self.config.mode}, bits={self.config.bits}, symmetric={self.config.symmetric}"


def observe_tensor(x: torch.Tensor, q: FakeQuantizePerTensor) -> torch.Tensor:
    """y = q(x) through gs_observe_tensor on the current stream (no sync)."""
    who = "observe_tensor"
    if not (isinstance(x, torch.Tensor) and x.is_cuda):
        raise ValueError(f"{who}: x must be a CUDA (HIP) tensor")
    if x.dtype != torch.float32:
        raise ValueError(f"{who}: x dtype must be float32; got {x.dtype}")
    if x.dim() == 0 or x.numel() == 0:
        raise ValueError(f"{who}: x must be a non-empty tensor with at least one dimension")
    if q.observer_stats.device != x.device and q.config.mode == "min_max":
        raise ValueError(f"{who}: quantizer stats on {q.observer_stats.device}, x on {x.device}")
    lib = _lib.load()
    xc = x.contiguous()
    cols = xc.shape[-1]
    rows = xc.numel() // cols
    y = torch.empty_like(xc)
    a = _lib.GsObserveTensorArgs()
    a.x, a.y = xc.data_ptr(), y.data_ptr()
    a.rows, a.cols, a.ld = rows, cols, cols
    a.q = q.observer()
    need = lib.gs_observe_tensor_scratch_bytes(ctypes.byref(a))
    if need < 0:
        _lib.raise_for(int(need), lib)
    with _lib.on_device(x.device):
        handle = _lib.current_stream_handle(x.device)
        scratch = torch.empty((int(need),), dtype=torch.uint8, device=x.device)
        a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel()
        rc = lib.gs_observe_tensor(ctypes.byref(a), ctypes.c_void_p(handle))
        del scratch
    _lib.raise_for(rc, lib)
    return y
