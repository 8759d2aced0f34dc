"""Scan dispatch of the reference ``GRULayer`` (LarocheC/gru-triton
src/gru_qat/gru_layer.py), restated around this build's scans.

The reference layer sends a forward to ``_forward_fast_dispatch``
(gru_layer.py:234-302) when ``use_triton`` resolves to True
(gru_layer.py:110-124): the input projection builds ``gi [T, B, 3H]`` and one
scan entry point consumes it with the hidden quantizers' frozen parameters.
This module keeps the parts of that path that decide and feed the scan:

* ``_extract_h_quant_params`` -- gru_layer.py:30-48;
* ``fast_dispatch_eligible`` and ``resolve_use_triton`` -- the eligibility
  rule and the ``use_triton`` argument contract of gru_layer.py:110-124;
* ``forward_fast_dispatch`` -- gru_layer.py:183-192 (T/B checks, zero h0)
  and :260-302 (kind switch, ``h_T = out[-1]`` taken before the batch_first
  transpose);
* ``layer_forward`` -- GRULayer.forward (gru_layer.py:153-200) with a dense
  input side, through ``_forward_fast_dispatch`` (:234-302): x to time-major,
  the input projection (``input_projection``, :249-255), the scan.

* ``ScanLayer`` -- GRULayer's forward, calibrate and freeze (gru_layer.py:52-65,
  :153-302, :308-342) around these scans, with weights given as tensors and
  per-tensor quantizers (``quantizers.FakeQuantizePerTensor``); its
  calibration forwards run on the observer kernels (``observe``).

The cell module is not part of this build; ``layer_forward`` callers pass the
extracted weights (``extract_*`` helpers of the scan modules) and the frozen
quant tuples.
"""

from __future__ import annotations

import weakref
from typing import Any, Optional, Tuple

import torch

from ._common import QuantTuple

FAST_DISPATCH_KINDS = ("diagonal", "monarch", "butterfly")
# Hidden kinds this build also scans on the GPU, which the reference sends to
# its per-step loop (gru_layer.py:109-113).
EXTENDED_KINDS = ("dense", "circulant")


_SCALE_CACHE: "weakref.WeakKeyDictionary[Any, Tuple[int, int, float]]" = weakref.WeakKeyDictionary()


def _scale_value(scale: torch.Tensor) -> float:
    """``float(scale.item())``, read once per version of the tensor: a frozen
    scale is not written again, so later forwards skip the device-to-host
    sync that the reference pays on every call (gru_layer.py:48). Any
    in-place write bumps ``scale._version`` and forces a fresh read."""
    key = (scale.data_ptr(), scale._version)
    hit = _SCALE_CACHE.get(scale)
    if hit is not None and hit[:2] == key:
        return hit[2]
    value = float(scale.item())
    _SCALE_CACHE[scale] = (key[0], key[1], value)
    return value


def _extract_h_quant_params(quantizer: Any) -> QuantTuple:
    """``(scale, qmin, qmax)`` of a frozen, per-tensor, symmetric quantizer,
    else None (the scan then runs without in-kernel fake-quant).

    Mirrors gru_layer.py:30-48. The reference tests
    ``isinstance(quantizer, FakeQuantizePerTensor)``; the quantizer classes
    are not part of this build, so per-tensor is read from the quantizer's
    config (``config.axis is None``, the reference's per-tensor config) and a
    one-element scale. The reference reads the scale with ``.item()`` on
    every forward; here the value is cached per tensor version
    (``_scale_value``), so a frozen device scale costs one sync, not one per
    call.
    """
    cfg = quantizer.config
    if cfg.mode != "frozen":
        return None
    if getattr(cfg, "axis", None) is not None or quantizer.scale.numel() != 1:
        return None
    if not cfg.symmetric:
        return None
    scale = quantizer.scale
    value = _scale_value(scale) if isinstance(scale, torch.Tensor) else float(scale)
    return (value, int(quantizer.qmin), int(quantizer.qmax))


def fast_dispatch_eligible(kind: Optional[str], gate_layout: str, *, extended: bool = False) -> bool:
    """gru_layer.py:110-113: the hidden structure kind is diagonal, monarch or
    butterfly and the gate layout is fused (gi is one [T, B, 3H] tensor).

    ``extended=True`` adds EXTENDED_KINDS, the dense and circulant hidden
    kinds, which this build scans on the GPU too (the reference sends them to
    its per-step loop); the default is the reference's rule."""
    kinds = FAST_DISPATCH_KINDS + (EXTENDED_KINDS if extended else ())
    return kind in kinds and gate_layout == "fused"


def resolve_use_triton(use_triton: Any, kind: Optional[str], gate_layout: str, *,
                       extended: bool = False) -> bool:
    """gru_layer.py:115-124: "auto" follows eligibility; a truthy value on an
    ineligible configuration raises ValueError; falsy disables dispatch.
    ``extended`` as in ``fast_dispatch_eligible``."""
    eligible = fast_dispatch_eligible(kind, gate_layout, extended=extended)
    if use_triton == "auto":
        return eligible
    use = bool(use_triton)
    if use and not eligible:
        raise ValueError(
            "use_triton=True requires structure_hidden.kind in {'diagonal', 'monarch', 'butterfly'} "
            "and gate_layout='fused'."
        )
    return use


def forward_fast_dispatch(
    kind: str,
    gi: torch.Tensor,
    h0: Optional[torch.Tensor],
    hidden: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
    batch_first: bool = False,
    hidden2: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Runs the scan of ``kind`` on ``gi [T, B, 3H]`` (time-major, as the
    reference builds it after its batch_first transpose) and returns
    ``(out, h_T)``: out is [T, B, H], or [B, T, H] when ``batch_first``;
    h_T = out[-1] of the time-major result.

    ``hidden`` is Wh_diag [3, H] (diagonal), Wh_struct [3, nb, bs, bs]
    (monarch; ``hidden2`` the optional second factor), twiddles (butterfly),
    or, for the kinds this build adds (the reference routes them to its
    per-step loop), Wh_cat [3H, H] (dense) or Wh_circ [3, H] (circulant). ``h0`` None means
    zeros, as in gru_layer.py:191-192. An unknown kind raises RuntimeError
    (gru_layer.py:294-297).
    """
    if gi.dim() != 3:
        raise ValueError(f"gi must be [T, B, 3H]; got shape {tuple(gi.shape)}")
    T, B, threeH = gi.shape
    if T == 0:
        raise ValueError(f"seq length T must be > 0; got T={T}")
    if B == 0:
        raise ValueError(f"batch size B must be > 0; got B={B}")
    if h0 is None:
        h0 = gi.new_zeros(B, threeH // 3)
    kw = dict(h_in_quant=h_in_quant, h_out_quant=h_out_quant)
    if kind == "diagonal":
        from .scan_diagonal import gru_scan_diagonal

        out = gru_scan_diagonal(gi, h0, hidden, bh_cat, **kw)
    elif kind == "monarch":
        from .scan_monarch import gru_scan_monarch

        out = gru_scan_monarch(gi, h0, hidden, bh_cat, Wh_struct2=hidden2, **kw)
    elif kind == "butterfly":
        from .scan_butterfly import gru_scan_butterfly_triton

        out = gru_scan_butterfly_triton(gi, h0, hidden, bh_cat, **kw)
    elif kind == "dense":
        from .scan import gru_scan_persistent

        out = gru_scan_persistent(gi, h0, hidden, bh_cat, **kw)
    elif kind == "circulant":
        from .scan_circulant import gru_scan_circulant

        out = gru_scan_circulant(gi, h0, hidden, bh_cat, **kw)
    else:
        raise RuntimeError(f"unexpected dispatch kind {kind!r}")
    h_T = out[-1]
    if batch_first:
        out = out.transpose(0, 1)
    return out, h_T


def layer_forward(
    kind: str,
    x: torch.Tensor,
    h0: Optional[torch.Tensor],
    Wi_cat: torch.Tensor,
    bi_cat: Optional[torch.Tensor],
    hidden: torch.Tensor,
    bh_cat: torch.Tensor,
    *,
    x_quant: QuantTuple = None,
    w_quant: Optional[Tuple[int, int]] = None,
    h_in_quant: QuantTuple = None,
    h_out_quant: QuantTuple = None,
    batch_first: bool = False,
    hidden2: Optional[torch.Tensor] = None,
    input_kind: Optional[str] = None,
    wi_out_quant: Any = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """GRULayer's forward on the fast dispatch:
    ``x`` [T, B, I] (or [B, T, I] when ``batch_first``) -> ``(out, h_T)``.

    Follows gru_layer.py:169-200 (time-major x, T/B checks, zero h0) and
    :249-302. A dense input side (``input_kind`` None) gives
    ``gi = input_projection(x, Wi_cat, bi_cat, x_quant=..., w_quant=...)``
    (the reference's ``quant_x`` + ``quantize_input_weights`` + ``F.linear``,
    :249-255); a structured one (``input_kind`` "diagonal", "monarch" or
    "butterfly", ``Wi_cat`` then holding the stacked per-gate weights and
    ``wi_out_quant`` the output-side quantizers) gives
    ``gi = structured_input_projection(...)`` (``cell.structured_input_projection``,
    :256). Then the scan of ``kind`` (``forward_fast_dispatch``).
    Differentiable in x, h0 and every weight.
    """
    from .input_proj import input_projection
    from .struct_proj import structured_input_projection

    if x.dim() != 3:
        raise ValueError(f"x must be [T, B, I] (or [B, T, I] with batch_first); got shape {tuple(x.shape)}")
    if batch_first:
        x = x.transpose(0, 1)
    T, B, _ = x.shape
    if T == 0:
        raise ValueError(f"seq length T must be > 0; got T={T}")
    if B == 0:
        raise ValueError(f"batch size B must be > 0; got B={B}")
    if input_kind is None:
        gi = input_projection(x, Wi_cat, bi_cat, x_quant=x_quant, w_quant=w_quant)
    else:
        if w_quant is not None:
            raise ValueError("w_quant is the dense input side's weight quantizer; a structured input side "
                             "quantizes its outputs (wi_out_quant)")
        gi = structured_input_projection(x, input_kind, Wi_cat, bi_cat, x_quant=x_quant, out_quant=wi_out_quant)
    return forward_fast_dispatch(kind, gi, h0, hidden, bh_cat, h_in_quant=h_in_quant, h_out_quant=h_out_quant,
                                 batch_first=batch_first, hidden2=hidden2)



class ScanLayer(torch.nn.Module):
    """GRULayer's forward, calibrate and freeze around this build's scans, with
    the weights given as tensors instead of a cell (the cell and its recipe
    are not part of this build).

    Follows gru_layer.py: the ``use_triton`` and ``batch_first`` arguments
    (:52-65, resolved by ``resolve_use_triton`` as :110-124 with
    ``extended=True``: the dense and circulant kinds have fast scans here, so
    "auto" dispatches them too; a reference ``GRULayer`` keeps the reference
    rule),
    ``forward`` (:153-302), ``calibrate`` (:308-336) and ``freeze``
    (:338-339).

    * ``kind``: "dense", "diagonal", "monarch" or "butterfly"; ``Wi_cat``
      [3H, I] (or, with ``input_kind`` set, the stacked structured input
      weights of that kind, input size H, and ``wi_out_quant`` the per-gate
      output quantizers of ``structured_input_projection``), ``bi_cat`` [3H]
      or None, ``hidden`` (and ``hidden2``) and
      ``bh_cat`` as in ``forward_fast_dispatch``. They become parameters.
    * ``x_quant`` and ``h_quant``: ``QuantizerConfig`` of the per-tensor
      ``quant_x`` and of ``quant_h_in`` and ``quant_h_out`` (both built from
      one config, as the reference builds both from recipe.hidden,
      gru_cell.py:191-193), or None for no quantizer. ``w_bits``: the per-row
      symmetric input-weight fake-quant (quantize_input_weights), or None.

    With ``use_triton`` on, ``forward`` is the fast dispatch: quant_x is
    applied to the whole sequence, and the hidden quantizers reach the scan
    kernel only when frozen, per-tensor and symmetric (gru_layer.py:30-48);
    otherwise the scan runs without them, as in the reference. With it off,
    ``forward`` is the per-step path with every quantizer firing (the input
    projected once over the sequence, as with the reference's pre_batch_input)
    on the observer kernels (``gru_scan_observe``); that path has no autograd.
    """

    def __init__(self, kind: str, Wi_cat: torch.Tensor, bi_cat: Optional[torch.Tensor], hidden: torch.Tensor,
                 bh_cat: torch.Tensor, *, hidden2: Optional[torch.Tensor] = None, x_quant: Any = None,
                 h_quant: Any = None, w_bits: Optional[int] = None, use_triton: Any = "auto",
                 batch_first: bool = False, input_kind: Optional[str] = None, wi_out_quant: Any = None) -> None:
        super().__init__()
        from .quantizers import FakeQuantizePerTensor, QuantizerConfig

        if kind not in EXTENDED_KINDS + FAST_DISPATCH_KINDS:
            raise ValueError(f"kind must be one of dense, diagonal, monarch, butterfly, circulant; got {kind!r}")
        if input_kind is not None and input_kind not in FAST_DISPATCH_KINDS:
            raise ValueError(f"input_kind must be None (dense) or one of diagonal, monarch, butterfly; "
                             f"got {input_kind!r}")
        if input_kind is not None and w_bits is not None:
            raise ValueError("w_bits quantizes a dense input weight; a structured input side quantizes its "
                             "outputs (wi_out_quant)")
        self.kind = kind
        self.input_kind = input_kind
        self.wi_out_quant = wi_out_quant
        self.Wi_cat = torch.nn.Parameter(Wi_cat.detach().clone())
        self.bi_cat = torch.nn.Parameter(bi_cat.detach().clone()) if bi_cat is not None else None
        self.hidden = torch.nn.Parameter(hidden.detach().clone())
        self.hidden2 = torch.nn.Parameter(hidden2.detach().clone()) if hidden2 is not None else None
        self.bh_cat = torch.nn.Parameter(bh_cat.detach().clone())
        self.hidden_size = bh_cat.shape[0] // 3

        def make(cfg: Any) -> Optional[FakeQuantizePerTensor]:
            if cfg is None:
                return None
            from copy import deepcopy

            return FakeQuantizePerTensor(deepcopy(cfg) if isinstance(cfg, QuantizerConfig) else QuantizerConfig(**cfg))

        self.quant_x = make(x_quant)
        self.quant_h_in = make(h_quant)
        self.quant_h_out = make(h_quant)
        if w_bits is not None and not (2 <= int(w_bits) <= 16):
            raise ValueError(f"w_bits must be in [2, 16] or None; got {w_bits}")
        self.w_quant = None if w_bits is None else (-(2 ** (int(w_bits) - 1)) + 1, 2 ** (int(w_bits) - 1) - 1)
        self.use_triton = resolve_use_triton(use_triton, kind, "fused", extended=True)
        self.batch_first = batch_first

    def _x_side(self, x: torch.Tensor) -> Tuple[torch.Tensor, QuantTuple]:
        """quant_x on the fast dispatch: a frozen symmetric per-tensor quantizer
        goes to the input projection as a tuple (differentiable, fused into
        the GEMM's operand load); any other runs on the observer kernel."""
        q = self.quant_x
        if q is None:
            return x, None
        frozen = _extract_h_quant_params(q)
        if frozen is not None:
            return x, frozen
        return q(x), None

    def forward(self, x: torch.Tensor, h0: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if not self.use_triton:
            return self._forward_observe(x, h0)
        xin, x_tuple = self._x_side(x)
        h_in = _extract_h_quant_params(self.quant_h_in) if self.quant_h_in is not None else None
        h_out = _extract_h_quant_params(self.quant_h_out) if self.quant_h_out is not None else None
        return layer_forward(self.kind, xin, h0, self.Wi_cat, self.bi_cat, self.hidden, self.bh_cat,
                             x_quant=x_tuple, w_quant=self.w_quant, h_in_quant=h_in, h_out_quant=h_out,
                             batch_first=self.batch_first, hidden2=self.hidden2, input_kind=self.input_kind,
                             wi_out_quant=self.wi_out_quant)

    def _forward_observe(self, x: torch.Tensor, h0: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
        from .input_proj import input_projection
        from .observe import gru_scan_observe

        if x.dim() != 3:
            raise ValueError(f"x must be [T, B, I] (or [B, T, I] with batch_first); got shape {tuple(x.shape)}")
        if self.batch_first:
            x = x.transpose(0, 1)
        T, B, _ = x.shape
        if T == 0:
            raise ValueError(f"seq length T must be > 0; got T={T}")
        if B == 0:
            raise ValueError(f"batch size B must be > 0; got B={B}")
        with torch.no_grad():
            if h0 is None:
                h0 = x.new_zeros(B, self.hidden_size)
            xin = self.quant_x(x) if self.quant_x is not None else x
            if self.input_kind is None:
                gi = input_projection(xin, self.Wi_cat, self.bi_cat, x_quant=None, w_quant=self.w_quant)
            else:
                from .struct_proj import structured_input_projection

                gi = structured_input_projection(xin, self.input_kind, self.Wi_cat, self.bi_cat,
                                                 out_quant=self.wi_out_quant)
            out = gru_scan_observe(self.kind, gi, h0, self.hidden, self.bh_cat, quant_h_in=self.quant_h_in,
                                   quant_h_out=self.quant_h_out, hidden2=self.hidden2)
        h_T = out[-1]
        if self.batch_first:
            out = out.transpose(0, 1)
        return out, h_T

    @torch.no_grad()
    def calibrate(self, loader: Any, n_batches: int = 64, *, only_activations: bool = True) -> dict:
        """gru_layer.py:308-336: runs ``calibration.calibrate`` with use_triton
        off, so that the hidden quantizers fire every step; does not freeze."""
        from .calibration import calibrate as _calibrate

        saved = self.use_triton
        self.use_triton = False
        try:
            return _calibrate(self, loader, n_batches=n_batches, only_activations=only_activations)
        finally:
            self.use_triton = saved

    def freeze(self) -> None:
        """gru_layer.py:338-339 (cell.freeze_quantizers, gru_cell.py:538-549):
        every quantizer of the layer goes to frozen mode."""
        from .calibration import freeze_all

        freeze_all(self)

    def export_int_weights(self, bits: int = 8) -> dict:
        """int8 weight codes, scales and zero points plus the frozen activation
        scales (the export gru_cell.py:551-553 leaves as a TODO); see
        ``export.export_int_weights``."""
        from .export import export_int_weights

        return export_int_weights(self, bits)
