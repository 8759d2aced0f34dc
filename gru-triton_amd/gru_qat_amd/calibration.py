"""Calibration of the activation quantizers (LarocheC/gru-triton
src/gru_qat/calibration.py:31-126): switch them to min_max, reset their
running statistics, run forwards on a loader, return a summary; freezing is a
separate call (``freeze_all``, calibration.py:129-135).

The forwards run on the HIP observer kernels: a ``ScanLayer`` whose
``use_triton`` is off takes the observer path (``gru_scan_observe``), in
which the hidden quantizers fire every step, as the reference's per-step
path does.
"""

from __future__ import annotations

import contextlib
from typing import Any, Callable, Dict, Iterable, Iterator, List, Tuple, Union

import torch
import torch.nn as nn

from .quantizers import FakeQuantizePerTensor

# Leaf names of the quantizers that watch activations rather than weights
# (the cell's attribute names); calibrate touches only these by default.
ACTIVATION_NAMES = frozenset((
    "quant_x", "quant_h_in", "quant_h_out",
    "quant_gate_r", "quant_gate_z", "quant_gate_n",
    "quant_struct_Wi_r", "quant_struct_Wi_z", "quant_struct_Wi_n",
    "quant_struct_Wh_r", "quant_struct_Wh_z", "quant_struct_Wh_n",
))

Summary = Dict[str, Dict[str, Union[float, List[float], int, bool, None]]]

# How one loader item becomes a forward call.
_CALL_FORMS: Tuple[Tuple[type, Callable[[nn.Module, Any], Any]], ...] = (
    (torch.Tensor, lambda m, b: m(b)),
    (tuple, lambda m, b: m(*b)),
    (list, lambda m, b: m(*b)),
    (dict, lambda m, b: m(**b)),
)


def _quantizers(module: nn.Module, only_activations: bool) -> Iterator[Tuple[str, FakeQuantizePerTensor]]:
    for name, sub in module.named_modules():
        if isinstance(sub, FakeQuantizePerTensor) and (
                not only_activations or name.rpartition(".")[2] in ACTIVATION_NAMES):
            yield name, sub


def _forward(module: nn.Module, batch: Any) -> None:
    for kind, call in _CALL_FORMS:
        if isinstance(batch, kind):
            call(module, batch)
            return
    raise TypeError(f"calibrate: cannot feed a {type(batch).__name__} to the module; the loader must "
                    "yield a Tensor, a tuple or list of arguments, or a dict of keyword arguments")


@contextlib.contextmanager
def _evaluating(module: nn.Module) -> Iterator[None]:
    """eval() for the duration, then the module's own training flag back."""
    restore = module.training
    module.eval()
    try:
        yield
    finally:
        module.train(restore)


def _summarize(chosen: List[Tuple[str, FakeQuantizePerTensor]]) -> Summary:
    if not chosen:
        return {}
    # every quantizer's (running_min, running_max, initialized) in one copy to the host
    stats = torch.stack([q.observer_stats.detach().reshape(-1)[:3].to(torch.float32) for _, q in chosen]).cpu()
    return {name: {"running_min": float(row[0]), "running_max": float(row[1]), "bits": q.config.bits,
                   "axis": q.config.axis, "initialized": bool(row[2] != 0.0)}
            for (name, q), row in zip(chosen, stats)}


@torch.no_grad()
def calibrate(
    module: nn.Module,
    loader: Iterable[object],
    n_batches: int = 64,
    *,
    only_activations: bool = True,
    verbose: bool = False,
) -> Summary:
    """calibration.py:31-126. Puts the chosen quantizers (activation-side by
    default, every one with ``only_activations=False``) into min_max mode with
    empty statistics, runs up to ``n_batches`` loader items through the module
    in eval mode (Tensor: ``module(batch)``; tuple or list: ``module(*batch)``;
    dict: ``module(**batch)``; anything else: TypeError) and returns, per
    quantizer's qualified name, its running_min, running_max, bits, axis and
    initialized flag. Leaves the quantizers unfrozen."""
    chosen = list(_quantizers(module, only_activations))
    for _, q in chosen:
        q.config.mode = "min_max"
        q.reset_observer()
    with _evaluating(module):
        for done, batch in enumerate(loader, start=1):
            if done > n_batches:
                break
            _forward(module, batch)
            if verbose:
                print(f"calibrate: {done} of at most {n_batches} batches seen")
    return _summarize(chosen)


def freeze_all(module: nn.Module) -> None:
    """calibration.py:129-135: freeze every quantizer in ``module``."""
    for m in module.modules():
        if isinstance(m, FakeQuantizePerTensor):
            m.freeze()
