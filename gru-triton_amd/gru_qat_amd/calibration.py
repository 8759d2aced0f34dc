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

from typing import Dict, Iterable, List, Tuple, Union

import torch
import torch.nn as nn

from .quantizers import FakeQuantizePerTensor

ACTIVATION_NAMES = (
    "quant_x", "quant_h_in", "quant_h_out",
    "quant_gate_r", "quant_gate_z", "quant_gate_n",
    "quant_struct_Wi_r", "quant_struct_Wi_z", "quant_struct_Wi_n",
    "quant_struct_Wh_r", "quant_struct_Wh_z", "quant_struct_Wh_n",
)


@torch.no_grad()
def calibrate(
    module: nn.Module,
    loader: Iterable[object],
    n_batches: int = 64,
    *,
    only_activations: bool = True,
    verbose: bool = False,
) -> Dict[str, Dict[str, Union[float, List[float], int, bool, None]]]:
    """calibration.py:31-126: every (activation-side, unless
    ``only_activations`` is False) quantizer goes to min_max with fresh
    statistics; the module runs ``n_batches`` batches in eval mode (a tensor
    is ``module(batch)``, a tuple or list ``module(*batch)``, a dict
    ``module(**batch)``); the summary maps each quantizer's qualified name to
    running_min, running_max, bits, axis and initialized. Does not freeze."""
    quantizers: List[Tuple[str, FakeQuantizePerTensor]] = []
    for name, m in module.named_modules():
        if not isinstance(m, FakeQuantizePerTensor):
            continue
        leaf = name.rsplit(".", 1)[-1]
        if only_activations and leaf not in ACTIVATION_NAMES:
            continue
        quantizers.append((name, m))

    for _, m in quantizers:
        m.config.mode = "min_max"
        m.reset_observer()

    was_training = module.training
    module.eval()
    try:
        for i, batch in enumerate(loader):
            if i >= n_batches:
                break
            if isinstance(batch, torch.Tensor):
                module(batch)
            elif isinstance(batch, (tuple, list)):
                module(*batch)
            elif isinstance(batch, dict):
                module(**batch)
            else:
                raise TypeError(
                    f"calibrate: loader yielded unsupported type {type(batch)}; "
                    "expected Tensor / tuple / list / dict"
                )
            if verbose:
                print(f"[calibrate] batch {i + 1}/{n_batches}")
    finally:
        if was_training:
            module.train()

    summary: Dict[str, Dict[str, Union[float, List[float], int, bool, None]]] = {}
    for name, m in quantizers:
        stats = m.observer_stats.detach().cpu()
        summary[name] = {
            "running_min": float(stats[0]),
            "running_max": float(stats[1]),
            "bits": m.config.bits,
            "axis": m.config.axis,
            "initialized": bool(stats[2] != 0.0),
        }
    return summary


def freeze_all(module: nn.Module) -> None:
    """calibration.py:129-135: freeze every quantizer in ``module``."""
    for m in module.modules():
        if isinstance(m, FakeQuantizePerTensor):
            m.freeze()
