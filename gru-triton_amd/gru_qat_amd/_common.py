"""Argument validation shared by the scan wrappers.

Errors are ``ValueError`` (device, dtype, shape, quant tuple) or
``RuntimeError`` (capacity, HIP), never ``AssertionError``, so they survive
``python -O`` (reference contract: tests/test_scan_wrapper_validation.py:47-49).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

QuantTuple = Optional[Tuple[float, int, int]]


def require_cuda(who: str, **tensors: torch.Tensor) -> None:
    dev = None
    for v in tensors.values():  # fast path: every tensor on one CUDA device
        if not (isinstance(v, torch.Tensor) and v.is_cuda):
            break
        if dev is None:
            dev = v.device
        elif v.device != dev:
            break
    else:
        return
    bad = {k: v.device for k, v in tensors.items() if not (isinstance(v, torch.Tensor) and v.is_cuda)}
    if bad:
        devs = ", ".join(f"{k}={v.device if isinstance(v, torch.Tensor) else type(v).__name__}"
                         for k, v in tensors.items())
        names = ", ".join(tensors)
        raise ValueError(f"{who}: {names} must all be CUDA (HIP) tensors; got devices {devs}")
    dev = next(iter(tensors.values())).device
    other = {k: v.device for k, v in tensors.items() if v.device != dev}
    if other:
        raise ValueError(f"{who}: all tensors must be on {dev}; got {other}")


_F32 = torch.float32


def cuda_f32(*tensors) -> bool:
    """Whether every argument is an fp32 tensor on one CUDA device: the common
    case, checked with integer device ordinals (building torch.device objects
    and keyword dicts costs the host a few microseconds a call). Callers run
    require_cuda and require_f32 when it is False, for their exact errors."""
    try:
        d = tensors[0].get_device()
        if d < 0:
            return False
        for t in tensors:
            if t.dtype is not _F32 or t.get_device() != d:
                return False
    except AttributeError:
        return False
    return True


def require_f32(who: str, **tensors: torch.Tensor) -> None:
    for k, v in tensors.items():
        if v.dtype != torch.float32:
            raise ValueError(f"{who}: {k} dtype must be float32; got {v.dtype}")


def split_gi(who: str, gi: torch.Tensor) -> Tuple[int, int, int]:
    if gi.dim() != 3:
        raise ValueError(f"{who}: gi must be [T, B, 3H]; got shape {tuple(gi.shape)}")
    T, B, three_h = gi.shape
    if three_h % 3 != 0 or three_h == 0:
        raise ValueError(f"{who}: gi last dim must be 3*H with H > 0; got {three_h}")
    if T == 0:
        raise ValueError(f"seq length T must be > 0; got T={T}")
    if B == 0:
        raise ValueError(f"batch size B must be > 0; got B={B}")
    return T, B, three_h // 3


def check_common(who: str, gi: torch.Tensor, h0: torch.Tensor, bh_cat: torch.Tensor) -> Tuple[int, int, int]:
    s = gi.shape
    if len(s) == 3:  # fast path: every check passes
        T, B, G3 = s
        if T > 0 and B > 0 and G3 > 0 and G3 % 3 == 0 and h0.shape == (B, G3 // 3) and bh_cat.shape == (G3,):
            return T, B, G3 // 3
    T, B, H = split_gi(who, gi)
    if tuple(h0.shape) != (B, H):
        raise ValueError(f"h0 shape must be (B, H)=({B}, {H}); got {tuple(h0.shape)}")
    if tuple(bh_cat.shape) != (3 * H,):
        raise ValueError(f"bh_cat shape must be (3H,)=({3 * H},); got {tuple(bh_cat.shape)}")
    return T, B, H


def check_quant(q: QuantTuple, name: str) -> QuantTuple:
    if q is None:
        return None
    try:
        scale, qmin, qmax = q
    except (TypeError, ValueError):
        raise ValueError(f"{name} must be None or a (scale, qmin, qmax) tuple; got {q!r}") from None
    scale = float(scale)
    # the kernels' division-free quotient needs 1 / scale normal and code * scale finite
    if not (2.0 ** -126 <= scale <= 2.0 ** 64):
        raise ValueError(f"{name} scale must be in [2^-126, 2^64]; got {scale}")
    if int(qmin) > int(qmax):
        raise ValueError(f"{name} qmin must be <= qmax; got {qmin} > {qmax}")
    return (scale, int(qmin), int(qmax))


# Training forwards of the dense and single-factor Monarch scans store gh
# ([T, B, 3H] fp32, 75 % more saved activations than the reference) so that
# their backward skips the recompute GEMM. set_save_gh(False) turns that off:
# the backward then recomputes gh, as the reference does (scan.py:388-421).
_SAVE_GH = True


def set_save_gh(enabled: bool) -> None:
    """Whether training forwards store gh for the backward (default True)."""
    global _SAVE_GH
    _SAVE_GH = bool(enabled)


def save_gh_default(*tensors: Optional[torch.Tensor]) -> bool:
    """The forward stores gh when the switch is on, grad mode is on and any
    tensor input requires a gradient."""
    return _SAVE_GH and torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)
