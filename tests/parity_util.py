"""Helpers shared by the GPU parity tests (not collected by pytest)."""

from __future__ import annotations

import sys
from typing import Dict, Optional

import torch

from gru_qat_amd.configs import make_config, run_config
from oracle import gru_oracle as O

FP32_TOL = 1e-5  # north-star bound on max |out - oracle| for fp32 outputs and h_T


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_dev(cfg: Dict[str, object], dev: torch.device) -> Dict[str, object]:
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}


def run_both(cfg: Dict[str, object], dev: torch.device):
    """Runs the HIP scan and the CPU oracle on the same inputs; returns (kernel, oracle)."""
    log(f"[parity] {cfg['name']} kind={cfg['kind']} T,B,H={cfg['T']},{cfg['B']},{cfg['H']} "
        f"qin={cfg['h_in_quant'] is not None} qout={cfg['h_out_quant'] is not None} w2={cfg.get('w2') is not None}")
    out = run_config(to_dev(cfg, dev))
    torch.cuda.synchronize(dev)
    return out.cpu(), O.scan_config(cfg)


def assert_fp32_parity(cfg: Dict[str, object], dev: torch.device, tol: float = FP32_TOL) -> float:
    out, ref = run_both(cfg, dev)
    assert out.shape == ref.shape
    assert torch.isfinite(out).all()
    err = (out - ref).abs().max().item()
    err_hT = (out[-1] - ref[-1]).abs().max().item()
    log(f"[parity]   max|out-oracle|={err:.3e} max|hT-oracle|={err_hT:.3e}")
    assert err <= tol, f"max abs err {err:.3e} > {tol:.1e}"
    assert err_hT <= tol
    return err


def assert_fp32_teacher_forced(cfg: Dict[str, object], dev: torch.device, tol: float = FP32_TOL) -> float:
    """For configs with q_in and no q_out: every step within ``tol`` of the
    oracle's step from the kernel's own previous output, so that a q_in
    rounding-boundary flip (the kernel's and the oracle's fp32 states differ by
    ~1e-7, and one level moves the next step by up to ~3e-4) cannot propagate.
    The free-running difference is reported."""
    assert cfg["h_out_quant"] is None
    out, ref = run_both(cfg, dev)
    assert torch.isfinite(out).all()
    pre = O.teacher_forced_prequant(cfg, out)
    err = (out - pre).abs().max().item()
    log(f"[parity]   teacher-forced max|out-oracle|={err:.3e}; free running {(out - ref).abs().max().item():.3e}")
    assert err <= tol, f"max abs err {err:.3e} > {tol:.1e}"
    return err


def assert_quant_parity(cfg: Dict[str, object], dev: torch.device, prequant_tol: float = 2e-6,
                        max_flip_frac: float = 1e-3, free_bound: Optional[float] = None,
                        min_clipped: int = 0) -> Dict[str, float]:
    """Bit-exact codes wherever the pre-quant fp32 values agree.

    Step by step (teacher forcing): the oracle recomputes the pre-q_out state of
    step t from the kernel's own h_{t-1}. Where that value lies farther than
    ``prequant_tol`` from a rounding boundary of q_out, the kernel's code must
    equal the oracle's code exactly; within that band a one-code difference is
    allowed (the two fp32 pre-quant values may straddle the boundary). The
    kernel's output must also be exactly code * scale.

    Free running (kernel and oracle each on their own trajectory): a flip near
    a boundary moves the next step's pre-quant values of every unit the map
    mixes it into, so later codes may differ too. ``free_bound`` bounds that
    divergence, max |out - oracle|, in quantization steps (scale units); with
    no flip the two trajectories must be identical. ``min_clipped`` asserts
    that the in-scan clamp fired at least that many times (codes past qmin or
    qmax before the clamp).
    """
    q = cfg["h_out_quant"]
    assert q is not None
    out, ref_free = run_both(cfg, dev)
    pre = O.teacher_forced_prequant(cfg, out)
    scale = torch.tensor(q[0])
    code_k = torch.round(out / scale)
    assert torch.equal(out, code_k * scale), "kernel output is not code * scale"
    code_o = O.quant_codes(pre, q)
    x = pre / scale
    dist = (x - torch.floor(x) - 0.5).abs() * scale  # distance to nearest boundary, in h units
    near = dist <= prequant_tol
    clipped = (torch.round(x) < q[1]) | (torch.round(x) > q[2])
    mism = code_k != code_o
    hard = mism & ~near
    assert not hard.any(), (
        f"{int(hard.sum())} code mismatches away from rounding boundaries; first at "
        f"{[int(i) for i in hard.nonzero()[0]]}"
    )
    assert ((code_k - code_o).abs() <= 1).all()
    flips = int(mism.sum())
    frac = flips / mism.numel()
    free_diff = int((out != ref_free).sum())
    free_steps = (out - ref_free).abs().max().item() / q[0]
    n_clipped = int(clipped.sum())
    log(f"[parity]   teacher-forced code flips={flips} ({frac:.2e}), all within {prequant_tol:.0e} of a "
        f"boundary; clipped={n_clipped}; free-running: {free_diff} elements differ "
        f"({free_diff / out.numel():.2e}), max {free_steps:.2f} steps")
    assert frac <= max_flip_frac
    assert n_clipped >= min_clipped, f"the in-scan clamp fired {n_clipped} times, expected >= {min_clipped}"
    if free_bound is not None:
        assert free_steps <= free_bound, f"free-running divergence {free_steps:.2f} steps > {free_bound}"
    if flips == 0:
        # every step's code equals the oracle's given the same h_{t-1}, so by
        # induction from h0 the free-running trajectories are identical
        assert free_diff == 0, f"no teacher-forced flip, yet {free_diff} free-running elements differ"
    return {"flips": flips, "free_diff": free_diff, "free_steps": free_steps, "clipped": n_clipped}


def small_cfg(idx: int, shape, seed: int = 0, **over) -> Dict[str, object]:
    cfg = make_config(idx, shape=shape, seed=seed)
    cfg.update(over)
    return cfg
