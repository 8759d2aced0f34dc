"""A persistent scan whose bounded wait gives up is never silent.

The condition is forced from the host: the test writes a poll bound of 1 into
the workspace's override word, so the kernels' own bounded waits run out almost
at once while every kernel still exits normally (no fault, no hang); a wait
whose words arrive by its second check still completes, so a launch is
repeated until one gives up. Then:

* every output element written after the failed wait is NaN, and every
  element that is not NaN equals the oracle (no value computed from stale
  inputs passes as valid);
* the next persistent launch on that stream raises ``PersistentScanFault`` (a
  ``RuntimeError``), read from the pinned host mirror without synchronising;
* the launch after that is correct again: the fault word names the launch that
  raised it, so it cuts no later launch's waits short;
* a stale value planted in the fault word does not disturb a launch.
"""

from __future__ import annotations

import contextlib

import pytest
import torch

import gru_qat_amd
from gru_qat_amd import _lib
from gru_qat_amd.configs import make_config, run_config
from gru_qat_amd.scan import gru_scan_backward_persistent
from oracle import gru_oracle as O
from parity_util import FP32_TOL, log, to_dev

pytestmark = pytest.mark.gpu

SPIN_WORD = 16  # control word holding the poll bound override (0 = default)
FAULT_WORD = 0


def _words(dev: torch.device) -> torch.Tensor:
    handle = torch.cuda.current_stream(dev).cuda_stream
    return _lib._ws_cache[(dev.index, handle)].view(torch.int32)


@contextlib.contextmanager
def poll_bound_of_one(dev: torch.device):
    """Launches queued inside the block run with a poll bound of 1; the
    override is cleared on the way out whatever happens inside."""
    words = _words(dev)
    words[SPIN_WORD] = 1  # queued on the stream before the next launch
    try:
        yield
    finally:
        words[SPIN_WORD] = 0
        torch.cuda.synchronize(dev)


def _cases():
    # dense remote mode (8 workgroups per group), two-factor Monarch fused (nb | bs)
    # and split (nb does not divide bs) kernels
    dense = make_config(1, shape=(16, 8, 512))
    fused = make_config(3, shape=(12, 8, 512))
    fused.update(h_in_quant=None, h_out_quant=None)
    split = make_config(3, shape=(8, 5, 240), seed=2)
    g = torch.Generator().manual_seed(5)
    nb, bs = 5, 48
    split["w"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
    split["w2"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
    split.update(h_in_quant=None, h_out_quant=None)
    return {"dense": dense, "monarch2_fused": fused, "monarch2_split": split}


CASES = _cases()


def _check_partial(out: torch.Tensor, ref: torch.Tensor) -> int:
    nan = torch.isnan(out)
    keep = ~nan
    assert keep.any() or nan.all()
    if keep.any():
        err = (out[keep] - ref[keep]).abs().max().item()
        assert err <= FP32_TOL, f"a value written before the give-up differs from the oracle by {err:.3e}"
    return int(nan.sum())


@pytest.mark.parametrize("name", list(CASES))
def test_forward_give_up_is_nan_then_raises(dev, name):
    cfg = CASES[name]
    d = to_dev(cfg, dev)
    ref = O.scan_config(cfg)
    log(f"[faults] {name}: normal launch")
    out = run_config(d)
    torch.cuda.synchronize(dev)
    assert (out.cpu() - ref).abs().max().item() <= FP32_TOL
    # A wait gives up only when its words are not there by the second check, so
    # a small grid can get through a launch without one; repeat until one does.
    # A launch that did not give up must be exact and leave the fault word clear.
    n_nan = 0
    for attempt in range(20):
        log(f"[faults] {name}: launch with a poll bound of 1 (attempt {attempt})")
        with poll_bound_of_one(dev):
            out = run_config(d)
        n_nan = _check_partial(out.cpu(), ref)
        log(f"[faults] {name}: {n_nan} of {out.numel()} outputs NaN")
        if n_nan:
            break
        assert gru_qat_amd.workspace_faults(dev) == 0, "a launch with no NaN output reported a give-up"
    assert n_nan > 0, "20 launches with a poll bound of 1 never gave up a wait"
    with pytest.raises(gru_qat_amd.PersistentScanFault):
        run_config(d)
    assert issubclass(gru_qat_amd.PersistentScanFault, RuntimeError)
    out = run_config(d)
    torch.cuda.synchronize(dev)
    err = (out.cpu() - ref).abs().max().item()
    log(f"[faults] {name}: launch after the fault: max|out-oracle|={err:.3e}")
    assert err <= FP32_TOL
    assert gru_qat_amd.workspace_faults(dev) == 1  # the word still names the faulted launch
    assert gru_qat_amd.workspace_faults(dev) == 0


def test_backward_give_up_is_nan_then_raises(dev):
    cfg = make_config(1, shape=(12, 8, 512))
    d = {k: cfg[k].to(dev) for k in ("gi", "h0", "w", "bh")}
    out = gru_qat_amd.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"])
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(1)).to(dev)
    torch.cuda.synchronize(dev)
    ref = O.scan_backward(cfg, out.cpu(), dout.cpu())
    for attempt in range(20):
        log(f"[faults] dense backward with a poll bound of 1 (attempt {attempt})")
        with poll_bound_of_one(dev):
            grads = gru_scan_backward_persistent(d["gi"], d["h0"], d["w"], d["bh"], out, dout)
        dgi = grads[0].cpu()
        if torch.isnan(dgi).any():
            break
        assert gru_qat_amd.workspace_faults(dev) == 0, "a launch with no NaN gradient reported a give-up"
    assert torch.isnan(dgi).any(), "20 launches with a poll bound of 1 never gave up a wait"
    with pytest.raises(gru_qat_amd.PersistentScanFault):
        gru_scan_backward_persistent(d["gi"], d["h0"], d["w"], d["bh"], out, dout)
    grads = gru_scan_backward_persistent(d["gi"], d["h0"], d["w"], d["bh"], out, dout)
    torch.cuda.synchronize(dev)
    for k, g in zip(("dgi", "dh0", "dw", "dbh"), grads):
        r = ref[k]
        err = (g.cpu() - r).abs().max().item()
        assert err <= 1e-4 * max(1.0, r.abs().max().item()), f"{k}: {err:.3e}"
    gru_qat_amd.workspace_faults(dev)


@pytest.mark.parametrize("name", ["dense", "monarch2_fused"])
def test_stale_fault_word_does_not_disturb_a_launch(dev, name):
    cfg = CASES[name]
    d = to_dev(cfg, dev)
    ref = O.scan_config(cfg)
    run_config(d)
    torch.cuda.synchronize(dev)
    words = _words(dev)
    try:
        for stale in (1, 12345, -1):
            words[FAULT_WORD] = stale
            out = run_config(d)
            torch.cuda.synchronize(dev)
            err = (out.cpu() - ref).abs().max().item()
            log(f"[faults] {name}: stale fault word {stale}: max|out-oracle|={err:.3e}")
            assert err <= FP32_TOL
        gru_qat_amd.check_faults(dev)
    finally:
        words[FAULT_WORD] = 0
