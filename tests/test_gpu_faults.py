"""A persistent scan whose bounded wait gives up is never silent.

The condition is forced from the host, deterministically: the test writes
into the workspace's poll-bound override word a small bound and a step F whose
exchange the kernels treat as late (the waits that check it see every word of
tag tag_base + F as not yet arrived: the XCD-id exchange, tag tag_base + 1,
which the dense and fused two-factor kernels and the dense backward run with
their first exchange, and every exchange of the split two-factor kernel), so
exactly that exchange runs out through the kernels' own bounded waits while
every kernel still exits normally (no fault, no hang). Then:

* the outputs up to the forced exchange equal the oracle, and every output
  element from it on is NaN (no value computed from stale inputs passes as
  valid);
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


BOUND = 4096   # polls before a wait gives up: far more than an on-time exchange takes


@contextlib.contextmanager
def forced_late_exchange(dev: torch.device, step: int, bound: int = BOUND):
    """Launches queued inside the block run with exchange `step` forced late
    and a poll bound of `bound`; the override is cleared on the way out
    whatever happens inside."""
    words = _words(dev)
    words[SPIN_WORD] = (step << 24) | bound  # queued on the stream before the next launch
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


# The exchange forced late per kernel and the first step whose output is then
# NaN. Dense and fused: F = 1, the XCD-id exchange that runs with the first
# exchange of q_in(h_0), which step 1 needs. Split: F = 2, the z exchange of
# step 1 (its second exchange of step t carries tag tag_base + t + 1).
FORCED = {"dense": 1, "monarch2_fused": 1, "monarch2_split": 2}
FIRST_NAN = {"dense": 1, "monarch2_fused": 1, "monarch2_split": 1}


@pytest.mark.parametrize("name", list(CASES))
def test_forward_give_up_is_nan_then_raises(dev, name):
    cfg = CASES[name]
    d = to_dev(cfg, dev)
    ref = O.scan_config(cfg)
    log(f"[faults] {name}: normal launch")
    out = run_config(d)
    torch.cuda.synchronize(dev)
    assert (out.cpu() - ref).abs().max().item() <= FP32_TOL
    log(f"[faults] {name}: launch with exchange {FORCED[name]} forced late")
    with forced_late_exchange(dev, FORCED[name]):
        out = run_config(d)
    out = out.cpu()
    s = FIRST_NAN[name]
    log(f"[faults] {name}: {int(torch.isnan(out).sum())} of {out.numel()} outputs NaN")
    assert not torch.isnan(out[:s]).any(), "an output before the forced exchange is NaN"
    assert (out[:s] - ref[:s]).abs().max().item() <= FP32_TOL
    assert torch.isnan(out[s:]).all(), "an output from the forced exchange on is not NaN"
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


@pytest.mark.parametrize("name", list(CASES))
def test_bound_alone_gives_no_fault(dev, name):
    """The bound the forced test uses, with no exchange forced: every wait is
    met long before it, so the launch is exact and raises nothing."""
    cfg = CASES[name]
    d = to_dev(cfg, dev)
    ref = O.scan_config(cfg)
    with forced_late_exchange(dev, step=0):
        out = run_config(d)
    assert (out.cpu() - ref).abs().max().item() <= FP32_TOL
    assert gru_qat_amd.workspace_faults(dev) == 0


def test_backward_give_up_is_nan_then_raises(dev):
    """The dense backward's recurrence walks t down from T - 1; its first
    exchange (with the XCD-id words, tag tag_base + 1, forced late here)
    carries D_{T-2}, which reverse step 1 needs, so the gradients of steps
    T-2 and T-1 are exact and those of steps 0 .. T-3 (and dh0) NaN."""
    FORCED = 1
    cfg = make_config(1, shape=(12, 8, 512))
    T = cfg["T"]
    d = {k: cfg[k].to(dev) for k in ("gi", "h0", "w", "bh")}
    out = gru_qat_amd.gru_scan_forward_persistent(d["gi"], d["h0"], d["w"], d["bh"])
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(1)).to(dev)
    torch.cuda.synchronize(dev)
    ref = O.scan_backward(cfg, out.cpu(), dout.cpu())
    log(f"[faults] dense backward with exchange {FORCED} forced late")
    with forced_late_exchange(dev, FORCED):
        grads = gru_scan_backward_persistent(d["gi"], d["h0"], d["w"], d["bh"], out, dout)
    dgi, dh0 = grads[0].cpu(), grads[1].cpu()
    keep = T - 1 - FORCED
    assert torch.isnan(dgi[:keep]).all() and torch.isnan(dh0).all()
    assert not torch.isnan(dgi[keep:]).any()
    bar = 1e-4 * max(1.0, ref["dgi"].abs().max().item())
    assert (dgi[keep:] - ref["dgi"][keep:]).abs().max().item() <= bar
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
