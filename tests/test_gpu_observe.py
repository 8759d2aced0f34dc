"""GPU parity of the observer path (calibration): the dense form of every
hidden map, the tensor quantizer and the observer scan through the C ABI,
against the oracle's restatement of the reference's per-step path with its
quantizers firing (quantizers.py:63-156, gru_layer.py:205-223, 308-342).

Bars: maps and fp32 outputs within 1e-5 (maps 1e-6); scales, zero points and
running statistics bit-exact where the kernel and the oracle reduce the same
tensor (the kernel's own h_{t-1}), within 1e-5 relative where they reduce a
pre-quant state computed twice (GEMM vs F.linear); codes bit-exact wherever
the pre-quant value lies farther than 2e-6 from a rounding boundary (teacher
forcing: each step restarts from the kernel's own previous output)."""

from __future__ import annotations

import math

import pytest
import torch

import gru_qat_amd as G
from gru_qat_amd.configs import make_config
from oracle import gru_oracle as O
from parity_util import log, to_dev

pytestmark = pytest.mark.gpu

SHAPES = {0: (8, 4, 64), 1: (8, 4, 64), 2: (6, 5, 100), 3: (8, 4, 64), 4: (6, 3, 64)}
BIG = {1: (4, 32, 512), 4: (3, 64, 1024)}


def _cfg(idx, shape=None, seed=0):
    return make_config(idx, shape=shape if shape is not None else SHAPES[idx], seed=seed)


def _run(cfg, dev, q_in=None, q_out=None, trace=True):
    d = to_dev(cfg, dev)
    log(f"[observe] {cfg['name']} kind={cfg['kind']} T,B,H={cfg['T']},{cfg['B']},{cfg['H']} "
        f"q_in={None if q_in is None else q_in.config.mode} q_out={None if q_out is None else q_out.config.mode}")
    with torch.no_grad():
        res = G.gru_scan_observe(cfg["kind"], d["gi"], d["h0"], d["w"], d["bh"], quant_h_in=q_in, quant_h_out=q_out,
                                 hidden2=d.get("w2"), return_trace=trace)
    torch.cuda.synchronize(dev)
    return res


@pytest.mark.parametrize("idx", [0, 1, 3, 4])
def test_hidden_map_dense(dev, idx):
    cfg = _cfg(idx)
    d = to_dev(cfg, dev)
    M = G.hidden_map_dense(cfg["kind"], d["w"], cfg["H"], hidden2=d.get("w2")).cpu()
    ref = O.materialize_hidden(cfg)
    err = (M - ref).abs().max().item()
    log(f"[observe] map {cfg['name']}: max err {err:.2e}")
    assert err <= 1e-6
    if idx in (0, 1):
        assert torch.equal(M, ref)


def test_hidden_map_butterfly_large(dev):
    cfg = make_config(4, shape=(1, 1, 1024))
    M = G.hidden_map_dense("butterfly", cfg["w"].to(dev), 1024).cpu()
    ref = O.materialize_hidden(cfg)
    assert (M - ref).abs().max().item() <= 1e-5 * max(1.0, ref.abs().max().item())


@pytest.mark.parametrize("idx", [0, 1, 2, 3, 4])
def test_observe_without_quantizers_is_the_scan(dev, idx):
    cfg = _cfg(idx)
    cfg["h_in_quant"] = cfg["h_out_quant"] = None
    out, trace = _run(cfg, dev)
    ref = O.scan_config(cfg)
    err = (out.cpu() - ref).abs().max().item()
    log(f"[observe]   max|out-oracle|={err:.2e}")
    assert err <= 1e-5
    assert torch.all(trace.cpu() == torch.tensor([1.0, 0.0, 1.0, 0.0]))


def _frozen(scale):
    q = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="frozen"))
    q.scale = torch.tensor(scale)
    return q


def _codes_match(out_t, pre_t, s, zp, qmin, qmax, tol=2e-6):
    """Kernel codes equal the oracle's wherever the pre-quant value is farther
    than tol from a rounding boundary; returns the number of flips."""
    ck = torch.round(out_t / s + zp)
    assert torch.allclose((ck - zp) * s, out_t, rtol=0, atol=1e-6 * max(1.0, abs(s) * 256)), "not on the grid"
    x = pre_t / s + zp
    co = torch.clamp(torch.round(x), qmin, qmax)
    near = (x - torch.floor(x) - 0.5).abs() * s <= tol
    mism = ck != co
    assert not (mism & ~near).any(), f"{int((mism & ~near).sum())} code mismatches away from boundaries"
    return int(mism.sum())


@pytest.mark.parametrize("idx", [2, 3])
def test_observe_frozen_matches_frozen_scan(dev, idx):
    cfg = _cfg(idx)
    s = cfg["h_out_quant"][0]
    out, trace = _run(cfg, dev, _frozen(s), _frozen(s))
    out = out.cpu()
    assert torch.all(trace.cpu()[:, [0, 2]] == s)
    pre = O.teacher_forced_prequant(cfg, out)
    flips = _codes_match(out, pre, s, 0.0, -127, 127)
    log(f"[observe]   frozen: teacher-forced flips={flips}")


def _teacher_forced(cfg, out_k, st_in, st_out):
    """Per step from the kernel's own h_{t-1}: the oracle's q_in (scale, zp) and
    observer update on h_{t-1}, the pre-quant h_t and q_out's (scale, zp) and
    update on it. Returns (pre [T, B, H], scales [T, 4])."""
    c = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}
    gh_fn = O.gh_fn_for(c)
    T = c["gi"].shape[0]
    pre = torch.empty_like(out_k)
    sc = torch.empty(T, 4)
    for t in range(T):
        h = c["h0"] if t == 0 else out_k[t - 1]
        hq, (si, zi) = O.observer_forward(st_in, h)
        p = O.gru_step(c["gi"][t], h, gh_fn(hq))
        _, (so, zo) = O.observer_forward(st_out, p)
        pre[t] = p
        sc[t] = torch.tensor([si, zi, so, zo])
    return pre, sc


def _quant(mode, symmetric):
    return G.FakeQuantizePerTensor(G.QuantizerConfig(mode=mode, symmetric=symmetric))


@pytest.mark.parametrize("idx", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("mode,symmetric", [("min_max", True), ("dynamic", True), ("min_max", False)])
def test_observe_dynamic_teacher_forced(dev, idx, mode, symmetric):
    cfg = _cfg(idx)
    q_in, q_out = _quant(mode, symmetric).to(dev), _quant(mode, symmetric).to(dev)
    out, trace = _run(cfg, dev, q_in, q_out)
    out, trace = out.cpu(), trace.cpu()
    st_in = O.ObserverState(mode, symmetric=symmetric)
    st_out = O.ObserverState(mode, symmetric=symmetric)
    pre, sc = _teacher_forced(cfg, out, st_in, st_out)
    # q_in reduces the kernel's own tensors: exact
    assert torch.equal(trace[:, 0], sc[:, 0]), (trace[:, 0], sc[:, 0])
    assert torch.equal(trace[:, 1], sc[:, 1])
    # q_out reduces a pre-quant state computed by both sides
    assert torch.allclose(trace[:, 2], sc[:, 2], rtol=1e-5, atol=0)
    assert ((trace[:, 3] - sc[:, 3]).abs() <= 1).all()
    flips = 0
    for t in range(out.shape[0]):
        flips += _codes_match(out[t], pre[t], float(trace[t, 2]), float(trace[t, 3]), q_out.qmin, q_out.qmax)
    stats_in, stats_out = q_in.observer_stats.cpu(), q_out.observer_stats.cpu()
    if mode == "min_max":
        assert stats_in[2] == 1.0 and stats_out[2] == 1.0
        assert torch.equal(stats_in[:2], torch.stack([st_in.running_min, st_in.running_max]))
        assert torch.allclose(stats_out[:2], torch.stack([st_out.running_min, st_out.running_max]), rtol=1e-5,
                              atol=1e-7)
    else:
        assert stats_in[2] == 0.0 and stats_out[2] == 0.0  # dynamic mode leaves them alone
    log(f"[observe]   {mode} sym={symmetric}: teacher-forced flips={flips}; "
        f"stats_in={stats_in.tolist()} stats_out={stats_out.tolist()}")


@pytest.mark.parametrize("idx,shape", [(1, (1, 1, 8)), (3, (1, 2, 64)), (0, (2, 1, 5)), (4, (1, 1, 16))])
def test_observe_tiny(dev, idx, shape):
    """T = 1 (q_in sees only h0, no next-step q_in pass) and B = 1."""
    cfg = _cfg(idx, shape)
    q_in, q_out = _quant("min_max", True).to(dev), _quant("min_max", True).to(dev)
    out, trace = _run(cfg, dev, q_in, q_out)
    out, trace = out.cpu(), trace.cpu()
    st_in, st_out = O.ObserverState("min_max"), O.ObserverState("min_max")
    pre, sc = _teacher_forced(cfg, out, st_in, st_out)
    assert torch.equal(trace[:, 0], sc[:, 0])
    assert torch.allclose(trace[:, 2], sc[:, 2], rtol=1e-5)
    for t in range(out.shape[0]):
        _codes_match(out[t], pre[t], float(trace[t, 2]), 0.0, -127, 127)
    assert torch.equal(q_in.observer_stats.cpu()[:2], torch.stack([st_in.running_min, st_in.running_max]))


@pytest.mark.parametrize("idx", sorted(BIG))
def test_observe_large_batch(dev, idx):
    """B H up to 64K elements (256 reduction partials, K-split GEMM)."""
    cfg = _cfg(idx, BIG[idx])
    q_in, q_out = _quant("min_max", True).to(dev), _quant("min_max", True).to(dev)
    out, trace = _run(cfg, dev, q_in, q_out)
    out, trace = out.cpu(), trace.cpu()
    st_in, st_out = O.ObserverState("min_max"), O.ObserverState("min_max")
    pre, sc = _teacher_forced(cfg, out, st_in, st_out)
    assert torch.equal(trace[:, 0], sc[:, 0])
    assert torch.allclose(trace[:, 2], sc[:, 2], rtol=1e-5)
    for t in range(out.shape[0]):
        _codes_match(out[t], pre[t], float(trace[t, 2]), 0.0, -127, 127)


def test_statistics_accumulate_across_calls(dev):
    """A second call continues the running statistics (momentum 0.99), as
    calibration over several batches does."""
    q_in, q_out = _quant("min_max", True).to(dev), _quant("min_max", True).to(dev)
    st_in, st_out = O.ObserverState("min_max"), O.ObserverState("min_max")
    for seed in (0, 1):
        cfg = _cfg(1, seed=seed)
        out, _ = _run(cfg, dev, q_in, q_out)
        _teacher_forced(cfg, out.cpu(), st_in, st_out)
    assert torch.equal(q_in.observer_stats.cpu()[:2], torch.stack([st_in.running_min, st_in.running_max]))
    assert torch.allclose(q_out.observer_stats.cpu()[:2], torch.stack([st_out.running_min, st_out.running_max]),
                          rtol=1e-5)


@pytest.mark.parametrize("mode,symmetric", [("min_max", True), ("dynamic", False), ("frozen", True)])
def test_observe_tensor(dev, mode, symmetric):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 5, 33, generator=g) * 0.7 + 0.2
    q = _quant(mode, symmetric)
    if mode == "frozen":
        q.scale = torch.tensor(0.013)
    q = q.to(dev)
    st = O.ObserverState(mode, symmetric=symmetric, scale=0.013)
    with torch.no_grad():
        y = q(x.to(dev)).cpu()
        y2 = q(x.to(dev) * 2).cpu()
    ref, _ = O.observer_forward(st, x)
    ref2, _ = O.observer_forward(st, x * 2)
    assert torch.equal(y, ref) and torch.equal(y2, ref2)
    if mode == "min_max":
        assert torch.equal(q.observer_stats.cpu()[:2], torch.stack([st.running_min, st.running_max]))


def test_layer_calibrate_freeze_and_fast_forward(dev):
    """ScanLayer.calibrate runs the observer path over a loader, freeze turns
    the statistics into scales, and the fast dispatch then runs the frozen
    quantizers in the scan kernel; compared with the oracle's calibration of
    the same layer (free-running, so within 1e-3 relative) and, after freeze,
    with the oracle's frozen scan on the kernel's own scales."""
    T, B, H, I = 8, 4, 64, 48
    g = torch.Generator().manual_seed(5)
    k = 1.0 / math.sqrt(H)
    Wi = (torch.rand(3 * H, I, generator=g) * 2 - 1) * k
    bi = (torch.rand(3 * H, generator=g) * 2 - 1) * k
    Wh = (torch.rand(3 * H, H, generator=g) * 2 - 1) * k
    bh = (torch.rand(3 * H, generator=g) * 2 - 1) * k
    xs = [torch.randn(T, B, I, generator=g) for _ in range(3)]
    cfg = G.QuantizerConfig(mode="dynamic")
    layer = G.ScanLayer("dense", Wi, bi, Wh, bh, x_quant=cfg, h_quant=cfg, w_bits=8).to(dev)
    summary = layer.calibrate([x.to(dev) for x in xs], n_batches=2)
    assert layer.use_triton
    assert set(summary) == {"quant_x", "quant_h_in", "quant_h_out"}

    # the oracle's calibration of the same layer
    sx, si, so = O.ObserverState("min_max"), O.ObserverState("min_max"), O.ObserverState("min_max")
    Wq, _ = O.weight_fake_quant_rows(Wi, -127, 127)
    for x in xs[:2]:
        xq, _ = O.observer_forward(sx, x)
        gi = F_linear(xq, Wq, bi)
        O.observe_scan(gi, torch.zeros(B, H), lambda hq: O.gh_dense(hq, Wh, bh), si, so)
    for name, st in (("quant_x", sx), ("quant_h_in", si), ("quant_h_out", so)):
        got = summary[name]
        log(f"[observe] {name}: kernel ({got['running_min']:.6f}, {got['running_max']:.6f}) oracle "
            f"({float(st.running_min):.6f}, {float(st.running_max):.6f})")
        assert got["initialized"]
        assert got["running_min"] == pytest.approx(float(st.running_min), rel=1e-3)
        assert got["running_max"] == pytest.approx(float(st.running_max), rel=1e-3)
    assert summary["quant_x"]["running_min"] == float(sx.running_min)  # same tensors: exact

    layer.freeze()
    for q in (layer.quant_x, layer.quant_h_in, layer.quant_h_out):
        assert q.config.mode == "frozen"
    s_in = G.gru_layer._extract_h_quant_params(layer.quant_h_in)
    s_out = G.gru_layer._extract_h_quant_params(layer.quant_h_out)
    s_x = G.gru_layer._extract_h_quant_params(layer.quant_x)
    assert s_in is not None and s_out is not None and s_x is not None
    x = xs[2]
    with torch.no_grad():
        out, h_T = layer(x.to(dev))
    out = out.cpu()
    assert torch.equal(h_T.cpu(), out[-1])
    gi = O.input_projection(x, Wi, bi, x_quant=s_x, w_quant=(-127, 127))
    c = {"kind": "dense", "w": Wh, "bh": bh, "gi": gi, "h0": torch.zeros(B, H), "h_in_quant": s_in,
         "h_out_quant": s_out}
    pre = O.teacher_forced_prequant(c, out)
    # gi differs from the kernel's (GEMM vs F.linear) by ~1e-7: boundary band 1e-5
    _codes_match(out, pre, s_out[0], 0.0, -127, 127, tol=1e-5)


def F_linear(x, W, b):
    return torch.nn.functional.linear(x, W, b)


@pytest.mark.parametrize("modes", [("min_max", None), (None, "min_max"), ("frozen", "dynamic"), ("dynamic", "frozen")])
def test_observe_mixed_modes(dev, modes):
    """Each hidden quantizer in its own mode (or absent): the scales each step
    used and the statistics follow the oracle on the kernel's own trajectory."""
    cfg = _cfg(1)
    qs, sts = [], []
    for m in modes:
        if m is None:
            qs.append(None)
            sts.append(O.ObserverState("off"))
        elif m == "frozen":
            q = _quant("frozen", True)
            q.scale = torch.tensor(0.004)
            qs.append(q.to(dev))
            sts.append(O.ObserverState("frozen", scale=0.004))
        else:
            qs.append(_quant(m, True).to(dev))
            sts.append(O.ObserverState(m))
    out, trace = _run(cfg, dev, qs[0], qs[1])
    out, trace = out.cpu(), trace.cpu()
    pre, sc = _teacher_forced(cfg, out, sts[0], sts[1])
    assert torch.equal(trace[:, 0], sc[:, 0]) and torch.equal(trace[:, 1], sc[:, 1])
    assert torch.allclose(trace[:, 2], sc[:, 2], rtol=1e-5, atol=0)
    for t in range(out.shape[0]):
        if modes[1] is None:
            assert (out[t] - pre[t]).abs().max().item() <= 1e-5
        else:
            _codes_match(out[t], pre[t], float(trace[t, 2]), float(trace[t, 3]), -127, 127)
    for q, st in zip(qs, sts):
        if q is not None and q.config.mode == "min_max":
            got = q.observer_stats.cpu()[:2]
            want = torch.stack([st.running_min, st.running_max])
            assert torch.allclose(got, want, rtol=1e-5, atol=1e-7)


def test_observe_tensor_reports_the_applied_scale(dev):
    """gs_observe_tensor's `used` output holds the (scale, zero point) it applied."""
    import ctypes

    from gru_qat_amd import _lib

    x = (torch.randn(9, 17, generator=torch.Generator().manual_seed(4)) * 0.3 - 0.1).to(dev)
    q = _quant("dynamic", False).to(dev)
    y = torch.empty_like(x)
    used = torch.zeros(2, device=dev)
    a = _lib.GsObserveTensorArgs()
    a.x, a.y, a.used = x.data_ptr(), y.data_ptr(), used.data_ptr()
    a.rows, a.cols, a.ld = 9, 17, 17
    a.q = q.observer()
    lib = _lib.load()
    need = lib.gs_observe_tensor_scratch_bytes(ctypes.byref(a))
    scratch = torch.empty(int(need), dtype=torch.uint8, device=dev)
    a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel()
    assert lib.gs_observe_tensor(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)) == 0
    torch.cuda.synchronize(dev)
    st = O.ObserverState("dynamic", symmetric=False)
    ref, (s, zp) = O.observer_forward(st, x.cpu())
    assert torch.equal(y.cpu(), ref)
    assert used.cpu().tolist() == [s, zp]
