"""Backward of the differentiable scan entry points on the GPU against the
oracle's restatement of the reference backward (scan.py:1450-1550), computed
from the kernel's own forward output so that both walk the same trajectory.

Bar: every gradient within 1e-4 x max(1, max |oracle|) (fp32 recomputation of
the gates on the device vs the CPU, accumulated over T steps)."""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN, make_config
from oracle import gru_oracle as O

pytestmark = pytest.mark.gpu

COARSE = (0.05, -10, 10)


def _cfg(idx, shape, nb=None, two=False, q=None, seed=0):
    cfg = make_config(idx, shape=shape, seed=seed)
    T, B, H = shape
    if idx == 3:
        g = torch.Generator().manual_seed(seed + 7)
        bs = H // nb
        cfg["w"] = (torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5
        cfg["w2"] = ((torch.rand((3, nb, bs, bs), generator=g) * 2 - 1) / bs ** 0.5) if two else None
    cfg["h0"] = torch.randn(B, H, generator=torch.Generator().manual_seed(seed + 3)) * 0.3
    cfg["h_in_quant"] = q
    cfg["h_out_quant"] = q
    return cfg


def _run(cfg, dev, leaves):
    import gru_qat_amd as G

    kw = dict(h_in_quant=cfg["h_in_quant"], h_out_quant=cfg["h_out_quant"])
    kind = cfg["kind"]
    if kind == "dense":
        return G.gru_scan_persistent(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"], **kw)
    if kind == "diagonal":
        return G.gru_scan_diagonal(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"], **kw)
    if kind == "monarch":
        return G.gru_scan_monarch(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"],
                                  Wh_struct2=leaves.get("w2"), **kw)
    return G.gru_scan_butterfly_triton(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"], **kw)


CASES = [
    (1, (8, 5, 64), None, False), (1, (6, 4, 300), None, False), (0, (8, 5, 64), None, False),
    (3, (6, 4, 64), 4, False), (3, (6, 4, 64), 4, True), (4, (5, 3, 256), None, False),
    (4, (5, 3, 100), None, False),
    (0, (67, 9, 200), None, False), (0, (1, 2, 8), None, False),
    (1, (64, 32, 512), None, False), (1, (5, 37, 1000), None, False), (1, (3, 2, 8), None, False),
    (1, (1, 3, 16), None, False), (1, (7, 6, 128), None, False),
    (3, (16, 8, 512), 8, True), (3, (8, 6, 128), 8, False), (3, (5, 9, 96), 3, True),
    (4, (8, 6, 512), None, False), (4, (3, 2, 1000), None, False), (4, (1, 3, 256), None, False),
    # butterfly: seven spans of the recurrence (the last one short) with the twiddle gradient alongside
    (4, (37, 3, 256), None, False),
    # N = 1024 with H = N: the recurrence's folded cross-wave layers over every element
    (4, (6, 5, 1024), None, False), (0, (33, 3, 1024), None, False),
    # single-factor Monarch on the block-local path: blksz 16, 32, 64, 128, B not a multiple of the
    # rows per workgroup; blksz 48 takes the materialized path
    (3, (64, 32, 512), 8, False), (3, (9, 5, 512), 4, False), (3, (7, 3, 256), 8, False),
    (3, (11, 7, 64), 4, False), (3, (5, 3, 96), 2, False), (3, (1, 2, 64), 2, False),
]


@pytest.mark.parametrize("idx,shape,nb,two", CASES)
@pytest.mark.parametrize("q", [None, COARSE, Q_INT8_HIDDEN])
def test_backward_matches_oracle(dev, idx, shape, nb, two, q):
    cfg = _cfg(idx, shape, nb=nb, two=two, q=q)
    keys = ["gi", "h0", "bh"] + list(O.hidden_params(cfg))
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
    out = _run(cfg, dev, leaves)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
    ref = O.scan_backward(cfg, out.detach(), dout)
    for k, g in zip(keys, grads):
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        print(f"[bwd] {cfg['name']} {shape} q={q is not None} d{k}: max err {err:.3e} (|ref| {r.abs().max().item():.3e})")
        assert err <= 1e-4 * max(1.0, r.abs().max().item()), k


@pytest.mark.parametrize("idx,shape,nb,two", [(1, (9, 6, 128), None, False), (3, (6, 5, 64), 4, True),
                                              (3, (6, 5, 128), 2, False),
                                              (4, (5, 3, 64), None, False), (0, (9, 6, 40), None, False)])
def test_backward_is_deterministic_and_accepts_strided_inputs(dev, idx, shape, nb, two):
    """Two backward calls give bitwise-equal gradients (no atomics anywhere), and
    a gi that is a strided view (every other step of a longer sequence, batch
    rows of a wider tensor) gives the same gradients as its contiguous copy."""
    cfg = _cfg(idx, shape, nb=nb, two=two, q=COARSE)
    keys = ["gi", "h0", "bh"] + list(O.hidden_params(cfg))
    T, B, H = shape
    big = torch.randn(2 * T, B + 3, 3 * H, generator=torch.Generator().manual_seed(5))
    big[::2, :B] = cfg["gi"]
    gi_view = big.to(dev)[::2, :B]
    assert not gi_view.is_contiguous()
    dout = torch.randn((T, B, H), generator=torch.Generator().manual_seed(13)).to(dev)
    runs = []
    for gi_src in (gi_view, gi_view.contiguous(), gi_view.contiguous()):
        leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys if k != "gi"}
        leaves["gi"] = gi_src.detach().requires_grad_(True)
        out = _run(cfg, dev, leaves)
        runs.append(torch.autograd.grad(out, [leaves[k] for k in keys], dout))
    for a, b, c in zip(*runs):
        assert torch.equal(b, c)  # deterministic
        assert torch.equal(a, b)  # strided input == contiguous input


@pytest.mark.parametrize("q", [None, COARSE])
def test_butterfly_backward_materialized_fallback(dev, q):
    """Twiddles of H_PAD = 2048 for H = 600 exceed what the stage-wise kernels
    hold in LDS, so gs_butterfly_bwd takes the materialized-map path."""
    cfg = _cfg(4, (4, 3, 600), q=q)
    cfg["w"] = torch.randn((3, 1, 11, 1024, 2, 2), generator=torch.Generator().manual_seed(8)) * 0.5 ** 0.5
    keys = ["gi", "h0", "bh", "w"]
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
    out = _run(cfg, dev, leaves)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
    ref = O.scan_backward(cfg, out.detach().cpu(), dout.cpu())
    for k, g in zip(keys, grads):
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        print(f"[bwd] butterfly H_PAD=2048 d{k}: max err {err:.3e}")
        assert err <= 1e-4 * max(1.0, r.abs().max().item()), k


@pytest.mark.parametrize("idx,shape,nb", [(0, (13, 5, 96), None), (0, (4, 3, 1024), None), (3, (9, 5, 128), 8),
                                           (1, (6, 4, 64), None)])
@pytest.mark.parametrize("qin,qout", [(COARSE, None), (None, COARSE), (Q_INT8_HIDDEN, COARSE)])
def test_backward_one_sided_quantizers(dev, idx, shape, nb, qin, qout):
    """Only one of the hidden quantizers on, or two different ones: the
    gradients follow q_in's and q_out's clipped straight-through masks
    separately (each kernel variant of the quantizer modes)."""
    cfg = _cfg(idx, shape, nb=nb)
    cfg["h_in_quant"], cfg["h_out_quant"] = qin, qout
    keys = ["gi", "h0", "bh"] + list(O.hidden_params(cfg))
    leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
    out = _run(cfg, dev, leaves)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(17)).to(dev)
    grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
    ref = O.scan_backward(cfg, out.detach(), dout)
    for k, g in zip(keys, grads):
        r = ref["d" + k]
        err = (g.cpu() - r).abs().max().item()
        print(f"[bwd] {cfg['name']} {shape} qin={qin is not None} qout={qout is not None} d{k}: max err {err:.3e}")
        assert err <= 1e-4 * max(1.0, r.abs().max().item()), k


@pytest.mark.parametrize("shape", [(8, 5, 64), (6, 4, 300), (64, 32, 512), (5, 37, 1000), (3, 2, 8), (9, 6, 1024),
                                   (1, 3, 16), (1, 7, 512)])
@pytest.mark.parametrize("q", [None, COARSE, Q_INT8_HIDDEN])
def test_dense_saved_gh_matches_recompute(dev, shape, q):
    """The training forward also stores q_in(h_{t-1}) Wh^T of every step
    (gh_save) and the dense backward then skips its recompute GEMM (gh_saved).
    The forward's out is bit-identical with and without gh_save; the saved
    product matches q_in(h_{t-1}) Wh^T in float64 to 1e-5 x the row scale; the
    gradients of both backward paths agree to 1e-5 x max(1, max |grad|)."""
    from gru_qat_amd import scan as S

    T, B, H = shape
    cfg = _cfg(1, shape, q=q)
    x = {k: cfg[k].to(dev) for k in ("gi", "h0", "w", "bh")}
    out_plain = S.gru_scan_forward_persistent(x["gi"], x["h0"], x["w"], x["bh"], h_in_quant=q, h_out_quant=q)
    gh = torch.full((T, B, 3 * H), float("nan"), device=dev)
    out = S._dense_forward("test", x["gi"], x["h0"], x["w"], x["bh"], q, q, gh_save=gh)
    torch.cuda.synchronize(dev)
    assert torch.equal(out, out_plain)
    hprev = torch.cat([x["h0"][None], out[:-1]]).cpu().double()
    hq = O.fake_quant(hprev, q)
    want = hq @ cfg["w"].double().T
    scale = (hq.abs() @ cfg["w"].double().abs().T).clamp_min(1.0)
    err = ((gh.cpu().double() - want).abs() / scale).max().item()
    assert err <= 1e-5, f"saved gh off by {err:.3e} (relative to the row scale)"
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    args = (x["gi"], x["h0"], x["w"], x["bh"], out, dout, q, q)
    g_saved = S._dense_backward("test", *args, gh_saved=gh)
    g_recomp = S._dense_backward("test", *args)
    for name, a, b in zip(("dgi", "dh0", "dW", "dbh"), g_saved, g_recomp):
        tol = 1e-5 * max(1.0, b.abs().max().item())
        err = (a - b).abs().max().item()
        assert err <= tol, f"{name}: saved-gh path differs from the recompute by {err:.3e} (tol {tol:.3e})"


@pytest.mark.parametrize("shape,nb", [((8, 5, 64), 4), ((6, 4, 256), 8), ((64, 32, 512), 8), ((5, 37, 1024), 8),
                                      ((1, 3, 128), 2), ((7, 9, 128), 1)])
@pytest.mark.parametrize("q", [None, COARSE, Q_INT8_HIDDEN])
def test_monarch_saved_gh_matches_recompute(dev, shape, nb, q):
    """Single-factor Monarch (blksz 16 to 128): the training forward stores
    each step's bias-free q_in(h_{t-1}) W^T through gh_save; out is
    bit-identical with and without it, the saved product matches the block
    product in float64 to 1e-5 x the row scale, and the backward given
    gh_saved agrees with the recomputing backward to 1e-5 x max(1, max |grad|)."""
    from gru_qat_amd import scan_monarch as M

    T, B, H = shape
    bs = H // nb
    assert M.monarch_saves_gh(T, B, nb, bs, False)
    cfg = _cfg(3, shape, nb=nb, q=q)
    x = {k: cfg[k].to(dev) for k in ("gi", "h0", "w", "bh")}
    kw = dict(h_in_quant=q, h_out_quant=q)
    out_plain = M.gru_scan_monarch_forward(x["gi"], x["h0"], x["w"], x["bh"], **kw)
    gh = torch.full((T, B, 3 * H), float("nan"), device=dev)
    out = M.gru_scan_monarch_forward(x["gi"], x["h0"], x["w"], x["bh"], gh_save=gh, **kw)
    torch.cuda.synchronize(dev)
    assert torch.equal(out, out_plain)
    hprev = torch.cat([x["h0"][None], out[:-1]]).cpu().double()
    hq = O.fake_quant(hprev, q).reshape(T, B, nb, bs)
    W = cfg["w"].double()
    want = torch.einsum("tbni,gnoi->tbgno", hq, W).reshape(T, B, 3 * H)
    scale = torch.einsum("tbni,gnoi->tbgno", hq.abs(), W.abs()).reshape(T, B, 3 * H).clamp_min(1.0)
    err = ((gh.cpu().double() - want).abs() / scale).max().item()
    assert err <= 1e-5, f"saved gh off by {err:.3e} (relative to the row scale)"
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    args = (x["gi"], x["h0"], x["w"], x["bh"], out, dout)
    g_saved = M.gru_scan_monarch_backward(*args, gh_saved=gh, **kw)
    g_recomp = M.gru_scan_monarch_backward(*args, **kw)
    names = ("dgi", "dh0", "dW", "dbh")
    for name, a, b in zip(names, g_saved, g_recomp):
        a, b = (a[0], b[0]) if name == "dW" else (a, b)
        tol = 1e-5 * max(1.0, b.abs().max().item())
        err = (a - b).abs().max().item()
        assert err <= tol, f"{name}: saved-gh path differs from the recompute by {err:.3e} (tol {tol:.3e})"


def test_monarch_function_saves_gh_only_where_supported(dev):
    """gru_scan_monarch saves gh for the single-factor scan under grad mode,
    not for the two-factor scan or under no_grad; the gradients through the
    autograd function match the recomputing backward either way."""
    import gru_qat_amd as G
    from gru_qat_amd import scan_monarch as M

    for two in (False, True):
        cfg = _cfg(3, (6, 4, 256), nb=8, two=two)
        keys = ["gi", "h0", "w", "bh"] + (["w2"] if two else [])
        leaves = {k: cfg[k].to(dev).requires_grad_(True) for k in keys}
        out = G.gru_scan_monarch(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"],
                                 Wh_struct2=leaves.get("w2"))
        saved = out.grad_fn.saved_tensors
        assert (saved[-1] is not None) == (not two)
        dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(dev)
        grads = torch.autograd.grad(out, [leaves[k] for k in keys], dout)
        plain = {k: v.detach() for k, v in leaves.items()}
        dgi, dh0, dps, dbh = M.gru_scan_monarch_backward(plain["gi"], plain["h0"], plain["w"], plain["bh"],
                                                         out.detach(), dout, Wh_struct2=plain.get("w2"))
        want = [dgi, dh0, dps[0], dbh] + ([dps[1]] if two else [])
        order = ["gi", "h0", "w", "bh"] + (["w2"] if two else [])
        for k, g, w in zip(order, grads, want):
            tol = 1e-5 * max(1.0, w.abs().max().item())
            assert (g - w).abs().max().item() <= tol, k
        with torch.no_grad():
            out_ng = G.gru_scan_monarch(leaves["gi"], leaves["h0"], leaves["w"], leaves["bh"],
                                        Wh_struct2=leaves.get("w2"))
        assert out_ng.grad_fn is None
        assert torch.equal(out_ng, out.detach())


@pytest.mark.parametrize("shape", [(9, 4, 256), (6, 3, 1024)])
def test_butterfly_backward_in_a_graph_and_on_another_stream(dev, shape):
    """The butterfly backward runs its twiddle gradient on a second stream of
    its own, ordered by events: captured into a graph (fork and join through
    those events) and replayed three times, with eager work between the
    replays, each replay gives bitwise the eager gradients; so does a call on a
    stream other than the default one."""
    from gru_qat_amd.scan_butterfly import gru_scan_butterfly_backward

    cfg = _cfg(4, shape, q=COARSE)
    d = {k: cfg[k].to(dev) for k in ("gi", "h0", "w", "bh")}
    kw = dict(h_in_quant=cfg["h_in_quant"], h_out_quant=cfg["h_out_quant"])
    import gru_qat_amd as G

    out = G.gru_scan_butterfly_triton(d["gi"], d["h0"], d["w"], d["bh"], **kw).detach()
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(21)).to(dev)
    args = (d["gi"], d["h0"], d["w"], d["bh"], out, dout)
    want = [g.clone() for g in gru_scan_butterfly_backward(*args, **kw)]
    torch.cuda.synchronize(dev)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        got = gru_scan_butterfly_backward(*args, **kw)
    torch.cuda.current_stream(dev).wait_stream(side)
    for name, a, b in zip(("dgi", "dh0", "dtw", "dbh"), got, want):
        assert torch.equal(a, b), f"{name} differs on another stream"

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        gru_scan_butterfly_backward(*args, **kw)  # warm-up on the capture stream
        torch.cuda.synchronize(dev)
        with torch.cuda.graph(g, stream=s):
            captured = gru_scan_butterfly_backward(*args, **kw)
    torch.cuda.synchronize(dev)
    for rep in range(3):
        for c in captured:
            c.zero_()
        g.replay()
        torch.cuda.synchronize(dev)
        for name, a, b in zip(("dgi", "dh0", "dtw", "dbh"), captured, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
        eager = gru_scan_butterfly_backward(*args, **kw)  # eager work between the replays
        torch.cuda.synchronize(dev)
        assert torch.equal(eager[0], want[0])
