"""gs_dense_fwd_noalloc (no workspace, no allocation) against gs_dense_fwd.

Both entry points are called through the C ABI on the same inputs, two calls
in a row with the second one smaller, so the second runs on the static array
the first left behind. The dense kernel is deterministic, so the outputs must
be bit-identical; the fp32 case is also checked against the oracle (1e-5) and
the int8 case's codes against the oracle's (teacher forcing, through
parity_util's quant bar). A shape whose exchange words exceed the static
array is refused with ValueError before anything is launched.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from gru_qat_amd import _lib
from gru_qat_amd.configs import make_config
from oracle import gru_oracle as O
from parity_util import FP32_TOL, log

pytestmark = pytest.mark.gpu


def _args(d: dict, out: torch.Tensor) -> "_lib.GsArgs":
    gi, h0, w, bh = d["gi"], d["h0"], d["w"], d["bh"]
    T, B, threeH = gi.shape
    a = _lib.GsArgs()
    a.gi, a.h0, a.w, a.w2, a.bh, a.out = gi.data_ptr(), h0.data_ptr(), w.data_ptr(), None, bh.data_ptr(), out.data_ptr()
    a.T, a.B, a.H = T, B, threeH // 3
    a.sg_t, a.sg_b, a.sh0_b = gi.stride(0), gi.stride(1), h0.stride(0)
    a.so_t, a.so_b = out.stride(0), out.stride(1)
    a.q_in = _lib.make_quant(d["h_in_quant"], "h_in_quant")
    a.q_out = _lib.make_quant(d["h_out_quant"], "h_out_quant")
    return a


def _call(name: str, a: "_lib.GsArgs") -> None:
    lib = _lib.load()
    rc = getattr(lib, name)(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.raise_for(rc, lib)


def _run_pair(cfg: dict, dev: torch.device):
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}
    T, B, H = cfg["T"], cfg["B"], cfg["H"]
    ref_out = torch.empty((T, B, H), device=dev)
    a = _args(d, ref_out)
    lib = _lib.load()
    need = lib.gs_workspace_bytes(_lib.KIND_DENSE, ctypes.byref(a))
    assert need > 0
    ws = torch.zeros(int(need), dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _call("gs_dense_fwd", a)
    out = torch.full((T, B, H), float("nan"), device=dev)
    b = _args(d, out)  # workspace left NULL: the entry point takes none
    _call("gs_dense_fwd_noalloc", b)
    torch.cuda.synchronize(dev)
    return out.cpu(), ref_out.cpu()


def test_noalloc_matches_dense_fwd_twice(dev):
    # the second call is smaller than the first and reuses what the first left
    for idx, shape in ((2, (24, 32, 512)), (1, (9, 5, 256))):
        cfg = make_config(idx, shape=shape, seed=3)
        log(f"[noalloc] {cfg['name']} T,B,H={shape}")
        out, ref_out = _run_pair(cfg, dev)
        assert torch.equal(out, ref_out), f"max diff {(out - ref_out).abs().max().item():.3e}"
        if cfg["h_out_quant"] is None:
            err = (out - O.scan_config(cfg)).abs().max().item()
            log(f"[noalloc]   max|out-oracle|={err:.3e}")
            assert err <= FP32_TOL
        else:
            q = cfg["h_out_quant"]
            pre = O.teacher_forced_prequant(cfg, out)
            x = pre / q[0]
            near = (x - torch.floor(x) - 0.5).abs() * q[0] <= 2e-6
            mism = torch.round(out / q[0]) != O.quant_codes(pre, q)
            assert not (mism & ~near).any()


def test_noalloc_refuses_shapes_beyond_the_static_array(dev):
    T, B, H = 1, 1024, 1024  # 2 * B * H tagged words of 8 bytes: 16 MiB > 4 MiB
    cfg = make_config(1, shape=(T, B, H))
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}
    out = torch.empty((T, B, H), device=dev)
    with pytest.raises(ValueError, match="static scratch"):
        _call("gs_dense_fwd_noalloc", _args(d, out))


def test_noalloc_under_graph_capture_and_replay(dev):
    """gs_dense_fwd_noalloc captured in a HIP graph (torch.cuda.CUDAGraph):
    every replay, with eager calls of the same entry point and
    synchronisations between replays, returns the eager result bit for bit.
    Each replay's launch advances the device tag base by T, so no replay can
    accept a word an earlier one left."""
    cfg = make_config(1, shape=(16, 8, 512), seed=5)
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}
    T, B, H = cfg["T"], cfg["B"], cfg["H"]
    eager = torch.empty((T, B, H), device=dev)
    _call("gs_dense_fwd_noalloc", _args(d, eager))  # also sets the static array up outside the capture
    torch.cuda.synchronize(dev)
    want = eager.cpu()
    assert (want - O.scan_config(cfg)).abs().max().item() <= FP32_TOL
    out_g = torch.empty((T, B, H), device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _call("gs_dense_fwd_noalloc", _args(d, out_g))
    for i in range(4):
        out_g.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize(dev)
        log(f"[noalloc] replay {i}: {int((out_g.cpu() != want).sum())} elements differ")
        assert torch.equal(out_g.cpu(), want)
        again = torch.empty((T, B, H), device=dev)
        _call("gs_dense_fwd_noalloc", _args(d, again))
        torch.cuda.synchronize(dev)
        assert torch.equal(again.cpu(), want)
