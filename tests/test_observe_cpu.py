"""Observer path checks that need no GPU: the C ABI rejects bad observer
and map arguments before any device work, sizes its scratch, and the host
quantizer, calibration loop and ScanLayer follow the reference's contracts
(quantizers.py:63-156, calibration.py:31-126, gru_layer.py:308-342)."""

from __future__ import annotations

import ctypes

import pytest
import torch

import gru_qat_amd as G
from gru_qat_amd import _lib

FAKE = 0x1000  # never dereferenced: validation fails before any device access


def _obs(mode=_lib.OBS_DYNAMIC, symmetric=1, qmin=-127, qmax=127, scale=1.0, zp=0.0, stats=None):
    o = _lib.GsObserver()
    o.mode, o.symmetric, o.qmin, o.qmax, o.scale, o.zero_point = mode, symmetric, qmin, qmax, scale, zp
    o.stats = stats
    return o


def _oargs(kind=_lib.KIND_DENSE, T=4, B=3, H=8, **kw):
    a = _lib.GsObserveArgs()
    a.kind = kind
    a.gi = a.h0 = a.w = a.bh = a.out = FAKE
    a.T, a.B, a.H = T, B, H
    a.sg_t, a.sg_b, a.sh0_b, a.so_t, a.so_b = B * 3 * H, 3 * H, H, B * H, H
    a.q_in = kw.pop("q_in", _obs())
    a.q_out = kw.pop("q_out", _obs())
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_observe_scan_scratch_sizes():
    lib = _lib.load()
    a = _oargs()
    need = lib.gs_observe_scan_scratch_bytes(ctypes.byref(a))
    assert need > 0 and need % 256 == 0
    d = _oargs(kind=_lib.KIND_DIAGONAL)
    assert 0 < lib.gs_observe_scan_scratch_bytes(ctypes.byref(d)) < need  # no GEMM partials
    m = _oargs(kind=_lib.KIND_MONARCH, nblocks=2, blksz=4)
    assert lib.gs_observe_scan_scratch_bytes(ctypes.byref(m)) >= need + 3 * 8 * 8 * 4  # + the map
    b = _oargs(kind=_lib.KIND_BUTTERFLY, log_n=3, bfly_nblocks=1)
    assert lib.gs_observe_scan_scratch_bytes(ctypes.byref(b)) > need


@pytest.mark.parametrize("bad,msg", [
    (dict(q_in=_obs(mode=7)), b"not a GS_OBS_"),
    (dict(q_out=_obs(qmin=5, qmax=-5)), b"qmin"),
    (dict(q_in=_obs(mode=_lib.OBS_MIN_MAX)), b"stats buffer"),
    (dict(q_out=_obs(mode=_lib.OBS_FROZEN, scale=0.0)), b"finite scale"),
    (dict(q_in=_obs(symmetric=0, qmin=3, qmax=3)), b"qmax > qmin"),
    (dict(kind=9), b"unknown kind"),
    (dict(kind=_lib.KIND_MONARCH, nblocks=3, blksz=3), b"tile H"),
    (dict(kind=_lib.KIND_BUTTERFLY, log_n=2, bfly_nblocks=1), b"H_PAD"),
    (dict(T=0), b"T must be > 0"),
])
def test_observe_scan_rejects(bad, msg):
    lib = _lib.load()
    a = _oargs(**bad)
    assert lib.gs_observe_scan(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert msg in lib.gs_last_error()


def test_observe_scan_needs_scratch():
    lib = _lib.load()
    a = _oargs()
    assert lib.gs_observe_scan(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"scratch" in lib.gs_last_error()


def test_observe_tensor_rejects():
    lib = _lib.load()
    a = _lib.GsObserveTensorArgs()
    a.x = a.y = FAKE
    a.rows, a.cols, a.ld = 4, 8, 8
    a.q = _obs()
    assert lib.gs_observe_tensor_scratch_bytes(ctypes.byref(a)) > 0
    assert lib.gs_observe_tensor(ctypes.byref(a), None) == _lib.GS_ERR_INVALID  # no scratch
    a.ld = 4
    assert lib.gs_observe_tensor(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"ld" in lib.gs_last_error()


def test_hidden_map_rejects_and_sizes():
    lib = _lib.load()
    a = _lib.GsMapArgs()
    a.kind, a.H = _lib.KIND_BUTTERFLY, 8
    a.log_n, a.bfly_nblocks = 3, 1
    assert lib.gs_hidden_map_scratch_bytes(ctypes.byref(a)) == 2 * 3 * 8 * 8 * 4  # two [3, N, H] stage buffers
    a.H, a.log_n = 5, 3
    assert lib.gs_hidden_map_scratch_bytes(ctypes.byref(a)) == 2 * 512  # each 480 bytes, 256-aligned
    a.w = a.m = FAKE
    assert lib.gs_hidden_map_dense(ctypes.byref(a), None) == _lib.GS_ERR_INVALID  # no scratch
    a.kind, a.nblocks, a.blksz = _lib.KIND_MONARCH, 3, 2
    assert lib.gs_hidden_map_dense(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"tile H" in lib.gs_last_error()
    a.kind = _lib.KIND_DIAGONAL
    assert lib.gs_hidden_map_scratch_bytes(ctypes.byref(a)) == 0


# ---- host quantizer ------------------------------------------------------------------

def test_quantizer_qrange_and_buffers():
    q = G.FakeQuantizePerTensor(G.QuantizerConfig(bits=8))
    assert (q.qmin, q.qmax) == (-127, 127)
    a = G.FakeQuantizePerTensor(G.QuantizerConfig(bits=8, symmetric=False))
    assert (a.qmin, a.qmax) == (0, 255)
    assert set(dict(q.named_buffers())) == {"scale", "zero_point", "observer_stats"}
    assert float(q.running_min) == float("inf") and float(q.running_max) == float("-inf")
    assert not q._initialized
    q.running_min = torch.tensor(-1.0)
    q._initialized = True
    assert float(q.observer_stats[0]) == -1.0 and q._initialized
    q.reset_observer()
    assert not q._initialized and float(q.running_min) == float("inf")


@pytest.mark.parametrize("cfg", [dict(axis=0), dict(mode="lsq"), dict(bits=1)])
def test_quantizer_rejects(cfg):
    with pytest.raises(ValueError):
        G.FakeQuantizePerTensor(G.QuantizerConfig(**cfg))


def test_quantizer_freeze_matches_oracle_rule():
    from oracle import gru_oracle as O

    for symmetric in (True, False):
        q = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="min_max", symmetric=symmetric))
        q.running_min, q.running_max = torch.tensor(-0.3), torch.tensor(1.7)
        q._initialized = True
        q.freeze()
        st = O.ObserverState("min_max", symmetric=symmetric)
        st.running_min, st.running_max = torch.tensor(-0.3), torch.tensor(1.7)
        O.freeze_observer(st)
        assert q.config.mode == "frozen"
        assert torch.equal(q.scale, st.scale) and torch.equal(q.zero_point, st.zero_point)
    d = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="dynamic"))
    d.freeze()  # dynamic: only the mode changes (quantizers.py:98-107)
    assert d.config.mode == "frozen" and float(d.scale) == 1.0


def test_frozen_quantizer_feeds_fast_dispatch_tuple():
    q = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="min_max"))
    assert G.gru_layer._extract_h_quant_params(q) is None
    q.running_min, q.running_max = torch.tensor(-0.5), torch.tensor(1.0)
    q.freeze()
    s, lo, hi = G.gru_layer._extract_h_quant_params(q)
    assert (lo, hi) == (-127, 127) and s == pytest.approx(1.0 / 127)
    a = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="frozen", symmetric=False))
    assert G.gru_layer._extract_h_quant_params(a) is None  # affine never reaches the kernel


def test_forward_refuses_autograd():
    q = G.FakeQuantizePerTensor()
    with pytest.raises(RuntimeError, match="without autograd"):
        q(torch.zeros(2, 2, requires_grad=True))


# ---- calibration loop ----------------------------------------------------------------

class _Probe(torch.nn.Module):
    """Counts forwards and records how the batch arrived."""

    def __init__(self):
        super().__init__()
        self.quant_h_in = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="dynamic"))
        self.quant_w = G.FakeQuantizePerTensor(G.QuantizerConfig(mode="dynamic"))  # not an activation name
        self.calls = []

    def forward(self, *args, **kw):
        self.calls.append((len(args), sorted(kw), self.training))
        self.quant_h_in.observer_stats.copy_(torch.tensor([-1.0, 2.0, 1.0]))


def test_calibrate_loop_contract():
    m = _Probe()
    m.train()
    loader = [torch.zeros(1), (torch.zeros(1), torch.zeros(1)), {"x": torch.zeros(1)}, torch.zeros(1)]
    summary = G.calibrate(m, loader, n_batches=3)
    assert m.calls == [(1, [], False), (2, [], False), (0, ["x"], False)]
    assert m.training  # restored
    assert m.quant_h_in.config.mode == "min_max" and m.quant_w.config.mode == "dynamic"
    assert summary == {"quant_h_in": {"running_min": -1.0, "running_max": 2.0, "bits": 8, "axis": None,
                                      "initialized": True}}
    summary = G.calibrate(m, [], only_activations=False)
    assert set(summary) == {"quant_h_in", "quant_w"} and not summary["quant_w"]["initialized"]
    with pytest.raises(TypeError, match="cannot feed"):
        G.calibrate(m, [3])
    G.freeze_all(m)
    assert m.quant_h_in.config.mode == "frozen" and m.quant_w.config.mode == "frozen"


def test_scan_layer_construction():
    H, I = 8, 5
    layer = G.ScanLayer("dense", torch.zeros(3 * H, I), None, torch.zeros(3 * H, H), torch.zeros(3 * H),
                        x_quant=G.QuantizerConfig(mode="frozen"), h_quant=dict(mode="min_max"), w_bits=8)
    assert layer.use_triton and layer.w_quant == (-127, 127)
    assert layer.quant_h_in is not layer.quant_h_out
    assert layer.quant_h_in.config is not layer.quant_h_out.config
    names = {n for n, m in layer.named_modules() if isinstance(m, G.FakeQuantizePerTensor)}
    assert names == {"quant_x", "quant_h_in", "quant_h_out"}
    with pytest.raises(ValueError):
        G.ScanLayer("ldr", torch.zeros(3 * H, I), None, torch.zeros(3 * H, H), torch.zeros(3 * H))
    with pytest.raises(ValueError):
        G.ScanLayer("dense", torch.zeros(3 * H, I), None, torch.zeros(3 * H, H), torch.zeros(3 * H), w_bits=1)


# ---- int8 export ----------------------------------------------------------------------

def test_quantize_rows_rejects():
    lib = _lib.load()
    a = _lib.GsRowsArgs()
    a.w, a.scale, a.codes = FAKE, FAKE, FAKE
    a.rows, a.cols, a.qmin, a.qmax = 4, 8, -127, 127
    a.rows = 0
    assert lib.gs_quantize_rows(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    a.rows = 4
    a.qmin, a.qmax = -200, 200
    assert lib.gs_quantize_rows(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"int8 codes" in lib.gs_last_error()
    a.qmin, a.qmax = -127, 127
    a.codes = None
    assert lib.gs_quantize_rows(ctypes.byref(a), None) == _lib.GS_ERR_INVALID
    assert b"at least one" in lib.gs_last_error()


def test_export_requires_frozen_quantizers():
    H, I = 8, 5
    layer = G.ScanLayer("dense", torch.zeros(3 * H, I), None, torch.zeros(3 * H, H), torch.zeros(3 * H),
                        h_quant=G.QuantizerConfig(mode="min_max"))
    with pytest.raises(ValueError, match="freeze"):
        G.export._frozen(layer.quant_h_in)
