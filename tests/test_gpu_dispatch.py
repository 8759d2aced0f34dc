"""GRULayer scan dispatch on the GPU (reference src/gru_qat/gru_layer.py:260-302):
each kind routes to its HIP scan with the hidden quant tuples, h_T is the last
time-major step, batch_first only transposes the returned sequence."""

from __future__ import annotations

import pytest
import torch

from gru_qat_amd.configs import Q_INT8_HIDDEN
from gru_qat_amd.gru_layer import forward_fast_dispatch
from oracle import gru_oracle as O
from parity_util import FP32_TOL, small_cfg, to_dev

pytestmark = pytest.mark.gpu

KIND_OF = {0: "diagonal", 1: "dense", 3: "monarch", 4: "butterfly"}


@pytest.mark.parametrize("idx", [0, 1, 3, 4])
@pytest.mark.parametrize("batch_first", [False, True])
def test_dispatch_matches_oracle(dev, idx, batch_first):
    shape = (6, 5, 64) if idx != 4 else (6, 5, 256)
    cfg = small_cfg(idx, shape, h_in_quant=None, h_out_quant=None)
    d = to_dev(cfg, dev)
    out, h_T = forward_fast_dispatch(KIND_OF[idx], d["gi"], d["h0"], d["w"], d["bh"],
                                     hidden2=d.get("w2"), batch_first=batch_first)
    ref = O.scan_config(cfg)
    tm = out.transpose(0, 1) if batch_first else out
    assert tuple(out.shape) == ((5, 6, shape[2]) if batch_first else (6, 5, shape[2]))
    assert (tm.cpu() - ref).abs().max().item() <= FP32_TOL
    assert torch.equal(h_T, tm[-1])


def test_dispatch_quant_and_zero_h0(dev):
    cfg = small_cfg(3, (6, 4, 64), h_in_quant=Q_INT8_HIDDEN, h_out_quant=Q_INT8_HIDDEN)
    cfg["h0"] = torch.zeros_like(cfg["h0"])
    d = to_dev(cfg, dev)
    out, _ = forward_fast_dispatch("monarch", d["gi"], None, d["w"], d["bh"], hidden2=d["w2"],
                                   h_in_quant=Q_INT8_HIDDEN, h_out_quant=Q_INT8_HIDDEN)
    from gru_qat_amd.scan_monarch import gru_scan_monarch

    direct = gru_scan_monarch(d["gi"], d["h0"], d["w"], d["bh"], Wh_struct2=d["w2"],
                              h_in_quant=Q_INT8_HIDDEN, h_out_quant=Q_INT8_HIDDEN)
    assert torch.equal(out, direct)
    o = out.cpu()
    s = Q_INT8_HIDDEN[0]
    assert torch.equal(o, torch.round(o / s) * s)  # every output on the int8 grid
