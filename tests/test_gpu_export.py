"""GPU checks of the int8 export (gs_quantize_rows; the export_int_weights the
reference leaves as a TODO, gru_cell.py:551-553): the per-row codes and
scales equal the oracle's per-channel rule bit for bit (quantizers.py:188-199,
124-134), codes * scale is exactly the fake-quantized weight, and a layer
rebuilt from the dequantized export runs the same forward as the layer
with those fake-quantized weights."""

from __future__ import annotations

import math

import pytest
import torch

import gru_qat_amd as G
from gru_qat_amd.configs import make_config
from oracle import gru_oracle as O
from parity_util import log

pytestmark = pytest.mark.gpu


def _layer(idx, dev, I=40):
    cfg = make_config(idx, shape=(6, 4, 64))
    H = cfg["H"]
    g = torch.Generator().manual_seed(7)
    Wi = (torch.rand(3 * H, I, generator=g) * 2 - 1) / math.sqrt(I)
    bi = (torch.rand(3 * H, generator=g) * 2 - 1) / math.sqrt(I)
    qc = G.QuantizerConfig(mode="min_max")
    layer = G.ScanLayer(cfg["kind"], Wi, bi, cfg["w"], cfg["bh"], hidden2=cfg.get("w2"), x_quant=qc, h_quant=qc,
                        w_bits=8).to(dev)
    xs = [torch.randn(6, 4, I, generator=g).to(dev) for _ in range(2)]
    layer.calibrate(xs, n_batches=2)
    layer.freeze()
    return layer, cfg, xs


@pytest.mark.parametrize("idx", [0, 1, 3, 4])
def test_export_codes_and_scales(dev, idx):
    layer, cfg, _ = _layer(idx, dev)
    ex = layer.export_int_weights()
    log(f"[export] {cfg['name']}: keys {sorted(k for k, v in ex.items() if isinstance(v, torch.Tensor))}")
    hidden_name = {"dense": "Wh_cat", "diagonal": "Wh_diag", "monarch": "Wh_struct", "butterfly": "twiddles"}[
        cfg["kind"]]
    pairs = [("Wi_cat", layer.Wi_cat), (hidden_name, layer.hidden)]
    if layer.hidden2 is not None:
        pairs.append(("Wh_struct2", layer.hidden2))
    deq = G.dequantize_int_weights(ex)
    for name, w in pairs:
        codes, scale = ex[name].cpu(), ex[name + "_scale"].cpu()
        assert codes.dtype == torch.int8 and codes.shape == w.shape
        assert int(codes.abs().max()) == 127  # each row's absmax lands on +-127
        rows = scale.numel()
        w2 = w.detach().cpu().reshape(rows, -1)
        wq_ref, s_ref = O.weight_fake_quant_rows(w2, -127, 127)
        assert torch.equal(scale.reshape(-1), s_ref), name
        assert torch.equal(codes.reshape(rows, -1).float(), torch.round(w2 / s_ref.view(-1, 1)).clamp(-127, 127))
        assert torch.equal(deq[name].cpu().reshape(rows, -1), wq_ref), name
    for tag in ("x", "h_in", "h_out"):
        assert ex[f"{tag}_scale"] == pytest.approx(float(getattr(layer, "quant_" + tag).scale))
        assert ex[f"{tag}_zero_point"] == 0.0 and ex[f"{tag}_qrange"] == (-127, 127)


@pytest.mark.parametrize("idx", [1, 3])
def test_dequantized_export_runs_like_fake_quant_weights(dev, idx):
    layer, cfg, xs = _layer(idx, dev)
    ex = layer.export_int_weights()
    deq = G.dequantize_int_weights(ex)
    hidden_name = "Wh_cat" if cfg["kind"] == "dense" else "Wh_struct"
    # the same layer with its hidden weights replaced by their fake-quantized form
    with torch.no_grad():
        layer.hidden.copy_(deq[hidden_name])
        if layer.hidden2 is not None:
            layer.hidden2.copy_(deq["Wh_struct2"])
        out_a, _ = layer(xs[0])
        # a layer built from the export alone (w_bits=8 re-derives the same Wi codes)
        twin = G.ScanLayer(cfg["kind"], deq["Wi_cat"], ex["bi_cat"], deq[hidden_name], ex["bh_cat"],
                           hidden2=deq.get("Wh_struct2"), x_quant=G.QuantizerConfig(mode="frozen"),
                           h_quant=G.QuantizerConfig(mode="frozen"), w_bits=8).to(dev)
        for tag in ("x", "h_in", "h_out"):
            getattr(twin, "quant_" + tag).scale = torch.tensor(ex[f"{tag}_scale"], device=dev)
        out_b, _ = twin(xs[0])
    torch.cuda.synchronize(dev)
    diff = (out_a - out_b).abs().max().item()
    step = ex["h_out_scale"]
    log(f"[export] {cfg['name']}: max|layer - layer from export| = {diff:.3e} (one code = {step:.3e})")
    # Wi re-quantized from codes*scale keeps its codes; its scale may move by an ulp
    assert diff <= step + 1e-6
    assert (out_a != out_b).float().mean().item() < 0.01
