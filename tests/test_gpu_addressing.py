"""The two addressing variants of the diagonal scan give identical results.

The diagonal forward and backward kernels read and write their per-step
tensors through 32-bit raw buffer offsets when every byte offset of gi, out,
dout and dgi fits 32 bits, and through 64-bit global addresses otherwise (the
host decides per call). Here gi and out are strided views whose time stride
spans more than 4 GiB, which forces the global-address variant; the same
values laid out contiguously take the buffer variant. The two must agree bit
for bit (the arithmetic is the same), and both must match the oracle.
"""

from __future__ import annotations

import pytest
import torch

from oracle import gru_oracle as O

pytestmark = pytest.mark.gpu

T, B, H = 3, 4, 64
STRIDE_T = (1 << 30) + 64  # floats: (T - 1) * STRIDE_T * 4 bytes > 2^32


def _far_view(src: torch.Tensor, dev) -> torch.Tensor:
    """src [T, B, N] copied into a view whose time stride is STRIDE_T floats."""
    n = src.shape[1] * src.shape[2]
    big = torch.empty((src.shape[0] - 1) * STRIDE_T + n, device=dev)
    v = big.as_strided(tuple(src.shape), (STRIDE_T, src.shape[2], 1))
    v.copy_(src.to(dev))
    return v


@pytest.mark.parametrize("quant", [False, True])
def test_diagonal_global_and_buffer_addressing_agree(dev, quant):
    from gru_qat_amd import _lib

    g = torch.Generator().manual_seed(11)
    gi = torch.randn(T, B, 3 * H, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.1
    w = (torch.rand(3, H, generator=g) * 2 - 1) / H ** 0.5
    bh = (torch.rand(3 * H, generator=g) * 2 - 1) / H ** 0.5
    q = (1.0 / 127.0, -127, 127) if quant else None
    d = {k: v.to(dev) for k, v in dict(h0=h0, w=w, bh=bh).items()}

    out_near = torch.empty(T, B, H, device=dev)
    _lib.launch(_lib.KIND_DIAGONAL, "gs_diagonal_fwd", gi=gi.to(dev), h0=d["h0"], w=d["w"], w2=None, bh=d["bh"],
                out=out_near, h_in_quant=q, h_out_quant=q)
    gi_far = _far_view(gi, dev)
    out_far = _far_view(torch.zeros(T, B, H), dev)
    _lib.launch(_lib.KIND_DIAGONAL, "gs_diagonal_fwd", gi=gi_far, h0=d["h0"], w=d["w"], w2=None, bh=d["bh"],
                out=out_far, h_in_quant=q, h_out_quant=q)
    torch.cuda.synchronize(dev)
    a, b = out_near.cpu(), out_far.cpu()
    print(f"[addr] forward quant={quant}: {int((a != b).sum())} of {a.numel()} differ", flush=True)
    assert torch.equal(a, b)
    if not quant:
        ref = O.scan(gi, h0, lambda hq: O.gh_diagonal(hq, w, bh))
        assert (a - ref).abs().max().item() <= 1e-5

    dout = torch.randn(T, B, H, generator=g)
    grads = []
    for gi_v, out_v in ((gi.to(dev), out_near), (gi_far, out_far)):
        dgi = torch.empty(T, B, 3 * H, device=dev)
        dh0 = torch.empty(B, H, device=dev)
        dw_part = torch.empty(B, 3, H, device=dev)
        dbh_part = torch.empty(B, 3 * H, device=dev)
        _lib.launch_bwd(_lib.KIND_DIAGONAL, "gs_diagonal_bwd", gi=gi_v, h0=d["h0"], w=d["w"], w2=None, bh=d["bh"],
                        out=out_v, dout=dout.to(dev), dgi=dgi, dh0=dh0, dw_part=dw_part, dbh_part=dbh_part,
                        h_in_quant=q, h_out_quant=q)
        torch.cuda.synchronize(dev)
        grads.append([x.cpu() for x in (dgi, dh0, dw_part, dbh_part)])
    for name, x, y in zip(("dgi", "dh0", "dw_part", "dbh_part"), *grads):
        print(f"[addr] backward quant={quant} {name}: {int((x != y).sum())} of {x.numel()} differ", flush=True)
        assert torch.equal(x, y), name
