"""Writes tests/golden/butterfly_reference.safetensors: butterfly products of
the reference's Butterfly scan kernel, the only source that fixes its twiddle
convention (which of t[pair, m, m] / t[pair, m, 1 - m] multiplies self and
partner, the pair index, the stride order per chain; LarocheC/gru-triton
src/gru_qat/triton_kernels/scan_butterfly.py:261-317).

Run in the build container only (it reads /root/reference and needs triton):

    TRITON_INTERPRET=1 python tests/golden/make_butterfly_golden.py

The reference kernel gru_scan_butterfly_fwd_kernel runs unmodified under
Triton's CPU interpreter, launched with its wrapper's arguments
(scan_butterfly.py:432-458; the wrapper itself rejects CPU tensors). Step 0
copies h0 into three per-gate scratch buffers and runs every butterfly stage
on them (:241-317); the gate epilogue then calls libdevice.tanh (:351),
which the interpreter does not implement, so the launch stops there. On CPU
tensors the interpreter works in place, so the scratch buffers then hold
butterfly_g(h0) for each gate g and every row of program 0: those products
are the vectors recorded here. The script checks that the launch stopped at
that tanh call. The modules are loaded by file path so that
gru_qat/__init__.py, which imports the absent torch_structured, does not run.
Tests read the fixture only.
"""

from __future__ import annotations

import importlib
import math
import os
import sys
import traceback
import types

import torch
from safetensors.torch import save_file

REF_SRC = "/root/reference/src"
REF_FILE = os.path.join(REF_SRC, "gru_qat/triton_kernels/scan_butterfly.py")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "butterfly_reference.safetensors")
BLOCK_B = 4

# (name, B, H, nchains); B <= BLOCK_B so all rows belong to program 0
CASES = [
    ("h8_c1", 3, 8, 1),
    ("h6_c1", 2, 6, 1),      # H_PAD = 8 > H: zero-padded input
    ("h16_c2", 3, 16, 2),    # second chain runs decreasing strides
    ("h32_c1", 4, 32, 1),
    ("h12_c3", 2, 12, 3),    # H_PAD = 16, three chains
    ("h64_c2", 4, 64, 2),
]


def load_reference():
    if os.environ.get("TRITON_INTERPRET") != "1":
        raise SystemExit("set TRITON_INTERPRET=1")
    for name, sub in (("gru_qat", "gru_qat"), ("gru_qat.triton_kernels", "gru_qat/triton_kernels")):
        pkg = types.ModuleType(name)
        pkg.__path__ = [os.path.join(REF_SRC, sub)]
        sys.modules[name] = pkg
    return importlib.import_module("gru_qat.triton_kernels.scan_butterfly")


def tanh_line() -> int:
    with open(REF_FILE) as f:
        for i, line in enumerate(f, 1):
            if "libdevice.tanh(gin + r * gh_n)" in line:
                return i
    raise SystemExit("tanh call not found in the reference kernel")


def butterfly_products(mod, h0, tw, H):
    """Runs the reference kernel on one step until its tanh call; returns the
    scratch buffers [3, B, H_PAD] = butterfly_g(h0)."""
    import triton

    B = h0.shape[0]
    T = 1
    nblocks, log_n, n_div_2 = tw.shape[1], tw.shape[2], tw.shape[3]
    H_PAD = 2 * n_div_2
    gi = torch.zeros((T, B, 3 * H))
    bh = torch.zeros(3 * H)
    out = torch.zeros((T, B, H))
    scratch = torch.full((1, 4, BLOCK_B, H_PAD), float("nan"))
    try:
        mod.gru_scan_butterfly_fwd_kernel[(triton.cdiv(B, BLOCK_B),)](
            gi, h0, tw, bh, out, scratch, T, B,
            gi.stride(0), gi.stride(1), h0.stride(0),
            tw.stride(0), tw.stride(1), tw.stride(2), tw.stride(3), tw.stride(4), tw.stride(5),
            out.stride(0), out.stride(1),
            scratch.stride(0), scratch.stride(1), scratch.stride(2),
            1.0, -2**31, 2**31 - 1, 1.0, -2**31, 2**31 - 1,
            H=H, H_PAD=H_PAD, LOG_H_PAD=log_n, NBLOCKS=nblocks, BLOCK_B=BLOCK_B,
            QUANT_H_IN=False, QUANT_H_OUT=False,
        )
    except Exception as e:  # the interpreter raises at the first libdevice call
        frames = traceback.extract_tb(e.__cause__.__traceback__ if e.__cause__ else e.__traceback__)
        ref = [f for f in frames if os.path.samefile(f.filename, REF_FILE)] if frames else []
        if not ref or ref[-1].lineno != tanh_line():
            raise SystemExit(f"launch stopped elsewhere: {ref[-1] if ref else frames}")
    else:
        raise SystemExit("expected the interpreter to stop at libdevice.tanh")
    prod = scratch[0, :3, :B, :].clone()
    if torch.isnan(prod).any():
        raise SystemExit("scratch not fully written")
    return prod


def main() -> None:
    mod = load_reference()
    tensors = {}
    for i, (name, B, H, nchains) in enumerate(CASES):
        g = torch.Generator().manual_seed(100 + i)
        h_pad = 1 << max(1, (H - 1).bit_length())
        L = h_pad.bit_length() - 1
        tw = torch.randn((3, nchains, L, h_pad // 2, 2, 2), generator=g) * math.sqrt(0.5)
        h0 = torch.randn((B, H), generator=g)
        prod = butterfly_products(mod, h0, tw, H)
        tensors[f"{name}.twiddles"] = tw.contiguous()
        tensors[f"{name}.h"] = h0.contiguous()
        tensors[f"{name}.products"] = prod.contiguous()
        print(f"{name}: B={B} H={H} H_PAD={h_pad} chains={nchains} |products|max={prod.abs().max().item():.4f}")
    save_file(tensors, OUT)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
