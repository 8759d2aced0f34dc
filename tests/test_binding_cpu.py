"""The reference-side binding: what ``GRULayer._forward_fast_dispatch``
(reference src/gru_qat/gru_layer.py:260-293) imports and calls, checked
against this build's modules aliased under the reference's module names.

* ``tests/golden/reference_api.json`` holds the reference modules' public
  functions with their positional and keyword-only parameters (read from the
  reference's source text). Every one is provided under the same name with
  the same positional parameters, the hidden quant keywords default to None,
  and the reference's tiling keywords are accepted (and ignored), except the
  ones listed in NOT_PROVIDED with the reason.
* The extract helpers stack a cell's hidden weights the way the reference's
  docstrings state (scan_diagonal.py:33-63, scan_monarch.py:22-58,
  scan_butterfly.py:1142-1182): gates r, z, n on dim 0, biases concatenated
  r, z, n, zeros without bias, ValueError on a dense hidden side, and the
  stacked tensors stay connected to the cell's parameters for autograd.
"""

from __future__ import annotations

import ast
import importlib
import inspect
import json
import os
import sys

import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
API = json.load(open(os.path.join(HERE, "golden", "reference_api.json")))

ALIASES = {
    "gru_qat.triton_kernels.scan": "gru_qat_amd.scan",
    "gru_qat.triton_kernels.scan_diagonal": "gru_qat_amd.scan_diagonal",
    "gru_qat.triton_kernels.scan_monarch": "gru_qat_amd.scan_monarch",
    "gru_qat.triton_kernels.scan_butterfly": "gru_qat_amd.scan_butterfly",
}

NOT_PROVIDED = {
    "gru_scan_diagonal_forward_pytorch": "the reference's own PyTorch checker (oracle/ restates it for tests)",
    "gru_scan_diagonal_backward_pytorch": "the reference's own PyTorch checker",
    "gru_scan_monarch_forward_pytorch": "the reference's own PyTorch checker",
    "gru_scan_monarch_backward_pytorch": "the reference's own PyTorch checker",
    "extract_butterfly_factors": "returns torch_structured Butterfly modules (package absent here)",
    "gru_scan_butterfly": "per-step scan over torch_structured Butterfly modules (package absent here)",
}


@pytest.fixture
def aliased():
    saved = {k: sys.modules.get(k) for k in ALIASES}
    for ref, ours in ALIASES.items():
        sys.modules[ref] = importlib.import_module(ours)
    try:
        yield
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


def _positional(sig):
    kinds = (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)
    return [p for p in sig.parameters.values() if p.kind in kinds]


def test_reference_names_and_signatures(aliased):
    checked = 0
    for modname, funcs in API["modules"].items():
        mod = importlib.import_module(modname)
        assert mod.__name__ == ALIASES[modname]
        for name, spec in funcs.items():
            if name in NOT_PROVIDED:
                continue
            assert hasattr(mod, name), f"{modname}.{name} (reference line {spec['line']}) is missing"
            obj = getattr(mod, name)
            if spec.get("class"):
                assert isinstance(obj, type) and issubclass(obj, torch.autograd.Function), name
                checked += 1
                continue
            sig = inspect.signature(obj)
            pos = _positional(sig)
            want = spec["positional"]
            assert [p.name for p in pos[: len(want)]] == want, f"{name}: positional {[p.name for p in pos]} != {want}"
            assert all(p.default is not inspect.Parameter.empty for p in pos[len(want):]), name
            kw = {}
            for k, default in spec["keyword_only"].items():
                if k in ("h_in_quant", "h_out_quant"):
                    p = sig.parameters[k]
                    assert p.kind is inspect.Parameter.KEYWORD_ONLY and p.default is None, f"{name}.{k}"
                kw[k] = ast.literal_eval(default) if default is not None else None
            # a call with every reference argument binds (tiling knobs land in **kwargs)
            sig.bind(*range(len(want)), **kw)
            checked += 1
    assert checked >= 20


def test_not_provided_names_are_absent(aliased):
    for modname, funcs in API["modules"].items():
        mod = importlib.import_module(modname)
        for name in funcs:
            if name in NOT_PROVIDED:
                assert not hasattr(mod, name), f"{name} is provided after all; drop it from NOT_PROVIDED"


def test_fast_dispatch_imports_and_calls_bind(aliased):
    """The three import statements and calls of _forward_fast_dispatch, as
    text, run against the aliased modules."""
    for call in API["fast_dispatch"]["calls"]:
        ns: dict = {}
        exec(f"from {call['module']} import ({call['extract']}, {call['scan']})", ns)
        extract, scan = ns[call["extract"]], ns[call["scan"]]
        inspect.signature(extract).bind(object())
        inspect.signature(scan).bind(*range(API["fast_dispatch"]["scan_call"]["positional"]),
                                     **{k: None for k in API["fast_dispatch"]["scan_call"]["keywords"]})


# ---- extract helpers on cell-shaped modules --------------------------------------------------

def _weight_module(t: torch.Tensor) -> torch.nn.Module:
    m = torch.nn.Module()
    m.weight = torch.nn.Parameter(t)
    return m


def _butterfly_module(tw: torch.Tensor) -> torch.nn.Module:
    inner = torch.nn.Module()
    inner.twiddle = torch.nn.Parameter(tw)
    m = torch.nn.Module()
    m.b = inner
    return m


def make_cell(kind: str, H: int, bias: bool = True, nb: int = 4, chains: int = 1, seed: int = 0) -> torch.nn.Module:
    """A module shaped like the reference cell's hidden side: struct_Wh_{r,z,n}
    (``.weight``, or ``.b.twiddle`` for butterfly), b_h{r,z,n} or None,
    hidden_size and _hidden_dense."""
    g = torch.Generator().manual_seed(seed)
    cell = torch.nn.Module()
    cell.hidden_size = H
    cell._hidden_dense = False
    for gate in "rzn":
        if kind == "diagonal":
            mod = _weight_module(torch.rand(H, generator=g) * 2 - 1)
        elif kind == "monarch":
            bs = H // nb
            mod = _weight_module((torch.rand(nb, bs, bs, generator=g) * 2 - 1) / bs ** 0.5)
        else:
            n = 1 << max(1, (H - 1).bit_length())
            L = n.bit_length() - 1
            mod = _butterfly_module(torch.randn(1, chains, L, n // 2, 2, 2, generator=g) * 0.5 ** 0.5)
        setattr(cell, f"struct_Wh_{gate}", mod)
        if bias:
            setattr(cell, f"b_h{gate}", torch.nn.Parameter(torch.rand(H, generator=g) * 0.2 - 0.1))
        else:
            setattr(cell, f"b_h{gate}", None)
    return cell


EXTRACT = {
    "diagonal": ("gru_qat_amd.scan_diagonal", "extract_diagonal_factors"),
    "monarch": ("gru_qat_amd.scan_monarch", "extract_monarch_factors"),
    "butterfly": ("gru_qat_amd.scan_butterfly", "extract_butterfly_twiddles"),
}


def _gate_tensor(cell, kind, gate):
    m = getattr(cell, f"struct_Wh_{gate}")
    return m.b.twiddle.squeeze(0) if kind == "butterfly" else m.weight


@pytest.mark.parametrize("kind", list(EXTRACT))
@pytest.mark.parametrize("bias", [True, False])
def test_extract_stacks_gates_r_z_n(kind, bias):
    extract = getattr(importlib.import_module(EXTRACT[kind][0]), EXTRACT[kind][1])
    H = 24 if kind != "butterfly" else 20
    cell = make_cell(kind, H, bias=bias, nb=4, chains=2)
    W, bh = extract(cell)
    assert W.shape[0] == 3
    for i, gate in enumerate("rzn"):
        assert torch.equal(W[i], _gate_tensor(cell, kind, gate)), f"gate {gate} not at index {i}"
    if kind == "diagonal":
        assert tuple(W.shape) == (3, H)
    elif kind == "monarch":
        assert tuple(W.shape) == (3, 4, H // 4, H // 4)
    else:
        assert tuple(W.shape) == (3, 2, 5, 16, 2, 2)
    if bias:
        assert torch.equal(bh, torch.cat([cell.b_hr, cell.b_hz, cell.b_hn]))
    else:
        assert torch.equal(bh, torch.zeros(3 * H)) and bh.dtype == W.dtype
    # the stacked tensors stay connected to the cell's parameters
    (W.sum() + 2 * bh.sum()).backward()
    for gate in "rzn":
        m = getattr(cell, f"struct_Wh_{gate}")
        grad = m.b.twiddle.grad if kind == "butterfly" else m.weight.grad
        assert grad is not None and torch.equal(grad, torch.ones_like(grad))
        if bias:
            assert torch.equal(getattr(cell, f"b_h{gate}").grad, torch.full((H,), 2.0))


@pytest.mark.parametrize("kind", list(EXTRACT))
def test_extract_refuses_a_dense_hidden_side(kind):
    extract = getattr(importlib.import_module(EXTRACT[kind][0]), EXTRACT[kind][1])
    cell = make_cell(kind, 16)
    cell._hidden_dense = True
    with pytest.raises(ValueError, match="dense"):
        extract(cell)
