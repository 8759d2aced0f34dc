"""CPU oracle for the persistent GRU scan -- TEST INFRASTRUCTURE ONLY.

This module restates, in plain PyTorch on the CPU, the reference path that
the HIP kernels must match (LarocheC/gru-triton, the per-step
``GRUCellQuant`` path). Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
or the timed CPU baseline; the product path (``gru_qat_amd``) never calls it.

Functions and what they follow (reference file:line):
  fake_quant       src/gru_qat/ste.py:65-95 (q = round(x/s + zp), clamp, (q - zp)*s,
                   zp = 0) as used by FakeQuantize.forward, quantizers.py:89-96
  gru_step         src/gru_qat/gru_cell.py:437-464 (step_with_gi), gate order r, z, n,
                   raw h on the carry side, q_out before the carry
  gh_dense         gru_cell.py:453 (F.linear(hq, Wh_cat, bh_cat)), scan.py:1500
  gh_diagonal      triton_kernels/scan_diagonal.py:110-115, structure.py:213-217
  gh_monarch       triton_kernels/scan_monarch.py:107-113
  gh_monarch2      build-defined two-factor form P^T L P R (no reference counterpart)
  gh_circulant     structure.py:220-240 (_CirculantLinear: y = irfft(rfft(col) * rfft(x))),
                   restated as the circular convolution y[i] = sum_j col[(i - j) mod H] x[j]
  butterfly_apply  triton_kernels/scan_butterfly.py:276-317 (stage order, stride
                   direction per chain, pair index and twiddle element selection)
  scan             the T-step loops of scan_diagonal.py:79-124 / scan_monarch.py:74-127 /
                   gru_layer.py:212-223
  scan_backward    triton_kernels/scan.py:1450-1550 (_fake_quant and the recompute-based
                   _gru_scan_backward_pytorch): reverse walk, gates recomputed from
                   out[t-1], clipped-STE masks on q_out and q_in, dW accumulated against hq
  scan_ste         the forward with ste.py:17-95's STERound/STEClamp gradients, the
                   independent derivation scan_backward is pinned against (autograd)
  weight_fake_quant_rows
                   quantizers.py:188-199 (per-channel min/max over every dim but axis 0)
                   and :124-134 (symmetric: scale = max(|max|, |min|).clamp(1e-8) / qmax,
                   zp = 0), then ste.py:65-95
  input_projection gru_layer.py:249-255 (xq = quant_x(x); Wi_cat = quantize_input_weights();
                   gi = F.linear(xq, Wi_cat, bi_cat)); with ste=True torch's autograd of the
                   reference quantizers: clipped STE on x (frozen scale), and the dynamic
                   per-row weight quantizer through fake_quant_rows_dynamic
  fake_quant_rows_dynamic
                   FakeQuantizePerChannel on axis 0 in dynamic mode (quantizers.py:188-199,
                   :124-134) into fake_quant_ste (ste.py:17-95, STERound / STEClamp): the scale
                   is computed from the tensor and not detached, so autograd carries gradient
                   through it to each row's max and min
  structured_input_projection
                   gru_cell.py:466-503: per gate quant_struct_Wi_g(struct_Wi_g(quant_x(x))) + b_ig,
                   concatenated r, z, n; the per-gate maps are the hidden-side kinds
  ObserverState, observer_forward, scale_zp_from_min_max, update_observer, freeze_observer
                   quantizers.py:63-156 and :176-181 (per-tensor FakeQuantize: modes frozen,
                   dynamic, min_max; scale and zero point from a min and max, symmetric or
                   affine; the running-statistics update with momentum 0.99; freeze)
  observe_scan     the per-step path with quant_h_in/quant_h_out firing (gru_layer.py:212-223
                   over step_with_gi, gru_cell.py:437-464), as GRULayer.calibrate
                   (gru_layer.py:308-336) runs it

Pins (tests/test_oracle.py; the backward in tests/test_oracle_backward.py
against torch.autograd through scan_ste, in float64): round-half-even and clipping known answers
(tests/test_ste.py:12-61 of the reference), an exhaustive boundary sweep of
fake_quant against exact rational arithmetic, nn.GRUCell closed forms for the
dense, diagonal and Monarch maps (weight_ih = I, weight_hh = the materialised
hidden map), an independent permutation-matrix construction of the
two-factor Monarch map and its reduction to the single-factor map, identity
and single-stage closed forms of the butterfly, float64 brute force, and
golden vectors produced from the reference's own butterfly kernel
(tests/golden/). The observers (tests/test_oracle_observe.py): frozen and off
modes reduce observe_scan to scan; known answers of the symmetric and affine
scale rules; the code-range invariants of a dynamic quantizer (a symmetric
one puts its largest |x| on code +-qmax, an affine one spans [qmin, qmax]);
the running statistics against their float64 recursion; freeze against the
scale rule applied by hand.
"""

from __future__ import annotations

from typing import Callable, Optional, Tuple

import torch
import torch.nn.functional as F

QuantTuple = Optional[Tuple[float, int, int]]


def fake_quant(x: torch.Tensor, q: QuantTuple) -> torch.Tensor:
    """Frozen per-tensor symmetric fake-quant with the reference's op order."""
    if q is None:
        return x
    scale, qmin, qmax = q
    s = torch.tensor(scale, dtype=x.dtype)
    zp = torch.tensor(0.0, dtype=x.dtype)
    v = torch.round(x / s + zp)
    v = torch.clamp(v, qmin, qmax)
    return (v - zp) * s


def quant_codes(x: torch.Tensor, q: Tuple[float, int, int]) -> torch.Tensor:
    """Integer codes clamp(round(x / s)) as fp32 (the reference never
    materialises int8; codes are integer-valued floats)."""
    scale, qmin, qmax = q
    s = torch.tensor(scale, dtype=x.dtype)
    return torch.clamp(torch.round(x / s), qmin, qmax)


def gru_step(gi_t: torch.Tensor, h: torch.Tensor, gh: torch.Tensor) -> torch.Tensor:
    """One GRU update from the two projections; returns the pre-q_out h."""
    gi_r, gi_z, gi_n = gi_t.chunk(3, dim=-1)
    gh_r, gh_z, gh_n = gh.chunk(3, dim=-1)
    r = torch.sigmoid(gi_r + gh_r)
    z = torch.sigmoid(gi_z + gh_z)
    n = torch.tanh(gi_n + r * gh_n)
    return (1.0 - z) * n + z * h


# ---- hidden maps (include bias) -----------------------------------------------------

def gh_dense(hq: torch.Tensor, Wh_cat: torch.Tensor, bh: torch.Tensor) -> torch.Tensor:
    return F.linear(hq, Wh_cat, bh)


def gh_diagonal(hq: torch.Tensor, Wh_diag: torch.Tensor, bh: torch.Tensor) -> torch.Tensor:
    H = hq.shape[-1]
    b = bh.view(3, H)
    return torch.cat([Wh_diag[0] * hq + b[0], Wh_diag[1] * hq + b[1], Wh_diag[2] * hq + b[2]], dim=-1)


def gh_monarch(hq: torch.Tensor, Wh_struct: torch.Tensor, bh: torch.Tensor) -> torch.Tensor:
    B, H = hq.shape
    _, nb, bs, _ = Wh_struct.shape
    gh = torch.einsum("bni,gnoi->bgno", hq.view(B, nb, bs), Wh_struct)
    return (gh.reshape(B, 3, H) + bh.view(3, H)).reshape(B, 3 * H)


def monarch_perm(nb: int, bs: int) -> torch.Tensor:
    """perm[c * nb + a] = a * bs + c, so (P z) = z[perm]."""
    c = torch.arange(bs).repeat_interleave(nb)
    a = torch.arange(nb).repeat(bs)
    return a * bs + c


def gh_monarch2(hq: torch.Tensor, R: torch.Tensor, L: torch.Tensor, bh: torch.Tensor) -> torch.Tensor:
    B, H = hq.shape
    _, nb, bs, _ = R.shape
    perm = monarch_perm(nb, bs)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(H)
    z = torch.einsum("bni,gnoi->bgno", hq.view(B, nb, bs), R).reshape(B, 3, H)
    u = z[:, :, perm]
    v = torch.einsum("bgni,gnoi->bgno", u.reshape(B, 3, nb, bs), L).reshape(B, 3, H)
    y = v[:, :, inv]
    return (y + bh.view(3, H)).reshape(B, 3 * H)


def circulant_matrix(col: torch.Tensor) -> torch.Tensor:
    """C [H, H] with C[i][j] = col[(i - j) mod H]: y = C x is the circular
    convolution of col and x."""
    H = col.shape[-1]
    idx = (torch.arange(H).unsqueeze(1) - torch.arange(H).unsqueeze(0)) % H
    return col[idx]


def gh_circulant(hq: torch.Tensor, Wh_circ: torch.Tensor, bh: torch.Tensor) -> torch.Tensor:
    """structure.py:220-240 for the three gates: [C(col_r) hq; C(col_z) hq; C(col_n) hq] + bh."""
    parts = [hq @ circulant_matrix(Wh_circ[g]).t() for g in range(3)]
    return torch.cat(parts, dim=-1) + bh


def butterfly_apply(x: torch.Tensor, tw_g: torch.Tensor) -> torch.Tensor:
    """One gate's butterfly on rows of x [B, N]; tw_g is [nchains, L, N/2, 2, 2]."""
    nchains, L, n2 = tw_g.shape[0], tw_g.shape[1], tw_g.shape[2]
    N = 2 * n2
    i = torch.arange(N)
    for c in range(nchains):
        for s in range(L):
            ls = s if c % 2 == 0 else L - 1 - s
            stride = 1 << ls
            partner = i ^ stride
            m = (i >> ls) & 1
            pair = (i >> (ls + 1)) * stride + (i & (stride - 1))
            t_ss = tw_g[c, s, pair, m, m]
            t_sp = tw_g[c, s, pair, m, 1 - m]
            x = t_ss * x + t_sp * x[:, partner]
    return x


def gh_butterfly(hq: torch.Tensor, twiddles: torch.Tensor, bh: torch.Tensor) -> torch.Tensor:
    B, H = hq.shape
    N = 2 * twiddles.shape[3]
    xp = F.pad(hq, (0, N - H))
    parts = [butterfly_apply(xp, twiddles[g])[:, :H] for g in range(3)]
    return torch.cat(parts, dim=-1) + bh


# ---- scans --------------------------------------------------------------------------

GhFn = Callable[[torch.Tensor], torch.Tensor]


def scan(gi: torch.Tensor, h0: torch.Tensor, gh_fn: GhFn, h_in_quant: QuantTuple = None,
         h_out_quant: QuantTuple = None) -> torch.Tensor:
    T = gi.shape[0]
    out = torch.empty(T, *h0.shape, dtype=gi.dtype)
    h = h0
    for t in range(T):
        h_new = gru_step(gi[t], h, gh_fn(fake_quant(h, h_in_quant)))
        h_new = fake_quant(h_new, h_out_quant)
        out[t] = h_new
        h = h_new
    return out


def gh_fn_for(cfg: dict) -> GhFn:
    kind = cfg["kind"]
    w, bh = cfg["w"], cfg["bh"]
    if kind == "dense":
        return lambda hq: gh_dense(hq, w, bh)
    if kind == "diagonal":
        return lambda hq: gh_diagonal(hq, w, bh)
    if kind == "monarch":
        if cfg.get("w2") is not None:
            w2 = cfg["w2"]
            return lambda hq: gh_monarch2(hq, w, w2, bh)
        return lambda hq: gh_monarch(hq, w, bh)
    if kind == "butterfly":
        return lambda hq: gh_butterfly(hq, w, bh)
    if kind == "circulant":
        return lambda hq: gh_circulant(hq, w, bh)
    raise ValueError(kind)


def _cpu(cfg: dict) -> dict:
    return {k: (v.detach().cpu() if isinstance(v, torch.Tensor) else v) for k, v in cfg.items()}


def scan_config(cfg: dict) -> torch.Tensor:
    """Runs the oracle on a config dict (see gru_qat_amd.configs); CPU tensors."""
    c = _cpu(cfg)
    return scan(c["gi"], c["h0"], gh_fn_for(c), c.get("h_in_quant"), c.get("h_out_quant"))


def teacher_forced_prequant(cfg: dict, out_kernel: torch.Tensor) -> torch.Tensor:
    """Pre-q_out hidden state of every step, computed by the oracle from the
    kernel's own previous output (h_{t-1} = out_kernel[t-1], h_{-1} = h0).

    Comparing quant codes of this against the kernel's codes checks every step
    in isolation, so one boundary flip cannot propagate into later steps.
    """
    c = _cpu(cfg)
    gi, h0 = c["gi"], c["h0"]
    ok = out_kernel.detach().cpu()
    gh_fn = gh_fn_for(c)
    T = gi.shape[0]
    pre = torch.empty_like(ok)
    for t in range(T):
        h = h0 if t == 0 else ok[t - 1]
        pre[t] = gru_step(gi[t], h, gh_fn(fake_quant(h, c.get("h_in_quant"))))
    return pre


def materialize_hidden(cfg: dict) -> torch.Tensor:
    """The hidden map of a config as a dense [3H, H] matrix (gh = hq @ M.T + bh),
    obtained by pushing identity rows through the oracle's map."""
    c = _cpu(cfg)
    H = c["H"] if "H" in c else c["h0"].shape[-1]
    eye = torch.eye(H, dtype=c["bh"].dtype)
    zero_b = torch.zeros_like(c["bh"])
    cz = dict(c)
    cz["bh"] = zero_b
    return gh_fn_for(cz)(eye).t().contiguous()


# ---- backward ---------------------------------------------------------------------

def fake_quant_mask(x: torch.Tensor, q: Tuple[float, int, int]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Forward fake-quant and the clipped-STE mask (scan.py:1450-1457):
    mask = round(x / s) inside [qmin, qmax]."""
    scale, qmin, qmax = q
    s = torch.tensor(scale, dtype=x.dtype)
    qu = torch.round(x / s)
    mask = (qu >= qmin) & (qu <= qmax)
    return qu.clamp(qmin, qmax) * s, mask


class _FakeQuantSTE(torch.autograd.Function):
    """fake_quant with the reference's gradient: STERound is the identity and
    STEClamp passes the gradient where round(x / s) lies in [qmin, qmax]
    (ste.py:17-63), so d out / d x = mask."""

    @staticmethod
    def forward(ctx, x, scale, qmin, qmax):  # type: ignore[override]
        xq, mask = fake_quant_mask(x, (scale, qmin, qmax))
        ctx.save_for_backward(mask)
        return xq

    @staticmethod
    def backward(ctx, g):  # type: ignore[override]
        (mask,) = ctx.saved_tensors
        return g * mask, None, None, None


def fake_quant_ste(x: torch.Tensor, q: QuantTuple) -> torch.Tensor:
    return x if q is None else _FakeQuantSTE.apply(x, *q)


class _STERound(torch.autograd.Function):
    """ste.py:17-37: round half to even forward, identity backward."""

    @staticmethod
    def forward(ctx, x):  # type: ignore[override]
        return torch.round(x)

    @staticmethod
    def backward(ctx, g):  # type: ignore[override]
        return g


class _STEClamp(torch.autograd.Function):
    """ste.py:40-62: clamp forward, gradient only inside [qmin, qmax]."""

    @staticmethod
    def forward(ctx, x, qmin, qmax):  # type: ignore[override]
        ctx.save_for_backward(x)
        ctx.qmin, ctx.qmax = qmin, qmax
        return torch.clamp(x, qmin, qmax)

    @staticmethod
    def backward(ctx, g):  # type: ignore[override]
        (x,) = ctx.saved_tensors
        return g * ((x >= ctx.qmin) & (x <= ctx.qmax)), None, None


def fake_quant_rows_dynamic(W: torch.Tensor, qmin: int, qmax: int) -> torch.Tensor:
    """Per-row (axis 0) symmetric fake-quant with the scale computed from W
    itself, differentiable as the reference's autograd differentiates it:
    FakeQuantizePerChannel._compute_scale_zp (quantizers.py:188-199: amin and
    amax over every dim but 0, keepdim), the symmetric rule (:124-134: scale =
    max(|max|, |min|).clamp(1e-8) / qmax, zp = zeros_like(scale)) and
    fake_quant_ste (ste.py:65-95: (STEClamp(STERound(W / scale + zp)) - zp) *
    scale). Nothing is detached, so the gradient also flows through the scale."""
    x_min = W.amin(dim=1, keepdim=True)
    x_max = W.amax(dim=1, keepdim=True)
    absmax = torch.maximum(x_max.abs(), x_min.abs()).clamp(min=1e-8)
    scale = absmax / qmax
    zp = torch.zeros_like(scale)
    q = _STERound.apply(W / scale + zp)
    q = _STEClamp.apply(q, qmin, qmax)
    return (q - zp) * scale


def hidden_params(cfg: dict) -> Tuple[str, ...]:
    """Keys of the hidden-map parameters of a config (w, and w2 for two-factor Monarch)."""
    return ("w", "w2") if cfg.get("w2") is not None else ("w",)


def gh_map_nobias(cfg: dict) -> Callable[..., torch.Tensor]:
    """The hidden map without bias as a function of (hq, *params) for the keys
    of hidden_params(cfg); differentiable in every argument."""
    kind = cfg["kind"]
    if kind == "dense":
        return lambda hq, w: hq @ w.t()
    if kind == "diagonal":
        return lambda hq, w: (w.unsqueeze(1) * hq.unsqueeze(0)).permute(1, 0, 2).reshape(hq.shape[0], -1)
    if kind == "monarch":
        zero = torch.zeros(3 * cfg["h0"].shape[-1], dtype=cfg["gi"].dtype)
        if cfg.get("w2") is not None:
            return lambda hq, w, w2: gh_monarch2(hq, w, w2, zero)
        return lambda hq, w: gh_monarch(hq, w, zero)
    if kind == "butterfly":
        zero = torch.zeros(3 * cfg["h0"].shape[-1], dtype=cfg["gi"].dtype)
        return lambda hq, w: gh_butterfly(hq, w, zero)
    if kind == "circulant":
        zero = torch.zeros(3 * cfg["h0"].shape[-1], dtype=cfg["gi"].dtype)
        return lambda hq, w: gh_circulant(hq, w, zero)
    raise ValueError(kind)


def scan_ste(cfg: dict) -> torch.Tensor:
    """Differentiable forward (STE on both quantizers): the autograd pin for
    scan_backward. cfg tensors may require grad."""
    gi, h0, bh = cfg["gi"], cfg["h0"], cfg["bh"]
    params = [cfg[k] for k in hidden_params(cfg)]
    gmap = gh_map_nobias(cfg)
    qin, qout = cfg.get("h_in_quant"), cfg.get("h_out_quant")
    h = h0
    outs = []
    for t in range(gi.shape[0]):
        hq = fake_quant_ste(h, qin)
        h_new = gru_step(gi[t], h, gmap(hq, *params) + bh)
        h = fake_quant_ste(h_new, qout)
        outs.append(h)
    return torch.stack(outs, dim=0)


def scan_backward(cfg: dict, out: torch.Tensor, dout: torch.Tensor, _mutation: str = "") -> dict:
    """Restates _gru_scan_backward_pytorch (scan.py:1460-1550) for every hidden
    kind: walk t from T-1 to 0, recompute the gates from h_{t-1} = out[t-1]
    (h0 at t = 0), push dout[t] plus the carried gradient through q_out's mask,
    the gate derivatives and the hidden map, and carry
    dh_{t-1} = dh_t * z + mask_in * (d gh / d hq)^T dgh. The hidden map's
    vector-Jacobian products (with respect to hq and to its parameters) come
    from autograd on the map, which for the dense kind are dgh @ Wh_cat and
    dgh^T @ hq exactly as in the reference.

    Returns {"dgi", "dh0", "dbh", "d<param key>" ...}; CPU tensors.
    ``_mutation`` plants a known mistake for the tests that show the autograd
    pin catches it: "dgh_n_without_r" or "ignore_mask_in".
    """
    c = _cpu(cfg)
    gi, h0, bh = c["gi"], c["h0"], c["bh"]
    out = out.detach().cpu()
    dout = dout.detach().cpu()
    keys = hidden_params(c)
    params = [c[k] for k in keys]
    gmap = gh_map_nobias(c)
    qin, qout = c.get("h_in_quant"), c.get("h_out_quant")
    T = gi.shape[0]
    H = h0.shape[-1]
    dgi = torch.zeros_like(gi)
    dparams = [torch.zeros_like(p) for p in params]
    dbh = torch.zeros_like(bh)
    dh_acc = torch.zeros_like(h0)
    for t in reversed(range(T)):
        h_prev = h0 if t == 0 else out[t - 1]
        if qin is not None:
            hq, mask_in = fake_quant_mask(h_prev, qin)
        else:
            hq, mask_in = h_prev, None
        with torch.enable_grad():
            hq_req = hq.detach().requires_grad_(True)
            p_req = [p.detach().requires_grad_(True) for p in params]
            gh_nob = gmap(hq_req, *p_req)
        gh = gh_nob.detach() + bh
        gi_r, gi_z, gi_n = gi[t].split(H, dim=-1)
        gh_r, gh_z, gh_n = gh.split(H, dim=-1)
        r = torch.sigmoid(gi_r + gh_r)
        z = torch.sigmoid(gi_z + gh_z)
        n = torch.tanh(gi_n + r * gh_n)
        h_raw = (1.0 - z) * n + z * h_prev
        dh_t = dout[t] + dh_acc
        if qout is not None:
            dh_t = dh_t * fake_quant_mask(h_raw, qout)[1]
        dn = dh_t * (1.0 - z)
        dz = dh_t * (h_prev - n)
        dh_direct = dh_t * z
        dgn = dn * (1.0 - n * n)
        dr = dgn * gh_n
        dgh_n = dgn if _mutation == "dgh_n_without_r" else dgn * r
        dgz = dz * z * (1.0 - z)
        dgr = dr * r * (1.0 - r)
        dgi[t] = torch.cat([dgr, dgz, dgn], dim=-1)
        dgh = torch.cat([dgr, dgz, dgh_n], dim=-1)
        grads = torch.autograd.grad(gh_nob, [hq_req] + p_req, dgh)
        dh_via = grads[0] if (mask_in is None or _mutation == "ignore_mask_in") else grads[0] * mask_in
        for acc, g in zip(dparams, grads[1:]):
            acc += g
        dbh += dgh.sum(dim=0)
        dh_acc = dh_direct + dh_via
    res = {"dgi": dgi, "dh0": dh_acc, "dbh": dbh}
    for k, d in zip(keys, dparams):
        res["d" + k] = d
    return res


# ---- input projection ----------------------------------------------------------------

def weight_fake_quant_rows(W: torch.Tensor, qmin: int, qmax: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row symmetric fake-quant of W [N, I]; returns (W_q, scale [N])."""
    x_min = W.amin(dim=1, keepdim=True)
    x_max = W.amax(dim=1, keepdim=True)
    absmax = torch.maximum(x_max.abs(), x_min.abs()).clamp(min=1e-8)
    scale = absmax / qmax
    q = torch.round(W / scale).clamp(qmin, qmax)
    return q * scale, scale.view(-1)


def input_projection(x: torch.Tensor, W: torch.Tensor, b: Optional[torch.Tensor], x_quant: QuantTuple = None,
                     w_quant: Optional[Tuple[int, int]] = None, ste: bool = False) -> torch.Tensor:
    """gi = F.linear(q_x(x), W_q, b) on x [..., I]."""
    if x_quant is not None:
        xq = fake_quant_ste(x, x_quant) if ste else fake_quant(x, x_quant)
    else:
        xq = x
    if w_quant is not None:
        W = fake_quant_rows_dynamic(W, w_quant[0], w_quant[1]) if ste else \
            weight_fake_quant_rows(W, w_quant[0], w_quant[1])[0]
    return F.linear(xq, W, b)


def _out_quant(y: torch.Tensor, oq, ste: bool) -> torch.Tensor:
    """One gate's output quantizer: None, a frozen per-tensor (scale, qmin,
    qmax) or ("rows", qmin, qmax), the dynamic per-row quantizer."""
    if oq is None:
        return y
    if oq[0] == "rows":
        return fake_quant_rows_dynamic(y, oq[1], oq[2]) if ste else \
            fake_quant_rows_dynamic(y.detach(), oq[1], oq[2]).detach()
    return fake_quant_ste(y, oq) if ste else fake_quant(y, oq)


def structured_input_projection(x: torch.Tensor, kind: str, w: torch.Tensor, b: Optional[torch.Tensor],
                                x_quant: QuantTuple = None, out_quant=(None, None, None),
                                ste: bool = False, y_value: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gi [..., 3H] of a structured input side (gru_cell.py:466-503): q_x over
    the whole sequence, each gate's map (the hidden-side map of ``kind`` with
    weights w, input size = H), the gate's output quantizer (_out_quant), its
    bias, concatenation r, z, n.

    ``y_value`` (optional, [N, 3H]) replaces the maps' output values while
    keeping their gradient: the output quantizers then see exactly the values
    a kernel under test produced (teacher forcing), so a backward can be
    checked without the rounding-boundary flips that a different summation
    order causes in the forward."""
    H = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, H)
    xq = (fake_quant_ste(x2, x_quant) if ste else fake_quant(x2, x_quant)) if x_quant is not None else x2
    cfg = {"kind": kind, "w": w, "h0": torch.zeros(1, H, dtype=x.dtype), "gi": torch.zeros(1, 1, 3 * H, dtype=x.dtype)}
    y = gh_map_nobias(cfg)(xq, w)
    if y_value is not None:
        y = y + (y_value.reshape(y.shape).to(y.dtype) - y).detach()
    parts = []
    for g in range(3):
        o = _out_quant(y[:, g * H:(g + 1) * H], out_quant[g], ste)
        if b is not None:
            o = o + b[g * H:(g + 1) * H]
        parts.append(o)
    return torch.cat(parts, dim=-1).reshape(*lead, 3 * H)



# ---- observers (calibration) -----------------------------------------------------------

class ObserverState:
    """A per-tensor FakeQuantize's state (quantizers.py:63-96): mode
    ("off", "frozen", "dynamic", "min_max"), the range of _qrange
    (quantizers.py:119-122), the frozen scale and zero point and the running
    statistics."""

    def __init__(self, mode: str, bits: int = 8, symmetric: bool = True, scale: float = 1.0,
                 zero_point: float = 0.0) -> None:
        self.mode = mode
        self.symmetric = symmetric
        if symmetric:
            self.qmin, self.qmax = -(2 ** (bits - 1)) + 1, 2 ** (bits - 1) - 1
        else:
            self.qmin, self.qmax = 0.0, 2.0**bits - 1.0
        self.scale = torch.tensor(scale, dtype=torch.float32)
        self.zero_point = torch.tensor(zero_point, dtype=torch.float32)
        self.running_min = torch.tensor(float("inf"))
        self.running_max = torch.tensor(float("-inf"))
        self.initialized = False


def scale_zp_from_min_max(st: ObserverState, x_min: torch.Tensor,
                          x_max: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """quantizers.py:124-134."""
    if st.symmetric:
        absmax = torch.maximum(x_max.abs(), x_min.abs()).clamp(min=1e-8)
        scale = absmax / st.qmax
        zp = torch.zeros_like(scale)
    else:
        scale = (x_max - x_min).clamp(min=1e-8) / (st.qmax - st.qmin)
        zp = torch.round(st.qmin - x_min / scale)
    return scale, zp


def update_observer(st: ObserverState, x: torch.Tensor) -> None:
    """The per-tensor branch of _update_observer (quantizers.py:136-156)."""
    cur_min = x.detach().min()
    cur_max = x.detach().max()
    if not st.initialized:
        st.running_min = cur_min
        st.running_max = cur_max
        st.initialized = True
    else:
        momentum = 0.99
        st.running_min = momentum * st.running_min + (1 - momentum) * cur_min
        st.running_max = momentum * st.running_max + (1 - momentum) * cur_max


def observer_forward(st: ObserverState, x: torch.Tensor) -> Tuple[torch.Tensor, Tuple[float, float]]:
    """FakeQuantize.forward (quantizers.py:84-96) with FakeQuantizePerTensor's
    scale rule (:176-181) and fake_quant_ste's forward (ste.py:65-95); returns
    the output and the (scale, zero point) applied."""
    if st.mode == "off":
        return x, (1.0, 0.0)
    if st.mode == "frozen":
        scale, zp = st.scale, st.zero_point
    else:
        scale, zp = scale_zp_from_min_max(st, x.min(), x.max())
        if st.mode == "min_max":
            update_observer(st, x)
    q = torch.round(x / scale + zp)
    q = torch.clamp(q, st.qmin, st.qmax)
    return (q - zp) * scale, (float(scale), float(zp))


def freeze_observer(st: ObserverState) -> None:
    """FakeQuantize.freeze (quantizers.py:98-107)."""
    if st.mode == "min_max":
        st.scale, st.zero_point = scale_zp_from_min_max(st, st.running_min, st.running_max)
    st.mode = "frozen"


def observe_scan(gi: torch.Tensor, h0: torch.Tensor, gh_fn: GhFn, q_in: ObserverState,
                 q_out: ObserverState) -> Tuple[torch.Tensor, torch.Tensor]:
    """The per-step path with quant_h_in / quant_h_out firing
    (gru_layer.py:212-223 over step_with_gi, gru_cell.py:437-464); returns out
    [T, B, H] and the (scale, zp) of q_in and q_out used per step [T, 4]."""
    T = gi.shape[0]
    out = torch.empty(T, *h0.shape, dtype=gi.dtype)
    trace = torch.empty(T, 4, dtype=torch.float32)
    h = h0
    for t in range(T):
        hq, (si, zi) = observer_forward(q_in, h)
        h_new = gru_step(gi[t], h, gh_fn(hq))
        h_new, (so, zo) = observer_forward(q_out, h_new)
        out[t] = h_new
        trace[t] = torch.tensor([si, zi, so, zo])
        h = h_new
    return out, trace
