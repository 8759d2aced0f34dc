"""ctypes binding of libgruscan.so (the C ABI declared in include/gruscan.h).

The library is built in-tree by ``make -C gru-triton_amd/csrc`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing
or cannot be loaded, every scan entry point raises ``RuntimeError``.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import struct
import threading
import weakref
from typing import Callable, Optional, Tuple

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgruscan.so")

GS_OK = 0
GS_ERR_INVALID = -1
GS_ERR_CAPACITY = -2
GS_ERR_HIP = -3

KIND_DENSE = 0
KIND_DIAGONAL = 1
KIND_MONARCH = 2
KIND_BUTTERFLY = 3
KIND_CIRCULANT = 4
KIND_DENSE_TILED = 5  # size queries of the batch-tiled dense entry points

# Every symbol include/gruscan.h declares.
EXPORTS = (
    "gs_dense_fwd",
    "gs_dense_fwd_tiled",
    "gs_dense_fwd_i8w",
    "gs_dense_fwd_tiled_i8w",
    "gs_weight_codes",
    "gs_dense_fwd_noalloc",
    "gs_diagonal_fwd",
    "gs_monarch_fwd",
    "gs_circulant_fwd",
    "gs_butterfly_fwd",
    "gs_butterfly_fwd_generic",
    "gs_diagonal_bwd",
    "gs_dense_bwd",
    "gs_dense_bwd_tiled",
    "gs_monarch_bwd",
    "gs_butterfly_bwd",
    "gs_input_proj",
    "gs_input_proj_bwd",
    "gs_input_proj_bwd_workspace_bytes",
    "gs_struct_input_proj",
    "gs_struct_input_proj_scratch_bytes",
    "gs_struct_input_proj_bwd",
    "gs_struct_input_proj_bwd_scratch_bytes",
    "gs_quantize_rows",
    "gs_hidden_map_dense",
    "gs_hidden_map_scratch_bytes",
    "gs_hidden_map_grad",
    "gs_observe_tensor",
    "gs_observe_tensor_scratch_bytes",
    "gs_observe_scan",
    "gs_observe_scan_scratch_bytes",
    "gs_workspace_bytes",
    "gs_bwd_workspace_bytes",
    "gs_bwd_scratch_bytes",
    "gs_workspace_status",
    "gs_last_error",
    "gs_abi_version",
)

ABI_VERSION = 5

QuantTuple = Optional[Tuple[float, int, int]]


class GsQuant(ctypes.Structure):
    _fields_ = [
        ("enabled", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("qmin", ctypes.c_int32),
        ("qmax", ctypes.c_int32),
    ]


class GsArgs(ctypes.Structure):
    _fields_ = [
        ("gi", ctypes.c_void_p),
        ("h0", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("bh", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("fault_mirror", ctypes.c_void_p),
        ("T", ctypes.c_int64),
        ("B", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("sg_t", ctypes.c_int64),
        ("sg_b", ctypes.c_int64),
        ("sh0_b", ctypes.c_int64),
        ("so_t", ctypes.c_int64),
        ("so_b", ctypes.c_int64),
        ("nblocks", ctypes.c_int64),
        ("blksz", ctypes.c_int64),
        ("log_n", ctypes.c_int64),
        ("bfly_nblocks", ctypes.c_int64),
        ("q_in", GsQuant),
        ("q_out", GsQuant),
        ("gh_save", ctypes.c_void_p),
    ]


class GsBwdArgs(ctypes.Structure):
    _fields_ = [
        ("gi", ctypes.c_void_p),
        ("h0", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("bh", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("dgi", ctypes.c_void_p),
        ("dh0", ctypes.c_void_p),
        ("dw_part", ctypes.c_void_p),
        ("dw2_part", ctypes.c_void_p),
        ("dbh_part", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("fault_mirror", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_int64),
        ("T", ctypes.c_int64),
        ("B", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("sg_t", ctypes.c_int64),
        ("sg_b", ctypes.c_int64),
        ("sh0_b", ctypes.c_int64),
        ("so_t", ctypes.c_int64),
        ("so_b", ctypes.c_int64),
        ("nblocks", ctypes.c_int64),
        ("blksz", ctypes.c_int64),
        ("log_n", ctypes.c_int64),
        ("bfly_nblocks", ctypes.c_int64),
        ("q_in", GsQuant),
        ("q_out", GsQuant),
        ("gh_saved", ctypes.c_void_p),
    ]


class GsProjArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("gi", ctypes.c_void_p),
        ("x_q", ctypes.c_void_p),
        ("w_q", ctypes.c_void_p),
        ("w_scale", ctypes.c_void_p),
        ("M", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("I", ctypes.c_int64),
        ("sx", ctypes.c_int64),
        ("sgi", ctypes.c_int64),
        ("q_x", GsQuant),
        ("q_w", GsQuant),
        ("x_codes", ctypes.c_void_p),
        ("w_codes", ctypes.c_void_p),
    ]


class GsProjBwdArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("x_q", ctypes.c_void_p),
        ("dgi", ctypes.c_void_p),
        ("dx", ctypes.c_void_p),
        ("dw", ctypes.c_void_p),
        ("dbias", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("M", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("I", ctypes.c_int64),
        ("sx", ctypes.c_int64),
        ("sdgi", ctypes.c_int64),
        ("sdx", ctypes.c_int64),
        ("q_x", GsQuant),
        ("w_raw", ctypes.c_void_p),
        ("w_scale", ctypes.c_void_p),
        ("q_w", GsQuant),
    ]


class GsOQuant(ctypes.Structure):
    _fields_ = [
        ("mode", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("qmin", ctypes.c_int32),
        ("qmax", ctypes.c_int32),
    ]


class GsSProjArgs(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("gi", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("y_scale", ctypes.c_void_p),
        ("x_q", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_int64),
        ("M", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("sx", ctypes.c_int64),
        ("sgi", ctypes.c_int64),
        ("nblocks", ctypes.c_int64),
        ("blksz", ctypes.c_int64),
        ("log_n", ctypes.c_int64),
        ("bfly_nblocks", ctypes.c_int64),
        ("q_x", GsQuant),
        ("q_out", GsOQuant * 3),
    ]


class GsSProjBwdArgs(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("x_q", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("y_scale", ctypes.c_void_p),
        ("dgi", ctypes.c_void_p),
        ("dx", ctypes.c_void_p),
        ("dw", ctypes.c_void_p),
        ("dbias", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_int64),
        ("M", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("sx", ctypes.c_int64),
        ("sdgi", ctypes.c_int64),
        ("sdx", ctypes.c_int64),
        ("nblocks", ctypes.c_int64),
        ("blksz", ctypes.c_int64),
        ("log_n", ctypes.c_int64),
        ("bfly_nblocks", ctypes.c_int64),
        ("q_x", GsQuant),
        ("q_out", GsOQuant * 3),
    ]


class GsRowsArgs(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("codes", ctypes.c_void_p),
        ("w_q", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("qmin", ctypes.c_int32),
        ("qmax", ctypes.c_int32),
    ]


class GsMapArgs(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("w", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("m", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("nblocks", ctypes.c_int64),
        ("blksz", ctypes.c_int64),
        ("log_n", ctypes.c_int64),
        ("bfly_nblocks", ctypes.c_int64),
    ]


OBS_OFF = 0
OBS_FROZEN = 1
OBS_DYNAMIC = 2
OBS_MIN_MAX = 3


class GsObserver(ctypes.Structure):
    _fields_ = [
        ("mode", ctypes.c_int32),
        ("symmetric", ctypes.c_int32),
        ("qmin", ctypes.c_int32),
        ("qmax", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("zero_point", ctypes.c_float),
        ("stats", ctypes.c_void_p),
    ]


class GsObserveTensorArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("used", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("ld", ctypes.c_int64),
        ("q", GsObserver),
    ]


class GsObserveArgs(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("gi", ctypes.c_void_p),
        ("h0", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("bh", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("trace", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_int64),
        ("T", ctypes.c_int64),
        ("B", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("sg_t", ctypes.c_int64),
        ("sg_b", ctypes.c_int64),
        ("sh0_b", ctypes.c_int64),
        ("so_t", ctypes.c_int64),
        ("so_b", ctypes.c_int64),
        ("nblocks", ctypes.c_int64),
        ("blksz", ctypes.c_int64),
        ("log_n", ctypes.c_int64),
        ("bfly_nblocks", ctypes.c_int64),
        ("q_in", GsObserver),
        ("q_out", GsObserver),
    ]


_lib = None
_lib_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libgruscan.so once (after torch, so it binds torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libgruscan.so not found at {LIB_PATH}; build it with "
                "`make -C gru-triton_amd/csrc` or __graft_entry__.build()"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name in ("gs_dense_fwd", "gs_dense_fwd_tiled", "gs_dense_fwd_noalloc", "gs_diagonal_fwd", "gs_monarch_fwd",
                     "gs_butterfly_fwd", "gs_butterfly_fwd_generic"):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.POINTER(GsArgs), ctypes.c_void_p]
            fn.restype = ctypes.c_int
        for name in ("gs_diagonal_bwd", "gs_dense_bwd", "gs_dense_bwd_tiled", "gs_monarch_bwd", "gs_butterfly_bwd"):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.POINTER(GsBwdArgs), ctypes.c_void_p]
            fn.restype = ctypes.c_int
        lib.gs_input_proj.argtypes = [ctypes.POINTER(GsProjArgs), ctypes.c_void_p]
        lib.gs_input_proj.restype = ctypes.c_int
        lib.gs_input_proj_bwd.argtypes = [ctypes.POINTER(GsProjBwdArgs), ctypes.c_void_p]
        lib.gs_input_proj_bwd.restype = ctypes.c_int
        lib.gs_input_proj_bwd_workspace_bytes.argtypes = [ctypes.POINTER(GsProjBwdArgs)]
        lib.gs_input_proj_bwd_workspace_bytes.restype = ctypes.c_int64
        for name, argt in (("gs_struct_input_proj", GsSProjArgs), ("gs_struct_input_proj_bwd", GsSProjBwdArgs)):
            run = getattr(lib, name)
            run.argtypes = [ctypes.POINTER(argt), ctypes.c_void_p]
            run.restype = ctypes.c_int
            size = getattr(lib, name + "_scratch_bytes")
            size.argtypes = [ctypes.POINTER(argt)]
            size.restype = ctypes.c_int64
        for name, argt in (("gs_hidden_map", GsMapArgs), ("gs_observe_tensor", GsObserveTensorArgs),
                           ("gs_observe_scan", GsObserveArgs)):
            run = getattr(lib, name if name != "gs_hidden_map" else "gs_hidden_map_dense")
            run.argtypes = [ctypes.POINTER(argt), ctypes.c_void_p]
            run.restype = ctypes.c_int
            size = getattr(lib, name + "_scratch_bytes")
            size.argtypes = [ctypes.POINTER(argt)]
            size.restype = ctypes.c_int64
        lib.gs_hidden_map_grad.argtypes = [ctypes.POINTER(GsMapArgs), ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_void_p]
        lib.gs_hidden_map_grad.restype = ctypes.c_int
        lib.gs_quantize_rows.argtypes = [ctypes.POINTER(GsRowsArgs), ctypes.c_void_p]
        lib.gs_quantize_rows.restype = ctypes.c_int
        lib.gs_weight_codes.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.gs_weight_codes.restype = ctypes.c_int
        lib.gs_workspace_bytes.argtypes = [ctypes.c_int, ctypes.POINTER(GsArgs)]
        lib.gs_workspace_bytes.restype = ctypes.c_int64
        lib.gs_bwd_workspace_bytes.argtypes = [ctypes.c_int, ctypes.POINTER(GsBwdArgs)]
        lib.gs_bwd_workspace_bytes.restype = ctypes.c_int64
        lib.gs_bwd_scratch_bytes.argtypes = [ctypes.c_int, ctypes.POINTER(GsBwdArgs)]
        lib.gs_bwd_scratch_bytes.restype = ctypes.c_int64
        lib.gs_workspace_status.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.gs_workspace_status.restype = ctypes.c_int
        lib.gs_last_error.argtypes = []
        lib.gs_last_error.restype = ctypes.c_char_p
        lib.gs_abi_version.argtypes = []
        lib.gs_abi_version.restype = ctypes.c_int
        if lib.gs_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"libgruscan.so ABI version {lib.gs_abi_version()} != expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
        return lib


_QUANT_OFF = GsQuant(0, 1.0, -(2**31), 2**31 - 1)


def make_quant(q: QuantTuple, name: str) -> GsQuant:
    if q is None:
        return _QUANT_OFF  # copied into the args struct on assignment
    try:
        scale, qmin, qmax = q
    except (TypeError, ValueError):
        raise ValueError(f"{name} must be None or a (scale, qmin, qmax) tuple; got {q!r}") from None
    return GsQuant(1, float(scale), int(qmin), int(qmax))


def raise_for(rc: int, lib: ctypes.CDLL) -> None:
    if rc == GS_OK:
        return
    msg = lib.gs_last_error().decode("utf-8", "replace")
    if rc == GS_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)


# ---- per-(device, stream) workspace cache ----------------------------------------
# A workspace is zeroed once when allocated. Every launch leaves its control
# words ready for the next launch ordered after it on the same stream, so
# launches on one stream share a workspace; distinct streams get distinct
# workspaces. The persistent kernels tag exchanged words with a 32-bit step
# counter kept in the workspace; before that counter could wrap, the
# workspace is zeroed again (the host mirrors the step count it has issued).
_ws_cache: dict = {}
_ws_steps: dict = {}
_ws_lock = threading.Lock()
_TAG_LIMIT = (1 << 32) - (1 << 24)

# ---- fault mirrors and cross-stream order of persistent launches -------------------
# Each (device, stream) has one pinned host word (torch's pinned allocator is
# hipHostMalloc) that the persistent kernels' last workgroup writes when a
# bounded wait of the launch gave up. The next persistent launch on that
# stream reads it (a host memory read, no synchronisation) and raises
# RuntimeError, so a launch that ran out of its wait cannot pass unnoticed;
# its output is NaN from the failed step on in any case.
_mirrors: dict = {}


class PersistentScanFault(RuntimeError):
    """A persistent scan launched earlier on this stream gave up a bounded
    wait: its workgroups were not all resident at once (another kernel held
    the device's CUs), and its output is NaN from the failed step on."""


def _mirror(dev: torch.device, stream_handle: int):
    key = (dev.index, stream_handle)
    m = _mirrors.get(key)
    if m is None:
        t = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        m = _mirrors[key] = (t, t.numpy())
    return m


def _raise_if_faulted(m, what: str) -> None:
    if m[1][0] != 0:
        value = int(m[1][0])
        m[1][0] = 0
        raise PersistentScanFault(
            f"{what}: a persistent scan launched earlier on this stream ran out of its bounded wait "
            f"(fault value {value}); its output is invalid (NaN from the failed step on). Another kernel "
            "holding the device's compute units while the scan ran is the usual cause.")


def check_faults(device: Optional[torch.device] = None) -> None:
    """Raises PersistentScanFault if a completed persistent launch on any
    stream of ``device`` (all devices when None) gave up a wait. Reads the
    host mirrors only: launches still running are not covered (use
    ``workspace_faults``, which synchronises, for those)."""
    for (dev, _), m in list(_mirrors.items()):
        if device is None or device.index == dev:
            _raise_if_faulted(m, "check_faults")


# Persistent scans on one device run one at a time: their grids fill the
# device, and two of them running at once would each wait for workgroups the
# other holds until their bounded waits give up. Launches on one stream are
# ordered already; when a persistent launch goes on a stream other than the
# device's previous one, that stream first waits for everything queued on the
# previous stream (torch's wait_stream: one event, recorded only on a switch).
# Entries are (raw stream handle, torch stream object); the object is built
# only when the device's persistent launches change streams.
_last_stream: dict = {}


def _order_after_previous(dev: torch.device, handle: int, current: Callable[[], "torch.cuda.Stream"]) -> None:
    prev = _last_stream.get(dev.index)
    if prev is not None and prev[0] == handle:
        return
    stream = current()
    if prev is not None:
        stream.wait_stream(prev[1])
    _last_stream[dev.index] = (handle, stream)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


_NO_SWITCH = contextlib.nullcontext()


def on_device(dev: torch.device):
    """torch.cuda.device(dev), or a no-op context when dev is already the
    current device (the common case; entering and leaving torch's context
    costs the host a few microseconds)."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _NO_SWITCH
    return torch.cuda.device(dev)


def current_stream_handle(dev: torch.device) -> int:
    """The raw handle of the current stream of `dev` (without building a
    torch Stream object, which costs the host about 2.5 us per call)."""
    if _raw_stream is not None:
        return int(_raw_stream(dev.index if dev.index is not None else torch.cuda.current_device()))
    return torch.cuda.current_stream(dev).cuda_stream


def workspace(device: torch.device, stream_handle: int, nbytes: int, steps: int = 0) -> torch.Tensor:
    key = (device.index, stream_handle)
    with _ws_lock:
        ws = _ws_cache.get(key)
        if ws is None or ws.numel() < nbytes:
            size = max(nbytes, 4096)
            if ws is not None:
                size = max(size, 2 * ws.numel())
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
            _ws_cache[key] = ws
            _ws_steps[key] = 0
        if steps:
            if _ws_steps[key] + steps + 1 >= _TAG_LIMIT:
                ws.zero_()
                _ws_steps[key] = 0
            _ws_steps[key] += steps
        return ws


def workspace_faults(device: Optional[torch.device] = None) -> int:
    """Read and clear the fault word of every cached workspace and its host
    mirror (synchronises each stream); returns how many were set.

    Nonzero means a persistent kernel ran out of its bounded wait and the output
    of that launch is invalid.
    """
    lib = load()
    total = 0
    with _ws_lock:
        items = list(_ws_cache.items())
    for (dev, stream_handle), ws in items:
        if device is not None and device.index != dev:
            continue
        rc = lib.gs_workspace_status(ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                     ctypes.c_void_p(stream_handle))
        if rc < 0:
            raise_for(rc, lib)
        total += rc
        m = _mirrors.get((dev, stream_handle))
        if m is not None:
            m[1][0] = 0
    return total


_FN_CACHE: dict = {}


def _entry(lib: ctypes.CDLL, fn_name: str):
    fn = _FN_CACHE.get(fn_name)
    if fn is None:
        fn = _FN_CACHE[fn_name] = getattr(lib, fn_name)
    return fn


def _check_gh(name: str, gh: torch.Tensor, gi: torch.Tensor) -> None:
    """gh_save / gh_saved must be a contiguous fp32 [T, B, 3H] tensor on gi's device."""
    if gh.shape != gi.shape or gh.dtype != torch.float32 or not gh.is_contiguous() or gh.device != gi.device:
        raise ValueError(f"{name} must be a contiguous float32 tensor of shape {tuple(gi.shape)} on {gi.device}; "
                         f"got {tuple(gh.shape)} {gh.dtype} on {gh.device}")


# gs_args packed by one call: 9 pointer / byte-count words, 12 int64 sizes and
# strides, the two gs_quant (int32, float, int32, int32), gh_save. The layout
# is that of the ctypes GsArgs above (checked bytewise by the CPU tests);
# building a ctypes Structure field by field cost the host about 4 us a call.
GS_ARGS = struct.Struct("<9Q12q" "ifii" "ifii" "Q")
_QOFF = (0, 1.0, -(2**31), 2**31 - 1)
_TAGGED = (KIND_DENSE, KIND_MONARCH, KIND_CIRCULANT)
_RAW_FN: dict = {}
_NEED: dict = {}  # workspace bytes per (kind, sizes, quant) of the tagged kinds


def _raw_entry(lib: ctypes.CDLL, fn_name: str):
    """The entry point as a function of (packed gs_args bytes, stream handle), or
    for the int8-weight entry points of (packed gs_args bytes, codes, scales, stream handle)."""
    fn = _RAW_FN.get(fn_name)
    if fn is None:
        fn = lib[fn_name]  # an independent function object: its argtypes do not touch getattr(lib, ...)
        if fn_name in ("gs_dense_fwd_i8w", "gs_dense_fwd_tiled_i8w"):
            fn.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        else:
            fn.argtypes = [ctypes.c_char_p, ctypes.c_void_p]
        fn.restype = ctypes.c_int
        _RAW_FN[fn_name] = fn
    return fn


# id(w) -> (weak reference to w, (data_ptr, _version), result); the entry goes
# when w does. (A WeakKeyDictionary would compare two tensors with ==.)
_CODES_CACHE: dict = {}


def weight_codes(w: torch.Tensor) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """Per-row int8 codes [rows, cols] and scales [rows] whose fp32 products
    reproduce the fake-quantized weight w [rows, cols] (fp32 on the GPU) element
    for element (``gs_weight_codes``), or None when a row is not such a product.
    Found once per version of w: the verdict costs one device-to-host read, and
    a frozen weight is not written again (any in-place write bumps ``_version``).
    Under HIP graph capture, where that read cannot happen, an uncached weight
    gets None (the fp32 kernels); a call before the capture caches it."""
    key = (w.data_ptr(), w._version)
    hit = _CODES_CACHE.get(id(w))
    if hit is not None and hit[0]() is w and hit[1] == key:
        return hit[2]
    if torch.cuda.is_current_stream_capturing():
        return None
    lib = _lib if _lib is not None else load()
    rows, cols = w.shape
    src = w.contiguous()
    codes = torch.empty((rows, cols), dtype=torch.int8, device=w.device)
    scale = torch.empty(rows, dtype=torch.float32, device=w.device)
    exact = torch.empty(rows, dtype=torch.int32, device=w.device)
    with torch.cuda.device(w.device):
        rc = lib.gs_weight_codes(src.data_ptr(), rows, cols, codes.data_ptr(), scale.data_ptr(), exact.data_ptr(),
                                 current_stream_handle(w.device))
    raise_for(rc, lib)
    res = (codes, scale) if bool(exact.all()) else None
    wid = id(w)
    _CODES_CACHE[wid] = (weakref.ref(w, lambda _r, wid=wid: _CODES_CACHE.pop(wid, None)), key, res)
    return res


def _qfields(q: QuantTuple, name: str) -> tuple:
    if q is None:
        return _QOFF
    try:
        scale, qmin, qmax = q
    except (TypeError, ValueError):
        raise ValueError(f"{name} must be None or a (scale, qmin, qmax) tuple; got {q!r}") from None
    return (1, float(scale), int(qmin), int(qmax))


def launch(kind: int, fn_name: str, *, gi: torch.Tensor, h0: torch.Tensor, w: torch.Tensor,
           w2: Optional[torch.Tensor], bh: torch.Tensor, out: torch.Tensor,
           h_in_quant: QuantTuple, h_out_quant: QuantTuple, nblocks: int = 0, blksz: int = 0,
           log_n: int = 0, bfly_nblocks: int = 0, gh_save: Optional[torch.Tensor] = None,
           contiguous: bool = False, w_codes: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
    """Fill gs_args from fp32 device tensors and call the entry point on the
    current torch stream of gi's device. contiguous: the caller guarantees that
    gi, h0 and out are contiguous (the wrappers make them so), which fixes their
    strides without reading them.

    Kept short on the host: the arguments packed by one struct call, the
    workspace size query once per shape for the kinds whose workspace depends
    on it (dense and Monarch), and the device switch only when gi's device is
    not current. The short scans (diagonal, single-factor Monarch) take about
    as long on the GPU as a launch does on the host."""
    lib = _lib if _lib is not None else load()
    T, B, G3 = gi.shape
    H = G3 // 3
    if gh_save is not None:
        _check_gh("gh_save", gh_save, gi)
    qi = _qfields(h_in_quant, "h_in_quant")
    qo = _qfields(h_out_quant, "h_out_quant")
    ptrs = (gi.data_ptr(), h0.data_ptr(), w.data_ptr(), w2.data_ptr() if w2 is not None else 0, bh.data_ptr(),
            out.data_ptr())
    if contiguous:
        sizes = (T, B, H, B * G3, G3, H, B * H, H, nblocks, blksz, log_n, bfly_nblocks)
    else:
        sg, so = gi.stride(), out.stride()
        sizes = (T, B, H, sg[0], sg[1], h0.stride(0), so[0], so[1], nblocks, blksz, log_n, bfly_nblocks)
    gh_ptr = gh_save.data_ptr() if gh_save is not None else 0
    tagged = kind in _TAGGED
    need = 0  # the diagonal and butterfly forwards use no workspace beyond the cached minimum
    if tagged:
        key = (kind, sizes, w2 is None, qi, qo, gh_ptr == 0)
        need = _NEED.get(key)
        if need is None:
            a = GS_ARGS.pack(*ptrs, 0, 0, 0, *sizes, *qi, *qo, gh_ptr)
            fn = lib["gs_workspace_bytes"]
            fn.argtypes = [ctypes.c_int, ctypes.c_char_p]
            fn.restype = ctypes.c_int64
            need = int(fn(kind, a))
            if need < 0:
                raise_for(need, lib)
            _NEED[key] = need
    dev = gi.device
    codes = (w_codes[0].data_ptr(), w_codes[1].data_ptr()) if w_codes is not None else None
    if dev.index == torch.cuda.current_device():
        rc = _launch_current(lib, fn_name, ptrs, sizes, qi, qo, gh_ptr, dev, need, T if tagged else 0, codes)
    else:
        with torch.cuda.device(dev):
            rc = _launch_current(lib, fn_name, ptrs, sizes, qi, qo, gh_ptr, dev, need, T if tagged else 0, codes)
    raise_for(rc, lib)


def _launch_current(lib: ctypes.CDLL, fn_name: str, ptrs: tuple, sizes: tuple, qi: tuple, qo: tuple, gh_ptr: int,
                    dev: torch.device, need: int, steps: int, codes: Optional[tuple] = None) -> int:
    handle = current_stream_handle(dev)
    ws = workspace(dev, handle, need, steps=steps)
    mirror = 0
    if steps:  # a persistent kernel: fault mirror and cross-stream order
        m = _mirror(dev, handle)
        _raise_if_faulted(m, fn_name)
        _order_after_previous(dev, handle, lambda: torch.cuda.current_stream(dev))
        mirror = m[0].data_ptr()
    a = GS_ARGS.pack(*ptrs, ws.data_ptr(), ws.numel(), mirror, *sizes, *qi, *qo, gh_ptr)
    if codes is not None:
        return _raw_entry(lib, fn_name)(a, codes[0], codes[1], handle)
    return _raw_entry(lib, fn_name)(a, handle)


# gs_bwd_args packed by one call: 12 tensor pointers, the workspace (pointer,
# bytes), the fault mirror, the scratch (pointer, bytes), 12 int64 sizes and
# strides, the two gs_quant, gh_saved (layout of the ctypes GsBwdArgs).
GS_BWD_ARGS = struct.Struct("<12QQqQQq12q" "ifii" "ifii" "Q")
_BWD_NEED: dict = {}  # (workspace, scratch) bytes per (kind, sizes, quant, optional inputs)


def launch_bwd(kind: int, fn_name: str, *, gi: torch.Tensor, h0: torch.Tensor, w: torch.Tensor,
               w2: Optional[torch.Tensor], bh: torch.Tensor, out: torch.Tensor, dout: torch.Tensor,
               dgi: torch.Tensor, dh0: torch.Tensor, dw_part: Optional[torch.Tensor],
               dbh_part: torch.Tensor, h_in_quant: QuantTuple, h_out_quant: QuantTuple,
               dw2_part: Optional[torch.Tensor] = None,
               nblocks: int = 0, blksz: int = 0, log_n: int = 0, bfly_nblocks: int = 0,
               gh_saved: Optional[torch.Tensor] = None) -> None:
    """Fill gs_bwd_args from fp32 device tensors (dout, dgi, dh0 and the
    partials contiguous) and call a backward entry point on the current torch
    stream of gi's device, with the stream's cached workspace when the kind
    needs one. The workspace and scratch sizes are queried once per shape."""
    lib = _lib if _lib is not None else load()
    T, B, G3 = gi.shape
    if gh_saved is not None:
        _check_gh("gh_saved", gh_saved, gi)
    ptrs = (gi.data_ptr(), h0.data_ptr(), w.data_ptr(), w2.data_ptr() if w2 is not None else 0, bh.data_ptr(),
            out.data_ptr(), dout.data_ptr(), dgi.data_ptr(), dh0.data_ptr(),
            dw_part.data_ptr() if dw_part is not None else 0, dw2_part.data_ptr() if dw2_part is not None else 0,
            dbh_part.data_ptr())
    sg, so = gi.stride(), out.stride()
    sizes = (T, B, G3 // 3, sg[0], sg[1], h0.stride(0), so[0], so[1], nblocks, blksz, log_n, bfly_nblocks)
    qi = _qfields(h_in_quant, "h_in_quant")
    qo = _qfields(h_out_quant, "h_out_quant")
    gh_ptr = gh_saved.data_ptr() if gh_saved is not None else 0
    key = (kind, sizes, w2 is None, dw_part is None, dw2_part is None, qi, qo, gh_ptr == 0)
    needs = _BWD_NEED.get(key)
    if needs is None:
        a = GS_BWD_ARGS.pack(*ptrs, 0, 0, 0, 0, 0, *sizes, *qi, *qo, gh_ptr)
        sizes_fn = []
        for name in ("gs_bwd_workspace_bytes", "gs_bwd_scratch_bytes"):
            fn = lib[name]
            fn.argtypes = [ctypes.c_int, ctypes.c_char_p]
            fn.restype = ctypes.c_int64
            n = int(fn(kind, a))
            if n < 0:
                raise_for(n, lib)
            sizes_fn.append(n)
        needs = _BWD_NEED[key] = tuple(sizes_fn)
    need, scratch_need = needs
    dev = gi.device
    with on_device(dev):
        handle = current_stream_handle(dev)
        ws_ptr = ws_bytes = mirror = 0
        if need > 0:
            ws = workspace(dev, handle, need, steps=T)
            ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
            m = _mirror(dev, handle)
            _raise_if_faulted(m, fn_name)
            _order_after_previous(dev, handle, lambda: torch.cuda.current_stream(dev))
            mirror = m[0].data_ptr()
        scratch = None
        sc_ptr = 0
        if scratch_need > 0:
            # plain scratch from torch's stream-aware caching allocator
            # (allocations are 512-byte aligned); kept alive until the launch is queued
            scratch = torch.empty((scratch_need,), dtype=torch.uint8, device=dev)
            sc_ptr = scratch.data_ptr()
        a = GS_BWD_ARGS.pack(*ptrs, ws_ptr, ws_bytes, mirror, sc_ptr, scratch_need, *sizes, *qi, *qo, gh_ptr)
        rc = _raw_entry(lib, fn_name)(a, handle)
        del scratch
    raise_for(rc, lib)
