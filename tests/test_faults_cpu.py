"""Host logic around the persistent kernels' fault word (no GPU needed)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gru_qat_amd import _lib


def test_mirror_raises_once_and_clears():
    word = np.zeros(1, dtype=np.int32)
    m = (None, word)
    _lib._raise_if_faulted(m, "probe")  # clear: nothing raised
    word[0] = 65  # a launch with tag base 64 gave up
    with pytest.raises(_lib.PersistentScanFault, match="fault value 65"):
        _lib._raise_if_faulted(m, "probe")
    assert word[0] == 0
    _lib._raise_if_faulted(m, "probe")
    assert issubclass(_lib.PersistentScanFault, RuntimeError)


class _FakeStream:
    def __init__(self, handle):
        self.cuda_stream = handle
        self.waited = []

    def wait_stream(self, other):
        self.waited.append(other.cuda_stream)


class _Dev:
    def __init__(self, index):
        self.index = index


def test_persistent_launches_wait_for_the_previous_stream():
    saved = dict(_lib._last_stream)
    _lib._last_stream.clear()
    try:
        a, b = _FakeStream(11), _FakeStream(22)
        dev = _Dev(7)
        order = lambda d, s: _lib._order_after_previous(d, s.cuda_stream, lambda: s)  # noqa: E731
        order(dev, a)
        order(dev, a)
        assert a.waited == []  # same stream: ordered already
        order(dev, b)
        assert b.waited == [11]
        order(dev, a)
        assert a.waited == [22]
        other = _FakeStream(33)
        order(_Dev(8), other)  # another device: independent
        assert other.waited == []
    finally:
        _lib._last_stream.clear()
        _lib._last_stream.update(saved)


def test_args_structs_carry_the_fault_mirror():
    """gs_args / gs_bwd_args field order matches include/gruscan.h: the mirror
    sits right after workspace_bytes."""
    for cls in (_lib.GsArgs, _lib.GsBwdArgs):
        names = [f[0] for f in cls._fields_]
        i = names.index("workspace_bytes")
        assert names[i + 1] == "fault_mirror"
        assert dict(cls._fields_)["fault_mirror"] is ctypes.c_void_p
