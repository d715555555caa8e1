"""Transport calls into libafd: pinned flag pages, the fused send / reply, stream memops.

Replaces the libcuda ctypes bindings the reference transport uses
(``python/sgl_asap_plugin/transport/cuda_wrapper.py``: ``memcpy_async``, ``write32/64``,
``wait32`` at :258-270) with the calls of ``include/afd.h``: ``afd_send`` (backpressure waits,
payload copies and doorbells of one message in one call), ``afd_reply`` (partial-sum copies
and done counters of one job) and ``afd_wait_replies``. All of them only enqueue on the given
stream; failures raise the exception classes of ``_lib.check``.

Done flags are 64-bit message counters that only grow and are waited on with ``>=``, so a
store of any later count releases every earlier wait. The F side gates its stream on a
doorbell word with an equality test on the word's 32-bit sequence field: the producer rings
the next doorbell of a slot only after the F side answered the current one, so the field holds
the awaited value or an older one while the gate waits.
"""

from __future__ import annotations

import ctypes

import numpy as np

from .. import _lib
from .layout import SEQ_MASK

WAIT_GEQ, WAIT_EQ = _lib.AFD_WAIT_GEQ, _lib.AFD_WAIT_EQ


class HostPage:
    """Pinned, coherent, zero-filled host memory the GPU reads and writes with memops (the
    doorbell page, the done-counter page). ``words`` is a uint64 numpy view the host reads
    and writes with plain loads and stores."""

    def __init__(self, nbytes: int):
        ptr = ctypes.c_void_p()
        _lib.call("afd_host_alloc", ctypes.byref(ptr), nbytes)
        self.ptr = ptr.value
        self.nbytes = nbytes
        buf = (ctypes.c_uint8 * nbytes).from_address(self.ptr)
        self.words = np.frombuffer(buf, dtype=np.uint64)

    def addr(self, offset: int) -> int:
        return self.ptr + offset

    def load(self, offset: int) -> int:
        return int(self.words[offset // 8])

    def store(self, offset: int, value: int) -> None:
        self.words[offset // 8] = np.uint64(value)

    def release(self) -> None:
        if self.ptr:
            self.words = None
            _lib.call("afd_host_free", self.ptr)
            self.ptr = 0


def send(desc: _lib.AfdSendDesc, stream: int) -> None:
    """Enqueue one message (``afd_send``): backpressure waits, payload copies, doorbells."""
    _lib.check(_lib.lib().afd_send(ctypes.byref(desc), stream), "afd_send")


def reply(rows: "ctypes.Array", count: int, stream: int) -> None:
    """Enqueue the answers of ``count`` rows (``afd_reply``): copies, then done counters."""
    _lib.check(_lib.lib().afd_reply(rows, count, stream), "afd_reply")


def wait_replies(addrs, seq: int, stream: int) -> None:
    """Park ``stream`` until every done counter at ``addrs`` holds at least ``seq``."""
    arr = (ctypes.c_void_p * len(addrs))(*addrs)
    _lib.check(_lib.lib().afd_wait_replies(arr, len(addrs), seq, stream), "afd_wait_replies")


def gate_on_doorbell(stream: int, addr: int, seq: int) -> None:
    """Park ``stream`` until the sequence field of the doorbell word at ``addr`` equals the
    low 32 bits of ``seq``."""
    _lib.call("afd_stream_wait64", stream, addr, seq & SEQ_MASK, SEQ_MASK, WAIT_EQ)


def copy_async(dst: int, src: int, nbytes: int, stream: int) -> None:
    _lib.call("afd_copy_async", dst, src, nbytes, stream)


def write64(stream: int, addr: int, value: int) -> None:
    """Enqueue a 64-bit store of ``value`` at ``addr`` after the stream's earlier work."""
    _lib.call("afd_stream_write64", stream, addr, value)


def wait64(stream: int, addr: int, value: int, mask: int = 0xFFFFFFFFFFFFFFFF, cond: int = WAIT_GEQ) -> None:
    """Park ``stream`` until the 64-bit word at ``addr`` satisfies ``cond`` against ``value``
    under ``mask`` (default: the whole word >= ``value``)."""
    _lib.call("afd_stream_wait64", stream, addr, value & 0xFFFFFFFFFFFFFFFF, mask, cond)
