"""Transport primitives over libafd: pinned flag pages, device copies, 64-bit stream memops.

Replaces the libcuda ctypes bindings the reference transport uses
(``python/sgl_asap_plugin/transport/cuda_wrapper.py``: ``memcpy_async``, ``write32/64``,
``wait32`` at :258-270). All calls only enqueue on the given stream; failures raise the
exception classes of ``_lib.check`` (``HIPError`` for a HIP runtime error).

Sequence numbers are compared with the EQ condition on their low 32 bits. With the
protocol's backpressure (a slot's next message is sent only after the previous reply
landed) a flag can only hold seq - 1 or seq when a wait for seq runs, so equality is the
wrap-safe form of the reference's cyclic GEQ wait (HIP's GEQ is a plain unsigned compare).
"""

from __future__ import annotations

import ctypes

import numpy as np

from .. import _lib
from .layout import SEQ_MASK

WAIT_GEQ, WAIT_EQ, WAIT_AND, WAIT_NOR = _lib.AFD_WAIT_GEQ, _lib.AFD_WAIT_EQ, _lib.AFD_WAIT_AND, _lib.AFD_WAIT_NOR


class HostPage:
    """Pinned, coherent, zero-filled host memory the GPU can read and write with memops
    (the doorbell page and the done-flag page). ``words`` is a uint64 numpy view the host
    reads and writes with plain loads and stores."""

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


def copy_async(dst: int, src: int, nbytes: int, stream: int) -> None:
    _lib.call("afd_copy_async", dst, src, nbytes, stream)


def write64(stream: int, addr: int, value: int) -> None:
    """Enqueue a 64-bit store of ``value`` at ``addr`` after the stream's earlier work."""
    _lib.call("afd_stream_write64", stream, addr, value)


def wait64(stream: int, addr: int, value: int, mask: int = SEQ_MASK, cond: int = WAIT_EQ) -> None:
    """Park ``stream`` until the 64-bit word at ``addr`` satisfies ``cond`` against
    ``value`` under ``mask`` (default: low 32 bits equal ``value``)."""
    _lib.call("afd_stream_wait64", stream, addr, value & 0xFFFFFFFFFFFFFFFF, mask, cond)
