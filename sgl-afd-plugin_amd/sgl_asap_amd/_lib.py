"""ctypes binding of libafd.so, the gfx950 C ABI declared in include/afd.h.

The reference binds libcuda the same way (``python/sgl_asap_plugin/transport/cuda_wrapper.py:33``
loads it with ctypes; ``_bind`` at :96-106 turns every non-zero result into ``CUDAError``).
Here every non-zero status raises the exception class the reference raises for the same
condition. There is no fallback: if the library is missing, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libafd.so")

AFD_OK = 0
AFD_ERR_ARG = -1
AFD_ERR_SHAPE = -2
AFD_ERR_UNSUPPORTED = -3
AFD_ERR_HIP = -4
AFD_ERR_WORKSPACE = -5

AFD_W_MXFP4 = 1
AFD_W_FP8_BLOCK = 2

AFD_A_FP8, AFD_A_BF16 = 0, 1

AFD_ACT_SWIGLU = 0
AFD_ACT_SITU = 1
AFD_ACT_SWIGLU_LIMIT = 2

AFD_WAIT_GEQ, AFD_WAIT_EQ, AFD_WAIT_AND, AFD_WAIT_NOR = 0, 1, 2, 3

AFD_WALK_STATIC, AFD_WALK_DYNAMIC = 0, 1

# afd_abi_version() of the library these structures match
ABI_VERSION = 6

# Every entry point include/afd.h declares; tests check the library exports all of them.
EXPORTED = (
    "afd_abi_version",
    "afd_status_string",
    "afd_last_hip_error",
    "afd_workspace_layout",
    "afd_pack_mxfp4",
    "afd_pack_fp8_block",
    "afd_repack_mxfp4",
    "afd_repack_fp8_block",
    "afd_quant_mxfp8",
    "afd_quant_fp8_1x128",
    "afd_quant_act",
    "afd_route",
    "afd_moe_ffn",
    "afd_moe_ffn_q",
    "afd_moe_ffn_answer",
    "afd_moe_ffn_batch",
    "afd_moe_ffn_noalloc",
    "afd_moe_ffn_job",
    "afd_job_set",
    "afd_moe_ffn_profiled",
    "afd_finalize",
    "afd_combine",
    "afd_silu_mul",
    "afd_host_alloc",
    "afd_host_free",
    "afd_copy_async",
    "afd_stream_write64",
    "afd_stream_wait64",
    "afd_send",
    "afd_reply",
    "afd_wait_replies",
)

AFD_MAX_F = 16
AFD_NOALLOC_SCRATCH_BYTES = 128 << 20


class HIPError(RuntimeError):
    """A HIP runtime call failed (the reference's ``CUDAError(name, code)``)."""

    def __init__(self, name: str, code: int):
        super().__init__(f"{name} failed: hipError_t {code}")
        self.name, self.code = name, code


class AfdMoeCfg(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("topk", ctypes.c_int32),
        ("expert_lo", ctypes.c_int32),
        ("num_local", ctypes.c_int32),
        ("weight_fmt", ctypes.c_int32),
        ("activation", ctypes.c_int32),
        ("act_alpha", ctypes.c_float),
        ("act_limit", ctypes.c_float),
        ("tile_walk", ctypes.c_int32),
        ("act_fmt", ctypes.c_int32),
    ]


class AfdExpertWeights(ctypes.Structure):
    _fields_ = [
        ("w13", ctypes.c_void_p),
        ("s13", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("s2", ctypes.c_void_p),
    ]


class AfdJob(ctypes.Structure):
    """afd_job: a job described in device memory (afd_moe_ffn_job reads it when it runs)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("xq", ctypes.c_void_p),
        ("xs", ctypes.c_void_p),
        ("ids", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("n", ctypes.c_int64),
    ]


AFD_MAX_BATCH = 8


class AfdBatchJob(ctypes.Structure):
    """afd_batch_job: one job of a batched expert call (afd_moe_ffn_batch)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("xq", ctypes.c_void_p),
        ("xs", ctypes.c_void_p),
        ("ids", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("done", ctypes.c_void_p),
        ("value", ctypes.c_uint64),
        ("n", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class AfdWsLayout(ctypes.Structure):
    _fields_ = [
        ("total", ctypes.c_uint64),
        ("xq", ctypes.c_uint64),
        ("xs", ctypes.c_uint64),
        ("counts", ctypes.c_uint64),
        ("offsets", ctypes.c_uint64),
        ("padded_offsets", ctypes.c_uint64),
        ("sorted_pairs", ctypes.c_uint64),
        ("pair_pos", ctypes.c_uint64),
        ("tile_expert", ctypes.c_uint64),
        ("num_tiles", ctypes.c_uint64),
        ("hist", ctypes.c_uint64),
        ("hq", ctypes.c_uint64),
        ("hs", ctypes.c_uint64),
        ("y", ctypes.c_uint64),
        ("np_max", ctypes.c_int64),
        ("block_m", ctypes.c_int32),
        ("max_tiles", ctypes.c_int32),
    ]


class AfdSendDesc(ctypes.Structure):
    """afd_send_desc: one message to every F rank (afd_send)."""

    _fields_ = [
        ("num_f", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("x_bytes", ctypes.c_uint64),
        ("xs", ctypes.c_void_p),
        ("xs_bytes", ctypes.c_uint64),
        ("ids", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("ids_bytes", ctypes.c_uint64),
        ("xs_off", ctypes.c_uint64),
        ("ids_off", ctypes.c_uint64),
        ("w_off", ctypes.c_uint64),
        ("done_min", ctypes.c_uint64),
        ("region", ctypes.c_void_p * AFD_MAX_F),
        ("bell", ctypes.c_void_p * AFD_MAX_F),
        ("word", ctypes.c_uint64 * AFD_MAX_F),
        ("done", ctypes.c_void_p * AFD_MAX_F),
    ]


class AfdReplyDesc(ctypes.Structure):
    """afd_reply_desc: one row's answer (afd_reply)."""

    _fields_ = [
        ("src", ctypes.c_void_p),
        ("dst", ctypes.c_void_p),
        ("bytes", ctypes.c_uint64),
        ("done", ctypes.c_void_p),
        ("value", ctypes.c_uint64),
    ]


_P = ctypes.c_void_p
_I32, _I64, _U64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
_SIGS = {
    "afd_abi_version": ([], _I32),
    "afd_status_string": ([_I32], ctypes.c_char_p),
    "afd_last_hip_error": ([], _I32),
    "afd_workspace_layout": ([ctypes.POINTER(AfdMoeCfg), _I32, ctypes.POINTER(AfdWsLayout)], _I32),
    "afd_pack_mxfp4": ([_P, _I64, _I32, _I32, _I32, _P, _P], _I32),
    "afd_pack_fp8_block": ([_P, _I64, _I32, _I32, _I32, _P, _P, _P], _I32),
    "afd_repack_mxfp4": ([_P, _P, _I64, _I32, _I32, _I32, _P, _P], _I32),
    "afd_repack_fp8_block": ([_P, _I64, _I32, _I32, _I32, _P, _P], _I32),
    "afd_quant_mxfp8": ([_P, _I64, _I32, _P, _P, _P], _I32),
    "afd_quant_fp8_1x128": ([_P, _I64, _I32, _P, _P, _P], _I32),
    "afd_route": ([_P, _I32, ctypes.POINTER(AfdMoeCfg), _P, _U64, _P], _I32),
    "afd_moe_ffn": (
        [ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), _P, _P, _P, _I32, _P, _U64, _P, _P],
        _I32,
    ),
    "afd_moe_ffn_noalloc": (
        [ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), _P, _P, _P, _I32, _P, _P],
        _I32,
    ),
    "afd_quant_act": ([ctypes.POINTER(AfdMoeCfg), _P, _I32, _P, _P, _P], _I32),
    "afd_moe_ffn_job": ([ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), _P, _I32, _I32, _P, _U64, _P], _I32),
    "afd_job_set": ([_P, ctypes.POINTER(AfdJob), _P], _I32),
    "afd_moe_ffn_q": (
        [ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), _P, _P, _P, _P, _I32, _P, _U64, _P, _P],
        _I32,
    ),
    "afd_moe_ffn_answer": (
        [ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), _P, _P, _P, _P, _P, _I32, _P, _U64, _P, _P,
         _U64, _P],
        _I32,
    ),
    "afd_moe_ffn_batch": (
        [ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), ctypes.POINTER(AfdBatchJob), _I32, _P,
         _U64, _P],
        _I32,
    ),
    "afd_moe_ffn_profiled": (
        [ctypes.POINTER(AfdMoeCfg), ctypes.POINTER(AfdExpertWeights), _P, _P, _P, _I32, _P, _U64, _P, _P,
         ctypes.POINTER(ctypes.c_void_p)],
        _I32,
    ),
    "afd_finalize": ([_P, _P, _P, _I32, _I32, _I32, _P, _P], _I32),
    "afd_combine": ([ctypes.POINTER(ctypes.c_void_p), _I32, _P, _P, _I64, _P], _I32),
    "afd_silu_mul": ([_P, _I64, _I32, _P, _P], _I32),
    "afd_host_alloc": ([ctypes.POINTER(ctypes.c_void_p), _U64], _I32),
    "afd_host_free": ([_P], _I32),
    "afd_copy_async": ([_P, _P, _U64, _P], _I32),
    "afd_stream_write64": ([_P, _P, _U64], _I32),
    "afd_stream_wait64": ([_P, _P, _U64, _U64, _I32], _I32),
    "afd_send": ([ctypes.POINTER(AfdSendDesc), _P], _I32),
    "afd_reply": ([ctypes.POINTER(AfdReplyDesc), _I32, _P], _I32),
    "afd_wait_replies": ([ctypes.POINTER(ctypes.c_void_p), _I32, _U64, _P], _I32),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it was not built (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing: build it with `make -C sgl-afd-plugin_amd/csrc` "
                        "(or __graft_entry__.build()); the expert path has no non-HIP fallback"
                    )
                handle = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in _SIGS.items():
                    fn = getattr(handle, name)
                    fn.argtypes, fn.restype = args, res
                if handle.afd_abi_version() != ABI_VERSION:
                    raise ImportError(
                        f"{LIB_PATH} has ABI version {handle.afd_abi_version()}, this binding "
                        f"expects {ABI_VERSION}: rebuild it"
                    )
                _lib = handle
    return _lib


def check(status: int, name: str) -> None:
    """Raise the reference's exception class for a non-zero afd_status."""
    if status == AFD_OK:
        return
    L = lib()
    msg = f"{name}: {L.afd_status_string(status).decode()}"
    if status == AFD_ERR_HIP:
        raise HIPError(name, int(L.afd_last_hip_error()))
    if status == AFD_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise ValueError(msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
