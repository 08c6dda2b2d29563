"""ctypes binding of libosh_hip.so (the C ABI declared in include/osh_hip.h).

This is the same surface a C# P/Invoke class binds.  The library must have
been built (`python -m onnxsharp_amd.build`); there is no CPU fallback: a
missing library raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libosh_hip.so")

OSH_OK = 0
OSH_E_INVALID = -1
OSH_E_UNSUPPORTED = -2
OSH_E_DEVICE = -3
OSH_E_NOMEM = -4

ACT_NONE, ACT_RELU, ACT_SILU, ACT_SIGMOID = 0, 1, 2, 3
PAD_NOTSET, PAD_SAME_UPPER, PAD_SAME_LOWER, PAD_VALID = 0, 1, 2, 3
AUTO_PAD = {"NOTSET": PAD_NOTSET, "SAME_UPPER": PAD_SAME_UPPER, "SAME_LOWER": PAD_SAME_LOWER, "VALID": PAD_VALID}
ACTIVATIONS = {None: ACT_NONE, "Relu": ACT_RELU, "Silu": ACT_SILU}


class OshError(RuntimeError):
    """A non-OK status from the library (message from osh_last_error)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"osh status {status}: {message}")
        self.status = status


class OshUnsupported(OshError):
    """OSH_E_UNSUPPORTED: the backend does not take this op (the emitter refuses it)."""


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 32), ("compute_units", C.c_int),
                ("clock_khz", C.c_int), ("total_mem", C.c_size_t), ("lds_per_block", C.c_size_t)]


class ConvAttrs(C.Structure):
    _fields_ = [("group", C.c_int), ("auto_pad", C.c_int),
                ("n_kernel_shape", C.c_int), ("kernel_shape", C.c_int * 2),
                ("n_strides", C.c_int), ("strides", C.c_int * 2),
                ("n_pads", C.c_int), ("pads", C.c_int * 4),
                ("n_dilations", C.c_int), ("dilations", C.c_int * 2)]


class ConvParams(C.Structure):
    _fields_ = [(f, C.c_int) for f in ("n", "c", "h", "w", "m", "kh", "kw", "group", "sh", "sw", "dh", "dw",
                                       "pt", "pl", "pb", "pr", "oh", "ow")]


PW_1X1, PW_DW3X3 = 0, 1
PW_MAX_SRC, PW_MAX_STAGES, PW_MAX_CHAINS = 3, 5, 3


class PwStage(C.Structure):
    """osh_pw_stage: one stage of a pointwise chain (include/osh_hip.h)."""
    _fields_ = [("kind", C.c_int), ("m", C.c_int), ("act", C.c_int), ("nsrc", C.c_int),
                ("src_stage", C.c_int * PW_MAX_SRC), ("src", C.c_void_p * PW_MAX_SRC), ("src_c", C.c_int * PW_MAX_SRC),
                ("w", C.c_void_p), ("bias", C.c_void_p), ("res_stage", C.c_int), ("res", C.c_void_p),
                ("y", C.c_void_p)]


class PwChain(C.Structure):
    """osh_pw_chain: stages over one H x W map."""
    _fields_ = [("h", C.c_int), ("w", C.c_int), ("nstages", C.c_int), ("stage", PwStage * PW_MAX_STAGES)]


class PoolParams(C.Structure):
    _fields_ = [(f, C.c_int) for f in ("n", "c", "h", "w", "kh", "kw", "sh", "sw", "pt", "pl", "oh", "ow")]


_vp, _i, _i64, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
_i64p = C.POINTER(C.c_int64)

_SIGS = {
    "osh_last_error": ([], C.c_char_p),
    "osh_init": ([_i, C.POINTER(DeviceInfo)], _i),
    "osh_device_count": ([C.POINTER(C.c_int)], _i),
    "osh_device_synchronize": ([], _i),
    "osh_kernel_log": ([_i, C.c_char_p, _sz, C.POINTER(C.c_int)], _i),
    "osh_config_set": ([C.c_char_p, _i], _i),
    "osh_config_get": ([C.c_char_p, C.POINTER(C.c_int)], _i),
    "osh_malloc": ([C.POINTER(_vp), _sz], _i),
    "osh_free": ([_vp], _i),
    "osh_host_alloc": ([C.POINTER(_vp), _sz], _i),
    "osh_host_free": ([_vp], _i),
    "osh_memcpy_h2d": ([_vp, _vp, _sz, _vp], _i),
    "osh_memcpy_d2h": ([_vp, _vp, _sz, _vp], _i),
    "osh_memcpy_d2d": ([_vp, _vp, _sz, _vp], _i),
    "osh_memset_d8": ([_vp, _i, _sz, _vp], _i),
    "osh_stream_create": ([C.POINTER(_vp)], _i),
    "osh_stream_destroy": ([_vp], _i),
    "osh_stream_sync": ([_vp], _i),
    "osh_event_create": ([C.POINTER(_vp)], _i),
    "osh_event_destroy": ([_vp], _i),
    "osh_event_record": ([_vp, _vp], _i),
    "osh_event_elapsed_ms": ([_vp, _vp, C.POINTER(C.c_float)], _i),
    "osh_stream_wait_event": ([_vp, _vp], _i),
    "osh_conv_infer_shape": ([C.POINTER(ConvAttrs), _i64p, _i64p, _i64p], _i),
    "osh_conv_resolve": ([C.POINTER(ConvAttrs), _i64p, _i64p, C.POINTER(ConvParams)], _i),
    "osh_conv_packed_weight_bytes": ([C.POINTER(ConvParams), C.POINTER(_sz)], _i),
    "osh_conv_pack_weights": ([C.POINTER(ConvParams), _vp, _vp, _vp], _i),
    "osh_conv_forget_pack": ([_vp, _sz], _i),
    "osh_pw_chain_f32": ([_i, C.POINTER(PwChain), _vp], _i),
    "osh_conv2d_f32": ([C.POINTER(ConvParams), _vp, _vp, _vp, _i, _vp, _vp], _i),
    "osh_conv2d_add_f32": ([C.POINTER(ConvParams), _vp, _vp, _vp, _i, _vp, _vp, _vp], _i),
    "osh_conv2d_group_f32": ([_i, C.POINTER(ConvParams), _vp, _vp, _vp, _i, _vp, _vp, _vp], _i),
    "osh_conv2d_pair_f32": ([C.POINTER(ConvParams), C.POINTER(ConvParams), _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp,
                             _vp, _vp], _i),
    "osh_conv2d_pair_check": ([C.POINTER(ConvParams), C.POINTER(ConvParams), _i], _i),
    "osh_gemm_f32": ([_i, _i, _i, _vp, _i, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _vp], _i),
    "osh_gemm_f32_batched": ([_i, _i, _i, _i, _vp, _i, _i64, _vp, _i, _i64, _vp, _i, _vp, _i, _i64, _vp], _i),
    "osh_matmul_infer_shape": ([_i64p, _i, _i64p, _i, _i64p, C.POINTER(C.c_int)], _i),
    "osh_gemm_ex_workspace_bytes": ([_i, _i, _i, _i, _i, C.POINTER(_sz)], _i),
    "osh_gemm_ex_f32": ([_i, _i, _i, _i, _i, C.c_float, _vp, _vp, C.c_float, _vp, _i64, _vp, _vp, _vp], _i),
    "osh_dqmm_packed_weight_bytes": ([_i, _i, C.POINTER(_sz)], _i),
    "osh_dqmm_scratch_bytes": ([_i, _i, C.POINTER(_sz)], _i),
    "osh_dqmm_pack_weights": ([_i, _i, _vp, _i, _vp, _i, _vp, _vp], _i),
    "osh_dqmm_u8s8": ([_i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "osh_dqmm_u8s8_noalloc": ([_i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp], _i),
    "osh_matmul_integer": ([_i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _vp], _i),
    "osh_dynamic_quantize_linear": ([_i64, _vp, _vp, _vp, _vp, _vp], _i),
    "osh_activation_f32": ([_i64, _vp, _i, _vp, _vp], _i),
    "osh_add_f32": ([_i64, _vp, _vp, _vp, _vp], _i),
    "osh_maxpool2d_f32": ([C.POINTER(PoolParams), _vp, _vp, _vp], _i),
    "osh_maxpool_chain3_f32": ([_i, _i, _i, _i, _i, _vp, _i64, _vp, _vp, _vp, _i64, _vp], _i),
    "osh_dfl_f32": ([_i, _i, _i, _i, _vp, _i64, _vp, _i64, _vp], _i),
    "osh_resize_nearest_f32": ([_i, _i, _i, _i, _i, _i, _vp, _vp, _i64, _vp], _i),
    "osh_transpose_f32": ([_i, _i, _i, _vp, _i64, _vp, _i64, _vp], _i),
    "osh_softmax_f32": ([_i64, _i, C.c_float, _vp, _vp, _vp], _i),
    "osh_attention_f32": ([_i, _i, _i, _i, C.c_float, _vp, _i64, _vp, _vp], _i),
    "osh_graph_begin": ([_vp], _i),
    "osh_graph_end": ([_vp, C.POINTER(_vp)], _i),
    "osh_graph_launch": ([_vp, _vp], _i),
    "osh_graph_destroy": ([_vp], _i),
    "osh_graph_builder_create": ([C.POINTER(_vp)], _i),
    "osh_graph_add_captured": ([_vp, _vp, C.POINTER(_vp), _i, C.POINTER(_vp)], _i),
    "osh_graph_add_captured_flat": ([_vp, _vp, C.POINTER(_vp), _i, C.POINTER(_vp), C.POINTER(_vp)], _i),
    "osh_graph_instantiate": ([_vp, C.POINTER(_vp)], _i),
    "osh_graph_builder_destroy": ([_vp], _i),
}

# Every symbol include/osh_hip.h declares (checked by the CPU test suite).
EXPORTED = tuple(_SIGS)

_lib = None


def lib():
    """Load libosh_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: build it with `python -m onnxsharp_amd.build` "
                          "(there is no CPU fallback)")
        l = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            f = getattr(l, name)
            f.argtypes = args
            f.restype = res
        _lib = l
    return _lib


def last_error() -> str:
    return lib().osh_last_error().decode(errors="replace")


def check(status: int) -> None:
    if status != OSH_OK:
        msg = last_error()
        raise (OshUnsupported if status == OSH_E_UNSUPPORTED else OshError)(status, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def dims64(shape) -> "C.Array":
    arr = (C.c_int64 * max(1, len(shape)))()
    for i, d in enumerate(shape):
        arr[i] = int(d)
    return arr


def kernel_log(reset: bool = True) -> list:
    """Names ("kernel<template arguments>") of the kernels the calling thread
    launched since the last reset, in launch order (osh_kernel_log)."""
    n = C.c_int()
    call("osh_kernel_log", 0, None, 0, C.byref(n))
    size = 256 * (min(n.value, 4096) + 1)
    buf = C.create_string_buffer(size)
    call("osh_kernel_log", 1 if reset else 0, buf, size, C.byref(n))
    return [s for s in buf.value.decode().split("\n") if s]
