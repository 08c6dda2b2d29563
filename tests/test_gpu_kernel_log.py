"""GPU: the launch log (osh_kernel_log) names the kernels a call ran -- the
tile that first-use tuning chose -- in the form rocprofv3 prints
("kernel<template arguments>"), so a bench line or a per-op profile can say
what it measured (the per-op kernel names of Net.ProfileAll,
src/OnnxSharp/Core/Net.cs:282-332)."""
import ctypes as C

import numpy as np
import pytest
import torch

from onnxsharp_amd import native as N, synth
from onnxsharp_amd.layers import ConvLayer, DynamicQuantizeMatMulLayer

pytestmark = pytest.mark.gpu


def test_log_names_each_launch_in_order(cuda):
    x = torch.from_numpy(synth.uniform(31, (1, 32, 24, 24))).to(cuda)
    w = torch.from_numpy(synth.normal(32, (64, 32, 3, 3), 0, 0.05)).to(cuda)
    b = torch.from_numpy(synth.normal(33, (64,), 0, 0.01)).to(cuda)
    layer = ConvLayer(pads=[1, 1, 1, 1], fused_activation="Silu")
    layer.forward(x, w, b)  # packs, tunes
    torch.cuda.synchronize()
    N.kernel_log(reset=True)
    layer.forward(x, w, b)
    torch.cuda.synchronize()
    names = N.kernel_log(reset=True)
    assert len(names) == 1, names
    assert names[0].startswith("conv16"), names
    assert "<" in names[0] and "(" not in names[0] and not names[0].startswith("void"), names
    # the log was reset: nothing since
    assert N.kernel_log(reset=True) == []


def test_log_counts_and_dqmm_pipeline(cuda):
    a = torch.from_numpy(synth.normal(41, (64, 96))).to(cuda)
    wq = torch.from_numpy(synth.randint(42, (96, 48), -127, 127, np.int8)).to(cuda)
    ws = torch.from_numpy(synth.uniform(43, (48,), 0.001, 0.02)).to(cuda)
    layer = DynamicQuantizeMatMulLayer()
    layer.forward(a, wq, None, ws, None)
    torch.cuda.synchronize()
    N.kernel_log(reset=True)
    layer.forward(a, wq, None, ws, None)
    torch.cuda.synchronize()
    n = C.c_int()
    N.call("osh_kernel_log", 0, None, 0, C.byref(n))
    names = N.kernel_log(reset=True)
    launches = C.c_int()
    N.call("osh_config_get", b"dqmm_launches", C.byref(launches))
    assert n.value == len(names) == launches.value, (n.value, names, launches.value)
    assert all(s.startswith("dqmm_") for s in names), names
    # a buffer that is too small is refused with a message
    N.kernel_log(reset=False)
    layer.forward(a, wq, None, ws, None)
    torch.cuda.synchronize()
    small = C.create_string_buffer(4)
    st = N.lib().osh_kernel_log(0, small, 4, None)
    assert st == N.OSH_E_INVALID and "bytes" in N.last_error()
    N.kernel_log(reset=True)
