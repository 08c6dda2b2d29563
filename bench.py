"""Benchmark of the dense-contraction hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all]

A step is one pass of the hot path on resident synthetic inputs.  The default
(--config all) times every workload in one process and prints ONE JSON line:
the headline is the 3x3 stride-1 pad-1 Conv + bias + fused SiLU on
X[1,64,160,160] U(0,1), W[64,64,3,3] N(0,0.05), b[64] N(0,0.01) (the shape the
reference publishes a CPU number for); "configs" holds the others, each with
its own step time, rate and roofline:
  c1   MatMul + Add(bias) fused: A[1024,768] x B[768,768] + bias[768], U(-1,1)
  c2   the headline conv
  c3a  1x1 conv 256->128 @ 80x80 + bias + SiLU
  c3b  3x3 stride-2 conv 128->256, 80x80 -> 40x40 + bias + SiLU
  c3c  C2f bottleneck block 128->128 @ 80x80 (1x1, 3x3, 3x3 + residual Add, 1x1; concat/split by slices)
  c4   YOLO11n frame at 640x640 (87 convolutions + C2PSA attention + SPPF/upsample/concat/add glue),
       replayed as one HIP graph; random N(0,0.05) weights, input U(0,1); DFL/NMS stay on the host
  c5   int8 DynamicQuantizeMatMul A f32[512,512] N(0,1), W s8[512,2048], per-column scales, bias
--config <name> times one workload alone (profiling runs); --config copy is a
64 MiB device-to-device copy that calibrates the HBM byte counters.

`value` is whole-job TFLOP/s (TOP/s for c5) from HIP events on the launch
stream over exactly K back-to-back steps (single-launch workloads: the K
launches recorded once as a HIP graph after the warm-up and replayed, so host
launch cost is not in the figure; `ms_per_step_eager` gives the same K steps
issued one by one; `--eager` makes that the value); `roofline` prices the
dominant kernel against the MI355X peak, with the HBM bytes per launch the
committed rocprofv3 counter summaries give; `cpu_baseline` times the CPU
oracle (a C restatement of the reference's CPU kernels, in the order the
reference's kernel for that shape uses on an AVX-512 host; the NCHWc layers
through a blocked AVX-512 restatement of NchwcConv) on this host at 4
threads and at all available cores, beside the reference's own published
figure where it has one.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"fp32_mfma_tflops": 157.3, "int8_tops": 5000.0, "hbm_gbs": 8000.0}
METRIC = "conv/GEMM TFLOP/s + % MI355X MFMA peak; ms/frame YOLO11n-shape 640²"


def host_info() -> dict:
    info = {"model": "", "flags": [], "logical_cpus": os.cpu_count()}
    try:
        txt = open("/proc/cpuinfo").read()
        for line in txt.splitlines():
            if line.startswith("model name") and not info["model"]:
                info["model"] = line.split(":", 1)[1].strip()
            if line.startswith("flags"):
                fl = set(line.split(":", 1)[1].split())
                info["flags"] = sorted(f for f in ("avx2", "fma", "avx512f", "avx512vl", "avx512_vnni", "avx_vnni")
                                       if f in fl)
                break
        cores = {(l.split(":")[1].strip()) for l in txt.splitlines() if l.startswith("core id")}
        sockets = {(l.split(":")[1].strip()) for l in txt.splitlines() if l.startswith("physical id")}
        info["physical_cores"] = max(1, len(cores)) * max(1, len(sockets))
    except OSError:
        pass
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    return info


class Workload:
    name = ""
    flops = 0.0        # algorithmic flops (or int ops) per step
    bytes = 0.0        # algorithmic HBM bytes per step (each tensor read or written once)
    bound = "mfma"
    peak = PEAK["fp32_mfma_tflops"]
    dtype = "f32"
    kernel = ""
    config: dict = {}

    def step(self):
        raise NotImplementedError

    def cpu_step(self, oracle):
        raise NotImplementedError


def _t(x, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


class ConvWorkload(Workload):
    graphable = True

    def __init__(self, dev, name, xs, ws, stride, act, kernel, seed):
        import torch
        from onnxsharp_amd import native as N, synth
        from onnxsharp_amd.layers import ConvLayer
        self.name = name
        self.kernel = kernel
        k = ws[2]
        pad = (k - 1) // 2
        self.layer = ConvLayer(strides=[stride, stride], pads=[pad] * 4, fused_activation=act)
        self.x_np = synth.uniform(seed, xs)
        self.w_np = synth.normal(seed + 1, ws, 0.0, 0.05)
        self.b_np = synth.normal(seed + 2, (ws[0],), 0.0, 0.01)
        self.x, self.w, self.b = _t(self.x_np, dev), _t(self.w_np, dev), _t(self.b_np, dev)
        p, buf = self.layer.prepack_weights(xs, self.w)
        self.p, self.wbuf = p, buf
        self.y = torch.empty((p.n, p.m, p.oh, p.ow), dtype=torch.float32, device=dev)
        self.flops = 2.0 * p.n * p.m * (p.c // p.group) * p.kh * p.kw * p.oh * p.ow
        self.bytes = 4.0 * (self.x.numel() + self.w.numel() + self.b.numel() + self.y.numel())
        self.act = N.ACTIVATIONS[act]
        self.fn = N.lib().osh_conv2d_f32
        self.args = (C.byref(p), C.c_void_p(self.x.data_ptr()), C.c_void_p(buf.data_ptr()),
                     C.c_void_p(self.b.data_ptr()), self.act, C.c_void_p(self.y.data_ptr()))
        self.config = {"workload": f"conv{k}x{k} s{stride} p{pad} {xs[1]}->{ws[0]} @{xs[2]}x{xs[3]} + bias"
                                   + (f" + {act}" if act else ""),
                       "x": list(xs), "w": list(ws), "stride": stride, "pads": [pad] * 4,
                       "inputs": "x U(0,1), w N(0,0.05), b N(0,0.01), splitmix64 seeds "
                                 f"{seed},{seed + 1},{seed + 2}"}

    def step(self, stream):
        st = self.fn(*self.args, stream)
        if st != 0:
            from onnxsharp_amd import native as N
            N.check(st)

    def cpu_order(self, oracle):
        p = self.p
        k = oracle.conv_reference_kernel(self.x_np.shape, self.w_np.shape, (p.sh, p.sw), (p.pt, p.pl),
                                         (p.dh, p.dw), p.group, (p.oh, p.ow))
        return {oracle.KERNEL_NCHWC: "NchwcConv chain (ib -> ky -> kx -> lane16, NchwcConv.cs:533-605)"
                                     + (", blocked AVX-512 kernel with its reorders (NchwcConv.cs:247-665)"
                                        if oracle.nchwc_avx512_ok() else ", scalar loop (no AVX-512 here)"),
                oracle.KERNEL_WINOGRAD: "Winograd F(2x2,3x3) (Winograd.cs)",
                oracle.KERNEL_DEPTHWISE: "DepthwiseConv (ky -> kx)"}.get(
            k, "im2col / pointwise GEMM chain (ic -> ky -> kx, ConvKernels.cs:464-563)")

    def cpu_step(self, oracle):
        p = self.p
        y = oracle.conv_reference(self.x_np, self.w_np, self.b_np, (p.sh, p.sw), (p.pt, p.pl), (p.dh, p.dw),
                                  p.group, (p.oh, p.ow))
        return oracle.silu_ref(y)


class GemmWorkload(Workload):
    graphable = True

    def __init__(self, dev):
        import torch
        from onnxsharp_amd import native as N, synth
        self.name = "c1"
        self.kernel = "gemm16_kernel"
        m, k, n = 1024, 768, 768
        self.a_np = synth.uniform(101, (m, k), -1, 1)
        self.b_np = synth.uniform(102, (k, n), -1, 1)
        self.bias_np = synth.uniform(103, (n,), -1, 1)
        self.a, self.b, self.bias = _t(self.a_np, dev), _t(self.b_np, dev), _t(self.bias_np, dev)
        self.c = torch.empty((m, n), dtype=torch.float32, device=dev)
        self.flops = 2.0 * m * n * k
        self.bytes = 4.0 * (m * k + k * n + n + m * n)
        self.fn = N.lib().osh_gemm_f32
        self.args = (m, n, k, C.c_void_p(self.a.data_ptr()), k, C.c_void_p(self.b.data_ptr()), n,
                     C.c_void_p(self.bias.data_ptr()), None, None, N.ACT_NONE, C.c_void_p(self.c.data_ptr()), n)
        self.config = {"workload": "MatMul+Add(bias) fused, A[1024x768] . B[768x768] + bias[768]",
                       "inputs": "U(-1,1), splitmix64 seeds 101,102,103"}

    def step(self, stream):
        st = self.fn(*self.args, stream)
        if st != 0:
            from onnxsharp_amd import native as N
            N.check(st)

    def cpu_order(self, oracle):
        return "GemmKernel k-ascending FMA chain from the column bias (GemmKernel.cs:1130-1207)"

    def cpu_step(self, oracle):
        return oracle.gemm_f32(self.a_np, self.b_np, col_bias=self.bias_np)


class DqmmWorkload(Workload):
    graphable = True

    def __init__(self, dev):
        import torch
        from onnxsharp_amd import native as N, synth
        from onnxsharp_amd.layers import DynamicQuantizeMatMulLayer
        self.name = "c5"
        self.kernel = "dqmm_fused"  # the quantize + GEMM launch (of whichever tile shape)
        self.dtype = "int8"
        self.bound = "hbm"
        m, k, n = 512, 512, 2048
        self.a_np = synth.normal(201, (m, k))
        self.w_np = synth.randint(202, (k, n), -127, 127, np.int8)
        self.ws_np = synth.uniform(203, (n,), 0.001, 0.02)
        self.bias_np = synth.normal(204, (n,), 0, 0.01)
        self.a, self.w = _t(self.a_np, dev), _t(self.w_np, dev)
        self.ws, self.bias = _t(self.ws_np, dev), _t(self.bias_np, dev)
        self.layer = DynamicQuantizeMatMulLayer()
        self.out = self.layer.forward(self.a, self.w, None, self.ws, self.bias)  # packs W, sizes scratch
        self.flops = 2.0 * m * n * k
        self.bytes = 4.0 * m * k + k * n + 4.0 * m * n + 8.0 * n
        self.fn = N.lib().osh_dqmm_u8s8
        self.args = (m, k, n, C.c_void_p(self.a.data_ptr()), C.c_void_p(self.layer._packed[1].data_ptr()),
                     C.c_void_p(self.ws.data_ptr()), n, C.c_void_p(self.bias.data_ptr()),
                     C.c_void_p(self.out.data_ptr()), None, None, C.c_void_p(self.layer._scratch.data_ptr()))
        self.config = {"workload": "int8 DynamicQuantizeMatMul A f32[512x512] -> u8, W s8[512x2048], "
                                   "per-column scales, bias",
                       "inputs": "A N(0,1), W uniform{-127..127}, w_scale U(0.001,0.02), bias N(0,0.01), "
                                 "splitmix64 seeds 201-204"}

    def step(self, stream):
        st = self.fn(*self.args, stream)
        if st != 0:
            from onnxsharp_amd import native as N
            N.check(st)

    def cpu_order(self, oracle):
        return ("Quantizer.MinMax + QuantizeAndWiden, then the F32 GEMM of the widened operands "
                "(QuantizedMatMulOps.cs:115-201)")

    def cpu_step(self, oracle):
        # the reference's CPU route: quantize and widen A, then the F32 GEMM of
        # the widened operands (weights widened once); dqmm's output bits
        return oracle.dqmm_widened_gemm(self.a_np, self.w_np, None, self.ws_np, self.bias_np)


class FrameWorkload(Workload):
    """A block of ops (yolo11n.Model) per step: the launches recorded once as
    a HIP graph and replayed, inputs resident on the device.
    ONNXSHARP_HIP_FRAME_MODE: "graph" (default, one serial HIP graph),
    "segments" (per-stream segments as child graphs of one DAG), "flat" (the
    same DAG of plain kernel nodes) or "eager" (launches issued from the host
    on the planned streams)."""

    def __init__(self, dev, name, model, x_np, label):
        from onnxsharp_amd import yolo11n
        self.name = name
        self.kernel = label
        self.model = model
        self.fr = yolo11n.Frame(self.model, dev)
        self.x_np = x_np
        self.fr.set_input(self.x_np)
        self.fr.run()
        self.fr.sync()
        self.mode = os.environ.get("ONNXSHARP_HIP_FRAME_MODE", "graph")
        if self.mode not in ("graph", "segments", "flat", "eager"):
            raise SystemExit(f"ONNXSHARP_HIP_FRAME_MODE={self.mode!r}: expected graph, segments, flat or eager")
        if self.mode != "eager":
            self.fr.capture(parallel=self.mode in ("segments", "flat"), flat=self.mode == "flat")
        self.stream = self.fr.stream
        self.flops = self.model.flops
        # each tensor read or written once per op that touches it
        self.bytes = 4.0 * sum(op.x.c * op.x.h * op.x.w + op.w.size + op.b.size + op.y.c * op.y.h * op.y.w
                               for op in self.model.convs)

    def step(self, stream):
        if self.mode == "eager":
            self.fr.run()
        else:
            self.fr.launch()

    def cpu_order(self, oracle):
        from collections import Counter
        kinds = Counter()
        for op in self.model.convs:
            k = oracle.conv_reference_kernel((1, op.x.c, op.x.h, op.x.w), op.w.shape, (op.s, op.s),
                                             (op.k // 2, op.k // 2), (1, 1), op.group, (op.y.h, op.y.w))
            kinds[k] += 1
        return ("each conv on the kernel ConvLayer.Forward picks on an AVX-512 host (DnnOps.cs:437-482): "
                + ", ".join(f"{v} {k}" for k, v in sorted(kinds.items())))

    def cpu_step(self, oracle):
        from oracle import yolo_frame
        return yolo_frame.Frame(self.model).run(oracle, self.x_np)

    def host_roundtrip_ms(self, frames=20):
        """ms per step with the input copied in and the outputs copied out
        through pinned host memory (PCIe included)."""
        import torch
        from onnxsharp_amd import native as N
        hin = torch.from_numpy(self.x_np).pin_memory()
        outs = self.fr.outputs()
        houts = [torch.empty(t.shape, dtype=t.dtype).pin_memory() for t in outs]
        nb_in = hin.numel() * 4
        dst_in = C.c_void_p(self.model.input.tensor.data_ptr())

        def frame():
            N.call("osh_memcpy_h2d", dst_in, C.c_void_p(hin.data_ptr()), nb_in, self.stream)
            self.step(self.stream)
            for h, d in zip(houts, outs):
                N.call("osh_memcpy_d2h", C.c_void_p(h.data_ptr()), C.c_void_p(d.data_ptr()), h.numel() * 4,
                       self.stream)
            N.call("osh_stream_sync", self.stream)

        for _ in range(3):
            frame()
        t0 = time.perf_counter()
        for _ in range(frames):
            frame()
        return (time.perf_counter() - t0) / frames * 1e3


class YoloWorkload(FrameWorkload):
    """One YOLO11n frame per step (about a hundred launches in one graph)."""

    def __init__(self, dev):
        from onnxsharp_amd import synth, yolo11n
        model = yolo11n.build(640)
        super().__init__(dev, "c4", model, synth.uniform(4000, (1, 3, 640, 640)), "yolo11n frame (HIP graph)")
        nconv = len(self.model.convs)
        nlaunch = len(self.fr.model.ops)
        self.config = {"workload": "YOLO11n backbone+neck+head, batch 1, 640x640, FP32 NCHW, "
                                   f"{nconv} convs + attention/SPPF/upsample glue as {nlaunch} launches "
                                   "(grouped and paired convs, residual Adds fused) in one HIP graph",
                       "input": "U(0,1) [1,3,640,640], splitmix64 seed 4000",
                       "weights": "N(0,0.05) conv weights, N(0,0.01) biases (BatchNorm folded), splitmix64 seeded per layer from its node name and model seed 7000",
                       "conv_gflop": round(sum(o.flops for o in self.model.convs) / 1e9, 4),
                       "outputs": "3 head tensors [1,144,80,80], [1,144,40,40], [1,144,20,20]; "
                                  "DFL/NMS on the host"}


class C2fWorkload(FrameWorkload):
    """One depthwise-free C2f bottleneck block per step (four convolutions,
    the shortcut Add folded into the second 3x3 conv), as one HIP graph."""

    def __init__(self, dev):
        from onnxsharp_amd import synth, yolo11n
        model = yolo11n.build_c2f(80, 128, 128, 1, True)
        super().__init__(dev, "c3c", model, synth.uniform(3300, (1, 128, 80, 80)), "C2f block (HIP graph)")
        self.config = {"workload": "C2f(128->128, n=1, shortcut) @ 80x80, batch 1, FP32 NCHW: cv1 1x1 128->128 "
                                   "+SiLU, split 64/64, bottleneck 3x3 64->64 +SiLU -> 3x3 64->64 +SiLU + residual "
                                   "Add, concat 192, cv2 1x1 192->128 +SiLU",
                       "input": "U(0,1) [1,128,80,80], splitmix64 seed 3300",
                       "weights": "N(0,0.05) conv weights, N(0,0.01) biases, splitmix64 seeded per layer from its node name and model seed 9000",
                       "conv_gflop": round(sum(o.flops for o in self.model.convs) / 1e9, 4),
                       "launches": len(self.fr.model.ops)}


class CopyWorkload(Workload):
    """Plain 64 MiB device copy: its FETCH_SIZE / WRITE_SIZE counter readings
    calibrate the per-dispatch HBM traffic of the other workloads."""

    def __init__(self, dev):
        import torch
        from onnxsharp_amd import native as N
        self.name = "copy"
        self.kernel = "__amd_rocclr_copyBuffer"
        self.bound = "hbm"
        self.nbytes = 64 << 20
        self.src = torch.ones(self.nbytes // 4, dtype=torch.float32, device=dev)
        self.dst = torch.empty_like(self.src)
        self.flops = 0.0
        self.bytes = 2.0 * self.nbytes
        self.fn = N.lib().osh_memcpy_d2d
        self.args = (C.c_void_p(self.dst.data_ptr()), C.c_void_p(self.src.data_ptr()), self.nbytes)
        self.config = {"workload": "device-to-device copy of 64 MiB (counter calibration)"}

    def step(self, stream):
        st = self.fn(*self.args, stream)
        if st != 0:
            from onnxsharp_amd import native as N
            N.check(st)


def make_workload(name, dev):
    if name == "c2":
        return ConvWorkload(dev, "c2", (1, 64, 160, 160), (64, 64, 3, 3), 1, "Silu", "", 1)
    if name == "c3a":
        return ConvWorkload(dev, "c3a", (1, 256, 80, 80), (128, 256, 1, 1), 1, "Silu", "", 11)
    if name == "c3b":
        return ConvWorkload(dev, "c3b", (1, 128, 80, 80), (256, 128, 3, 3), 2, "Silu", "", 21)
    if name == "c1":
        return GemmWorkload(dev)
    if name == "c5":
        return DqmmWorkload(dev)
    if name == "c4":
        return YoloWorkload(dev)
    if name == "c3c":
        return C2fWorkload(dev)
    if name == "copy":
        return CopyWorkload(dev)
    raise SystemExit(f"unknown --config {name}")


def time_gpu(wl, steps, warmup, graph=True, marks=False):
    """(device ms over exactly `steps` back-to-back steps, host wall s, eager
    device ms or None).  Single-launch workloads (wl.graphable) are timed as
    one HIP graph holding the `steps` launches, recorded after the warm-up
    (which also runs the first-use tile tuning), so the figure is the device's
    and not the Python launch loop's; the same steps issued one by one are
    timed too and reported beside it.  Frame workloads replay their own graph
    per step.  With `marks`, a 1-byte fill kernel runs just before and just
    after each timed region (outside its events), so that a kernel trace of
    the run can tell the timed dispatches from the warm-up's."""
    import torch
    from onnxsharp_amd import native as N
    sp = getattr(wl, "stream", None)
    own = None
    use_graph = graph and getattr(wl, "graphable", False)
    if sp is None:
        if use_graph:  # capture needs a stream of its own
            own = C.c_void_p()
            N.call("osh_stream_create", C.byref(own))
            sp = own
        else:
            sp = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for _ in range(warmup):
        wl.step(sp)
    N.call("osh_stream_sync", sp)
    torch.cuda.synchronize()
    e0, e1 = C.c_void_p(), C.c_void_p()
    N.call("osh_event_create", C.byref(e0))
    N.call("osh_event_create", C.byref(e1))
    mark_buf = torch.empty(64, dtype=torch.uint8, device="cuda") if marks else None

    def mark():
        if mark_buf is not None:
            N.call("osh_memset_d8", C.c_void_p(mark_buf.data_ptr()), 0, 1, sp)

    def timed(run):
        N.call("osh_stream_sync", sp)
        mark()
        t0 = time.perf_counter()
        N.call("osh_event_record", e0, sp)
        run()
        N.call("osh_event_record", e1, sp)
        mark()
        N.call("osh_stream_sync", sp)
        wall = time.perf_counter() - t0
        ms = C.c_float()
        N.call("osh_event_elapsed_ms", e0, e1, C.byref(ms))
        return ms.value, wall

    def eager():
        for _ in range(steps):
            wl.step(sp)

    eager_ms = None
    if use_graph:
        g = C.c_void_p()
        N.call("osh_graph_begin", sp)
        try:
            eager()
        finally:
            N.call("osh_graph_end", sp, C.byref(g))
        N.call("osh_graph_launch", g, sp)  # one untimed replay
        ms, wall = timed(lambda: N.call("osh_graph_launch", g, sp))
        eager_ms, _ = timed(eager)
        N.call("osh_graph_destroy", g)
    else:
        ms, wall = timed(eager)
    N.call("osh_event_destroy", e0)
    N.call("osh_event_destroy", e1)
    if own is not None:
        N.call("osh_stream_destroy", own)
    return ms, wall, eager_ms


CPU_LABEL = "C++ restatement of OnnxSharp CPU kernels, not the C# binary"
CPU_IMPL = ("oracle/osh_oracle.c: C, gcc -O3 -mavx2 -mfma -ffp-contract=off, explicit fmaf chains, a persistent "
            "pthread pool; where the host has AVX-512: the NCHWc-gate 3x3 layers through a blocked restatement of "
            "NchwcConv (input reorder, 2 output blocks x 8 pixels per step, output reorder), GEMM chains (MatMul, "
            "pointwise convs, the widened DQM GEMM) register-blocked 8 x 32 over packed panels, vector SiLU; "
            "each bit-identical to the scalar loops the parity tests pin")
# The reference's own published CPU figures for these workloads (4 threads,
# its AVX-512 host), printed beside the port's timing.
REFERENCE_PUBLISHED = {
    "c2": {"ms_per_step": 4.28, "reorder_ms": 0.24, "threads": 4,
           "source": "bench.md:1977 (NchwcConv 64->64 160x160, 220.6 GMAC/s; input/output reorder 0.24 ms beside)"},
    "c4": {"ms_per_frame": 30.4, "threads": 4, "source": "bench.md:3108 (yolo11n 640x640 median, onnxsharp)"},
}
# CPU seconds per thread count: the headline gets the longest sample
CPU_BUDGET = {"c2": 10.0, "c3b": 4.0, "c4": 4.0, "c1": 2.0, "c3a": 2.0, "c3c": 2.0, "c5": 2.0}
CONFIGS = ("c1", "c2", "c3a", "c3b", "c3c", "c4", "c5")


def reference_paths(flags) -> dict:
    """Which reference CPU kernels fire on this host's ISA."""
    f = set(flags)
    return {"NchwcConv (needs AVX-512F, NchwcConv.cs:43)": "avx512f" in f,
            "GemmKernel MR=12 (needs AVX-512VL, GemmKernel.cs:452-454)": "avx512f" in f and "avx512vl" in f,
            "FirstConv (needs AVX-512F)": "avx512f" in f,
            "DynamicQuantizeMatMul": "F32 GEMM path on every ISA (QuantizedMatMulOps.cs:170-183)"}


def cpu_baseline(wl, threads, budget_s):
    """(rate, steps, seconds, per-step ms list) of the oracle on this host."""
    from oracle import oracle
    oracle.set_threads(threads)
    wl.cpu_step(oracle)  # warm
    times, t0 = [], time.perf_counter()
    while True:
        t1 = time.perf_counter()
        wl.cpu_step(oracle)
        times.append((time.perf_counter() - t1) * 1e3)
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return wl.flops * len(times) / el / 1e12, len(times), el, times


def cpu_leg(wl, budget_s, hi):
    from oracle import oracle
    unit = "TOP/s" if wl.dtype == "int8" else "TFLOP/s"
    v4, n4, el4, t4 = cpu_baseline(wl, 4, budget_s)
    cpu = {"value": round(v4, 5), "unit": unit, "cores": 4, "kind": "port",
           "label": CPU_LABEL, "impl": CPU_IMPL, "order": wl.cpu_order(oracle),
           "avx512_nchwc": bool(oracle.nchwc_avx512_ok()),
           "ms_per_step_median": round(float(np.median(t4)), 3), "ms_per_step_min": round(min(t4), 3),
           "sample": f"{n4} full steps of the same workload in {el4:.1f} s (4 threads)"}
    allc = int(min(hi.get("affinity_cpus") or 4, hi.get("physical_cores") or 4))
    if allc != 4:
        va, na, ela, ta = cpu_baseline(wl, allc, budget_s)
        cpu["all_cores"] = {"value": round(va, 5), "cores": allc,
                            "ms_per_step_median": round(float(np.median(ta)), 3),
                            "ms_per_step_min": round(min(ta), 3), "sample": f"{na} steps in {ela:.1f} s"}
    if wl.name in REFERENCE_PUBLISHED:
        cpu["reference_published"] = REFERENCE_PUBLISHED[wl.name]
    return cpu


def read_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    try:
        d = json.load(open(path))
        return d.get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def step_kernels(wl):
    """Names of the kernels one step launches, after the warm-up's first-use
    tuning has fixed every tile (one extra step issued from the host)."""
    import torch
    from onnxsharp_amd import native as N
    torch.cuda.synchronize()
    N.kernel_log(reset=True)
    if hasattr(wl, "fr"):
        wl.fr.run()
        wl.fr.sync()
    else:
        wl.step(C.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return N.kernel_log(reset=True)


def measure(wl, args):
    """GPU figures of one workload: step time, rate and roofline."""
    ms, wall, eager_ms = time_gpu(wl, args.steps, args.warmup, graph=not args.eager, marks=args.trace_marks)
    ms_step = ms / args.steps
    rate = wl.flops / (ms_step * 1e-3) / 1e12
    if wl.bound == "hbm":
        achieved = wl.bytes / (ms_step * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK["hbm_gbs"], "unit": "GB/s",
                "frac": round(achieved / PEAK["hbm_gbs"], 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(rate, 3), "peak": PEAK["fp32_mfma_tflops"], "unit": "TFLOP/s",
                "frac": round(rate / PEAK["fp32_mfma_tflops"], 4)}
    roof["traffic"] = read_traffic(wl.name)
    names = step_kernels(wl)
    if hasattr(wl, "fr"):
        from collections import Counter
        roof["kernel"] = wl.kernel
        roof["kernels_per_step"] = dict(Counter(names).most_common())
    else:
        # the dominant kernel: the only one, or the one the workload names
        main = [n for n in names if n.startswith(wl.kernel)] or names
        roof["kernel"] = main[0] if main else wl.kernel
        roof["kernels_per_step"] = names
    roof["algorithmic_per_launch"] = {"flops": wl.flops, "bytes": wl.bytes}
    out = {"value": round(rate, 3), "unit": "TOP/s" if wl.dtype == "int8" else "TFLOP/s",
           "ms_per_step": round(ms_step, 5), "dtype": wl.dtype, "config": wl.config, "roofline": roof,
           "wall_s": round(wall, 4)}
    if wl.dtype == "int8":
        out["frac_of_int8_mfma_peak"] = round(rate / PEAK["int8_tops"], 4)
    if eager_ms is not None:
        out["timing"] = f"HIP events around one HIP graph of the {args.steps} launches (recorded after the warm-up)"
        out["ms_per_step_eager"] = round(eager_ms / args.steps, 5)
    elif getattr(wl, "graphable", False):
        out["timing"] = "HIP events around the launches issued one by one"
    else:
        out["timing"] = "HIP events around the frame graph replayed once per step"
    if wl.name in ("c4", "c3c"):
        key = "frame" if wl.name == "c4" else "block"
        out[f"ms_per_{key}"] = round(ms_step, 4)
        if not args.no_host_copies:
            out[f"ms_per_{key}_with_host_copies"] = round(wl.host_roundtrip_ms(), 4)
        if getattr(wl, "mode", "") == "graph" and not args.eager and not args.trace_marks:
            out[f"ms_per_{key}_one_graph"] = round(repeated_graph_ms(wl, min(args.steps, 50)), 5)
    return out


def repeated_graph_ms(wl, reps):
    """ms per step with `reps` steps' launches recorded into one graph (as the
    one-launch configs are timed) instead of one graph replay per step: the
    difference is what each replay's own start costs."""
    from onnxsharp_amd import native as N
    fr, st = wl.fr, wl.fr.stream
    g = C.c_void_p()
    N.call("osh_graph_begin", st)
    try:
        for _ in range(reps):
            for c in fr._calls:
                c(st)
    finally:
        N.call("osh_graph_end", st, C.byref(g))
    e0, e1 = C.c_void_p(), C.c_void_p()
    N.call("osh_event_create", C.byref(e0))
    N.call("osh_event_create", C.byref(e1))
    try:
        N.call("osh_graph_launch", g, st)  # one untimed replay
        best = None
        for _ in range(3):
            N.call("osh_stream_sync", st)
            N.call("osh_event_record", e0, st)
            N.call("osh_graph_launch", g, st)
            N.call("osh_event_record", e1, st)
            N.call("osh_stream_sync", st)
            ms = C.c_float()
            N.call("osh_event_elapsed_ms", e0, e1, C.byref(ms))
            best = ms.value if best is None else min(best, ms.value)
    finally:
        N.call("osh_event_destroy", e0)
        N.call("osh_event_destroy", e1)
        N.call("osh_graph_destroy", g)
    return best / reps


def launch_table(wl, reps=7, replays=40):
    """Each launch's share of a frame graph's replay time.  Graphs of the
    frame's first j launches (j = 1 .. L, the serial order the frame graph
    records) are replayed `replays` times, `reps` times over; t(j) is the
    median time per replay, and launch j's share is t(j) - t(j-1), so the
    shares add up to t(L), the whole frame.  Each share is the time the
    launch adds where it stands in the frame (its gap to the previous kernel
    included), measured with HIP events and no tracer."""
    import torch
    from onnxsharp_amd import native as N
    fr = wl.fr
    ops, calls = fr.model.ops, fr._calls
    st = fr.stream
    names = []
    for c in calls:  # the kernels each launch runs (tiles already tuned)
        N.kernel_log(reset=True)
        c(st)
        N.call("osh_stream_sync", st)
        names.append(N.kernel_log(reset=True))
    e0, e1 = C.c_void_p(), C.c_void_p()
    N.call("osh_event_create", C.byref(e0))
    N.call("osh_event_create", C.byref(e1))
    t = [0.0]
    for j in range(1, len(calls) + 1):
        g = C.c_void_p()
        N.call("osh_graph_begin", st)
        try:
            for c in calls[:j]:
                c(st)
        finally:
            N.call("osh_graph_end", st, C.byref(g))
        for _ in range(5):
            N.call("osh_graph_launch", g, st)
        samples = []
        for _ in range(reps):
            N.call("osh_stream_sync", st)
            N.call("osh_event_record", e0, st)
            for _ in range(replays):
                N.call("osh_graph_launch", g, st)
            N.call("osh_event_record", e1, st)
            N.call("osh_stream_sync", st)
            ms = C.c_float()
            N.call("osh_event_elapsed_ms", e0, e1, C.byref(ms))
            samples.append(ms.value * 1e3 / replays)
        N.call("osh_graph_destroy", g)
        t.append(float(np.median(samples)))
    N.call("osh_event_destroy", e0)
    N.call("osh_event_destroy", e1)
    rows = []
    for j, op in enumerate(ops):
        share = t[j + 1] - t[j]
        fl = float(getattr(op, "flops", 0.0) or 0.0)
        rows.append({"launch": j, "op": op.name, "kind": type(op).__name__, "kernels": names[j],
                     "us": round(share, 3), "gflop": round(fl / 1e9, 4),
                     "tflops": round(fl / (share * 1e-6) / 1e12, 2) if share > 0 and fl else None})
    return {"frame_us": round(t[-1], 3), "launches": len(ops), "sum_us": round(sum(r["us"] for r in rows), 3),
            "method": f"graphs of the first j launches, median of {reps} x {replays} replays each; "
                      "share(j) = t(j) - t(j-1)", "rows": rows}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="all",
                    help="all (default: every workload, C2 as the headline) or one of "
                         + ", ".join(CONFIGS) + ", copy")
    ap.add_argument("--cpu-seconds", type=float, default=None,
                    help="CPU seconds per thread count (default: per workload, 2-10 s)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-host-copies", action="store_true",
                    help="c3c/c4: skip the extra timing with PCIe copies")
    ap.add_argument("--eager", action="store_true",
                    help="time the steps issued one by one (default: one HIP graph of the K launches)")
    ap.add_argument("--trace-marks", action="store_true",
                    help="run a 1-byte fill kernel just before and after each timed region, so that a "
                         "kernel trace can pick out the timed dispatches")
    ap.add_argument("--launch-table", action="store_true",
                    help="c3c/c4: print each launch's share of the frame graph's time (one JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU (every box here has one MI355X); "
              f"--gpus {args.gpus} is not supported. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from onnxsharp_amd import native as N
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    info = N.DeviceInfo()
    N.call("osh_init", 0, C.byref(info))
    dev = torch.device("cuda", 0)

    if args.config == "copy":
        wl = make_workload("copy", dev)
        ms, _, _ = time_gpu(wl, args.steps, args.warmup, graph=not args.eager)
        ms_step = ms / args.steps
        gbs = wl.bytes / (ms_step * 1e-3) / 1e9
        print(json.dumps({"metric": "device copy GB/s", "value": round(gbs, 1), "unit": "GB/s",
                          "ms_per_step": round(ms_step, 5), "bytes_per_step": wl.bytes}), flush=True)
        return

    if args.launch_table:
        if args.config not in ("c3c", "c4"):
            raise SystemExit("--launch-table needs --config c3c or c4")
        wl = make_workload(args.config, dev)
        time_gpu(wl, args.steps, args.warmup)
        tab = launch_table(wl)
        tab.update({"config": args.config, "workload": wl.config.get("workload"),
                    "device": info.name.decode()})
        print(json.dumps(tab), flush=True)
        wl.fr.close()
        return

    names = CONFIGS if args.config == "all" else (args.config,)
    headline = "c2" if args.config == "all" else args.config
    hi = host_info() if not args.no_cpu else None
    results = {}
    for name in names:
        print(f"bench: {name}", file=sys.stderr, flush=True)
        wl = make_workload(name, dev)
        r = measure(wl, args)
        if not args.no_cpu:
            budget = args.cpu_seconds if args.cpu_seconds is not None else CPU_BUDGET.get(name, 2.0)
            r["cpu_baseline"] = cpu_leg(wl, budget, hi)
        results[name] = r
        if hasattr(wl, "fr"):
            wl.fr.close()
        del wl
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    h = results[headline]
    out = {
        "metric": METRIC,
        "value": h["value"],
        "unit": h["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": h["dtype"],
        "data": "synthetic",
        "config": h["config"],
        "device": {"name": info.name.decode(), "arch": info.arch.decode(), "cus": info.compute_units},
        "roofline": h["roofline"],
        "cpu_baseline": h.get("cpu_baseline"),
    }
    for k in ("timing", "ms_per_step_eager", "wall_s", "ms_per_frame", "ms_per_frame_with_host_copies",
              "ms_per_frame_one_graph", "ms_per_block", "ms_per_block_with_host_copies", "ms_per_block_one_graph",
              "frac_of_int8_mfma_peak"):
        if k in h:
            out[k] = h[k]
    if hi is not None:
        out["host"] = hi
        out["reference_paths"] = reference_paths(hi.get("flags", []))
    if len(results) > 1:
        out["configs"] = {k: v for k, v in results.items() if k != headline}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
