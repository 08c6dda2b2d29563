"""GPU parity of the YOLO11n frame (87 convolutions, C2PSA attention, SPPF,
upsampling, concat/split/add glue) against the oracle.

* Per op: every op of the frame (built with the head's DFL/Sigmoid decode, and
  with the launch fusions applied) runs on the device on the device's own
  inputs, and its output must equal the oracle's output for those same inputs
  bit for bit: each kernel sums in the order of the reference's kernel for
  that shape (NCHWc chain, im2col chain, GEMM chain, depthwise, SoftmaxRow's
  lane order, ...).
* End to end: the frame's three head tensors (and, with the decode, the DFL
  and Sigmoid outputs) against an independent restatement of the network
  (oracle/yolo11n_net.py) run from the same input, bit for bit.
* The frame recorded as a HIP graph replays to the eager result, bit for bit,
  with host work and other launches between replays.
SiLU runs in the exact (reference polynomial) mode throughout."""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_fp32_close, fp32_violations
from onnxsharp_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture()
def exact_silu():
    from onnxsharp_amd import native as N
    N.call("osh_config_set", b"exact_silu", 1)
    yield
    N.call("osh_config_set", b"exact_silu", 0)


def _frame(cuda, size, decode=False, chains=False):
    from onnxsharp_amd import yolo11n
    model = yolo11n.build(size, decode=decode)
    return model, yolo11n.Frame(model, cuda, chains=chains)


def _host(sl):
    import torch
    torch.cuda.synchronize()
    return np.ascontiguousarray(sl.buf.tensor[:, sl.c0:sl.c0 + sl.c].cpu().numpy())


@pytest.mark.parametrize("size,chains", [(128, False), (640, False), (640, True)])
def test_yolo_per_op_parity(cuda, oracle, exact_silu, size, chains):
    # 640 is the benchmarked frame: map-size-tuned tiles at 80/40/20, the
    # grouped head launches over three scales and the one-launch C2PSA
    # attention at n = 400 (at 128 the attention takes the five-launch path)
    from oracle import yolo_frame as YO
    from onnxsharp_amd import yolo11n as Y
    model, fr = _frame(cuda, size, decode=True, chains=chains)
    try:
        print(f"per-op parity at {size}x{size}, chains={chains}: {len(fr.model.ops)} launches", flush=True)
        fr.set_input(synth.uniform(4242, (1, 3, size, size)))
        worst = (0.0, "")
        assert len(fr.model.ops) < len(model.ops)  # the residual Adds run inside their convs
        for i, launch in enumerate(fr.model.ops):
            # a GroupConvOp is one launch of independent convs, a ChainOp one
            # launch of convs in chains: check each conv against the oracle
            # run one by one over host copies of the buffers the launch
            # touches, taken before it (later stages read earlier outputs)
            members = launch.ops if isinstance(launch, (Y.GroupConvOp, Y.ChainOp, Y.PairOp)) else [launch]
            reads, writes = Y.op_access(launch)
            host = {}
            for sl in reads + writes:
                if id(sl.buf) not in host:
                    host[id(sl.buf)] = _host(Y.whole(sl.buf)).copy()
            fr._calls[i](fr.stream)
            fr.sync()
            for op in members:
                oin = [np.ascontiguousarray(host[id(s.buf)][:, s.c0:s.c0 + s.c]) for s in YO.op_inputs(op)]
                ref = YO.run_op(oracle, op, oin)
                host[id(op.y.buf)][:, op.y.c0:op.y.c0 + op.y.c] = ref
                if isinstance(launch, Y.PairOp) and op is launch.a and not launch.store_mid:
                    continue  # the intermediate stayed on chip: its oracle value feeds b
                got = _host(op.y)
                what = f"op {i} {type(op).__name__} {op.name}"
                nbad, dmax = fp32_violations(got, ref)
                assert_fp32_close(got, ref, what)
                assert np.array_equal(got, ref), f"{what}: not bit-identical (max |d| {dmax:.3e})"
        kinds = sorted({type(l).__name__ for l in fr.model.ops})
        print(f"{len(fr.model.ops)} ops bit-identical ({', '.join(kinds)})", flush=True)
        if size == 640:  # the launches that only the 640 frame takes were checked
            assert any(isinstance(l, Y.AttentionOp) for l in fr.model.ops)
            assert any(isinstance(l, Y.GroupConvOp) for l in fr.model.ops)
            assert any(isinstance(l, Y.ChainOp) for l in fr.model.ops) == chains
    finally:
        fr.close()


@pytest.mark.parametrize("size", [320, 640])
def test_yolo_end_to_end(cuda, oracle, exact_silu, size):
    # against the independent restatement of the network (oracle/yolo11n_net.py,
    # written without the device package's builder), so the frame's wiring is
    # checked along with its arithmetic
    from oracle import yolo11n_net
    model, fr = _frame(cuda, size)
    print(f"end to end at {size}x{size}", flush=True)
    try:
        x = synth.uniform(4243, (1, 3, size, size))
        fr.set_input(x)
        fr.run()
        fr.sync()
        got = [t.cpu().numpy() for t in fr.outputs()]
        ref = yolo11n_net.forward(oracle, x)
        for i, (g, r) in enumerate(zip(got, ref)):
            d = np.abs(g.astype(np.float64) - r)
            print(f"head {i} {g.shape}: max|d| {d.max():.3e}, range {np.abs(r).max():.3e}", flush=True)
            assert np.isfinite(g).all()
            assert np.array_equal(g, r), f"head {i}: max |d| {d.max():.3e}"
    finally:
        fr.close()


def test_yolo_640_graph_default_silu_within_tolerance(cuda, oracle):
    # the benchmarked configuration: the 640 frame replayed as one HIP graph
    # with the default (fast) SiLU epilogue, against the independent oracle
    # network with the reference polynomial; FP32 bar |d| <= 1e-5 + 1e-4 |ref|
    # on all three head tensors
    from oracle import yolo11n_net
    size = 640
    model, fr = _frame(cuda, size)
    try:
        x = synth.uniform(4000, (1, 3, size, size))
        fr.set_input(x)
        fr.run()
        fr.sync()
        fr.capture()
        for t in fr.outputs():
            t.fill_(float("nan"))
        fr.launch()
        fr.sync()
        got = [t.cpu().numpy() for t in fr.outputs()]
        ref = yolo11n_net.forward(oracle, x)
        for i, (g, r) in enumerate(zip(got, ref)):
            nbad, dmax = fp32_violations(g, r)
            rel = float((np.abs(g.astype(np.float64) - r) / (1e-5 + np.abs(r))).max())
            print(f"head {i} {g.shape}: max|d| {dmax:.3e}, max |d|/(1e-5+|ref|) {rel:.3e}", flush=True)
            assert_fp32_close(g, r, f"head {i}")
    finally:
        fr.close()


def test_yolo_end_to_end_without_nchwc(cuda, oracle, exact_silu):
    # the 640 frame on a reference host without NchwcConv (nchwc = 0): its 30
    # NCHWc layers take Winograd (40x40, 20x20) or the im2col chain; pairs and
    # grouped launches that would sum another chain fall back to single
    # launches; the heads equal the independent network's, bit for bit
    from onnxsharp_amd import native as N
    from oracle import yolo11n_net
    size = 640
    old = C.c_int()
    N.call("osh_config_get", b"nchwc", C.byref(old))
    N.call("osh_config_set", b"nchwc", 0)
    try:
        model, fr = _frame(cuda, size)
        try:
            print(f"end to end at {size}x{size} with nchwc=0: {len(fr.model.ops)} launches", flush=True)
            x = synth.uniform(4247, (1, 3, size, size))
            fr.set_input(x)
            N.kernel_log(reset=True)
            fr.run()
            fr.sync()
            names = N.kernel_log(reset=True)
            got = [t.cpu().numpy() for t in fr.outputs()]
        finally:
            fr.close()
    finally:
        N.call("osh_config_set", b"nchwc", old.value)
    assert any(n.startswith("wino_f23") for n in names), names
    ref = yolo11n_net.forward(oracle, x, nchwc=0)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert np.array_equal(g, r), f"head {i}: max |d| {np.abs(g - r).max():.3e}"
    on = yolo11n_net.forward(oracle, x, nchwc=1)
    assert not all(np.array_equal(g, r) for g, r in zip(got, on))


def test_yolo_decoded_heads_end_to_end(cuda, oracle, exact_silu):
    # the frame with the head's DFL and class Sigmoid on the device, against
    # the independent network's decode, bit for bit
    from oracle import yolo11n_net
    size = 640
    model, fr = _frame(cuda, size, decode=True)
    try:
        x = synth.uniform(4245, (1, 3, size, size))
        fr.set_input(x)
        fr.run()
        fr.sync()
        got = [t.cpu().numpy() for t in fr.outputs()]
        ref = yolo11n_net.forward(oracle, x, decode=True)
        for i, (g, r) in enumerate(zip(got, ref)):
            assert g.shape == r.shape == (1, 84, size // (8 << i), size // (8 << i))
            assert np.array_equal(g, r), f"decoded head {i}: max |d| {np.abs(g - r).max():.3e}"
    finally:
        fr.close()


@pytest.mark.parametrize("parallel,flat", [(False, False), (True, False), (True, True)],
                         ids=["chain", "segments", "flat"])
def test_yolo_graph_replay_matches_eager(cuda, parallel, flat):
    import torch
    from onnxsharp_amd import native as N
    model, fr = _frame(cuda, 128)
    try:
        x = synth.uniform(4244, (1, 3, 128, 128))
        fr.set_input(x)
        torch.cuda.synchronize()
        fr.run()
        fr.sync()
        eager = [t.cpu().numpy().copy() for t in fr.outputs()]
        print(f"capturing {len(model.ops)} ops (parallel={parallel}, flat={flat})", flush=True)
        fr.capture(parallel=parallel, flat=flat)
        print("captured", flush=True)
        for rep in range(3):
            print(f"replay {rep}", flush=True)
            for t in fr.outputs():
                t.fill_(float("nan"))  # the replay must rewrite every output
            torch.cuda.synchronize()
            fr.launch()
            fr.sync()
            got = [t.cpu().numpy() for t in fr.outputs()]
            for g, e in zip(got, eager):
                assert np.array_equal(g, e), f"replay {rep} differs from the eager frame"
            # unrelated device work between replays
            scratch = torch.randn(1 << 20, device=cuda)
            N.call("osh_activation_f32", scratch.numel(), C.c_void_p(scratch.data_ptr()), N.ACT_RELU,
                   C.c_void_p(scratch.data_ptr()), None)
            torch.cuda.synchronize()
    finally:
        fr.close()


@pytest.mark.parametrize("size,shortcut", [(80, True), (36, False)])
def test_c2f_block_is_bit_exact(cuda, oracle, exact_silu, size, shortcut):
    # every op of the C2f block is an exact restatement (1x1 convs: the GEMM
    # chain; 3x3 convs: the NCHWc chain; the shortcut Add folded into the
    # second 3x3 conv's epilogue), so the whole block matches the oracle bit
    # for bit, eagerly and as a replayed graph
    import torch
    from oracle import yolo_frame as YO
    from onnxsharp_amd import yolo11n
    model = yolo11n.build_c2f(size, 128, 128, 1, shortcut)
    fr = yolo11n.Frame(model, cuda)
    try:
        x = synth.uniform(4246 + size, (1, 128, size, size))
        fr.set_input(x)
        fr.run()
        fr.sync()
        got = fr.outputs()[0].cpu().numpy()
        ref = YO.Frame(model).run(oracle, x)[0]
        assert np.array_equal(got, ref), f"max |d| {np.abs(got - ref).max():.3e}"
        fr.capture()
        fr.outputs()[0].fill_(float("nan"))
        torch.cuda.synchronize()
        fr.launch()
        fr.sync()
        assert np.array_equal(fr.outputs()[0].cpu().numpy(), ref)
    finally:
        fr.close()
