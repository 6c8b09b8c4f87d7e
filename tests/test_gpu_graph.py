"""Whole-graph and seam parity on the GPU: IrGraphs installed as programs,
the run_kernel handler seam, the run_node arena seam, and error mapping —
against the oracle's eval_graph_cpu / eval_graph_reference restatement."""
import os

import numpy as np
import pytest

import catnn_amd
import oracle
from catnn_amd import (CatError, DeviceHandler, IrGraph, IrNode, OpenOp, Program, Tensor,
                       TensorType, arena_conflict, configs)
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _check_graph(device, g, x, bound_abs=None, tol=TOL):
    prog = Program(device, g)
    got = prog.forward(x)
    want = oracle.eval_graph(g, x.numpy())
    want_ref = oracle.eval_graph(g, x.numpy(), reference=True)
    err, err_ref = rel_l2(got.numpy(), want), rel_l2(got.numpy(), want_ref)
    mx = float(np.max(np.abs(got.numpy() - want)))
    print(f"{g.name}: rel_l2 cpu={err:.2e} ref={err_ref:.2e} max_abs={mx:.2e}")
    assert got.numpy().shape == want.shape
    assert err < tol and err_ref < tol
    if bound_abs is not None:
        assert mx < bound_abs
    allocs, reserved = prog.arena()
    assert arena_conflict(allocs) is None
    assert reserved <= sum(a.bytes for a in allocs)
    prog.free()
    return got


def test_mlp_catnn_example_e2e(device):
    # crates/catnn-rt/tests/e2e.rs:8-17: examples/mlp.catnn, lcg input seed 1, < 1e-4
    spec = catnn_amd.parse_catnn(open(os.path.join(GOLDEN, "mlp.catnn")).read())
    g = catnn_amd.lower_architecture(catnn_amd.to_architecture(spec))
    g.fusions = catnn_amd.propose_fusions(g)
    _check_graph(device, g, Tensor.lcg(TensorType.f32([4, 16]), 1), bound_abs=1e-4)


def test_transformer_block_spec_e2e(device):
    # e2e.rs:20-27: transformer_block_spec(2, 8, 16, 4), lcg input seed 11, < 1e-4
    g = catnn_amd.lower_architecture(catnn_amd.transformer_block_spec(2, 8, 16, 4))
    g.fusions = catnn_amd.propose_fusions(g)
    _check_graph(device, g, Tensor.lcg(TensorType.f32([2, 8, 16]), 11), bound_abs=1e-4)


def test_transformer_catnn_example(device):
    spec = catnn_amd.parse_catnn(open(os.path.join(GOLDEN, "transformer.catnn")).read())
    g = catnn_amd.lower_architecture(catnn_amd.to_architecture(spec))
    # `attention mha 8 16 4` is seq 8, d_model 16, 4 heads on batch 2
    _check_graph(device, g, Tensor.lcg(TensorType.f32([2, 8, 16]), 3), bound_abs=1e-4)


def test_config1_mlp(device):
    w = configs.config1()
    _check_graph(device, w.graph, w.x)


@pytest.mark.parametrize("causal", [True, False])
def test_config3_block_small(device, causal):
    w = configs.config3(batch=2, seq=128, d=256, heads=4, ffn=1024, causal=causal)
    _check_graph(device, w.graph, w.x)


def test_config3_block_ragged_seq(device):
    w = configs.config3(batch=1, seq=77, d=128, heads=2, ffn=256, causal=True)
    _check_graph(device, w.graph, w.x)


def test_config4_moe_small(device):
    w = configs.config4(batch=2, seq=64, d=128, n_experts=4, top_k=2, inter=96)
    _check_graph(device, w.graph, w.x)


def test_unfused_graph_matches_fused(device):
    w = configs.config1(batch=64)
    fused = Program(device, w.graph).forward(w.x)
    w.graph.fusions = []
    plain = Program(device, w.graph).forward(w.x)
    assert np.array_equal(fused.data, plain.data)


def test_run_kernel_seam_and_events(device):
    h = DeviceHandler(device)
    device.clear_events()
    r = np.random.default_rng(3)
    node = IrNode(5, "fc", OpenOp.linear(24, 40, True), TensorType.f32([3, 7, 40]),
                  {"w": Tensor.from_numpy(r.standard_normal((24, 40)).astype(np.float32)),
                   "b": Tensor.from_numpy(r.standard_normal(40).astype(np.float32))})
    x = Tensor.from_numpy(r.standard_normal((3, 7, 24)).astype(np.float32))
    y = h.run_kernel(node, [x])
    assert y.ty == TensorType.f32([3, 7, 40])
    want = oracle.linear(x.numpy(), node.params["w"].numpy(), node.params["b"].numpy())
    assert rel_l2(y.numpy(), want) < TOL
    ev = device.events()
    assert [e[2] for e in ev] == [0, 1] and ev[0][1] == "fc" and ev[0][0] < ev[1][0]
    assert ev[1][3] == y.checksum()
    # pass-through ops keep their input's type (eval_cpu returns x.clone())
    t = h.run_kernel(IrNode(6, "t", OpenOp.transpose(0, 1), TensorType.f32([7, 3, 40])), [y])
    assert t.ty == y.ty and np.array_equal(t.data, y.data)
    # Identity with no inputs → zeros of output_ty (mod.rs:22-24)
    z = h.run_kernel(IrNode(7, "z", OpenOp.identity(), TensorType.f32([2, 3])), [])
    assert z.ty == TensorType.f32([2, 3]) and not z.data.any()


def test_event_stamps_are_device_times(device):
    # A node's KernelStart → KernelEnd span is the device time of its
    # kernels: a 2048³ fp32 GEMM (17.2 GFLOP) cannot finish in less than
    # 17.2e9 / 157.3e12 s = 109 µs on MI355X's matrix cores, however fast the
    # host enqueues it; the host-side enqueue of the same call takes far less.
    h = DeviceHandler(device)
    r = np.random.default_rng(6)
    n = 2048
    node = IrNode(9, "big", OpenOp.linear(n, n, False), TensorType.f32([n, n]),
                  {"w": Tensor.from_numpy(r.standard_normal((n, n)).astype(np.float32))})
    x = Tensor.from_numpy(r.standard_normal((n, n)).astype(np.float32))
    h.run_kernel(node, [x])  # warm-up
    device.clear_events()
    y = h.run_kernel(node, [x])
    ev = device.events()
    assert [e[2] for e in ev] == [0, 1]
    span_ns = ev[1][0] - ev[0][0]
    print(f"  device span {span_ns / 1e3:.1f} us")
    assert 109_000 <= span_ns < 50_000_000
    assert ev[1][3] == y.checksum()


def test_run_kernel_every_executable_op(device):
    h = DeviceHandler(device)
    r = np.random.default_rng(4)
    x = Tensor.from_numpy(r.standard_normal((2, 8, 16)).astype(np.float32))
    x2 = Tensor.from_numpy(r.standard_normal((2, 8, 16)).astype(np.float32))
    bias = Tensor.from_numpy(r.standard_normal(16).astype(np.float32))
    g = Tensor.from_numpy(r.standard_normal(16).astype(np.float32))
    ty = x.ty
    cases = [
        (IrNode(1, "r", OpenOp.relu(), ty), [x]),
        (IrNode(1, "g", OpenOp.gelu(), ty), [x]),
        (IrNode(1, "s", OpenOp.softmax(-1), ty), [x]),
        (IrNode(1, "a", OpenOp.add(), ty), [x, x2]),
        (IrNode(1, "ab", OpenOp.add(), ty), [x, bias]),
        (IrNode(1, "ra", OpenOp.residual_add(), ty), [x, x2]),
        (IrNode(1, "m", OpenOp.mul(), ty), [x, x2]),
        (IrNode(1, "ln", OpenOp.layer_norm(1), ty, {"gamma": g, "beta": bias}), [x]),
        (IrNode(1, "mm", OpenOp.matmul(), TensorType.f32([2, 8, 4]),
                {"w": Tensor.from_numpy(r.standard_normal((16, 4)).astype(np.float32))}), [x]),
        (IrNode(1, "at", OpenOp.attention(4, 16, 4), ty,
                {p: Tensor.from_numpy((r.standard_normal((16, 16)) * 0.25).astype(np.float32))
                 for p in ("wq", "wk", "wv", "wo")}), [x]),
    ]
    for node, ins in cases:
        got = h.run_kernel(node, ins).numpy()
        want = oracle.eval_node(node, [t.numpy() for t in ins])
        err = rel_l2(got, want)
        print(f"{node.name}: {err:.2e}")
        assert got.shape == want.shape and err < TOL, node.name


def test_error_kinds(device):
    h = DeviceHandler(device)
    x = Tensor.zeros(TensorType.f32([2, 8]))
    bad_w = IrNode(1, "fc", OpenOp.linear(9, 4, False), TensorType.f32([2, 4]),
                   {"w": Tensor.zeros(TensorType.f32([9, 4]))})
    with pytest.raises(CatError) as e:
        h.run_kernel(bad_w, [x])
    assert e.value.kind == "ShapeMismatch"
    ln = IrNode(1, "ln", OpenOp.layer_norm(1), x.ty, {"beta": Tensor.zeros(TensorType.f32([8]))})
    with pytest.raises(CatError) as e:
        h.run_kernel(ln, [x])
    assert e.value.kind == "UnknownPort" and "gamma" in str(e.value)
    emb = IrNode(1, "emb", OpenOp("embedding", (10, 4)), TensorType.f32([2, 8, 4]))
    with pytest.raises(CatError) as e:
        h.run_kernel(emb, [x])
    assert e.value.kind == "UnknownPort" and "w" in str(e.value)  # mod.rs:82-85
    mla = IrNode(1, "mla", OpenOp("mla", (2, 4, 4, 4, 4, 4, 10000)), TensorType.f32([2, 8]))
    with pytest.raises(CatError) as e:
        h.run_kernel(mla, [x])
    assert e.value.kind == "Unsupported"
    with pytest.raises(CatError) as e:
        h.run_kernel(IrNode(1, "r", OpenOp.relu(), x.ty), [])
    assert e.value.kind == "Wiring"
    g = IrGraph("cyc")
    g.add_node(IrNode(0, "a", OpenOp.relu(), x.ty))
    g.add_node(IrNode(1, "b", OpenOp.relu(), x.ty))
    g.add_edge(0, 1)
    g.add_edge(1, 0)
    g.outputs.append(1)
    with pytest.raises(CatError) as e:
        Program(device, g)
    assert e.value.kind == "Wiring"


def test_run_node_on_arena_buffers(device):
    r = np.random.default_rng(5)
    m, k, n = 64, 48, 80
    x = r.standard_normal((m, k)).astype(np.float32)
    w = r.standard_normal((k, n)).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32)
    res = r.standard_normal((m, n)).astype(np.float32)
    device.arena_reserve(1 << 20)
    device.bind("act:0", 0, x.nbytes)
    device.bind("param:fc:w", 1 << 16, w.nbytes)
    device.bind("param:fc:b", 1 << 17, b.nbytes)
    device.bind("act:skip", 1 << 18, res.nbytes)
    device.bind("act:2", 1 << 19, m * n * 4)
    for bid, arr in [("act:0", x), ("param:fc:w", w), ("param:fc:b", b), ("act:skip", res)]:
        device.upload(bid, arr)
    node = IrNode(1, "fc", OpenOp.linear(k, n, True), TensorType.f32([m, n]),
                  {"w": Tensor.from_numpy(w), "b": Tensor.from_numpy(b)})
    import ctypes
    from catnn_amd._lib import CTensor, check, lib
    from catnn_amd.ir import ctensor
    cnode, keep = node.to_c(with_data=False)
    ids = (ctypes.c_char_p * 1)(b"act:0")
    tys = (CTensor * 1)(ctensor(ty=TensorType.f32([m, k])))
    device.clear_events()
    check(lib.catnn_hip_run_node(device.handle, ctypes.byref(cnode), ids, tys, 1, b"act:2", 3, b"act:skip"))
    got = device.download("act:2", (m, n))
    want = oracle.add(res, oracle.gelu(oracle.linear(x, w, b)))
    assert rel_l2(got, want) < TOL
    # KernelStart/KernelEnd stamped on the device, the output's checksum on KernelEnd
    ev = device.events()
    assert [(e[1], e[2]) for e in ev] == [("fc", 0), ("fc", 1)] and ev[0][0] < ev[1][0]
    assert ev[1][3] == Tensor.from_numpy(got).checksum()
    device.trace_checksums(False)
    check(lib.catnn_hip_run_node(device.handle, ctypes.byref(cnode), ids, tys, 1, b"act:2", 3, b"act:skip"))
    device.trace_checksums(True)
    ev2 = device.events()
    assert len(ev2) == 4 and ev2[3][3] == 0 and ev2[1][0] < ev2[2][0] < ev2[3][0]
    with pytest.raises(CatError) as e:
        device.download("act:nope", (1,))
    assert e.value.kind == "UnknownPort"
    with pytest.raises(CatError) as e:
        device.bind("too_big", 1 << 20, 8)
    assert e.value.kind == "Fibration"
    device.arena_reserve(0)


def test_program_arena_aliases_dead_activations(device):
    w = configs.config1(batch=32)
    prog = Program(device, w.graph)
    allocs, reserved = prog.arena()
    acts = [a for a in allocs if a.id.startswith("act:")]
    # input, two fused Linear+ReLU outputs and the final output: the first
    # activation is dead once fc2 has read it, so fc3's output reuses its bytes.
    assert arena_conflict(allocs) is None
    assert reserved < sum(a.bytes for a in allocs)
    assert {a.id for a in acts} == {"act:0", "act:2", "act:4", "act:5"}
    prog.free()


def test_graph_from_serde_json_runs(device):
    # The hand-written serde form of a Linear(4→3, bias) → ReLU graph.
    import json

    from catnn_amd import CGraph

    text = open(os.path.join(GOLDEN, "mlp_ir.json")).read()
    doc = json.loads(text)
    w = np.array(doc["nodes"]["1"]["params"]["w"]["data"], np.float32).reshape(4, 3)
    b = np.array(doc["nodes"]["1"]["params"]["b"]["data"], np.float32)
    x = Tensor.lcg(TensorType.f32([2, 4]), 5)
    got = Program(device, CGraph.from_json(text)).forward(x).numpy()
    want = oracle.relu(oracle.linear(x.numpy(), w, b))
    assert rel_l2(got, want) < TOL


def test_json_blob_graph_matches_the_ir_graph(device):
    from catnn_amd import CGraph, Trainer, to_serde_json

    w = configs.config3(batch=1, seq=64, d=128, heads=2, ffn=256, causal=True)
    lean, blob = to_serde_json(w.graph, inline=False)
    cg = CGraph.from_json(lean, blob)
    a = Program(device, cg).forward(w.x).numpy()
    b = Program(device, w.graph).forward(w.x).numpy()
    assert np.array_equal(a, b)
    tgt = Tensor(w.x.ty, np.zeros(w.x.ty.numel(), np.float32))
    t1, t2 = Trainer(device, cg, 0.05), Trainer(device, w.graph, 0.05)
    t1.set_batch(w.x, tgt)
    t2.set_batch(w.x, tgt)
    assert t1.step() == t2.step()
    assert np.array_equal(t1.grad(5, "w", (128, 256)), t2.grad(5, "w", (128, 256)))
