"""adjoint_of on the GPU, node by node (catnn_hip_run_adjoint through
DeviceHandler.adjoint_of), against the oracle's restatement of
crates/catnn-compile/src/kernel/adjoint.rs:762-951 on the same seeded inputs
and cotangent.  The seam runs the trainer's fp32 precision (every GEMM on
six-part split operands, everything else fp32), so every input and
parameter cotangent is held to the fp32 bar: relative L2 1e-4."""
import numpy as np
import pytest

import oracle
import oracle_train as ot
from catnn_amd import CatError, DeviceHandler, IrGraph, IrNode, OpenOp, Tensor, TensorType, Trainer
from conftest import rel_l2

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 1e-2


def _t(a):
    return Tensor.from_numpy(np.ascontiguousarray(a, np.float32))


def _check(device, node, ins, tol, seed=0):
    r = np.random.default_rng(seed)
    ins = [np.asarray(a, np.float32) for a in ins]
    out = oracle.eval_node(node, ins)
    dy = r.standard_normal(out.shape).astype(np.float32)
    print(f"[adjoint] {node.name} {node.op.kind} ins={[a.shape for a in ins]}", flush=True)
    dx, dp = DeviceHandler(device).adjoint_of(node, [_t(a) for a in ins], None, _t(dy))
    dx_o, dp_o = ot.adjoint_of(node, ins, out, dy)
    assert len(dx) == len(dx_o) == len(ins)
    for i, (a, b) in enumerate(zip(dx, dx_o)):
        assert a.ty.shape == ins[i].shape
        e = rel_l2(a.numpy(), np.asarray(b).reshape(ins[i].shape))
        print(f"  dx[{i}] rel_l2 {e:.2e}")
        assert e < tol, (node.name, i, e)
    assert list(dp) == list(node.params)
    # A cotangent the mathematics makes exactly zero (GQA with window 1:
    # dwq = dwk = 0) is held relative to the node's largest one instead.
    scale = max([float(np.linalg.norm(np.asarray(v, np.float64))) for v in dp_o.values()] + [1e-30])
    for port, g in dp.items():
        want = np.asarray(dp_o[port]).reshape(node.params[port].ty.shape)
        if np.any(want):
            e = rel_l2(g.numpy(), want)
        else:
            e = float(np.linalg.norm(g.numpy().astype(np.float64))) / scale
        print(f"  d{port} rel_l2 {e:.2e}")
        assert g.ty.shape == tuple(node.params[port].ty.shape)
        assert e < tol, (node.name, port, e)
    return dx, dp


@pytest.mark.parametrize("m,k,n,bias", [(64, 128, 96, True), (37, 784, 10, True), (256, 512, 512, False)])
def test_linear(device, m, k, n, bias):
    r = np.random.default_rng(k + n)
    params = {"w": _t(r.standard_normal((k, n)) / np.sqrt(k))}
    if bias:
        params["b"] = _t(r.standard_normal(n))
    node = IrNode(3, "fc", OpenOp.linear(k, n, bias), TensorType.f32([m, n]), params)
    _check(device, node, [r.standard_normal((m, k))], FP32_TOL)


@pytest.mark.parametrize("op", ["relu", "gelu", "identity"])
def test_elementwise(device, op):
    r = np.random.default_rng(1)
    x = r.standard_normal((33, 65)) * 2
    node = IrNode(1, op, getattr(OpenOp, op)(), TensorType.f32([33, 65]))
    dx, _ = _check(device, node, [x], FP32_TOL)


@pytest.mark.parametrize("op", ["add", "residual_add"])
def test_two_input_add(device, op):
    r = np.random.default_rng(2)
    a, b = r.standard_normal((4, 50)), r.standard_normal((4, 50))
    node = IrNode(5, op, getattr(OpenOp, op)(), TensorType.f32([4, 50]))
    dx, _ = _check(device, node, [a, b], FP32_TOL)
    assert np.array_equal(dx[0].numpy(), dx[1].numpy())  # dy to both inputs (adjoint.rs:778-784)


@pytest.mark.parametrize("rows,cols", [(64, 128), (9, 1000)])
def test_layer_norm(device, rows, cols):
    r = np.random.default_rng(cols)
    node = IrNode(2, "ln", OpenOp.layer_norm(1), TensorType.f32([rows, cols]),
                  {"gamma": _t(1 + 0.1 * r.standard_normal(cols)), "beta": _t(0.1 * r.standard_normal(cols))})
    _check(device, node, [r.standard_normal((rows, cols)) * 2 + 0.5], FP32_TOL)


@pytest.mark.parametrize("rows,cols", [(64, 1024), (9, 100)])
def test_rms_norm(device, rows, cols):
    r = np.random.default_rng(cols + 1)
    node = IrNode(2, "rms", OpenOp.rms_norm(10), TensorType.f32([rows, cols]),
                  {"w": _t(1 + 0.1 * r.standard_normal(cols))})
    _check(device, node, [r.standard_normal((rows, cols)) * 2 + 0.5], FP32_TOL)


def test_softmax_and_mul(device):
    r = np.random.default_rng(10)
    sm = IrNode(1, "sm", OpenOp.softmax(), TensorType.f32([7, 333]))
    _check(device, sm, [3 * r.standard_normal((7, 333))], FP32_TOL)
    mul = IrNode(2, "mul", OpenOp.mul(), TensorType.f32([4, 50]))
    _check(device, mul, [r.standard_normal((4, 50)), r.standard_normal((4, 50))], FP32_TOL)


def test_softmax_mul_graph_step(device):
    # in → fc → softmax → mul(softmax, fc): the softmax adjoint reads its own
    # output after its consumer's adjoint has run.
    r = np.random.default_rng(11)
    g = IrGraph("sm")
    ty = TensorType.f32([16, 64])
    g.add_node(IrNode(0, "in", OpenOp.identity(), ty))
    g.add_node(IrNode(1, "fc", OpenOp.linear(64, 64), ty,
                      {"w": _t(r.standard_normal((64, 64)) / 8), "b": _t(r.standard_normal(64) * 0.1)}))
    g.add_node(IrNode(2, "sm", OpenOp.softmax(), ty))
    g.add_node(IrNode(3, "mul", OpenOp.mul(), ty))
    for a, b in ((0, 1), (1, 2), (2, 3), (1, 3)):
        g.add_edge(a, b)
    g.inputs, g.outputs = [0], [3]
    x = r.standard_normal((16, 64)).astype(np.float32)
    tgt = r.standard_normal((16, 64)).astype(np.float32)
    tr = Trainer(device, g, 0.05)
    tr.set_batch(_t(x), _t(tgt))
    loss = tr.step()
    loss_o, grads_o, _ = ot.train_step(g, x, tgt, 0.05)
    assert abs(loss - loss_o) <= 2e-3 * max(1.0, abs(loss_o))
    for nid, dp in grads_o.items():
        for port, go in dp.items():
            shape = tuple(g.nodes[nid].params[port].ty.shape)
            e = rel_l2(tr.grad(nid, port, shape), np.asarray(go).reshape(shape))
            print(f"  grad {g.nodes[nid].name}.{port}: {e:.2e}")
            assert e < BF16_TOL, (nid, port, e)
    tr.free()


def test_embedding(device):
    # The table's cotangent sums each row's tokens in token order, as the
    # reference does: bit-exact.  Ids repeat; the ids get zero.
    r = np.random.default_rng(8)
    V, H = 50, 1024
    ids = r.integers(0, V, (2, 300)).astype(np.float32)
    ids[0, :3] = [1.5, -2.0, 49.4]
    node = IrNode(1, "emb", OpenOp.embedding(V, H), TensorType.f32([2, 300, H]),
                  {"w": _t(r.standard_normal((V, H)))})
    dy = r.standard_normal((2, 300, H)).astype(np.float32)
    dx, dp = DeviceHandler(device).adjoint_of(node, [_t(ids)], None, _t(dy))
    assert not dx[0].numpy().any()
    assert np.array_equal(dp["w"].numpy(), ot.embedding_backward(ids, (V, H), dy))
    with pytest.raises(CatError) as e:
        DeviceHandler(device).adjoint_of(node, [_t(np.full((2, 300), 50.0))], None, _t(dy))
    assert e.value.kind == "ShapeMismatch"


@pytest.mark.parametrize("gate", [None, 0.7])
def test_mix(device, gate):
    r = np.random.default_rng(6)
    params = {} if gate is None else {"gate": _t([gate])}
    node = IrNode(3, "mix", OpenOp.mix(), TensorType.f32([5, 300]), params)
    ins = [r.standard_normal((5, 300)), r.standard_normal((5, 300))]
    _check(device, node, ins, FP32_TOL)
    if gate is None:
        # The reference reports a [1] gate cotangent even for a Mix without a
        # gate param (adjoint.rs:918-927); run_adjoint returns one cotangent
        # per param the node holds, so a gate-less Mix gets none.
        x = [np.asarray(a, np.float32) for a in ins]
        dy = np.ones((5, 300), np.float32)
        _, dp_o = ot.adjoint_of(node, x, oracle.eval_node(node, x), dy)
        _, dp = DeviceHandler(device).adjoint_of(node, [_t(a) for a in x], None, _t(dy))
        assert list(dp_o) == ["gate"] and dp == {}


def test_mix_graph_step(device):
    # in → relu, gelu → mix(relu, gelu) with a trained gate; the gate's and
    # the input path's cotangents through a whole step, against the fp32 step.
    r = np.random.default_rng(7)
    g = IrGraph("mix")
    ty = TensorType.f32([16, 64])
    g.add_node(IrNode(0, "in", OpenOp.identity(), ty))
    g.add_node(IrNode(1, "fc", OpenOp.linear(64, 64), ty,
                      {"w": _t(r.standard_normal((64, 64)) / 8), "b": _t(r.standard_normal(64) * 0.1)}))
    g.add_node(IrNode(2, "a", OpenOp.relu(), ty))
    g.add_node(IrNode(3, "b", OpenOp.gelu(), ty))
    g.add_node(IrNode(4, "mix", OpenOp.mix(), ty, {"gate": _t([0.3])}))
    for a, b in ((0, 1), (1, 2), (1, 3), (2, 4), (3, 4)):
        g.add_edge(a, b)
    g.inputs, g.outputs = [0], [4]
    x = r.standard_normal((16, 64)).astype(np.float32)
    tgt = r.standard_normal((16, 64)).astype(np.float32)
    tr = Trainer(device, g, 0.05)
    tr.set_batch(_t(x), _t(tgt))
    loss = tr.step()
    loss_o, grads_o, _ = ot.train_step(g, x, tgt, 0.05)
    assert abs(loss - loss_o) <= 2e-3 * max(1.0, abs(loss_o))
    for nid, dp in grads_o.items():
        for port, go in dp.items():
            shape = tuple(g.nodes[nid].params[port].ty.shape)
            e = rel_l2(tr.grad(nid, port, shape), np.asarray(go).reshape(shape))
            print(f"  grad {g.nodes[nid].name}.{port}: {e:.2e}")
            assert e < BF16_TOL, (nid, port, e)
    tr.free()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("heads,dh", [(2, 64), (4, 32), (1, 128)])  # the MFMA adjoint's head sizes
def test_attention(device, causal, heads, dh):
    r = np.random.default_rng(3)
    d, b, s = 128, 2, 96
    params = {p: _t(0.05 * r.standard_normal((d, d))) for p in ("wq", "wk", "wv", "wo")}
    node = IrNode(4, "attn", OpenOp.attention(heads, d, dh, causal), TensorType.f32([b, s, d]), params)
    _check(device, node, [r.standard_normal((b, s, d))], FP32_TOL)


@pytest.mark.parametrize("T,H,I", [(64, 128, 256), (37, 100, 52)])
def test_swiglu(device, T, H, I):
    r = np.random.default_rng(T + I)
    params = {"w1": _t(r.standard_normal((H, I)) / np.sqrt(H)), "w3": _t(r.standard_normal((H, I)) / np.sqrt(H)),
              "w2": _t(r.standard_normal((I, H)) / np.sqrt(I))}
    node = IrNode(4, "sw", OpenOp.swiglu(H, I), TensorType.f32([T, H]), params)
    _check(device, node, [r.standard_normal((T, H))], FP32_TOL)


def test_moe(device):
    r = np.random.default_rng(4)
    E, k, H, I, T = 4, 2, 128, 96, 200
    params = {"gate": _t(0.5 * r.standard_normal((H, E)))}
    for e in range(E):
        params[f"e{e}.w1"] = _t(0.05 * r.standard_normal((H, I)))
        params[f"e{e}.w3"] = _t(0.05 * r.standard_normal((H, I)))
        params[f"e{e}.w2"] = _t(0.05 * r.standard_normal((I, H)))
    node = IrNode(6, "moe", OpenOp.moe(E, k, H, I), TensorType.f32([T, H]), params)
    _check(device, node, [r.standard_normal((T, H))], FP32_TOL)


def test_adjoint_errors(device):
    h = DeviceHandler(device)
    node = IrNode(1, "r", OpenOp.relu(), TensorType.f32([4]))
    with pytest.raises(CatError) as e:
        h.adjoint_of(node, [], None, _t(np.ones(4)))
    assert e.value.kind == "Wiring"
    with pytest.raises(CatError) as e:
        h.adjoint_of(node, [_t(np.ones(4))], None, _t(np.ones(5)))
    assert e.value.kind == "ShapeMismatch"
    rt = IrNode(1, "rt", OpenOp.router(4, 2), TensorType.f32([2, 4]))  # STE lives inside MoE
    with pytest.raises(CatError) as e:
        h.adjoint_of(rt, [_t(np.ones((2, 4)))], None, _t(np.ones((2, 4))))
    assert e.value.kind == "Unlawful"
    mla = IrNode(1, "mla", OpenOp("mla", (2, 4, 4, 4, 4, 4, 10000)), TensorType.f32([2, 8]))
    with pytest.raises(CatError) as e:  # not executable on this backend
        h.adjoint_of(mla, [_t(np.ones((2, 8)))], None, _t(np.ones((2, 8))))
    assert e.value.kind == "Unsupported"
    fc = IrNode(1, "fc", OpenOp.linear(8, 4, False), TensorType.f32([2, 4]), {"w": _t(np.ones((8, 4)))})
    with pytest.raises(CatError) as e:
        h.adjoint_of(fc, [_t(np.ones((2, 7)))], None, _t(np.ones((2, 4))))
    assert e.value.kind == "ShapeMismatch"


def test_repeated_adjoint_calls_reuse_the_plan_and_take_new_values(device):
    # The training wave calls adjoint_of on the same node every step with new
    # parameter values and inputs: the cached one-node plan must take them.
    h = DeviceHandler(device)
    device.clear_events()
    for step in range(3):
        r = np.random.default_rng(100 + step)
        params = {"w": _t(r.standard_normal((96, 64)) / 10), "b": _t(r.standard_normal(64))}
        node = IrNode(3, "fc", OpenOp.linear(96, 64, True), TensorType.f32([32, 64]), params)
        x = r.standard_normal((32, 96)).astype(np.float32)
        out = oracle.eval_node(node, [x])
        dy = r.standard_normal(out.shape).astype(np.float32)
        dx, dp = h.adjoint_of(node, [_t(x)], None, _t(dy))
        dx_o, dp_o = ot.adjoint_of(node, [x], out, dy)
        assert rel_l2(dx[0].numpy(), dx_o[0]) < FP32_TOL
        for port in ("w", "b"):
            assert rel_l2(dp[port].numpy(), np.asarray(dp_o[port]).reshape(params[port].ty.shape)) < FP32_TOL
        ev = device.events()[-2:]
        # note_kernel("{name}.bwd", dy.checksum()) (coord.rs:412), stamped on the device
        assert [(e[1], e[2]) for e in ev] == [("fc.bwd", 0), ("fc.bwd", 1)] and ev[0][0] < ev[1][0]
        assert ev[1][3] == Tensor.from_numpy(dy).checksum()


# GqaAttention (gqa_backward, adjoint.rs:287-440): d_head 32, 64 and 128 take
# the MFMA adjoint kernels, other head sizes the generic ones; grouped K/V
# heads, sliding windows, a ragged sequence and n_heads·head_dim ≠ d_model.
@pytest.mark.parametrize("B,S,D,nh,nkv,hd,window,theta", [
    (2, 128, 256, 4, 2, 64, None, 10000),
    (1, 200, 256, 4, 1, 64, 50, 1000000),
    (1, 130, 128, 2, 2, 64, 1, 10000),
    (2, 9, 32, 4, 2, 8, 3, 10000),
    (1, 77, 48, 6, 2, 10, None, 500),
    (1, 150, 128, 4, 2, 32, 40, 10000),
    (1, 140, 256, 2, 1, 128, None, 10000),
])
def test_gqa(device, B, S, D, nh, nkv, hd, window, theta):
    r = np.random.default_rng(S + nh)
    qw, kw = nh * hd, nkv * hd
    params = {"wq": _t(r.standard_normal((D, qw)) / np.sqrt(D)), "wk": _t(r.standard_normal((D, kw)) / np.sqrt(D)),
              "wv": _t(r.standard_normal((D, kw)) / np.sqrt(D)), "wo": _t(r.standard_normal((qw, D)) / np.sqrt(qw))}
    node = IrNode(4, "gqa", OpenOp.gqa_attention(nh, nkv, hd, D, window, theta), TensorType.f32([B, S, D]),
                  params)
    _check(device, node, [r.standard_normal((B, S, D))], FP32_TOL)
