"""One training step on the GPU (catnn_hip_train_*) against the oracle's
restatement of pipeline::reference_train (oracle_train.train_step, pinned
by test_oracle_adjoint.py against float64 autograd).

The device step runs its GEMMs on bf16 operands with fp32 accumulation, so
losses and gradients are held to the bf16 bar (rel L2 ≤ 1e-2).  The SGD
update is checked bit-exactly against p − lr·g on the device's own
gradient, and MoE routing bit-exactly wherever the router's input is the
exact graph input."""
import numpy as np
import pytest

import oracle_train as ot
from catnn_amd import (CatError, IrGraph, IrNode, OpenOp, Tensor, TensorType, Trainer,
                       arena_conflict, configs, synth)
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
LOSS_TOL = 2e-3


def _target(shape, seed):
    return Tensor(TensorType.f32(shape), synth.normal(int(np.prod(shape)), seed, 1.0))


def _shape(g, nid, port):
    return tuple(g.nodes[nid].params[port].ty.shape)


def _check_step(device, g, x, tgt, lr=0.05, grad_tol=BF16_TOL, loose=()):
    """One step on both sides; returns (trainer, oracle loss, worst error)."""
    print(f"[train] {g.name} x={x.ty.shape}", flush=True)
    tr = Trainer(device, g, lr)
    tr.set_batch(x, tgt)
    loss = tr.step()
    loss_o, grads_o, _ = ot.train_step(g, x.numpy(), tgt.numpy(), lr)
    print(f"  loss gpu={loss:.6f} oracle={loss_o:.6f}")
    assert abs(loss - loss_o) <= LOSS_TOL * max(1.0, abs(loss_o))
    out = g.outputs[-1]
    pred = tr.value(out, tuple(g.nodes[out].output_ty.shape))
    assert np.isfinite(pred).all()
    worst = 0.0
    for nid, dp in grads_o.items():
        for port, go in dp.items():
            shape = _shape(g, nid, port)
            gg = tr.grad(nid, port, shape)
            err = rel_l2(gg, go.reshape(shape))
            tol = grad_tol * (5 if (nid, port) in loose else 1)
            print(f"  grad {g.nodes[nid].name}.{port}: rel_l2={err:.2e}")
            assert err < tol, (g.nodes[nid].name, port, err)
            worst = max(worst, err)
            # Sgd::put on the device's own gradient, rounded as the reference rounds.
            p0 = g.nodes[nid].params[port].numpy().reshape(shape)
            p1 = tr.param(nid, port, shape)
            want = p0 - np.float32(lr) * gg
            assert np.array_equal(p1, want), (g.nodes[nid].name, port)
    allocs, reserved = tr.arena()
    assert arena_conflict(allocs) is None
    assert reserved < sum(a.bytes for a in allocs)  # dead buffers share space
    return tr, loss_o, worst


def test_mlp_relu_unaligned_k(device):
    # K = 784 and N = 10: the bf16 GEMM's element-load edges.
    w = configs.config1(batch=64)
    _check_step(device, w.graph, w.x, _target([64, 10], 11))


@pytest.mark.parametrize("causal", [True, False])
def test_block_mfma_head(device, causal):
    # d_head = 64: the MFMA attention adjoint kernels.
    w = configs.config3(batch=2, seq=128, d=128, heads=2, ffn=256, causal=causal)
    _check_step(device, w.graph, w.x, _target([2, 128, 128], 12))


def test_block_generic_head_ragged(device):
    # d_head = 32 and a sequence that is not a tile multiple: generic kernels.
    w = configs.config3(batch=1, seq=77, d=64, heads=2, ffn=96, causal=True)
    _check_step(device, w.graph, w.x, _target([1, 77, 64], 13))


def test_block_mfma_head_ragged(device):
    w = configs.config3(batch=1, seq=200, d=128, heads=2, ffn=256, causal=True)
    _check_step(device, w.graph, w.x, _target([1, 200, 128], 14))


def test_moe_layer_routing_bit_exact(device):
    # The router reads the exact graph input, so its top-k matches bit for bit.
    w = configs.config4(batch=2, seq=64, d=128, n_experts=4, top_k=2, inter=96)
    tr, _, _ = _check_step(device, w.graph, w.x, _target([2, 64, 128], 15))
    import oracle

    idx, _, _ = oracle.route(w.x.numpy().reshape(-1, 128), w.graph.nodes[1].params["gate"].numpy(), 2)
    assert np.array_equal(tr.routing(1, 128, 2), idx)


def test_block_plus_moe_config5_shape(device):
    w = configs.config5(batch=2, seq=128, d=128, heads=2, ffn=256, n_experts=4, top_k=2, inter=128)
    tr, _, _ = _check_step(device, w.graph, w.x, w.target)
    # The router here reads the block's bf16-GEMM output: top-k may differ on near ties.
    import oracle

    acts = {0: w.x.numpy()}
    g = w.graph
    for nid in oracle.topo(g)[1:]:
        preds = [e.src for e in g.edges if e.dst == nid]
        acts[nid] = oracle.eval_node(g.nodes[nid], [acts[p] for p in preds])
    idx, _, _ = oracle.route(acts[8].reshape(-1, 128), g.nodes[9].params["gate"].numpy(), 2)
    agree = float(np.mean(np.sort(tr.routing(9, 256, 2), 1) == np.sort(idx, 1)))
    print(f"  routing agreement {agree:.4f}")
    assert agree > 0.97


def test_block_plus_moe_ragged(device):
    w = configs.config5(batch=1, seq=77, d=128, heads=2, ffn=256, n_experts=4, top_k=2, inter=96)
    _check_step(device, w.graph, w.x, w.target)


def test_three_steps_follow_the_oracle(device):
    w = configs.config5(batch=1, seq=64, d=128, heads=2, ffn=256, n_experts=4, top_k=2, inter=128)
    g = w.graph
    tr = Trainer(device, g, w.lr)
    tr.set_batch(w.x, w.target)
    losses, losses_o = [], []
    for _ in range(3):
        losses.append(tr.step())
        loss_o, _, new = ot.train_step(g, w.x.numpy(), w.target.numpy(), w.lr)
        losses_o.append(loss_o)
        for nid, ports in new.items():
            for port, v in ports.items():
                g.nodes[nid].params[port] = Tensor(g.nodes[nid].params[port].ty, v.reshape(-1))
    print(f"  losses gpu={losses} oracle={losses_o}")
    assert losses[2] < losses[0]
    for a, b in zip(losses, losses_o):
        assert abs(a - b) <= LOSS_TOL * max(1.0, abs(b))


def test_training_error_kinds(device):
    ty = TensorType.f32([4, 8])
    g = IrGraph("sm")
    g.add_node(IrNode(0, "in", OpenOp.identity(), ty))
    g.add_node(IrNode(1, "sm", OpenOp.softmax(-1), ty))
    g.add_edge(0, 1)
    g.inputs.append(0)
    g.outputs.append(1)
    with pytest.raises(CatError) as e:
        Trainer(device, g)
    assert e.value.kind == "Unsupported"

    w = configs.config1(batch=8)
    tr = Trainer(device, w.graph)
    with pytest.raises(CatError) as e:
        tr.set_batch(Tensor.zeros(TensorType.f32([8, 783])), _target([8, 10], 1))
    assert e.value.kind == "ShapeMismatch"
    lin = next(n.id for n in w.graph.nodes.values() if n.op.kind == "linear")
    with pytest.raises(CatError) as e:
        tr.grad(lin, "nope", (1,))
    assert e.value.kind == "UnknownPort"
    with pytest.raises(CatError) as e:
        tr.value(lin, tuple(w.graph.nodes[lin].output_ty.shape))
    assert e.value.kind == "Unsupported"
    tr.free()
