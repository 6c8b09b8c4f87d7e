"""apply_update on the GPU: the standalone Sgd::put / Adam::put entry points
(catnn_hip_sgd_f32, catnn_hip_adam_f32) bit-exactly against the oracle's
restatement of crates/catnn-core/src/lens/optim.rs, and the training step
installed with OptimizerKind::Adam (catnn_hip_train_install_opt):

  * every update the device makes is bit-identical to Adam::put applied to
    the device's own gradient and moments, step after step;
  * the first step's gradients stay within the bf16 bar (rel L2 ≤ 1e-2) of
    the fp32 reference step (pipeline::reference_train with Adam), and the
    losses of three steps follow the reference's;
  * reset zeroes the moments and the step counter, and steps then repeat
    bit for bit.
"""
import copy
import ctypes

import numpy as np
import pytest

import oracle_train as ot
from catnn_amd import CatError, Tensor, TensorType, Trainer, configs, synth
from catnn_amd._lib import lib
from catnn_amd.device import adam, sgd
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _target(shape, seed):
    return Tensor(TensorType.f32(shape), synth.normal(int(np.prod(shape)), seed, 1.0))


@pytest.mark.parametrize("n", [1, 3, 1000, 100003])
@pytest.mark.parametrize("offset", [0, 1])
def test_update_entries_bit_exact(device, n, offset):
    # offset 1 shifts every buffer by one float: the unaligned (scalar) path.
    print(f"[adam] n={n} offset={offset}", flush=True)
    rng = np.random.default_rng(n + offset)
    p = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    m = (0.1 * rng.standard_normal(n)).astype(np.float32)
    v = (0.01 * rng.random(n)).astype(np.float32)
    bufs = [device.put(np.concatenate([np.zeros(offset, np.float32), a])) for a in (p, g, m, v)]
    ptr = [b.ptr.value + 4 * offset for b in bufs]
    for t, lr in ((0, 1e-3), (7, 0.05)):
        bufs[0].upload(np.concatenate([np.zeros(offset, np.float32), p]))
        bufs[2].upload(np.concatenate([np.zeros(offset, np.float32), m]))
        bufs[3].upload(np.concatenate([np.zeros(offset, np.float32), v]))
        adam(device, ptr[0], ptr[1], ptr[2], ptr[3], n, t, lr)
        device.sync()
        st = ot.AdamState((n,))
        st.m, st.v, st.t = m.copy(), v.copy(), t
        want = ot.adam(p, g, st, lr)
        got = [b.download((n + offset,))[offset:] for b in (bufs[0], bufs[2], bufs[3])]
        assert np.array_equal(got[0], want), (t, np.abs(got[0] - want).max())
        assert np.array_equal(got[1], st.m) and np.array_equal(got[2], st.v)
    bufs[0].upload(np.concatenate([np.zeros(offset, np.float32), p]))
    sgd(device, ptr[0], ptr[1], n, 0.05)
    device.sync()
    assert np.array_equal(bufs[0].download((n + offset,))[offset:], ot.sgd(p, g, 0.05))
    for b in bufs:
        b.free()


def test_update_entries_empty_and_errors(device):
    adam(device, None, None, None, None, 0, 0, 0.1)
    sgd(device, None, None, 0, 0.1)
    with pytest.raises(CatError) as e:
        adam(device, None, None, None, None, 4, 0, 0.1)
    assert e.value.kind == "InvalidArgument"
    with pytest.raises(CatError) as e:
        sgd(device, None, None, -1, 0.1)
    assert e.value.kind == "ShapeMismatch"


def _params(g):
    return [(nid, port, tuple(g.nodes[nid].params[port].ty.shape))
            for nid in sorted(g.nodes) for port in g.nodes[nid].params]


def _adam_steps(device, g, x, tgt, lr, steps=3):
    tr = Trainer(device, g, lr, opt="adam")
    tr.set_batch(x, tgt)
    states = {}
    prev = {(nid, port): g.nodes[nid].params[port].numpy().reshape(shape) for nid, port, shape in _params(g)}
    losses = []
    for k in range(steps):
        losses.append(tr.step())
        assert tr.adam_step() == k + 1
        for nid, port, shape in _params(g):
            gg = tr.grad(nid, port, shape)
            st = states.setdefault((nid, port), ot.AdamState(shape))
            want = ot.adam(prev[(nid, port)], gg, st, lr)
            got = tr.param(nid, port, shape)
            assert np.array_equal(got, want), (k, g.nodes[nid].name, port)
            assert np.array_equal(tr.moment(nid, port, "m", shape), st.m), (k, g.nodes[nid].name, port)
            assert np.array_equal(tr.moment(nid, port, "v", shape), st.v), (k, g.nodes[nid].name, port)
            prev[(nid, port)] = got
    return tr, losses, prev


@pytest.mark.parametrize("which", ["block", "block_moe"])
def test_trainer_adam_follows_the_reference(device, which):
    if which == "block":
        w = configs.config3(batch=2, seq=128, d=128, heads=2, ffn=256, causal=True)
        g, x, tgt = w.graph, w.x, _target([2, 128, 128], 21)
    else:
        w = configs.config5(batch=2, seq=128, d=128, heads=2, ffn=256, n_experts=4, top_k=2, inter=128)
        g, x, tgt = w.graph, w.x, w.target
    print(f"[adam-train] {which}", flush=True)
    lr = 1e-3
    tr, losses, _ = _adam_steps(device, g, x, tgt, lr)
    # The fp32 reference trajectory with Adam.
    states = {}
    losses_o = []
    first_grads = None
    cur = copy.deepcopy(g)
    for k in range(3):
        loss_o, grads_o, new = ot.train_step(cur, x.numpy(), tgt.numpy(), lr, opt="adam", adam_states=states)
        losses_o.append(loss_o)
        if first_grads is None:
            first_grads = grads_o
        for nid, ports in new.items():
            for port, val in ports.items():
                t = cur.nodes[nid].params[port]
                cur.nodes[nid].params[port] = Tensor(t.ty, np.asarray(val, np.float32).reshape(-1))
    print(f"  losses gpu {losses}  fp32 {losses_o}")
    for a, b in zip(losses, losses_o):
        assert abs(a - b) <= BF16_TOL * max(1.0, abs(b)), (losses, losses_o)
    # Step 1's gradients: Adam's first step sees the same gradient as SGD's.
    tr2 = Trainer(device, g, lr, opt="adam")
    tr2.set_batch(x, tgt)
    tr2.step()
    for nid, dp in first_grads.items():
        for port, go in dp.items():
            shape = tuple(g.nodes[nid].params[port].ty.shape)
            e = rel_l2(tr2.grad(nid, port, shape), go.reshape(shape))
            assert e < BF16_TOL, (g.nodes[nid].name, port, e)
    tr2.free()
    tr.free()


def test_trainer_adam_reset_repeats(device):
    w = configs.config4(batch=2, seq=64, d=128, n_experts=4, top_k=2, inter=96)
    g, x, tgt = w.graph, w.x, _target([2, 64, 128], 22)
    tr = Trainer(device, g, 1e-3, opt="adam")
    tr.set_batch(x, tgt)
    first = [tr.step() for _ in range(2)]
    p_first = tr.param(1, "gate", (128, 4))
    tr.reset()
    assert tr.adam_step() == 0
    assert not tr.moment(1, "gate", "m", (128, 4)).any()
    assert not tr.moment(1, "gate", "v", (128, 4)).any()
    again = [tr.step() for _ in range(2)]
    assert first == again
    assert np.array_equal(tr.param(1, "gate", (128, 4)), p_first)
    tr.free()


def test_trainer_optimizer_errors(device):
    w = configs.config1(batch=8)
    with pytest.raises(ValueError):
        Trainer(device, w.graph, 0.1, opt="rmsprop")
    from catnn_amd.device import graph_handle
    h, owned = graph_handle(w.graph)
    out = ctypes.c_void_p()
    try:
        rc = lib.catnn_hip_train_install_opt(device.handle, h, 7, ctypes.c_float(0.1), ctypes.byref(out))
        assert rc != 0 and not out.value
        assert b"unknown optimizer" in lib.catnn_hip_last_error()
    finally:
        if owned:
            lib.catnn_graph_free(h)
    tr = Trainer(device, w.graph, 0.1)  # SGD: no moments
    with pytest.raises(CatError) as e:
        tr.moment(1, "w", "m", (784, 512))
    assert e.value.kind == "Unsupported"
    tr.free()
