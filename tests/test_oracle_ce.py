"""Pins the oracle's cross_entropy (crates/catnn-compile/src/kernel/adjoint.rs:
123-145) and the LmHead arm of adjoint_of (adjoint.rs:903-913), on the CPU:

  * uniform logits, where the loss is ln V and d = 1/(V·rows) − onehot/rows;
  * log-softmax in float64 on random logits (loss and every element of d);
  * the rows of d sum to zero, and a target past the vocabulary is refused;
  * the LmHead adjoint against dx = dy·W and dW = dyᵀ·x in float64 (a
    transposed operand or a swapped product fails it);
  * one reference_train step of input → LmHead with class targets against
    the same float64 algebra.
"""
import numpy as np
import pytest

import oracle_train as ot
from catnn_amd import IrGraph, IrNode, OpenOp, Tensor, TensorType
from conftest import rel_l2


def _f64_ce(logits, t):
    z = logits.astype(np.float64)
    z = z - z.max(axis=1, keepdims=True)
    logp = z - np.log(np.exp(z).sum(axis=1, keepdims=True))
    rows = logits.shape[0]
    d = np.exp(logp) / rows
    d[np.arange(rows), t] -= 1.0 / rows
    return -logp[np.arange(rows), t].mean(), d


def test_uniform_logits_known_answer():
    rows, V = 4, 10
    t = np.array([0, 3, 9, 3], np.uint32)
    loss, d = ot.cross_entropy(np.zeros((rows, V), np.float32), t)
    assert abs(loss - np.log(V)) < 1e-6
    want = np.full((rows, V), 1.0 / (V * rows))
    want[np.arange(rows), t] -= 1.0 / rows
    assert np.allclose(d, want, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("rows,V", [(7, 50), (64, 1000), (3, 32000)])
def test_against_float64_log_softmax(rows, V):
    r = np.random.default_rng(V)
    logits = (3 * r.standard_normal((rows, V))).astype(np.float32)
    t = r.integers(0, V, rows).astype(np.uint32)
    loss, d = ot.cross_entropy(logits, t)
    lw, dw = _f64_ce(logits, t)
    assert abs(loss - lw) <= 1e-5 * max(1.0, abs(lw))
    assert rel_l2(d, dw) < 1e-5
    # Σ_j d = (Σ_j p − 1)/rows: the f32 softmax sum's rounding, which grows with V.
    assert np.abs(d.astype(np.float64).sum(axis=1)).max() < 1e-6 * max(1.0, V / 1000)


def test_target_past_the_vocabulary_is_refused():
    with pytest.raises(ValueError):
        ot.cross_entropy(np.zeros((2, 5), np.float32), [1, 5])


def test_lm_head_adjoint_against_float64():
    r = np.random.default_rng(1)
    T, H, V = 33, 24, 70
    x = r.standard_normal((T, H)).astype(np.float32)
    w = r.standard_normal((V, H)).astype(np.float32)
    dy = r.standard_normal((T, V)).astype(np.float32)
    dx, dw = ot.lm_head_backward(x, w, dy)
    assert dx.shape == (T, H) and dw.shape == (V, H)
    assert rel_l2(dx, dy.astype(np.float64) @ w.astype(np.float64)) < 1e-6
    assert rel_l2(dw, dy.astype(np.float64).T @ x.astype(np.float64)) < 1e-6


def test_train_step_with_class_targets():
    r = np.random.default_rng(2)
    T, H, V = 16, 12, 30
    x = r.standard_normal((T, H)).astype(np.float32)
    w = (0.3 * r.standard_normal((V, H))).astype(np.float32)
    t = r.integers(0, V, T).astype(np.uint32)
    g = IrGraph("lm")
    g.add_node(IrNode(0, "in", OpenOp.identity(), TensorType.f32([T, H])))
    g.add_node(IrNode(1, "lm", OpenOp.lm_head(H, V), TensorType.f32([T, V]),
                      {"w": Tensor(TensorType.f32([V, H]), w)}))
    g.add_edge(0, 1)
    g.inputs, g.outputs = [0], [1]
    loss, grads, new = ot.train_step(g, x, t, 0.1)
    lw, dlog = _f64_ce(x.astype(np.float64) @ w.astype(np.float64).T, t)
    assert abs(loss - lw) < 1e-5
    assert rel_l2(grads[1]["w"], dlog.T @ x.astype(np.float64)) < 1e-5
    assert np.allclose(new[1]["w"], w - np.float32(0.1) * grads[1]["w"], rtol=0, atol=1e-7)
