"""Pins the oracle's restatement of the reference adjoints (adjoint.rs) and
of one reference_train step against float64 torch autograd — an
independent derivation of the same gradients — and against the
reference's own known answers."""
import math

import numpy as np
import pytest
import torch

import oracle
import oracle_train as ot
from conftest import rel_l2

RNG = np.random.default_rng(99)
T64 = torch.float64


def _t(a, grad=False):
    return torch.tensor(np.asarray(a, np.float64), dtype=T64, requires_grad=grad)


def test_relu_backward_known_answer():
    # adjoint.rs:1006-1011
    assert ot.relu_backward(np.array([-1.0, 2.0, 0.0]), np.ones(3)).tolist() == [0.0, 1.0, 0.0]


def test_softmax_grad_rows_sum_to_zero():
    # adjoint.rs:1035-1042
    y = oracle.softmax_last(RNG.standard_normal((4, 9)))
    dx = ot.softmax_backward(y, RNG.standard_normal((4, 9)))
    assert np.allclose(dx.sum(-1), 0.0, atol=1e-6)


def test_sgd_known_answers():
    # optim.rs:163-176
    assert ot.sgd(np.array([1.0, 2.0]), np.array([1.0, -1.0]), 0.5).tolist() == [0.5, 2.5]
    assert ot.sgd(np.array([3.0, 4.0]), np.zeros(2), 0.1).tolist() == [3.0, 4.0]


def test_linear_backward_matches_autograd():
    x, w = RNG.standard_normal((6, 10)), RNG.standard_normal((10, 7))
    dy = RNG.standard_normal((6, 7))
    dx, dw, db = ot.linear_backward(x, w, dy)
    X, W = _t(x, True), _t(w, True)
    B = torch.zeros(7, dtype=T64, requires_grad=True)
    (X @ W + B).backward(_t(dy))
    assert rel_l2(dx, X.grad) < 1e-6 and rel_l2(dw, W.grad) < 1e-6 and rel_l2(db, B.grad) < 1e-6


def test_gelu_and_mse_backward_match_autograd():
    x, dy = RNG.standard_normal(500) * 3, RNG.standard_normal(500)
    X = _t(x, True)
    torch.nn.functional.gelu(X, approximate="tanh").backward(_t(dy))
    assert rel_l2(ot.gelu_backward(x, dy), X.grad) < 1e-5
    p, t = RNG.standard_normal((5, 8)), RNG.standard_normal((5, 8))
    loss, d = ot.mse_loss(p, t)
    P = _t(p, True)
    L = torch.mean((P - _t(t)) ** 2)
    L.backward()
    assert abs(loss - L.item()) < 1e-5 and rel_l2(d, P.grad) < 1e-6


def test_layer_norm_backward_matches_autograd():
    x = RNG.standard_normal((7, 32)) * 2 + 1
    g, dy = RNG.standard_normal(32), RNG.standard_normal((7, 32))
    dx, dg, db = ot.layer_norm_backward(x, g, dy, 1e-6)
    X, G, Bb = _t(x, True), _t(g, True), torch.zeros(32, dtype=T64, requires_grad=True)
    torch.nn.functional.layer_norm(X, (32,), G, Bb, eps=1e-6).backward(_t(dy))
    assert rel_l2(dx, X.grad) < 1e-4 and rel_l2(dg, G.grad) < 1e-5 and rel_l2(db, Bb.grad) < 1e-6


def _attn64(X, Wq, Wk, Wv, Wo, H, causal):
    B, S, D = X.shape
    dh = D // H
    q, k, v = [(X @ W).view(B, S, H, dh).transpose(1, 2) for W in (Wq, Wk, Wv)]
    ctx = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)
    return ctx.transpose(1, 2).reshape(B, S, D) @ Wo


@pytest.mark.parametrize("causal", [False, True])
def test_attention_backward_matches_autograd(causal):
    B, S, D, H = 2, 9, 16, 4
    x = RNG.standard_normal((B, S, D))
    ws = [RNG.standard_normal((D, D)) / math.sqrt(D) for _ in range(4)]
    dy = RNG.standard_normal((B, S, D))
    got = ot.attention_backward(x, *ws, H, D // H, dy, causal=causal)
    X, *W = [_t(a, True) for a in (x, *ws)]
    _attn64(X, *W, H, causal).backward(_t(dy))
    for g, ref in zip(got, [X.grad] + [w.grad for w in W]):
        assert rel_l2(g, ref) < 1e-4
    if causal:  # a wrong mask must not pass
        nc = ot.attention_backward(x, *ws, H, D // H, dy, causal=False)
        assert rel_l2(nc[0], X.grad) > 1e-2


def _swiglu64(X, W1, W3, W2):
    a, c = X @ W1, X @ W3
    return (a * torch.sigmoid(a) * c) @ W2


def test_swiglu_backward_matches_autograd():
    T, H, I = 5, 12, 20
    x = RNG.standard_normal((T, H))
    w1, w3 = RNG.standard_normal((H, I)) * 0.3, RNG.standard_normal((H, I)) * 0.3
    w2 = RNG.standard_normal((I, H)) * 0.3
    dy = RNG.standard_normal((T, H))
    got = ot.swiglu_backward(x, w1, w3, w2, dy)
    X, W1, W3, W2 = [_t(a, True) for a in (x, w1, w3, w2)]
    _swiglu64(X, W1, W3, W2).backward(_t(dy))
    for g, ref in zip(got, (X.grad, W1.grad, W3.grad, W2.grad)):
        assert rel_l2(g, ref) < 1e-5


def _moe64(X, G, W1, W3, W2, idx):
    """Dense float64 MoE with the routing indices held fixed (the STE:
    gradients flow through the softmax weights of the selected experts)."""
    logits = X @ G
    sel = torch.gather(logits, 1, torch.from_numpy(idx.astype(np.int64)))
    w = torch.softmax(sel, -1)
    out = torch.zeros_like(X)
    for j in range(idx.shape[1]):
        for e in range(W1.shape[0]):
            m = torch.from_numpy(idx[:, j] == e)
            if m.any():
                out[m] = out[m] + w[m, j:j + 1] * _swiglu64(X[m], W1[e], W3[e], W2[e])
    return out


def test_router_and_moe_backward_match_autograd():
    T, H, I, E, k = 11, 8, 12, 4, 2
    x = RNG.standard_normal((T, H))
    gate = RNG.standard_normal((H, E))
    w1, w3 = RNG.standard_normal((E, H, I)) * 0.3, RNG.standard_normal((E, H, I)) * 0.3
    w2 = RNG.standard_normal((E, I, H)) * 0.3
    dy = RNG.standard_normal((T, H))
    got = ot.moe_backward(x, gate, w1, w3, w2, k, dy)
    idx, _, _ = oracle.route(x.astype(np.float32), gate.astype(np.float32), k)
    X, G, W1, W3, W2 = [_t(a, True) for a in (x, gate, w1, w3, w2)]
    _moe64(X, G, W1, W3, W2, idx).backward(_t(dy))
    for g, ref in zip(got, (X.grad, G.grad, W1.grad, W3.grad, W2.grad)):
        assert rel_l2(g, ref) < 1e-4
    # the router's STE piece alone
    dwt = RNG.standard_normal((T, k))
    dx, dg = ot.router_backward_ste(x, gate, k, dwt)
    X2, G2 = _t(x, True), _t(gate, True)
    sel = torch.gather(X2 @ G2, 1, torch.from_numpy(idx.astype(np.int64)))
    (torch.softmax(sel, -1) * _t(dwt)).sum().backward()
    assert rel_l2(dx, X2.grad) < 1e-5 and rel_l2(dg, G2.grad) < 1e-5


def test_train_step_matches_autograd_on_block_plus_moe():
    from catnn_amd import configs

    g = configs.config5_graph(batch=1, seq=12, d=16, heads=2, ffn=32, n_experts=4, top_k=2, inter=24)
    x = RNG.standard_normal((1, 12, 16)).astype(np.float32)
    tgt = RNG.standard_normal((1, 12, 16)).astype(np.float32)
    loss, grads, new = ot.train_step(g, x, tgt, 0.05)
    # float64 torch restatement of the same graph
    P = {nid: {p: _t(t.numpy(), True) for p, t in n.params.items()} for nid, n in g.nodes.items()}
    X = _t(x)
    n = g.nodes

    def ln(h, nid):
        return torch.nn.functional.layer_norm(h, (16,), P[nid]["gamma"], P[nid]["beta"], eps=1e-6)

    h1 = ln(X, 1)
    a = _attn64(h1, P[2]["wq"], P[2]["wk"], P[2]["wv"], P[2]["wo"], 2, True)
    r1 = X + a
    f = torch.nn.functional.gelu(ln(r1, 4) @ P[5]["w"] + P[5]["b"], approximate="tanh")
    r2 = r1 + (f @ P[7]["w"] + P[7]["b"])
    mp = P[9]
    flat = r2.reshape(12, 16)
    idx, _, _ = oracle.route(flat.detach().numpy().astype(np.float32), mp["gate"].detach().numpy().astype(np.float32), 2)
    stack = lambda s: torch.stack([mp[f"e{e}.{s}"] for e in range(4)])
    out = _moe64(flat, mp["gate"], stack("w1"), stack("w3"), stack("w2"), idx)
    L = torch.mean((out.reshape(1, 12, 16) - _t(tgt)) ** 2)
    L.backward()
    assert abs(loss - L.item()) < 1e-4 * max(1.0, abs(L.item()))
    for nid, dp in grads.items():
        for port, gr in dp.items():
            assert rel_l2(gr, P[nid][port].grad) < 1e-3, (n[nid].name, port)
            assert np.allclose(new[nid][port], n[nid].params[port].numpy() - np.float32(0.05) * gr)


# ---------------------------------------------------------------------------
# The device-precision model (oracle_bf16): with rounding off it must be the
# reference algorithm; its rounding must be torch's bfloat16 rounding.

def test_bf16_round_known_answers_and_torch():
    import oracle_bf16 as ob

    one = 1.0
    vals = np.array([one, one + 2.0 ** -8, one + 3 * 2.0 ** -8, -2.5, 0.0, 3.0e38, 1e-40], np.float32)
    got = ob.bf16_round(vals)
    assert got[:3].tolist() == [1.0, 1.0, 1.0 + 2.0 ** -6]  # ties to even
    a = RNG.standard_normal(4096).astype(np.float32) * np.float32(10.0) ** RNG.integers(-20, 20, 4096)
    want = torch.tensor(np.concatenate([vals, a])).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ob.bf16_round(np.concatenate([vals, a])).astype(np.float32), want)
    # hi + lo carries 16 significant bits: |a − hi − lo| ≤ 2⁻¹⁶|a| (normal range)
    b = RNG.standard_normal(4096).astype(np.float32)
    hi, lo = ob.bf16_split(b)
    assert np.all(np.abs(b - hi - lo) <= 2.0 ** -16 * np.abs(b))


@pytest.mark.parametrize("which", ["mlp", "block_moe"])
def test_bf16_model_without_rounding_is_the_reference_step(which):
    import oracle_bf16 as ob
    from catnn_amd import configs

    if which == "mlp":
        w = configs.config1(batch=16)
        g, x = w.graph, w.x.numpy()
        tgt = RNG.standard_normal((16, 10)).astype(np.float32)
    else:
        w = configs.config5(batch=1, seq=24, d=32, heads=2, ffn=48, n_experts=4, top_k=2, inter=40)
        g, x, tgt = w.graph, w.x.numpy(), w.target.numpy()
    loss_o, grads_o, _ = ot.train_step(g, x, tgt, 0.05)
    loss_m, grads_m, _ = ob.train_step(g, x, tgt, policy=ob.WIDE)
    assert abs(loss_m - loss_o) < 1e-5 * max(1.0, loss_o)
    assert grads_m.keys() == grads_o.keys()
    for nid, dp in grads_o.items():
        assert dp.keys() == grads_m[nid].keys()
        for port, go in dp.items():
            assert rel_l2(grads_m[nid][port].reshape(go.shape), go) < 1e-4, (g.nodes[nid].name, port)


# ---- pins for oracle.mul, the Mul arm of adjoint_of and softmax_backward ----


def test_mul_is_the_elementwise_f32_product():
    # cpu.rs:100-109: y[i] = a[i]·b[i], one correctly rounded f32 product.
    # The float64 product of two f32 values is exact (48 significant bits),
    # so rounding it once to f32 is the reference value bit for bit.
    a = RNG.standard_normal(1000).astype(np.float32)
    b = (RNG.standard_normal(1000) * 7).astype(np.float32)
    want = (a.astype(np.float64) * b.astype(np.float64)).astype(np.float32)
    got = oracle.mul(a, b)
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()
    # signs and signed zeros come through as IEEE multiplication gives them
    assert oracle.mul(np.array([-2.0, 0.5, -0.0], np.float32),
                      np.array([3.0, -4.0, 5.0], np.float32)).tolist() == [-6.0, -2.0, -0.0]
    with pytest.raises(Exception):
        oracle.mul(np.ones(3, np.float32), np.ones(4, np.float32))


def _mul_node(shape):
    from catnn_amd import IrNode, OpenOp, TensorType

    return IrNode(2, "mul", OpenOp.mul(), TensorType.f32(list(shape)))


def test_mul_adjoint_matches_autograd_and_finite_differences():
    # adjoint.rs:785-799: d(x·y) = (dy·y, dy·x).  The two inputs differ, so a
    # swapped pair of cotangents fails both checks.
    x = RNG.standard_normal((5, 11))
    y = RNG.standard_normal((5, 11)) * 3 + 1
    dy = RNG.standard_normal((5, 11))
    node = _mul_node(x.shape)
    out = oracle.mul(x.astype(np.float32), y.astype(np.float32))
    (dx, dyy), dp = ot.adjoint_of(node, [x.astype(np.float32), y.astype(np.float32)], out,
                                  dy.astype(np.float32))
    assert dp == {}
    X, Y = _t(x, True), _t(y, True)
    (X * Y).backward(_t(dy))
    assert rel_l2(dx, X.grad) < 1e-6 and rel_l2(dyy, Y.grad) < 1e-6
    assert rel_l2(dyy, X.grad) > 0.1 and rel_l2(dx, Y.grad) > 0.1  # a swap is caught
    # central differences of <dy, x·y> in float64
    h = 1e-6
    f = lambda a, b: float(np.sum(dy * a * b))
    for (i, j) in [(0, 0), (2, 5), (4, 10)]:
        e = np.zeros_like(x)
        e[i, j] = h
        assert abs((f(x + e, y) - f(x - e, y)) / (2 * h) - dx[i, j]) < 1e-4 * (1 + abs(dx[i, j]))
        assert abs((f(x, y + e) - f(x, y - e)) / (2 * h) - dyy[i, j]) < 1e-4 * (1 + abs(dyy[i, j]))
    # single input: Mul passes dy through (adjoint.rs:786-787)
    (d1,), _ = ot.adjoint_of(node, [x.astype(np.float32)], x.astype(np.float32), dy.astype(np.float32))
    assert np.array_equal(d1, dy.astype(np.float32))


def test_softmax_backward_matches_autograd():
    # adjoint.rs:92-104: dx = y·(dy − Σ y·dy), against float64 autograd of
    # softmax.  A flipped sign or a dropped dot term both sum to zero per
    # row, so they pass the reference's own row-sum check; this one fails
    # them (checked below on planted mistakes).
    x = RNG.standard_normal((6, 17)) * 2
    dy = RNG.standard_normal((6, 17))
    X = _t(x, True)
    torch.softmax(X, -1).backward(_t(dy))
    y = oracle.softmax_last(x.astype(np.float32))
    got = ot.softmax_backward(y, dy.astype(np.float32))
    assert rel_l2(got, X.grad) < 1e-5
    yd = y.astype(np.float64)
    dot = np.sum(yd * dy, -1, keepdims=True)
    for wrong in (-yd * (dy - dot), yd * (dot - dy), yd * dy, yd * (dy - dot) * 2):
        assert rel_l2(wrong, X.grad) > 0.3
    # the same through adjoint_of's Softmax arm (reads the forward output)
    from catnn_amd import IrNode, OpenOp, TensorType

    node = IrNode(1, "sm", OpenOp.softmax(), TensorType.f32([6, 17]))
    (d,), dp = ot.adjoint_of(node, [x.astype(np.float32)], y, dy.astype(np.float32))
    assert dp == {} and rel_l2(d, X.grad) < 1e-5


def test_softmax_backward_finite_differences_and_closed_form():
    # central differences of <dy, softmax(x)> in float64 on one row
    x = RNG.standard_normal(9)
    dy = RNG.standard_normal(9)
    sm = lambda v: np.exp(v - v.max()) / np.exp(v - v.max()).sum()
    y = oracle.softmax_last(x.astype(np.float32)[None])
    got = ot.softmax_backward(y, dy.astype(np.float32)[None])[0]
    h = 1e-6
    for i in range(9):
        e = np.zeros(9)
        e[i] = h
        fd = (np.dot(dy, sm(x + e)) - np.dot(dy, sm(x - e))) / (2 * h)
        assert abs(fd - got[i]) < 2e-5 * (1 + abs(fd))
    # closed form: a constant cotangent moves nothing (softmax is invariant
    # to a shift of its output's dual), and a one-hot dy on a uniform row
    # gives (1/n)(e_i − 1/n).
    assert np.allclose(ot.softmax_backward(y, np.full((1, 9), 3.0, np.float32)), 0.0, atol=1e-6)
    n = 8
    u = np.full((1, n), 1.0 / n, np.float32)
    oh = np.zeros((1, n), np.float32)
    oh[0, 2] = 1.0
    want = (1.0 / n) * (oh - 1.0 / n)
    assert np.allclose(ot.softmax_backward(u, oh), want, atol=1e-7)
