"""catnn oracle, training side — TEST INFRASTRUCTURE ONLY.

numpy front end of the adjoint restatements in catnn_oracle.cpp and one
training step restating pipeline::reference_train
(crates/catnn-compile/src/pipeline.rs:476-547): forward in topo order with
eval_cpu, MSE (adjoint.rs:106-119), reverse topo with adjoint_of
(adjoint.rs:762-951) summing cotangents from several successors with
add_tensors (adjoint.rs:22-24), then apply_update (pipeline.rs:455-472) on
every parameter: Sgd::put (optim.rs:32-42) or Adam::put (optim.rs:95-118)
with its per-parameter state.  Pinned by tests/test_oracle_adjoint.py and
tests/test_oracle_adam.py.
"""
from __future__ import annotations

import ctypes

import numpy as np

import oracle
from oracle import _c, _f, _lib, _I64, _F

_SIG = {
    "orc_linear_backward": ([_F, _F, _F, _I64, _I64, _I64, _F, _F, _F], None),
    "orc_relu_backward": ([_F, _F, _F, _I64], None),
    "orc_gelu_backward": ([_F, _F, _F, _I64], None),
    "orc_softmax_backward": ([_F, _F, _F, _I64, _I64], None),
    "orc_mse_loss": ([_F, _F, _I64, _F], ctypes.c_float),
    "orc_layer_norm_backward": ([_F, _F, _F, _I64, _I64, ctypes.c_float, _F, _F, _F], None),
    "orc_attention_backward": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, ctypes.c_int32,
                                _F, _F, _F, _F, _F, _F], ctypes.c_int),
    "orc_swiglu_backward": ([_F, _F, _F, _F, _I64, _I64, _I64, _F, _F, _F, _F, _F], None),
    "orc_gqa_backward": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_double, _I64,
                          _F, _F, _F, _F, _F, _F], ctypes.c_int),
    "orc_router_backward_ste": ([_F, _F, _I64, _I64, _I64, _I64, _F, _F, _F], None),
    "orc_moe_backward": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, _F, _F, _F, _F, _F, _F],
                         None),
    "orc_sgd": ([_F, _F, _I64, ctypes.c_float], None),
    "orc_rmsnorm_backward": ([_F, _F, _F, _I64, _I64, ctypes.c_float, _F, _F], None),
    "orc_mix_backward": ([_F, _F, ctypes.c_float, _F, _I64, _F, _F], ctypes.c_float),
    "orc_embedding_backward": ([_F, _I64, _F, _I64, _I64, _F], None),
    "orc_cross_entropy": ([_F, ctypes.POINTER(ctypes.c_uint32), _I64, _I64, _F, _F], ctypes.c_int),
    "orc_powi": ([ctypes.c_float, ctypes.c_int32], ctypes.c_float),
    "orc_adam": ([_F, _F, _F, _F, _I64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                  ctypes.c_float], None),
}
for _name, (_args, _res) in _SIG.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res


def linear_backward(x, w, dy):
    x, w, dy = _c(x), _c(w), _c(dy)
    k, n = w.shape
    m = x.size // k
    dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty(n, np.float32)
    _lib.orc_linear_backward(_f(x), _f(w), _f(dy), m, k, n, _f(dx), _f(dw), _f(db))
    return dx, dw, db


def relu_backward(x, dy):
    x, dy = _c(x), _c(dy)
    dx = np.empty_like(x)
    _lib.orc_relu_backward(_f(x), _f(dy), _f(dx), x.size)
    return dx


def gelu_backward(x, dy):
    x, dy = _c(x), _c(dy)
    dx = np.empty_like(x)
    _lib.orc_gelu_backward(_f(x), _f(dy), _f(dx), x.size)
    return dx


def softmax_backward(y, dy):
    y, dy = _c(y), _c(dy)
    dx = np.empty_like(y)
    _lib.orc_softmax_backward(_f(y), _f(dy), _f(dx), y.size // y.shape[-1], y.shape[-1])
    return dx


def mse_loss(pred, target):
    pred, target = _c(pred), _c(target)
    d = np.empty_like(pred)
    loss = _lib.orc_mse_loss(_f(pred), _f(target), pred.size, _f(d))
    return float(loss), d


def cross_entropy(logits, targets):
    """adjoint.rs:123-145: (loss, d) for class ids `targets`, one per row."""
    logits = _c(logits)
    last = logits.shape[-1]
    rows = logits.size // last
    t = np.ascontiguousarray(targets, np.uint32).reshape(-1)
    assert t.size == rows, "ce targets"
    d = np.empty_like(logits)
    loss = np.zeros(1, np.float32)
    rc = _lib.orc_cross_entropy(_f(logits), t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), rows, last,
                                _f(d), _f(loss))
    if rc != 0:
        raise ValueError("target >= last")
    return float(loss[0]), d


def lm_head_backward(x, w, dy):
    """The LmHead arm of adjoint_of (adjoint.rs:903-913): linear_backward
    with wᵀ [H, V]; dW transposed back to [V, H]."""
    V, H = w.shape
    dx, dwt, _ = linear_backward(np.asarray(x, np.float32).reshape(-1, H), np.ascontiguousarray(w.T), dy.reshape(-1, V))
    return dx.reshape(np.shape(x)), np.ascontiguousarray(dwt.T)


def rmsnorm_backward(x, w, dy, eps):
    """adjoint.rs:147-198: (dx, dw)."""
    x, w, dy = _c(x), _c(w), _c(dy)
    last = x.shape[-1]
    dx, dw = np.empty_like(x), np.empty(last, np.float32)
    _lib.orc_rmsnorm_backward(_f(x), _f(w), _f(dy), x.size // last, last, np.float32(eps), _f(dx), _f(dw))
    return dx, dw


def embedding_backward(ids, table_shape, dy):
    """adjoint.rs:187-197 (ids as the adjoint_of arm converts them, :845)."""
    ids, dy = _c(ids), _c(dy)
    V, H = table_shape
    dw = np.empty((V, H), np.float32)
    _lib.orc_embedding_backward(_f(ids), ids.size, _f(dy), V, H, _f(dw))
    return dw


def mix_backward(a, b, gate, dy):
    """deepseek.rs:241-258: (da, db, dg)."""
    a, b, dy = _c(a), _c(b), _c(dy)
    da, db = np.empty_like(a), np.empty_like(b)
    dg = _lib.orc_mix_backward(_f(a), _f(b), np.float32(gate), _f(dy), a.size, _f(da), _f(db))
    return da, db, float(dg)


def layer_norm_backward(x, gamma, dy, eps=1e-6):
    x, gamma, dy = _c(x), _c(gamma), _c(dy)
    last = x.shape[-1]
    dx, dg, db = np.empty_like(x), np.empty(last, np.float32), np.empty(last, np.float32)
    _lib.orc_layer_norm_backward(_f(x), _f(gamma), _f(dy), x.size // last, last, np.float32(eps),
                                 _f(dx), _f(dg), _f(db))
    return dx, dg, db


def attention_backward(x, wq, wk, wv, wo, n_heads, d_head, dy, causal=False):
    x, dy = _c(x), _c(dy)
    B, S, D = x.shape
    dx = np.empty_like(x)
    dws = [np.empty((D, D), np.float32) for _ in range(4)]
    rc = _lib.orc_attention_backward(_f(x), _f(_c(wq)), _f(_c(wk)), _f(_c(wv)), _f(_c(wo)), B, S, D,
                                     n_heads, d_head, int(causal), _f(dy), _f(dx),
                                     *[_f(w) for w in dws])
    if rc:
        raise ValueError("attention head split")
    return (dx, *dws)


def gqa_backward(x, wq, wk, wv, wo, n_heads, n_kv, head_dim, theta, window, dy):
    """gqa_backward, adjoint.rs:287-440 (window None or ≤ 0: no sliding
    window): (dx, dwq, dwk, dwv, dwo)."""
    x, dy = _c(x), _c(dy)
    wq, wk, wv, wo = _c(wq), _c(wk), _c(wv), _c(wo)
    B, S, D = x.shape
    dx = np.empty_like(x)
    dws = [np.empty_like(w) for w in (wq, wk, wv, wo)]
    rc = _lib.orc_gqa_backward(_f(x), _f(wq), _f(wk), _f(wv), _f(wo), B, S, D, n_heads, n_kv, head_dim,
                               float(theta), 0 if window is None else int(window), _f(dy), _f(dx),
                               *[_f(w) for w in dws])
    if rc:
        raise ValueError("gqa shape")
    return (dx, *dws)


def swiglu_backward(x, w1, w3, w2, dy):
    x, dy = _c(x), _c(dy)
    H, I = w1.shape
    T = x.size // H
    dx = np.empty_like(x)
    dw1, dw3, dw2 = np.empty((H, I), np.float32), np.empty((H, I), np.float32), np.empty((I, H), np.float32)
    _lib.orc_swiglu_backward(_f(x), _f(_c(w1)), _f(_c(w3)), _f(_c(w2)), T, H, I, _f(dy), _f(dx),
                             _f(dw1), _f(dw3), _f(dw2))
    return dx, dw1, dw3, dw2


def router_backward_ste(x, gate, top_k, d_weights):
    x, gate, dwt = _c(x), _c(gate), _c(d_weights)
    H, E = gate.shape
    T = x.size // H
    dx, dg = np.empty_like(x), np.empty_like(gate)
    _lib.orc_router_backward_ste(_f(x), _f(gate), T, H, E, top_k, _f(dwt), _f(dx), _f(dg))
    return dx, dg


def moe_backward(x, gate, w1s, w3s, w2s, top_k, dy):
    x, gate, dy = _c(x), _c(gate), _c(dy)
    E, H, I = w1s.shape
    T = x.size // H
    dx, dg = np.empty_like(x), np.empty_like(gate)
    d1, d3, d2 = (np.empty_like(_c(a)) for a in (w1s, w3s, w2s))
    _lib.orc_moe_backward(_f(x), _f(gate), _f(_c(w1s)), _f(_c(w3s)), _f(_c(w2s)), T, H, I, E, top_k,
                          _f(dy), _f(dx), _f(dg), _f(d1), _f(d3), _f(d2))
    return dx, dg, d1, d3, d2


def sgd(p, g, lr):
    p = _c(p).copy()
    _lib.orc_sgd(_f(p), _f(_c(g)), p.size, np.float32(lr))
    return p


ADAM_DEFAULTS = (np.float32(0.9), np.float32(0.999), np.float32(1e-8))  # Adam::default, optim.rs:86-90


def powi(b, t):
    """f32::powi with a run-time exponent (binary exponentiation in f32)."""
    return np.float32(_lib.orc_powi(np.float32(b), int(t)))


class AdamState:
    """AdamState (optim.rs:63-76): moments m, v and the step counter t."""

    def __init__(self, shape):
        self.m = np.zeros(shape, np.float32)
        self.v = np.zeros(shape, np.float32)
        self.t = 0


def adam(p, g, state, lr, betas=ADAM_DEFAULTS):
    """Adam::put: returns the new parameter; `state` advances in place."""
    b1, b2, eps = betas
    p = _c(p).copy()
    g = _c(g)
    assert p.size == g.size == state.m.size
    _lib.orc_adam(_f(p), _f(g), _f(state.m), _f(state.v), p.size, state.t, np.float32(lr), b1, b2, eps)
    state.t = min(state.t + 1, 2**64 - 1)
    return p


def apply_update(p, g, opt, lr, state):
    """pipeline.rs:455-472: Sgd::put, or Adam::put creating the state on first use."""
    if opt == "sgd":
        return sgd(p, g, lr), state
    if state is None:
        state = AdamState(np.shape(p))
    return adam(p, g, state, lr), state


def adjoint_of(node, inputs, output, dy):
    """adjoint.rs:762-951 for the executable op set: (cotangents per input,
    {port: parameter cotangent})."""
    kind = node.op.kind
    x = inputs[0]
    P = {k: v.numpy() for k, v in node.params.items()}
    if kind in ("identity", "reshape", "transpose"):
        return [dy.copy()], {}
    if kind == "relu":
        return [relu_backward(x, dy)], {}
    if kind == "gelu":
        return [gelu_backward(x, dy)], {}
    if kind == "softmax":
        return [softmax_backward(output, dy)], {}
    if kind == "mul":  # adjoint.rs:787-800
        if len(inputs) == 1:
            return [dy.copy()], {}
        return [_c(dy) * _c(inputs[1]).reshape(dy.shape), _c(dy) * _c(x).reshape(dy.shape)], {}
    if kind in ("add", "residual_add"):
        return ([dy.copy()] if len(inputs) == 1 else [dy.copy(), dy.copy()]), {}
    if kind in ("linear", "matmul"):
        dx, dw, db = linear_backward(x, P["w"], dy)
        d = {"w": dw}
        if "b" in P:
            d["b"] = db
        return [dx.reshape(x.shape)], d
    if kind == "layer_norm":
        eps = np.float32(node.op.fields[0]) * np.float32(1e-6)
        dx, dg, db = layer_norm_backward(x, P["gamma"], dy, eps)
        return [dx], {"gamma": dg, "beta": db}
    if kind == "attention":
        heads, _, dh = node.op.fields
        dx, dwq, dwk, dwv, dwo = attention_backward(x, P["wq"], P["wk"], P["wv"], P["wo"], heads, dh, dy,
                                                    causal=bool(node.op.flags & 1))
        return [dx], {"wq": dwq, "wk": dwk, "wv": dwv, "wo": dwo}
    if kind == "gqa_attention":  # adjoint.rs:862-883
        nh, nkv, hd, _, window, theta = node.op.fields
        dx, dwq, dwk, dwv, dwo = gqa_backward(x, P["wq"], P["wk"], P["wv"], P["wo"], nh, nkv, hd,
                                              float(theta), None if window < 0 else window, dy)
        return [dx], {"wq": dwq, "wk": dwk, "wv": dwv, "wo": dwo}
    if kind == "swiglu":  # adjoint.rs:849-861
        dx, dw1, dw3, dw2 = swiglu_backward(x, P["w1"], P["w3"], P["w2"], dy)
        return [dx.reshape(np.shape(x))], {"w1": dw1, "w3": dw3, "w2": dw2}
    if kind == "embedding":
        # adjoint.rs:843-848: the ids get the zero cotangent.
        return [np.zeros_like(np.asarray(x, np.float32))], {"w": embedding_backward(x, P["w"].shape, dy)}
    if kind == "mix":
        # adjoint.rs:918-927: the gate cotangent is reported as a [1] tensor.
        g = float(P["gate"].reshape(-1)[0]) if "gate" in P else 0.0
        da, db, dg = mix_backward(x, inputs[1], g, dy)
        return [da, db], {"gate": np.array([dg], np.float32)}
    if kind == "rms_norm":
        eps = np.float32(node.op.fields[0]) * np.float32(1e-6)
        dx, dw = rmsnorm_backward(x, P["w"], dy, eps)
        return [dx], {"w": dw}
    if kind == "lm_head":
        dx, dw = lm_head_backward(x, P["w"], dy)
        return [dx], {"w": dw}
    if kind == "moe":
        E, k, _, _ = node.op.fields
        w1 = np.stack([P[f"e{e}.w1"] for e in range(E)])
        w3 = np.stack([P[f"e{e}.w3"] for e in range(E)])
        w2 = np.stack([P[f"e{e}.w2"] for e in range(E)])
        dx, dg, d1, d3, d2 = moe_backward(x, P["gate"], w1, w3, w2, k, dy)
        d = {"gate": dg}
        for e in range(E):
            d[f"e{e}.w1"], d[f"e{e}.w3"], d[f"e{e}.w2"] = d1[e], d3[e], d2[e]
        return [dx.reshape(x.shape)], d
    raise NotImplementedError(kind)


def train_step(graph, x, target, lr, opt="sgd", adam_states=None):
    """One step of pipeline::reference_train with `opt` ("sgd" or "adam"):
    returns (loss, {node_id: {port: grad}}, {node_id: {port: updated
    param}}).  The loss is loss_and_grad's (pipeline.rs:446-451): MSE
    against `target`, or cross-entropy when the output node is an LmHead, in
    which case `target` holds one class id per row (TrainTarget::Classes).
    For Adam, `adam_states` ({(node_id, port): AdamState}, updated in place)
    carries the moments between steps."""
    order = oracle.topo(graph)
    acts = {}
    for nid in order:
        node = graph.nodes[nid]
        if nid in graph.inputs:
            acts[nid] = np.asarray(x, np.float32)
            continue
        preds = [e.src for e in graph.edges if e.dst == nid]
        acts[nid] = oracle.eval_node(node, [acts[p] for p in preds])
    out_id = graph.outputs[-1]
    if graph.nodes[out_id].op.kind == "lm_head":
        loss, dy = cross_entropy(acts[out_id], target)
    else:
        loss, dy = mse_loss(acts[out_id], target)
    grads = {out_id: dy.reshape(acts[out_id].shape)}
    dparams = {}
    for nid in reversed(order):
        if nid in graph.inputs or nid not in grads:
            continue
        node = graph.nodes[nid]
        preds = [e.src for e in graph.edges if e.dst == nid]
        dxs, dp = adjoint_of(node, [acts[p] for p in preds], acts[nid], grads[nid])
        for p, dx in zip(preds, dxs):
            grads[p] = oracle.add(grads[p], dx) if p in grads else dx
        dparams[nid] = dp
    new = {}
    if adam_states is None:
        adam_states = {}
    for nid, dp in dparams.items():
        node = graph.nodes[nid]
        new[nid] = {}
        for port, g in dp.items():
            st = adam_states.get((nid, port))
            new[nid][port], st = apply_update(node.params[port].numpy(), g, opt, lr, st)
            if st is not None:
                adam_states[(nid, port)] = st
    return loss, dparams, new
