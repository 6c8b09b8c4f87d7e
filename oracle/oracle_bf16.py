"""Device-precision model of one training step — TEST INFRASTRUCTURE ONLY.

The algorithm of oracle_train.train_step (pipeline::reference_train with
MSE, crates/catnn-compile/src/pipeline.rs:476-547; the adjoints of
adjoint.rs:762-951), evaluated in float64 numpy with the GPU trainer's
declared rounding points (DEVICE): GEMM operands are rounded to bfloat16
(round to nearest even) or split into bf16 hi/lo pairs exactly where the
device does so (the attention core's products included: q, k, v, the
normalised softmax P, dO and dS), and nothing else is rounded —
accumulation, LayerNorm, activations, the softmax statistics, the router
and cotangent sums stay wide.
MoE routing is the reference's own fp32 router (oracle.route) on the fp32
router input, as on the device.

Under the WIDE policy no operand is rounded and the model is the plain
reference algorithm in float64: tests/test_oracle_adjoint.py pins that
mode against oracle_train.train_step, so a dropped term or a transposed
operand here fails there; the rounding points are the device's precision
policy and are what this model adds.
"""
from __future__ import annotations

import numpy as np

import oracle

F64 = np.float64


def bf16_round(a) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even), returned as float64."""
    u = np.ascontiguousarray(np.asarray(a, np.float32)).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(F64)


def _gelu(z):
    c = 0.7978845608028654
    return 0.5 * z * (1.0 + np.tanh(c * (z + 0.044715 * z ** 3)))


def _gelu_grad(z):
    c = 0.7978845608028654
    t = np.tanh(c * (z + 0.044715 * z ** 3))
    return 0.5 * (1.0 + t) + 0.5 * z * (1.0 - t * t) * c * (1.0 + 3.0 * 0.044715 * z * z)


def _silu(a):
    return a / (1.0 + np.exp(-a))


def _silu_grad(a):
    s = 1.0 / (1.0 + np.exp(-a))
    return s + a * s * (1.0 - s)


def bf16_split(a):
    """(hi, lo): hi = bf16(a), lo = bf16(a − hi), as float64."""
    hi = bf16_round(a)
    return hi, bf16_round(np.asarray(a, np.float32) - hi.astype(np.float32))


SITES = ("linear_fwd", "linear_bwd", "attn_fwd", "attn_bwd", "attn_core", "moe_fwd", "moe_bwd")
# The GPU trainer's policy: split-bf16 forward GEMMs for the attention
# projections (hi·hi + hi·lo + lo·hi); the MoE gate/up GEMM with its input
# split and the expert weights rounded ("xsplit": (hi + lo)·bf16(w)); plain
# bf16 operands for Linear, the rest of the MoE experts and every backward
# GEMM; the attention core's products on bf16 operands (attn_core: q, k, v,
# the normalised P, dO and dS rounded).
DEVICE = {"linear_fwd": "bf16", "attn_fwd": "split", "linear_bwd": "bf16", "attn_bwd": "bf16",
          "attn_core": "bf16", "moe_fwd": "xsplit", "moe_bwd": "bf16"}
WIDE = {site: "wide" for site in SITES}
BF16 = {site: "bf16" for site in SITES}


class Model:
    def __init__(self, policy=None):
        self.policy = dict(DEVICE if policy is None else policy)
        self.site = None

    def rb(self, a):
        """One GEMM operand as the current site rounds it (split sites: hi)."""
        if self.policy.get(self.site, "wide") == "wide":
            return np.asarray(a, F64)
        return bf16_round(a)

    def core_rb(self, dh):
        """Operand rounding of the attention core's products (site attn_core;
        the device's bf16 core covers d_head 64, other head sizes stay fp32)."""
        if self.policy.get("attn_core", "wide") == "bf16" and dh == 64:
            return bf16_round
        return lambda a: np.asarray(a, F64)

    def mm(self, a, b):
        if self.policy.get(self.site, "wide") == "split":
            ah, al = bf16_split(a)
            bh, bl = bf16_split(b)
            return ah @ bh + ah @ bl + al @ bh
        return self.rb(a) @ self.rb(b)

    # ------------------------------------------------------------ forward
    def forward(self, node, xs):
        """Returns (value, tape)."""
        rb = self.rb
        kind = node.op.kind
        self.site = {"linear": "linear_fwd", "matmul": "linear_fwd", "attention": "attn_fwd",
                     "moe": "moe_fwd"}.get(kind)
        P = {k: v.numpy().astype(F64) for k, v in node.params.items()}
        x = xs[0] if xs else np.zeros(node.output_ty.shape)
        if kind in ("identity", "reshape", "transpose"):
            return x.copy(), None
        if kind == "relu":
            return np.maximum(x, 0.0), None
        if kind == "gelu":
            return _gelu(x), None
        if kind in ("add", "residual_add"):
            return (x + xs[1] if len(xs) > 1 else x.copy()), None
        if kind in ("linear", "matmul"):
            w = P.get("w", next(iter(P.values())))
            K, N = w.shape
            y = self.mm(x.reshape(-1, K), w)
            if "b" in P:
                y = y + P["b"]
            return y.reshape(x.shape[:-1] + (N,)), None
        if kind == "layer_norm":
            eps = float(np.float32(node.op.fields[0]) * np.float32(1e-6))
            mu = x.mean(-1, keepdims=True)
            rstd = 1.0 / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
            return (x - mu) * rstd * P["gamma"] + P["beta"], (mu, rstd)
        if kind == "attention":
            heads, _, dh = node.op.fields
            B, S, D = x.shape
            wqkv = np.concatenate([P["wq"], P["wk"], P["wv"]], 1)
            qkv = self.mm(x.reshape(-1, D), wqkv).reshape(B, S, 3, heads, dh)
            q, k, v = (qkv[:, :, i].transpose(0, 2, 1, 3) for i in range(3))  # [B,H,S,dh]
            core = self.core_rb(dh)
            s = core(q) @ core(k).transpose(0, 1, 3, 2) / np.sqrt(dh)
            if node.op.flags & 1:
                s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            ctx = (core(p) @ core(v)).transpose(0, 2, 1, 3).reshape(B * S, D)
            y = self.mm(ctx, P["wo"])
            return y.reshape(B, S, D), (q, k, v, p, ctx, wqkv)
        if kind == "moe":
            E, K, H, _ = node.op.fields
            xt = x.reshape(-1, H)
            T = xt.shape[0]
            idx, w, _ = oracle.route(xt.astype(np.float32), node.params["gate"].numpy(), K)
            w = w.astype(F64)
            y = np.zeros((T, H))
            saved = {}
            if self.policy.get("moe_fwd") == "xsplit":
                hi, lo = bf16_split(xt)
                xb = hi + lo
            else:
                xb = rb(xt)
            for e in range(E):
                tok, j = np.nonzero(idx == e)
                if tok.size == 0:
                    continue
                a = xb[tok] @ rb(P[f"e{e}.w1"])
                c = xb[tok] @ rb(P[f"e{e}.w3"])
                h = rb(_silu(a) * c)
                ys = h @ rb(P[f"e{e}.w2"])
                np.add.at(y, tok, w[tok, j][:, None] * ys)
                saved[e] = (tok, j, rb(a), rb(c), h, ys)
            return y.reshape(x.shape), (idx, w, saved)
        raise NotImplementedError(kind)

    # ----------------------------------------------------------- backward
    def backward(self, node, xs, tape, dy):
        """Returns ([cotangent per input], {port: parameter cotangent})."""
        rb = self.rb
        kind = node.op.kind
        self.site = {"linear": "linear_bwd", "matmul": "linear_bwd", "attention": "attn_bwd",
                     "moe": "moe_bwd"}.get(kind)
        P = {k: v.numpy().astype(F64) for k, v in node.params.items()}
        x = xs[0] if xs else None
        if kind in ("identity", "reshape", "transpose"):
            return [dy.copy()], {}
        if kind in ("add", "residual_add"):
            return [dy.copy() for _ in xs], {}
        if kind == "relu":
            return [np.where(x > 0, dy, 0.0)], {}
        if kind == "gelu":
            return [dy * _gelu_grad(x)], {}
        if kind in ("linear", "matmul"):
            port = "w" if "w" in P else next(iter(P))
            w = P[port]
            K, N = w.shape
            dyb = rb(dy.reshape(-1, N))
            d = {port: rb(x.reshape(-1, K)).T @ dyb}
            if "b" in P:
                d["b"] = dy.reshape(-1, N).sum(0)
            return [(dyb @ rb(w).T).reshape(x.shape)], d
        if kind == "layer_norm":
            mu, rstd = tape
            C = x.shape[-1]
            xh = (x - mu) * rstd
            g = dy * P["gamma"]
            dx = rstd / C * (C * g - g.sum(-1, keepdims=True) - xh * (g * xh).sum(-1, keepdims=True))
            return [dx], {"gamma": (dy * xh).reshape(-1, C).sum(0), "beta": dy.reshape(-1, C).sum(0)}
        if kind == "attention":
            q, k, v, p, ctx, wqkv = tape
            heads, _, dh = node.op.fields
            B, S, D = x.shape
            dyb = rb(dy.reshape(-1, D))
            dwo = rb(ctx).T @ dyb
            dctx = (dyb @ rb(P["wo"]).T).reshape(B, S, heads, dh).transpose(0, 2, 1, 3)
            # D_i = Σ_d dO·O over the forward's context, as the device takes it
            # (equal to Σ_j dP·P when nothing is rounded); dS is rounded before
            # the 1/√dh scale.
            core = self.core_rb(dh)
            D_ = (dctx * ctx.reshape(B, S, heads, dh).transpose(0, 2, 1, 3)).sum(-1)[..., None]
            dv = core(p).transpose(0, 1, 3, 2) @ core(dctx)
            dp = core(dctx) @ core(v).transpose(0, 1, 3, 2)
            ds = core(p * (dp - D_))
            dq = ds @ core(k) / np.sqrt(dh)
            dk = ds.transpose(0, 1, 3, 2) @ core(q) / np.sqrt(dh)
            dqkv = np.stack([t.transpose(0, 2, 1, 3) for t in (dq, dk, dv)], 2).reshape(-1, 3 * D)
            dqkvb = rb(dqkv)
            dx = (dqkvb @ rb(wqkv).T).reshape(x.shape)
            dw = rb(x.reshape(-1, D)).T @ dqkvb
            return [dx], {"wq": dw[:, :D], "wk": dw[:, D:2 * D], "wv": dw[:, 2 * D:], "wo": dwo}
        if kind == "moe":
            idx, w, saved = tape
            E, K, H, _ = node.op.fields
            xt = x.reshape(-1, H)
            dyt = dy.reshape(-1, H)
            T = xt.shape[0]
            xb = rb(xt)
            dx = np.zeros((T, H))
            dwts = np.zeros((T, K))
            d = {}
            for e in range(E):
                I = P[f"e{e}.w1"].shape[1]
                d[f"e{e}.w1"], d[f"e{e}.w3"], d[f"e{e}.w2"] = np.zeros((H, I)), np.zeros((H, I)), np.zeros((I, H))
                if e not in saved:
                    continue
                tok, j, a, c, h, ys = saved[e]
                dwts[tok, j] = (ys * dyt[tok]).sum(1)
                dys = rb(w[tok, j][:, None] * dyt[tok])
                dh_ = dys @ rb(P[f"e{e}.w2"]).T
                da = rb(dh_ * c * _silu_grad(a))
                dc = rb(dh_ * _silu(a))
                np.add.at(dx, tok, da @ rb(P[f"e{e}.w1"]).T + dc @ rb(P[f"e{e}.w3"]).T)
                d[f"e{e}.w2"] = h.T @ dys
                d[f"e{e}.w1"] = xb[tok].T @ da
                d[f"e{e}.w3"] = xb[tok].T @ dc
            # router_backward_ste (adjoint.rs:255-284): softmax Jacobian on the selected subset
            dl = np.zeros((T, E))
            dot = (w * dwts).sum(1, keepdims=True)
            np.add.at(dl, (np.arange(T)[:, None].repeat(K, 1), idx), w * (dwts - dot))
            d["gate"] = xt.T @ dl
            dx += dl @ P["gate"].T
            return [dx.reshape(x.shape)], d
        raise NotImplementedError(kind)


def train_step(graph, x, target, policy=None):
    """(loss, {node_id: {port: grad}}, {moe node id: top-k indices}) under a
    rounding policy {site: "wide" | "bf16" | "split"} (default DEVICE)."""
    m = Model(policy)
    order = oracle.topo(graph)
    acts, tapes = {}, {}
    for nid in order:
        if nid in graph.inputs:
            acts[nid] = np.asarray(x, F64)
            continue
        preds = [e.src for e in graph.edges if e.dst == nid]
        acts[nid], tapes[nid] = m.forward(graph.nodes[nid], [acts[p] for p in preds])
    out = graph.outputs[-1]
    e = acts[out] - np.asarray(target, F64).reshape(acts[out].shape)
    loss = float((e * e).mean())
    grads = {out: 2.0 * e / e.size}
    dparams = {}
    for nid in reversed(order):
        if nid in graph.inputs or nid not in grads:
            continue
        preds = [e.src for e in graph.edges if e.dst == nid]
        dxs, dp = m.backward(graph.nodes[nid], [acts[p] for p in preds], tapes[nid], grads[nid])
        for p, dx in zip(preds, dxs):
            grads[p] = grads[p] + dx if p in grads else dx
        dparams[nid] = dp
    routing = {nid: t[0] for nid, t in tapes.items() if graph.nodes[nid].op.kind == "moe"}
    return loss, dparams, routing
