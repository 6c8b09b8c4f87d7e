"""catnn oracle — TEST INFRASTRUCTURE ONLY (the checker, never the product).

numpy front end of oracle/catnn_oracle.cpp, the CPU restatement of the
reference's kernels, plus graph evaluation restating
  * kernel::eval_cpu / eval_reference dispatch  (crates/catnn-compile/src/kernel/mod.rs:21-251)
  * eval_graph_cpu / eval_graph_reference       (crates/catnn-compile/src/lib.rs:48-90)
  * IrGraph::topo / preds                        (crates/catnn-compile/src/ir.rs:58-92)
over any graph object with `nodes` (id → node with .op.kind, .op.fields,
.op.flags, .params, .output_ty, .name), `edges` (.src, .dst), `inputs`,
`outputs`.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module.  Pinning of each kernel is described in catnn_oracle.cpp's
header and checked by tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libcatnn_oracle.so")


def build() -> str:
    subprocess.run(["make", "-B", "-C", HERE], check=True, capture_output=True)
    return LIB_PATH


if not os.path.exists(LIB_PATH):
    build()
_lib = ctypes.CDLL(LIB_PATH)

_F = ctypes.POINTER(ctypes.c_float)
_I32P = ctypes.POINTER(ctypes.c_int32)
_I64P = ctypes.POINTER(ctypes.c_int64)
_U64P = ctypes.POINTER(ctypes.c_uint64)
_I64 = ctypes.c_int64

_SIG = {
    "orc_lcg": ([ctypes.c_uint64, _F, _I64], None),
    "orc_checksum": ([_F, _I64], ctypes.c_uint64),
    "orc_max_abs_diff": ([_F, _F, _I64], ctypes.c_float),
    "orc_relu": ([_F, _F, _I64], None),
    "orc_gelu": ([_F, _F, _I64], None),
    "orc_softmax_last": ([_F, _F, _I64, _I64], None),
    "orc_ref_softmax_last": ([_F, _F, _I64, _I64], None),
    "orc_layer_norm": ([_F, _F, _F, _F, _I64, _I64, ctypes.c_float], None),
    "orc_ref_layer_norm": ([_F, _F, _F, _F, _I64, _I64, ctypes.c_float], None),
    "orc_add": ([_F, _I64, _F, _I64, _I64, _F], ctypes.c_int),
    "orc_mul": ([_F, _F, _F, _I64], ctypes.c_int),
    "orc_matmul_seq": ([_F, _F, _F, _I64, _I64, _I64], None),
    "orc_linear_seq": ([_F, _F, _F, _F, _I64, _I64, _I64], None),
    "orc_matmul": ([_F, _F, _F, _I64, _I64, _I64], None),
    "orc_linear": ([_F, _F, _F, _F, _I64, _I64, _I64], None),
    "orc_ref_linear": ([_F, _F, _F, _F, _I64, _I64, _I64], None),
    "orc_attention": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, ctypes.c_int32, _F],
                      ctypes.c_int),
    "orc_topk_softmax": ([_F, _I64, _I64, _I32P, _F], None),
    "orc_route": ([_F, _F, _I64, _I64, _I64, _I64, _I32P, _F, _F], None),
    "orc_swiglu": ([_F, _F, _F, _F, _I64, _I64, _I64, _F], None),
    "orc_ref_swiglu": ([_F, _F, _F, _F, _I64, _I64, _I64, _F], None),
    "orc_moe": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, _I64P, _I64, _F], None),
    "orc_ref_moe": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, _F], None),
    "orc_moe_permute": ([_I32P, _I64, _I64, _I64, _I32P, _I32P, _I32P, _I32P], ctypes.c_int),
    "orc_place_arena": ([_U64P, _U64P, _U64P, _I64, ctypes.c_uint64, _U64P, _I64P, _I64P],
                        ctypes.c_int),
    "orc_arena_conflict": ([_U64P, _U64P, _U64P, _U64P, _I64], ctypes.c_int),
    "orc_rmsnorm": ([_F, _F, _I64, _I64, ctypes.c_float, _F], None),
    "orc_embedding": ([_F, _I64, _F, _I64, _I64, _F], ctypes.c_int),
    "orc_gqa": ([_F, _F, _F, _F, _F, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_double, _I64, _F],
                ctypes.c_int),
    "orc_lm_head": ([_F, _F, _I64, _I64, _I64, _F], None),
    "orc_mix": ([_F, _F, ctypes.c_float, _I64, _F], None),
}
for _name, (_args, _res) in _SIG.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res


def _f(a):
    return None if a is None else a.ctypes.data_as(_F)


def _c(a, dtype=np.float32):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------- kernels

def lcg(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    _lib.orc_lcg(seed, _f(out), n)
    return out


def checksum(x) -> int:
    x = _c(x).reshape(-1)
    return int(_lib.orc_checksum(_f(x), x.size))


def relu(x):
    x = _c(x)
    y = np.empty_like(x)
    _lib.orc_relu(_f(x), _f(y), x.size)
    return y


def gelu(x):
    x = _c(x)
    y = np.empty_like(x)
    _lib.orc_gelu(_f(x), _f(y), x.size)
    return y


def softmax_last(x, reference=False):
    x = _c(x)
    y = np.empty_like(x)
    last = x.shape[-1] if x.ndim else 1
    fn = _lib.orc_ref_softmax_last if reference else _lib.orc_softmax_last
    fn(_f(x), _f(y), x.size // max(last, 1), last)
    return y


def layer_norm(x, gamma, beta, eps=1e-6, reference=False):
    x, g, b = _c(x), _c(gamma), _c(beta)
    y = np.empty_like(x)
    last = x.shape[-1]
    fn = _lib.orc_ref_layer_norm if reference else _lib.orc_layer_norm
    fn(_f(x), _f(g), _f(b), _f(y), x.size // last, last, np.float32(eps))
    return y


def add(a, b):
    a, b = _c(a), _c(b)
    y = np.empty_like(a)
    last = a.shape[-1] if a.ndim else a.size
    rc = _lib.orc_add(_f(a), a.size, _f(b), b.size, last, _f(y))
    if rc:
        raise ValueError(f"add {a.shape} vs {b.shape}")
    return y


def mul(a, b):
    a, b = _c(a), _c(b)
    if a.size != b.size:
        raise ValueError("mul length")
    y = np.empty_like(a)
    _lib.orc_mul(_f(a), _f(b), _f(y), a.size)
    return y


def _lin(fn, x, w, b):
    x, w = _c(x), _c(w)
    k, n = w.shape
    m = x.size // k
    y = np.empty(x.shape[:-1] + (n,), np.float32)
    fn(_f(x), _f(w), _f(None if b is None else _c(b)), _f(y), m, k, n)
    return y


def linear(x, w, b=None):
    """cpu::linear (f32x8 dot, OpenMP rows)."""
    return _lin(_lib.orc_linear, x, w, b)


def linear_seq(x, w, b=None):
    """cpu::linear_seq (sequential p order)."""
    return _lin(_lib.orc_linear_seq, x, w, b)


def ref_linear(x, w, b=None):
    """reference::linear (naïve, bias inside the sum)."""
    return _lin(_lib.orc_ref_linear, x, w, b)


def attention(x, wq, wk, wv, wo, n_heads, d_head, causal=False):
    x = _c(x)
    B, S, D = x.shape
    out = np.empty_like(x)
    rc = _lib.orc_attention(_f(x), _f(_c(wq)), _f(_c(wk)), _f(_c(wv)), _f(_c(wo)), B, S, D,
                            n_heads, d_head, int(causal), _f(out))
    if rc:
        raise ValueError("attention: n_heads*d_head > d_model")
    return out


def topk_softmax(logits, k):
    logits = _c(logits).reshape(-1)
    kk = min(k, logits.size)
    idx = np.empty(kk, np.int32)
    w = np.empty(kk, np.float32)
    _lib.orc_topk_softmax(_f(logits), logits.size, k, idx.ctypes.data_as(_I32P), _f(w))
    return idx, w


def route(x, gate, top_k):
    x, gate = _c(x), _c(gate)
    H, E = gate.shape
    T = x.size // H
    idx = np.empty((T, top_k), np.int32)
    w = np.empty((T, top_k), np.float32)
    logits = np.empty((T, E), np.float32)
    _lib.orc_route(_f(x), _f(gate), T, H, E, top_k, idx.ctypes.data_as(_I32P), _f(w), _f(logits))
    return idx, w, logits


def swiglu(x, w1, w3, w2, reference=False):
    x = _c(x)
    H, I = w1.shape
    T = x.size // H
    y = np.empty_like(x)
    fn = _lib.orc_ref_swiglu if reference else _lib.orc_swiglu
    fn(_f(x), _f(_c(w1)), _f(_c(w3)), _f(_c(w2)), T, H, I, _f(y))
    return y


def moe(x, gate, w1s, w3s, w2s, top_k, tokens=None, reference=False):
    """moe::moe (or moe::reference::moe).  w1s/w3s [E,H,I], w2s [E,I,H].
    `tokens` restricts the expert work to those token rows (others zero)."""
    x, gate = _c(x), _c(gate)
    E, H, I = w1s.shape
    T = x.size // H
    out = np.zeros_like(x)
    w1s, w3s, w2s = _c(w1s), _c(w3s), _c(w2s)
    if reference:
        assert tokens is None
        _lib.orc_ref_moe(_f(x), _f(gate), _f(w1s), _f(w3s), _f(w2s), T, H, I, E, top_k, _f(out))
    else:
        tok = None if tokens is None else np.ascontiguousarray(tokens, np.int64)
        _lib.orc_moe(_f(x), _f(gate), _f(w1s), _f(w3s), _f(w2s), T, H, I, E, top_k,
                     None if tok is None else tok.ctypes.data_as(_I64P),
                     0 if tok is None else tok.size, _f(out))
    return out


def rmsnorm(x, w, eps):
    """moe::rmsnorm, moe.rs:17-32."""
    x, w = _c(x), _c(w)
    y = np.empty_like(x)
    _lib.orc_rmsnorm(_f(x), _f(w), x.size // x.shape[-1], x.shape[-1], np.float32(eps), _f(y))
    return y


def embedding(ids, table):
    """Embedding arm of eval_cpu (mod.rs:81-96): [.., n] f32 ids → [.., n, H]."""
    ids, table = _c(ids), _c(table)
    V, H = table.shape
    y = np.empty(ids.shape + (H,), np.float32)
    if _lib.orc_embedding(_f(ids), ids.size, _f(table), V, H, _f(y)):
        raise ValueError("token id >= vocab")
    return y


def gqa(x, wq, wk, wv, wo, n_heads, n_kv, head_dim, theta, window=None):
    """moe::gqa, moe.rs:62-136 (window None: no sliding window)."""
    x = _c(x)
    B, S, D = x.shape
    y = np.empty_like(x)
    rc = _lib.orc_gqa(_f(x), _f(_c(wq)), _f(_c(wk)), _f(_c(wv)), _f(_c(wo)), B, S, D, n_heads, n_kv,
                      head_dim, float(theta), -1 if window is None else int(window), _f(y))
    if rc:
        raise ValueError("gqa shape")
    return y


def lm_head(x, w):
    """moe::lm_head, moe.rs:325-333 (w is [V, H])."""
    x, w = _c(x), _c(w)
    V, H = w.shape
    y = np.empty(x.shape[:-1] + (V,), np.float32)
    _lib.orc_lm_head(_f(x), _f(w), x.size // H, H, V, _f(y))
    return y


# ---- Mixtral-tiny (crates/catnn-compile/src/kernel/moe.rs:227-322, :418-455) ----

class MixtralConfig:
    """MixtralConfig::tiny (crates/catnn-core/src/spec/mixtral.rs:107-130):
    the fields moe::forward reads."""

    def __init__(self, vocab=32, hidden=32, inter=64, layers=2, heads=4, kv_heads=2, experts=4, top_k=2,
                 eps=1e-5, rope_theta=10000.0, sliding_window=8):
        self.vocab, self.hidden, self.inter, self.layers = vocab, hidden, inter, layers
        self.heads, self.kv_heads, self.experts, self.top_k = heads, kv_heads, experts, top_k
        self.eps, self.rope_theta, self.sliding_window = eps, rope_theta, sliding_window

    def head_dim(self):
        """MixtralConfig::head_dim, mixtral.rs:132-140."""
        if self.heads == 0 or self.hidden % self.heads:
            raise ValueError("hidden not divisible by heads")
        return self.hidden // self.heads


_U64 = (1 << 64) - 1


def mixtral_weights_seeded(cfg, seed):
    """MixtralWeights::seeded, moe.rs:246-285: one Tensor::lcg per weight,
    its seed the next state of s ← s·6364136223846793005 + 1 (wrapping)
    from s = seed, drawn in the reference's order (embed; per layer the
    experts' (w1, w3, w2), then wq, wk, wv, wo, gate; lm_head last); RMSNorm
    weights are ones."""
    h, mid, hd = cfg.hidden, cfg.inter, cfg.head_dim()
    kv = cfg.kv_heads * hd
    state = [seed & _U64]

    def nxt():
        state[0] = (state[0] * 6364136223846793005 + 1) & _U64
        return state[0]

    def draw(rows, cols):
        return lcg(rows * cols, nxt()).reshape(rows, cols)

    w = {"embed": draw(cfg.vocab, h), "layers": []}
    for _ in range(cfg.layers):
        experts = [(draw(h, mid), draw(h, mid), draw(mid, h)) for _ in range(cfg.experts)]
        layer = {"rms_attn": np.ones(h, np.float32), "wq": draw(h, h), "wk": draw(h, kv), "wv": draw(h, kv),
                 "wo": draw(h, h), "rms_moe": np.ones(h, np.float32), "gate": draw(h, cfg.experts),
                 "experts": experts}
        w["layers"].append(layer)
    w["final_norm"] = np.ones(h, np.float32)
    w["lm_head"] = draw(cfg.vocab, h)
    return w


def _mixtral(cfg, w, tokens, batch, seq, reference):
    if len(tokens) != batch * seq:
        raise ValueError("token batch*seq")
    h = cfg.hidden
    x = embedding(np.asarray(tokens, np.float32).reshape(batch, seq), w["embed"])
    for layer in w["layers"]:
        xn = rmsnorm(x, layer["rms_attn"], cfg.eps)
        attn = gqa(xn, layer["wq"], layer["wk"], layer["wv"], layer["wo"], cfg.heads, cfg.kv_heads,
                   cfg.head_dim(), cfg.rope_theta, cfg.sliding_window)
        x = add(x, attn)  # cpu::add (forward, moe.rs:309); x[i] += attn[i] (reference, :437-439)
        xn = rmsnorm(x, layer["rms_moe"], cfg.eps)
        w1, w3, w2 = (np.stack([e[i] for e in layer["experts"]]) for i in range(3))
        m = moe(xn.reshape(-1, h), layer["gate"], w1, w3, w2, cfg.top_k, reference=reference).reshape(x.shape)
        x = add(x, m)
    x = rmsnorm(x, w["final_norm"], cfg.eps)
    return lm_head(x, w["lm_head"])


def mixtral_forward(cfg, w, tokens, batch, seq):
    """moe::forward, moe.rs:288-322: embed → per layer x += gqa(rmsnorm(x)),
    x += moe(rmsnorm(x)) → rmsnorm → lm_head."""
    return _mixtral(cfg, w, tokens, batch, seq, reference=False)


def mixtral_forward_reference(cfg, w, tokens, batch, seq):
    """moe::reference::forward, moe.rs:418-455: the same chain with the
    naïve reference MoE (moe.rs:383-416)."""
    return _mixtral(cfg, w, tokens, batch, seq, reference=True)


def mix(a, b, gate):
    """deepseek::mix, deepseek.rs:229-239."""
    a, b = _c(a), _c(b)
    y = np.empty_like(a)
    _lib.orc_mix(_f(a), _f(b), np.float32(gate), a.size, _f(y))
    return y


def moe_permute(idx, n_experts):
    idx = np.ascontiguousarray(idx, np.int32)
    T, k = idx.shape
    counts = np.empty(n_experts, np.int32)
    offsets = np.empty(n_experts + 1, np.int32)
    sop = np.empty(T * k, np.int32)
    pos = np.empty(T * k, np.int32)
    p = lambda a: a.ctypes.data_as(_I32P)
    rc = _lib.orc_moe_permute(p(idx), T, k, n_experts, p(counts), p(offsets), p(sop), p(pos))
    if rc:
        raise ValueError("expert id out of range")
    return counts, offsets, sop, pos


def place_arena(reqs, cap):
    """reqs: list of (bytes, live_from, live_to).  Returns (offsets,
    placement order) or raises OverflowError(index)."""
    n = len(reqs)
    b = np.array([r[0] for r in reqs], np.uint64)
    f = np.array([r[1] for r in reqs], np.uint64)
    t = np.array([r[2] for r in reqs], np.uint64)
    off = np.zeros(n, np.uint64)
    order = np.zeros(n, np.int64)
    fail = ctypes.c_int64(-1)
    u = lambda a: a.ctypes.data_as(_U64P)
    rc = _lib.orc_place_arena(u(b), u(f), u(t), n, cap, u(off), order.ctypes.data_as(_I64P),
                              ctypes.byref(fail))
    if rc:
        raise OverflowError(fail.value)
    return off, order


def arena_conflict(bytes_, offsets, live_from, live_to) -> bool:
    a = [np.ascontiguousarray(v, np.uint64) for v in (bytes_, offsets, live_from, live_to)]
    return bool(_lib.orc_arena_conflict(*[v.ctypes.data_as(_U64P) for v in a], len(a[0])))


# --------------------------------------------------------------- graphs

def topo(graph):
    """IrGraph::topo, ir.rs:67-92."""
    indeg = {k: 0 for k in graph.nodes}
    for e in graph.edges:
        indeg[e.dst] += 1
    q = sorted(k for k, d in indeg.items() if d == 0)
    out = []
    while q:
        n = q.pop()
        out.append(n)
        for s in sorted(e.dst for e in graph.edges if e.src == n):
            indeg[s] -= 1
            if indeg[s] == 0:
                q.append(s)
    if len(out) != len(graph.nodes):
        raise ValueError("IR graph has a cycle")
    return out


def eval_node(node, inputs, reference=False):
    """kernel::eval_cpu (mod.rs:21-194) or eval_reference (mod.rs:197-251)
    for the executable op set."""
    kind = node.op.kind
    if not inputs and kind == "identity":
        return np.zeros(node.output_ty.shape, np.float32)
    x = inputs[0]
    P = {k: v.numpy() for k, v in node.params.items()}
    if kind in ("identity", "reshape", "transpose"):
        return x.copy()
    if kind == "relu":
        return relu(x)
    if kind == "gelu":
        return gelu(x)
    if kind == "softmax":
        return softmax_last(x, reference)
    if kind in ("add", "residual_add"):
        return add(x, inputs[1]) if len(inputs) > 1 else x.copy()
    if kind == "mul":
        return mul(x, inputs[1]) if len(inputs) > 1 else x.copy()
    if kind in ("linear", "matmul"):
        w = P.get("w", next(iter(P.values())))
        fn = ref_linear if reference else linear
        return fn(x, w, P.get("b"))
    if kind == "layer_norm":
        eps = np.float32(node.op.fields[0]) * np.float32(1e-6)
        return layer_norm(x, P["gamma"], P["beta"], eps, reference)
    if kind == "attention":
        heads, _, dh = node.op.fields
        return attention(x, P["wq"], P["wk"], P["wv"], P["wo"], heads, dh,
                         causal=bool(node.op.flags & 1))
    if kind == "moe":
        E, k, _, _ = node.op.fields
        w1 = np.stack([P[f"e{e}.w1"] for e in range(E)])
        w3 = np.stack([P[f"e{e}.w3"] for e in range(E)])
        w2 = np.stack([P[f"e{e}.w2"] for e in range(E)])
        return moe(x, P["gate"], w1, w3, w2, k)
    # Mixtral / DeepSeek arms of eval_cpu (mod.rs:74-131, :186-193); eval_reference
    # sends these to eval_cpu as well (mod.rs:240-249).
    if kind == "rms_norm":
        return rmsnorm(x, P["w"], np.float32(node.op.fields[0]) * np.float32(1e-6))
    if kind == "embedding":
        return embedding(x, P["w"])
    if kind == "swiglu":
        return swiglu(x, P["w1"], P["w3"], P["w2"])
    if kind == "gqa_attention":
        nh, nkv, hd, _, window, theta = node.op.fields
        return gqa(x, P["wq"], P["wk"], P["wv"], P["wo"], nh, nkv, hd, float(theta),
                   None if window < 0 else window)
    if kind == "lm_head":
        return lm_head(x, P["w"])
    if kind == "router":
        return x.copy()
    if kind == "mix":
        return mix(x, inputs[1], float(P["gate"][0]) if "gate" in P else 0.0)
    raise NotImplementedError(kind)


def eval_graph(graph, x, reference=False):
    """eval_graph_cpu / eval_graph_reference, lib.rs:48-90."""
    vals = {}
    for nid in topo(graph):
        node = graph.nodes[nid]
        if nid in graph.inputs:
            vals[nid] = np.asarray(x, np.float32)
            continue
        preds = [e.src for e in graph.edges if e.dst == nid]
        vals[nid] = eval_node(node, [vals[p] for p in preds], reference)
    return vals[graph.outputs[-1]]
