"""The benchmark configurations as IR graphs with seeded synthetic weights.

  1  MLP 256×(784→512→512→10), ReLU — the reference's `.catnn` spec path
     (parse_catnn → to_architecture → lower_architecture), weights
     N(0, 2/fan_in), biases 0, input U(−1, 1).
  2  MLP 8192×(4096→16384→4096), GELU — same path, weights N(0, 1/fan_in),
     biases N(0, 0.01), input N(0, 1).
  3  Pre-LN transformer block [8,1024,1024], 16 heads × 64, causal, FFN ×4
     with GELU, two residual adds — an explicit IrGraph (chain lowering
     cannot express the skips, lower.rs:38-55).  Weights N(0, 0.02),
     biases N(0, 0.02), γ = 1, β = 0, input N(0, 1).
  4  MoE layer: 16384 tokens × 1024, 8 SwiGLU experts 1024→3584→1024,
     top-2; gate N(0, 0.5), experts N(0, 0.02), input N(0, 1).
  5  Config 3's block followed by config 4's layer on its 8192 tokens, one
     training step against a N(0, 1) target.

Reading of N(0, c): in the fan-in forms N(0, 2/fan_in) and N(0, 1/fan_in)
(He and LeCun initialisation) c is the variance; in the constant forms
N(0, 0.02), N(0, 0.5) and N(0, 1) it is the standard deviation, GPT-2's
N(0, 0.02) convention.  (Read as a variance, 0.02 gives the block a gain of
≈4.5 per projection: config 5's first MSE is 2e10 and lr 0.05 turns the
weights to NaN within two steps, in the fp32 reference step as on the
device.)  Tensor i of config c is drawn from the SplitMix64 stream seeded
1000·c + i.  Every builder takes smaller shapes for parity tests.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from . import synth
from .ir import FusionGroup, IrGraph, IrNode, OpenOp, Tensor, TensorType
from .spec import lower_architecture, parse_catnn, propose_fusions, to_architecture

# Standard deviations of the constant-form normals.
W_STD = 0.02     # block and expert weights, block biases
GATE_STD = 0.5   # router weights


@dataclass
class Workload:
    name: str
    graph: IrGraph
    x: Tensor
    flops: int            # algorithmic FLOPs of one forward
    min_bytes: int        # compulsory HBM traffic of one forward
    tokens: int


def _seq(config: int):
    i = 0
    while True:
        yield 1000 * config + i
        i += 1


def mlp_text(name: str, batch: int, dims: List[int], act: str) -> str:
    lines = [f"network {name} batch {batch}"]
    for li in range(len(dims) - 1):
        lines.append(f"linear fc{li + 1} {dims[li]} {dims[li + 1]}")
        if li + 2 < len(dims):
            lines.append(f"{act} act{li + 1}")
    lines.append("compose sequential")
    return "\n".join(lines) + "\n"


def _mlp(config: int, name: str, batch: int, dims: List[int], act: str, w_var_num: float,
         bias_var: float, x_kind: str) -> Workload:
    arch = to_architecture(parse_catnn(mlp_text(name, batch, dims, act)))
    g = lower_architecture(arch)
    seeds = _seq(config)
    for node in g.nodes.values():
        if node.op.kind != "linear":
            continue
        fan_in, fan_out = node.op.fields[0], node.op.fields[1]
        node.params["w"] = Tensor(TensorType.f32([fan_in, fan_out]),
                                  synth.normal(fan_in * fan_out, next(seeds), w_var_num / fan_in))
        b = (synth.normal(fan_out, next(seeds), bias_var) if bias_var > 0
             else np.zeros(fan_out, np.float32))
        node.params["b"] = Tensor(TensorType.f32([fan_out]), b)
    g.fusions = propose_fusions(g)
    n_x = batch * dims[0]
    xs = (synth.uniform(n_x, next(seeds), -1.0, 1.0) if x_kind == "uniform"
          else synth.normal(n_x, next(seeds), 1.0))
    x = Tensor(TensorType.f32([batch, dims[0]]), xs)
    flops = sum(2 * batch * dims[i] * dims[i + 1] for i in range(len(dims) - 1))
    w_bytes = sum(4 * (dims[i] * dims[i + 1] + dims[i + 1]) for i in range(len(dims) - 1))
    act_bytes = 4 * batch * (dims[0] + dims[-1] + 2 * sum(dims[1:-1]))
    return Workload(name, g, x, flops, w_bytes + act_bytes, batch)


def config1(batch: int = 256) -> Workload:
    return _mlp(1, "mlp", batch, [784, 512, 512, 10], "relu", 2.0, 0.0, "uniform")


def config2(batch: int = 8192, d: int = 4096, hidden: int = 16384) -> Workload:
    return _mlp(2, "mlp_gemm", batch, [d, hidden, d], "gelu", 1.0, 0.01, "normal")


def attention_flops(batch: int, seq: int, heads: int, d_head: int, causal: bool) -> int:
    """QKᵀ and PV: 2·dh per (query, key) pair attended, each."""
    pairs = seq * (seq + 1) // 2 if causal else seq * seq
    return 2 * 2 * batch * heads * pairs * d_head


def config3(batch: int = 8, seq: int = 1024, d: int = 1024, heads: int = 16, ffn: int = 4096,
            causal: bool = True, _config: int = 3) -> Workload:
    seeds = _seq(_config)
    var = W_STD ** 2
    T = batch * seq
    ty = TensorType.f32([batch, seq, d])

    def w(shape):
        n = int(np.prod(shape))
        return Tensor(TensorType.f32(shape), synth.normal(n, next(seeds), var))

    g = IrGraph("prenorm_block")
    ones = lambda n: Tensor(TensorType.f32([n]), np.ones(n, np.float32))
    zeros = lambda n: Tensor(TensorType.f32([n]), np.zeros(n, np.float32))
    g.add_node(IrNode(0, "block.in", OpenOp.identity(), ty))
    g.add_node(IrNode(1, "ln1", OpenOp.layer_norm(1), ty, {"gamma": ones(d), "beta": zeros(d)}))
    g.add_node(IrNode(2, "attn", OpenOp.attention(heads, d, d // heads, causal), ty,
                      {"wq": w([d, d]), "wk": w([d, d]), "wv": w([d, d]), "wo": w([d, d])}))
    g.add_node(IrNode(3, "res1", OpenOp.residual_add(), ty))
    g.add_node(IrNode(4, "ln2", OpenOp.layer_norm(1), ty, {"gamma": ones(d), "beta": zeros(d)}))
    g.add_node(IrNode(5, "ff1", OpenOp.linear(d, ffn, True), TensorType.f32([batch, seq, ffn]),
                      {"w": w([d, ffn]), "b": w([ffn])}))
    g.add_node(IrNode(6, "ff_act", OpenOp.gelu(), TensorType.f32([batch, seq, ffn])))
    g.add_node(IrNode(7, "ff2", OpenOp.linear(ffn, d, True), ty, {"w": w([ffn, d]), "b": w([d])}))
    g.add_node(IrNode(8, "res2", OpenOp.residual_add(), ty))
    for s, t in [(0, 1), (1, 2), (0, 3), (2, 3), (3, 4), (4, 5), (5, 6), (6, 7), (3, 8), (7, 8)]:
        g.add_edge(s, t)
    g.inputs.append(0)
    g.outputs.append(8)
    g.fusions = propose_fusions(g)
    x = Tensor(ty, synth.normal(T * d, next(seeds), 1.0))
    dh = d // heads
    flops = (2 * T * d * 3 * d + attention_flops(batch, seq, heads, dh, causal) + 2 * T * d * d
             + 2 * 2 * T * d * ffn)
    w_bytes = 4 * (4 * d * d + 2 * d * ffn + ffn + d + 4 * d)
    act_bytes = 4 * T * (2 * d + 2 * d + 3 * d + d + d + d + ffn + ffn + d + d)
    wl = Workload("prenorm_block", g, x, flops, w_bytes + act_bytes, T)
    wl._seeds = seeds  # config 5 keeps drawing from the same stream
    return wl


def moe_weights(n_experts: int, hidden: int, inter: int, seeds, gate_var=GATE_STD ** 2,
                w_var=W_STD ** 2):
    gate = synth.normal(hidden * n_experts, next(seeds), gate_var).reshape(hidden, n_experts)
    w1 = np.empty((n_experts, hidden, inter), np.float32)
    w3 = np.empty((n_experts, hidden, inter), np.float32)
    w2 = np.empty((n_experts, inter, hidden), np.float32)
    for e in range(n_experts):
        w1[e] = synth.normal(hidden * inter, next(seeds), w_var).reshape(hidden, inter)
        w3[e] = synth.normal(hidden * inter, next(seeds), w_var).reshape(hidden, inter)
        w2[e] = synth.normal(inter * hidden, next(seeds), w_var).reshape(inter, hidden)
    return gate, w1, w3, w2


def config4(batch: int = 8, seq: int = 2048, d: int = 1024, n_experts: int = 8, top_k: int = 2,
            inter: int = 3584) -> Workload:
    seeds = _seq(4)
    T = batch * seq
    ty = TensorType.f32([batch, seq, d])
    gate, w1, w3, w2 = moe_weights(n_experts, d, inter, seeds)
    params = {"gate": Tensor(TensorType.f32([d, n_experts]), gate)}
    for e in range(n_experts):
        params[f"e{e}.w1"] = Tensor(TensorType.f32([d, inter]), w1[e])
        params[f"e{e}.w3"] = Tensor(TensorType.f32([d, inter]), w3[e])
        params[f"e{e}.w2"] = Tensor(TensorType.f32([inter, d]), w2[e])
    g = IrGraph("moe_layer")
    g.add_node(IrNode(0, "moe.in", OpenOp.identity(), ty))
    g.add_node(IrNode(1, "moe", OpenOp.moe(n_experts, top_k, d, inter), ty, params))
    g.add_edge(0, 1)
    g.inputs.append(0)
    g.outputs.append(1)
    x = Tensor(ty, synth.normal(T * d, next(seeds), 1.0))
    flops = 2 * T * d * n_experts + T * top_k * 2 * 3 * d * inter
    min_bytes = 4 * (2 * T * d + d * n_experts + 3 * n_experts * d * inter)
    return Workload("moe_layer", g, x, flops, min_bytes, T)


def _moe_params(n_experts, d, inter, seeds):
    gate, w1, w3, w2 = moe_weights(n_experts, d, inter, seeds)
    params = {"gate": Tensor(TensorType.f32([d, n_experts]), gate)}
    for e in range(n_experts):
        params[f"e{e}.w1"] = Tensor(TensorType.f32([d, inter]), w1[e])
        params[f"e{e}.w3"] = Tensor(TensorType.f32([d, inter]), w3[e])
        params[f"e{e}.w2"] = Tensor(TensorType.f32([inter, d]), w2[e])
    return params


@dataclass
class TrainWorkload:
    name: str
    graph: IrGraph
    x: Tensor
    target: Tensor
    lr: float
    flops: int          # forward + backward (2x forward), the reference's recompute excluded
    tokens: int


def config5(batch: int = 8, seq: int = 1024, d: int = 1024, heads: int = 16, ffn: int = 4096,
            n_experts: int = 8, top_k: int = 2, inter: int = 3584) -> TrainWorkload:
    """Config 5: the config-3 block followed by the config-4 MoE layer on the
    block's T = batch·seq tokens, one training step (forward, MSE against a
    N(0,1) target, reverse chain, SGD lr 0.05)."""
    blk = config3(batch, seq, d, heads, ffn, causal=True, _config=5)
    g = blk.graph
    g.name = "block_moe_train"
    seeds = blk._seeds
    ty = TensorType.f32([batch, seq, d])
    g.add_node(IrNode(9, "moe", OpenOp.moe(n_experts, top_k, d, inter), ty,
                      _moe_params(n_experts, d, inter, seeds)))
    g.add_edge(8, 9)
    g.outputs = [9]
    T = batch * seq
    target = Tensor(ty, synth.normal(T * d, next(seeds), 1.0))
    moe_flops = 2 * T * d * n_experts + T * top_k * 2 * 3 * d * inter
    fwd = blk.flops + moe_flops
    return TrainWorkload("block_moe_train", g, blk.x, target, 0.05, 3 * fwd, T)


def config5_graph(**kw) -> IrGraph:
    return config5(**kw).graph


@dataclass
class MixtralShape:
    """MixtralConfig fields the graph needs (crates/catnn-core/src/spec/mixtral.rs:
    107-130 gives the tiny values used as defaults)."""
    vocab: int = 32
    hidden: int = 32
    inter: int = 64
    layers: int = 2
    heads: int = 4
    kv_heads: int = 2
    experts: int = 4
    top_k: int = 2
    eps: float = 1e-5
    rope_theta: int = 10000
    sliding_window: Optional[int] = 8


def mixtral(batch: int = 2, seq: int = 4, shape: Optional[MixtralShape] = None, seed: int = 7) -> Workload:
    """The IrGraph of mixtral_architecture (mixtral.rs:180-292): tokens →
    embed → per layer rms_attn → gqa → rms_moe → moe → final_norm → lm_head,
    a plain chain (the architecture lowers without residual adds).  Weights
    are seeded normals scaled 1/fan_in (the RMSNorm weights 1 + N(0, 0.01));
    token ids are uniform over the vocabulary, stored as f32 like every
    value the reference evaluates."""
    c = shape or MixtralShape()
    seeds = iter(range(1000 * seed, 1000 * seed + 100000))
    h, hd = c.hidden, c.hidden // c.heads
    eps_e6 = int(np.float32(c.eps) * np.float32(1e6))  # (eps · 1e6) as u32, in f32

    def normal(shape, var):
        n = int(np.prod(shape))
        return Tensor(TensorType.f32(shape), synth.normal(n, next(seeds), var).reshape(shape))

    def norm_w():
        return Tensor(TensorType.f32([h]), 1.0 + synth.normal(h, next(seeds), 0.01))

    ty = TensorType.f32([batch, seq, h])
    g = IrGraph(f"mixtral_{c.layers}l_{h}")
    g.add_node(IrNode(0, "tokens", OpenOp.identity(), TensorType.f32([batch, seq])))
    g.inputs.append(0)
    nodes = [IrNode(1, "embed", OpenOp.embedding(c.vocab, h), ty, {"w": normal([c.vocab, h], 1.0)})]
    for layer in range(c.layers):
        gqa_params = {"wq": normal([h, h], 1.0 / h), "wk": normal([h, c.kv_heads * hd], 1.0 / h),
                      "wv": normal([h, c.kv_heads * hd], 1.0 / h), "wo": normal([h, h], 1.0 / h)}
        moe_params = {"gate": normal([h, c.experts], 1.0 / h)}
        for e in range(c.experts):
            moe_params[f"e{e}.w1"] = normal([h, c.inter], 1.0 / h)
            moe_params[f"e{e}.w3"] = normal([h, c.inter], 1.0 / h)
            moe_params[f"e{e}.w2"] = normal([c.inter, h], 1.0 / c.inter)
        nid = len(nodes) + 1
        nodes += [
            IrNode(nid, f"L{layer}.rms_attn", OpenOp.rms_norm(eps_e6), ty, {"w": norm_w()}),
            IrNode(nid + 1, f"L{layer}.gqa",
                   OpenOp.gqa_attention(c.heads, c.kv_heads, hd, h, c.sliding_window, c.rope_theta), ty,
                   gqa_params),
            IrNode(nid + 2, f"L{layer}.rms_moe", OpenOp.rms_norm(eps_e6), ty, {"w": norm_w()}),
            IrNode(nid + 3, f"L{layer}.moe", OpenOp.moe(c.experts, c.top_k, h, c.inter), ty, moe_params),
        ]
    nid = len(nodes) + 1
    nodes += [IrNode(nid, "final_norm", OpenOp.rms_norm(eps_e6), ty, {"w": norm_w()}),
              IrNode(nid + 1, "lm_head", OpenOp.lm_head(h, c.vocab), TensorType.f32([batch, seq, c.vocab]),
                     {"w": normal([c.vocab, h], 1.0 / h)})]
    prev = 0
    for n in nodes:
        g.add_node(n)
        g.add_edge(prev, n.id)
        prev = n.id
    g.outputs.append(prev)
    T = batch * seq
    ids = synth.uniform(T, next(seeds), 0.0, float(c.vocab))
    x = Tensor(TensorType.f32([batch, seq]), np.minimum(np.floor(ids), c.vocab - 1).astype(np.float32))
    kvw = c.kv_heads * hd
    win = seq if c.sliding_window is None else min(seq, c.sliding_window)
    attn_pairs = sum(min(i + 1, win) for i in range(seq)) * batch
    per_layer = (2 * T * h * (2 * h + 2 * kvw) + 4 * attn_pairs * c.heads * hd +
                 2 * T * h * c.experts + T * c.top_k * 6 * h * c.inter)
    flops = c.layers * per_layer + 2 * T * h * c.vocab
    params = sum(t.data.size for n in g.nodes.values() for t in n.params.values())
    return Workload(g.name, g, x, flops, 4 * (params + T + T * c.vocab), T)
