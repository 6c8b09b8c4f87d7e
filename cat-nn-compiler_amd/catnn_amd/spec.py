"""From catnn's `.catnn` spec text to an IrGraph, for chain-wired networks.

Restates the reference's front half so graphs reach the backend exactly as
the Rust compiler would hand them over:
  * `parse_catnn`        — crates/catnn-core/src/spec/parse.rs:39-115
  * `Architecture`       — NetworkSpec::to_architecture (spec/ast.rs:100-165)
                           with the component constructors of
                           crates/catnn-core/src/lens/open.rs:57-181
  * `lower_architecture` — crates/catnn-compile/src/lower.rs:16-127 (Chain
                           wiring; params materialised with Tensor::lcg,
                           seed = id·1009 + 17 + port index)
  * `propose_fusions`    — crates/catnn-compile/src/place.rs:184-208
  * `mlp_spec`, `transformer_block_spec` — spec/dsl.rs:130-156
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

from ._lib import CatError
from .ir import FusionGroup, IrGraph, IrNode, OpenOp, Tensor, TensorType


@dataclass
class LayerSpec:
    op: str
    name: str
    args: Dict[str, int] = field(default_factory=dict)


@dataclass
class NetworkSpec:
    name: str = "net"
    batch: int = 1
    layers: List[LayerSpec] = field(default_factory=list)
    compose: str = "sequential"


def _usize(tok: Optional[str], what: str) -> int:
    try:
        v = int(tok)  # type: ignore[arg-type]
    except (TypeError, ValueError):
        raise CatError(9, f"{what} needs an integer")
    if v < 0:
        raise CatError(9, f"{what} needs an integer")
    return v


def _need(tok: Optional[str], what: str) -> str:
    if tok is None:
        raise CatError(9, f"missing {what}")
    return tok


def parse_catnn(src: str) -> NetworkSpec:
    """parse.rs:48-115."""
    spec = NetworkSpec()
    for lineno, raw in enumerate(src.splitlines()):
        line = raw.strip()
        if not line or line.startswith("#") or line.startswith("//"):
            continue
        toks = line.split()
        kw, rest = toks[0], toks[1:] + [None] * 4
        if kw == "network":
            spec.name = _need(rest[0], "network name")
            if rest[1] == "batch":
                spec.batch = _usize(rest[2], "batch")
        elif kw == "linear":
            spec.layers.append(LayerSpec("linear", _need(rest[0], "linear name"),
                                         {"in_features": _usize(rest[1], "in_features"),
                                          "out_features": _usize(rest[2], "out_features"),
                                          "bias": 1}))
        elif kw in ("relu", "gelu"):
            spec.layers.append(LayerSpec(kw, _need(rest[0], f"{kw} name")))
        elif kw == "softmax":
            spec.layers.append(LayerSpec("softmax", _need(rest[0], "softmax name"), {"axis": -1}))
        elif kw == "layernorm":
            spec.layers.append(LayerSpec("layer_norm", _need(rest[0], "layernorm name"),
                                         {"features": _usize(rest[1], "features")}))
        elif kw == "attention":
            spec.layers.append(LayerSpec("attention", _need(rest[0], "attention name"),
                                         {"seq": _usize(rest[1], "seq"),
                                          "d_model": _usize(rest[2], "d_model"),
                                          "n_heads": _usize(rest[3], "n_heads")}))
        elif kw == "compose":
            style = rest[0] or "sequential"
            if style not in ("sequential", "parallel"):
                raise CatError(9, f"unknown compose {style}")
            spec.compose = style
        else:
            raise CatError(9, f"line {lineno}: unknown keyword {kw}")
    if spec.batch == 0:
        spec.batch = 1
    return spec


@dataclass
class Component:
    """An `OpenComponent` reduced to what lowering reads: name, op, state
    ports (name → type, in declaration order) and input/output types."""
    name: str
    op: OpenOp
    state: List[Tuple[str, TensorType]]
    input: TensorType
    output: TensorType


@dataclass
class Architecture:
    id: str
    components: List[Component]
    materialize_params: bool = True

    def input(self) -> TensorType:
        return self.components[0].input


def _state_ports(op: OpenOp, in_features: Optional[int]) -> List[Tuple[str, TensorType]]:
    """OpenOp::state_interface, morphism.rs:247-342 (executable ops)."""
    if op.kind == "linear":
        i, o, bias = op.fields
        ports = [("w", TensorType.f32([i, o]))]
        if bias:
            ports.append(("b", TensorType.f32([o])))
        return ports
    if op.kind == "layer_norm":
        n = in_features or 1
        return [("gamma", TensorType.f32([n])), ("beta", TensorType.f32([n]))]
    if op.kind == "attention":
        d = op.fields[1]
        return [(p, TensorType.f32([d, d])) for p in ("wq", "wk", "wv", "wo")]
    if op.kind == "moe":
        e_count, _, hidden, inter = op.fields
        ports = [("gate", TensorType.f32([hidden, e_count]))]
        for e in range(e_count):
            ports += [(f"e{e}.w1", TensorType.f32([hidden, inter])),
                      (f"e{e}.w3", TensorType.f32([hidden, inter])),
                      (f"e{e}.w2", TensorType.f32([inter, hidden]))]
        return ports
    return []


def to_architecture(spec: NetworkSpec) -> Architecture:
    """NetworkSpec::to_architecture (ast.rs:100-165) + the open.rs
    constructors, checking that each component's input matches the previous
    output (CompositeSystem::then)."""
    batch = spec.batch or 1
    parts: List[Component] = []
    cur: Optional[TensorType] = None
    for layer in spec.layers:
        a = layer.args
        if layer.op == "linear":
            i, o = a["in_features"], a["out_features"]
            inp = cur if cur is not None else TensorType.f32([batch, i])
            last = inp.shape[-1] if inp.shape else 0
            if last != i:
                raise CatError(2, f"linear {layer.name}: last dim {last} != in_features {i}")
            out = TensorType.f32(list(inp.shape[:-1]) + [o]) if inp.shape else TensorType.f32([o])
            op = OpenOp.linear(i, o, bool(a.get("bias", 1)))
            parts.append(Component(layer.name, op, _state_ports(op, i), inp, out))
        elif layer.op in ("relu", "gelu", "softmax"):
            if cur is None:
                raise CatError(9, f"{layer.op} {layer.name} has no preceding interface")
            op = {"relu": OpenOp.relu(), "gelu": OpenOp.gelu(),
                  "softmax": OpenOp.softmax(a.get("axis", -1))}[layer.op]
            parts.append(Component(layer.name, op, [], cur, cur))
        elif layer.op == "layer_norm":
            if cur is None:
                raise CatError(9, f"layernorm {layer.name} has no preceding interface")
            op = OpenOp.layer_norm(1)  # eps_e6 = 1 (open.rs:131)
            parts.append(Component(layer.name, op, _state_ports(op, a["features"]), cur, cur))
        elif layer.op == "attention":
            d, h = a["d_model"], a["n_heads"]
            if h == 0 or d % h:
                raise CatError(2, f"d_model {d} not divisible by n_heads {h}")
            ty = TensorType.f32([batch, a["seq"], d])
            op = OpenOp.attention(h, d, d // h)
            parts.append(Component(layer.name, op, _state_ports(op, d), ty, ty))
        else:
            raise CatError(9, f"unsupported layer {layer.op}")
        if len(parts) > 1 and parts[-2].output != parts[-1].input:
            raise CatError(1, f"expected {parts[-2].output}, got {parts[-1].input}")
        cur = parts[-1].output
    if not parts:
        raise CatError(9, "network has no layers")
    return Architecture(spec.name, parts)


def lower_architecture(arch: Architecture) -> IrGraph:
    """lower.rs:16-127, Chain wiring."""
    g = IrGraph(arch.id)
    g.add_node(IrNode(0, f"{arch.id}.in", OpenOp.identity(), arch.input()))
    g.inputs.append(0)
    last = 0
    for idx, c in enumerate(arch.components, start=1):
        params = {}
        if arch.materialize_params:
            seed_base = idx * 1009 + 17
            for i, (pname, ty) in enumerate(c.state):
                params[pname] = Tensor.lcg(ty, seed_base + i)
        g.add_node(IrNode(idx, c.name, c.op, c.output, params))
        g.add_edge(last, idx)
        last = idx
    g.outputs.append(last)
    return g


def propose_fusions(graph: IrGraph, placement: Optional[Dict[str, str]] = None) -> List[FusionGroup]:
    """place.rs:184-208: consecutive (topo order) Linear → Relu/Gelu on the
    same device become one group."""
    order = graph.topo()
    place = placement or {}
    groups = []
    i = 0
    while i + 1 < len(order):
        a, b = graph.nodes[order[i]], graph.nodes[order[i + 1]]
        same = place.get(a.name) == place.get(b.name)
        if same and a.op.kind == "linear" and b.op.kind in ("relu", "gelu"):
            groups.append(FusionGroup(f"{a.name}+{b.name}", [a.name, b.name]))
            i += 2
        else:
            i += 1
    return groups


def mlp_spec(batch: int, din: int, hidden: int, dout: int) -> Architecture:
    """dsl.rs:130-136."""
    return to_architecture(NetworkSpec("mlp", batch, [
        LayerSpec("linear", "fc1", {"in_features": din, "out_features": hidden, "bias": 1}),
        LayerSpec("relu", "act"),
        LayerSpec("linear", "fc2", {"in_features": hidden, "out_features": dout, "bias": 1}),
    ]))


def transformer_block_spec(batch: int, seq: int, d_model: int, n_heads: int) -> Architecture:
    """dsl.rs:138-156 (the sequential stand-in: MHA → LN → FF → GELU → FF → LN)."""
    return to_architecture(NetworkSpec("transformer_block", batch, [
        LayerSpec("attention", "mha", {"seq": seq, "d_model": d_model, "n_heads": n_heads}),
        LayerSpec("layer_norm", "ln1", {"features": d_model}),
        LayerSpec("linear", "ff1", {"in_features": d_model, "out_features": 2 * d_model, "bias": 1}),
        LayerSpec("gelu", "ff_act"),
        LayerSpec("linear", "ff2", {"in_features": 2 * d_model, "out_features": d_model, "bias": 1}),
        LayerSpec("layer_norm", "ln2", {"features": d_model}),
    ]))
