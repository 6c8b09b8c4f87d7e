"""Host-side mirror of catnn's runtime data and IR types.

Same names and meaning as the reference:
  * `TensorType`, `Tensor`   — crates/catnn-core/src/tensor.rs:179-289
  * `OpenOp`                 — crates/catnn-core/src/category/morphism.rs:19-116
  * `IrNode`, `IrEdge`, `IrGraph` — crates/catnn-compile/src/ir.rs:13-97
  * `FusionGroup`            — crates/catnn-core/src/architecture/realization.rs:40-45

`IrGraph.topo()` runs the C++ implementation in the backend library (the
same Kahn order as ir.rs:67-92), so the order a test sees is the order the
device executor walks.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from ._lib import (CNode, COp, CParam, CTensor, CatError, MAX_RANK, check, lib)

DTYPES = ["f32", "f16", "bf16", "fp8", "fp4", "i32", "bool"]

# OpenOp discriminants (declaration order of the Rust enum).
OP_KINDS = [
    "identity", "linear", "relu", "gelu", "softmax", "layer_norm", "add", "mul",
    "matmul", "transpose", "reshape", "attention", "residual_add", "embedding",
    "rms_norm", "gqa_attention", "swiglu", "router", "moe", "lm_head", "mla",
    "deepseek_moe", "mix",
]
OP_NAMES = [  # OpenOp::name, morphism.rs:119-145
    "id", "linear", "relu", "gelu", "softmax", "layernorm", "add", "mul", "matmul",
    "transpose", "reshape", "attention", "residual_add", "embedding", "rmsnorm", "gqa",
    "swiglu", "router", "moe", "lm_head", "mla", "deepseek_moe", "mix",
]
FLAG_CAUSAL = 0x1


@dataclass(frozen=True)
class TensorType:
    """`TensorType { shape, dtype }` (tensor.rs:179-215)."""
    shape: tuple
    dtype: str = "f32"

    @staticmethod
    def f32(shape: Sequence[int]) -> "TensorType":
        return TensorType(tuple(int(d) for d in shape), "f32")

    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def bytes(self) -> int:
        size = {"f32": 4, "i32": 4, "f16": 2, "bf16": 2, "fp8": 1, "bool": 1, "fp4": 1}[self.dtype]
        return self.numel() * size

    def __str__(self) -> str:
        return f"{self.dtype}[{','.join(str(d) for d in self.shape)}]"


class Tensor:
    """`Tensor { ty, data: Vec<f32> }` (tensor.rs:223-289): storage is always
    row-major float32 on the host; `dtype` is a tag."""

    def __init__(self, ty: TensorType, data):
        arr = np.ascontiguousarray(np.asarray(data, dtype=np.float32).reshape(-1))
        if arr.size != ty.numel():
            raise CatError(2, f"data len {arr.size} != numel {ty.numel()}")
        self.ty = ty
        self.data = arr

    @staticmethod
    def zeros(ty: TensorType) -> "Tensor":
        return Tensor(ty, np.zeros(ty.numel(), np.float32))

    @staticmethod
    def ones(ty: TensorType) -> "Tensor":
        return Tensor(ty, np.ones(ty.numel(), np.float32))

    @staticmethod
    def from_numpy(arr: np.ndarray) -> "Tensor":
        arr = np.asarray(arr, dtype=np.float32)
        return Tensor(TensorType.f32(arr.shape), arr)

    @staticmethod
    def lcg(ty: TensorType, seed: int) -> "Tensor":
        """`Tensor::lcg` (tensor.rs:259-268), computed by the backend library."""
        out = np.empty(ty.numel(), np.float32)
        check(lib.catnn_tensor_lcg(seed & (2**64 - 1),
                                   out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out.size))
        return Tensor(ty, out)

    def numpy(self) -> np.ndarray:
        return self.data.reshape(self.ty.shape)

    def max_abs_diff(self, other: "Tensor") -> float:
        """`Tensor::max_abs_diff` (tensor.rs:270-277)."""
        if self.ty != other.ty:
            raise CatError(2, f"{self.ty} vs {other.ty}")
        if self.data.size == 0:
            return 0.0
        return float(np.max(np.abs(self.data - other.data)))

    def checksum(self) -> int:
        """`Tensor::checksum` (tensor.rs:279-288)."""
        out = ctypes.c_uint64()
        check(lib.catnn_tensor_checksum(self.data.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                        self.data.size, ctypes.byref(out)))
        return out.value

    def __repr__(self) -> str:
        return f"Tensor({self.ty})"


@dataclass(frozen=True)
class OpenOp:
    """An `OpenOp` variant: `kind` is the snake_case variant name, `fields`
    its fields in declaration order, `flags` backend extensions
    (FLAG_CAUSAL on Attention)."""
    kind: str
    fields: tuple = ()
    flags: int = 0

    def name(self) -> str:
        return OP_NAMES[OP_KINDS.index(self.kind)]

    # Constructors named after the variants.
    @staticmethod
    def identity():
        return OpenOp("identity")

    @staticmethod
    def linear(in_features: int, out_features: int, bias: bool = True):
        return OpenOp("linear", (in_features, out_features, int(bias)))

    @staticmethod
    def relu():
        return OpenOp("relu")

    @staticmethod
    def gelu():
        return OpenOp("gelu")

    @staticmethod
    def softmax(axis: int = -1):
        return OpenOp("softmax", (axis,))

    @staticmethod
    def layer_norm(eps_e6: int = 1):
        return OpenOp("layer_norm", (eps_e6,))

    @staticmethod
    def add():
        return OpenOp("add")

    @staticmethod
    def mul():
        return OpenOp("mul")

    @staticmethod
    def matmul():
        return OpenOp("matmul")

    @staticmethod
    def transpose(dim0: int, dim1: int):
        return OpenOp("transpose", (dim0, dim1))

    @staticmethod
    def reshape(out: Sequence[int]):
        return OpenOp("reshape", tuple(out))

    @staticmethod
    def attention(n_heads: int, d_model: int, d_head: int, causal: bool = False):
        return OpenOp("attention", (n_heads, d_model, d_head), FLAG_CAUSAL if causal else 0)

    @staticmethod
    def residual_add():
        return OpenOp("residual_add")

    @staticmethod
    def rms_norm(eps_e6: int = 1):
        return OpenOp("rms_norm", (eps_e6,))

    @staticmethod
    def embedding(vocab: int, hidden: int):
        return OpenOp("embedding", (vocab, hidden))

    @staticmethod
    def gqa_attention(n_heads: int, n_kv_heads: int, head_dim: int, d_model: int,
                      sliding_window=None, rope_theta: int = 10000):
        """sliding_window None (Option::None) is stored as −1."""
        return OpenOp("gqa_attention", (n_heads, n_kv_heads, head_dim, d_model,
                                        -1 if sliding_window is None else sliding_window, rope_theta))

    @staticmethod
    def swiglu(hidden: int, intermediate: int):
        return OpenOp("swiglu", (hidden, intermediate))

    @staticmethod
    def router(n_experts: int, top_k: int):
        return OpenOp("router", (n_experts, top_k))

    @staticmethod
    def lm_head(hidden: int, vocab: int):
        return OpenOp("lm_head", (hidden, vocab))

    @staticmethod
    def mix():
        return OpenOp("mix")

    @staticmethod
    def moe(n_experts: int, top_k: int, hidden: int, intermediate: int):
        return OpenOp("moe", (n_experts, top_k, hidden, intermediate))

    def to_c(self) -> COp:
        op = COp()
        op.kind = OP_KINDS.index(self.kind)
        op.flags = self.flags
        for i, v in enumerate(self.fields[:8]):
            op.a[i] = int(v)
        return op


def ctensor(t: Optional[Tensor] = None, ty: Optional[TensorType] = None,
            buf: Optional[np.ndarray] = None) -> CTensor:
    """A catnn_tensor view of `t` (or of a type, with `buf` as storage)."""
    c = CTensor()
    ty = t.ty if t is not None else ty
    if ty is not None:
        if len(ty.shape) > MAX_RANK:
            raise CatError(2, f"rank {len(ty.shape)} > {MAX_RANK}")
        for i, d in enumerate(ty.shape):
            c.dims[i] = d
        c.rank = len(ty.shape)
        c.dtype = DTYPES.index(ty.dtype)
    arr = t.data if t is not None else buf
    if arr is not None:
        c.data = arr.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    return c


@dataclass
class IrNode:
    """`IrNode { id, name, op, output_ty, params }` (ir.rs:17-24)."""
    id: int
    name: str
    op: OpenOp
    output_ty: TensorType
    params: Dict[str, Tensor] = field(default_factory=dict)

    def to_c(self, with_data: bool = True):
        """catnn_node plus the objects that keep its memory alive."""
        keep = [self.name.encode()]
        params = (CParam * max(len(self.params), 1))()
        for i, (port, t) in enumerate(self.params.items()):
            pb = port.encode()
            keep.append(pb)
            params[i].port = pb
            params[i].value = ctensor(t) if with_data else ctensor(ty=t.ty)
        node = CNode()
        node.id = self.id
        node.name = keep[0]
        node.op = self.op.to_c()
        node.output_ty = ctensor(ty=self.output_ty)
        node.params = params
        node.n_params = len(self.params)
        keep.append(params)
        return node, keep


@dataclass
class IrEdge:
    """`IrEdge { src, dst, src_port, dst_port }` (ir.rs:26-32)."""
    src: int
    dst: int
    src_port: str = "data"
    dst_port: str = "data"


@dataclass
class FusionGroup:
    """`FusionGroup { name, ops }` (realization.rs:40-45)."""
    name: str
    ops: List[str]


class IrGraph:
    """`IrGraph { name, nodes, edges, inputs, outputs }` (ir.rs:35-97), plus
    the `Realization.fusions` that apply to it."""

    def __init__(self, name: str):
        self.name = name
        self.nodes: Dict[int, IrNode] = {}
        self.edges: List[IrEdge] = []
        self.inputs: List[int] = []
        self.outputs: List[int] = []
        self.fusions: List[FusionGroup] = []

    def add_node(self, node: IrNode) -> IrNode:
        self.nodes[node.id] = node
        return node

    def add_edge(self, src: int, dst: int, src_port: str = "data", dst_port: str = "data"):
        self.edges.append(IrEdge(src, dst, src_port, dst_port))

    def node(self, id: int) -> Optional[IrNode]:
        return self.nodes.get(id)

    def preds(self, id: int) -> List[int]:
        """ir.rs:58-60: sources of edges into `id`, in edge order."""
        return [e.src for e in self.edges if e.dst == id]

    def succs(self, id: int) -> List[int]:
        return [e.dst for e in self.edges if e.src == id]

    def to_c(self):
        """A catnn_graph handle (caller frees with lib.catnn_graph_free)."""
        h = ctypes.c_void_p()
        check(lib.catnn_graph_new(self.name.encode(), ctypes.byref(h)))
        try:
            for n in self.nodes.values():
                cn, keep = n.to_c()
                check(lib.catnn_graph_add_node(h, ctypes.byref(cn)))
                del keep
            for e in self.edges:
                check(lib.catnn_graph_add_edge(h, e.src, e.dst, e.src_port.encode(),
                                               e.dst_port.encode()))
            for i in self.inputs:
                check(lib.catnn_graph_add_input(h, i))
            for o in self.outputs:
                check(lib.catnn_graph_add_output(h, o))
            for f in self.fusions:
                names = [s.encode() for s in f.ops]
                arr = (ctypes.c_char_p * max(len(names), 1))(*names)
                check(lib.catnn_graph_add_fusion(h, arr, len(names)))
        except Exception:
            lib.catnn_graph_free(h)
            raise
        return h

    def topo(self) -> List[int]:
        """Kahn order of ir.rs:67-92 (CatError Wiring on cycles)."""
        h = self.to_c()
        try:
            order = (ctypes.c_uint32 * max(len(self.nodes), 1))()
            n = ctypes.c_int32()
            check(lib.catnn_graph_topo(h, order, len(self.nodes), ctypes.byref(n)))
            return [int(order[i]) for i in range(n.value)]
        finally:
            lib.catnn_graph_free(h)
