"""IrGraph in the reference's serde JSON form (ir.rs:13-41 through
serde_json): load a graph the Rust compiler serialised, or write one.

`CGraph.from_json` parses in the backend (catnn_graph_from_json) and the
result installs like an IrGraph (`Program(dev, cgraph)`, `Trainer`).
`to_serde_json` is a second, pure-Python writer of the same encoding, kept
for the tests to cross-check the C++ one against.
"""
from __future__ import annotations

import ctypes
import json
from typing import Optional, Tuple

import numpy as np

from ._lib import check, lib
from .ir import IrGraph

_FP = ctypes.POINTER(ctypes.c_float)

# OpenOp kind → (serde variant name, field names in declaration order), morphism.rs:19-116.
SERDE_OPS = {
    "identity": ("identity", ()), "linear": ("linear", ("in_features", "out_features", "bias")),
    "relu": ("relu", ()), "gelu": ("gelu", ()), "softmax": ("softmax", ("axis",)),
    "layer_norm": ("layer_norm", ("eps_e6",)), "add": ("add", ()), "mul": ("mul", ()),
    "matmul": ("mat_mul", ()), "transpose": ("transpose", ("dim0", "dim1")),
    "reshape": ("reshape", ("out",)), "attention": ("attention", ("n_heads", "d_model", "d_head")),
    "residual_add": ("residual_add", ()), "embedding": ("embedding", ("vocab", "hidden")),
    "rms_norm": ("rms_norm", ("eps_e6",)),
    "gqa_attention": ("gqa_attention", ("n_heads", "n_kv_heads", "head_dim", "d_model", "sliding_window",
                                        "rope_theta")),
    "swiglu": ("swi_glu", ("hidden", "intermediate")), "router": ("router", ("n_experts", "top_k")),
    "moe": ("mo_e", ("n_experts", "top_k", "hidden", "intermediate")), "lm_head": ("lm_head", ("hidden", "vocab")),
    "mla": ("mla", ("n_heads", "q_lora", "kv_lora", "qk_nope", "qk_rope", "v_dim", "rope_theta")),
    "deepseek_moe": ("deep_seek_moe", ("n_routed", "n_shared", "top_k", "n_group", "topk_group", "hidden",
                                       "moe_intermediate", "routed_scale_milli")),
    "mix": ("mix", ()),
}


def _ty(t):
    return {"shape": {"dims": [int(d) for d in t.shape]}, "dtype": t.dtype}


def _op(op):
    name, fields = SERDE_OPS[op.kind]
    if not fields:
        return name
    if op.kind == "reshape":
        return {name: {"out": [int(d) for d in op.fields]}}
    body = {}
    for f, v in zip(fields, op.fields):
        if op.kind == "linear" and f == "bias":
            body[f] = bool(v)
        elif op.kind == "gqa_attention" and f == "sliding_window" and v < 0:
            body[f] = None  # Option::None
        else:
            body[f] = int(v)
    if op.kind == "attention" and op.flags & 1:
        body["causal"] = True
    return {name: body}


def to_serde_json(graph: IrGraph, inline: bool = True) -> Tuple[str, np.ndarray]:
    """serde_json::to_string of `graph` (+ the parameter blob when not inline)."""
    blob = []
    nodes = {}
    for nid, n in graph.nodes.items():
        params = {}
        for port, t in n.params.items():
            data = [None if not np.isfinite(v) else float(v) for v in t.data] if inline else []
            if not inline:
                blob.append(t.data)
            params[port] = {"ty": _ty(t.ty), "data": data}
        nodes[str(nid)] = {"id": nid, "name": n.name, "op": _op(n.op), "output_ty": _ty(n.output_ty),
                           "params": params}
    doc = {"name": graph.name, "nodes": nodes,
           "edges": [{"src": e.src, "dst": e.dst, "src_port": e.src_port, "dst_port": e.dst_port}
                     for e in graph.edges],
           "inputs": list(graph.inputs), "outputs": list(graph.outputs)}
    if graph.fusions:
        doc["fusions"] = [list(f.ops) for f in graph.fusions]
    b = np.concatenate(blob).astype(np.float32) if blob else np.zeros(0, np.float32)
    return json.dumps(doc, separators=(",", ":")), b


class CGraph:
    """A graph held by the backend (catnn_graph)."""

    def __init__(self, handle: ctypes.c_void_p):
        self.handle = handle

    @staticmethod
    def from_json(text, blob: Optional[np.ndarray] = None) -> "CGraph":
        raw = text.encode() if isinstance(text, str) else bytes(text)
        h = ctypes.c_void_p()
        if blob is not None:
            blob = np.ascontiguousarray(blob, np.float32)
            check(lib.catnn_graph_from_json(raw, len(raw), blob.ctypes.data_as(_FP), blob.size, ctypes.byref(h)))
        else:
            check(lib.catnn_graph_from_json(raw, len(raw), None, 0, ctypes.byref(h)))
        return CGraph(h)

    @staticmethod
    def from_ir(graph: IrGraph) -> "CGraph":
        return CGraph(graph.to_c())

    def to_json(self, inline: bool = True) -> Tuple[str, np.ndarray]:
        n, nb = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib.catnn_graph_to_json(self.handle, int(inline), None, 0, ctypes.byref(n), None, 0,
                                      ctypes.byref(nb)))
        buf = ctypes.create_string_buffer(n.value + 1)
        blob = np.empty(max(nb.value, 1), np.float32)
        check(lib.catnn_graph_to_json(self.handle, int(inline), buf, n.value + 1, ctypes.byref(n),
                                      blob.ctypes.data_as(_FP), blob.size, ctypes.byref(nb)))
        return buf.value.decode(), blob[: nb.value]

    def free(self):
        if self.handle:
            check(lib.catnn_graph_free(self.handle))
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
