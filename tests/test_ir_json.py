"""IrGraph serde-JSON ingest/export (catnn_graph_from_json / _to_json).

The backend's parser and writer are checked against an independent Python
writer of the same serde encoding (catnn_amd.irjson.to_serde_json), against
a hand-written fixture in serde_json's exact form (tests/golden/
mlp_ir.json: a graph as the reference's IrGraph derives would serialise
it), and for every OpenOp variant.  Host-only: no GPU needed."""
import json
import os

import numpy as np
import pytest

from catnn_amd import (CatError, CGraph, IrGraph, IrNode, OpenOp, Tensor, TensorType, configs,
                       to_serde_json)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "mlp_ir.json")


def _norm(x):
    """JSON value with every number as float32 (the tensors' precision)."""
    if isinstance(x, dict):
        return {k: _norm(v) for k, v in x.items()}
    if isinstance(x, list):
        return [_norm(v) for v in x]
    if isinstance(x, bool) or x is None or isinstance(x, str):
        return x
    return float(np.float32(x))


def _same(a_text, b_text):
    a, b = json.loads(a_text), json.loads(b_text)
    assert list(a["nodes"].keys()) == list(b["nodes"].keys())  # IndexMap order survives
    assert _norm(a) == _norm(b)


def test_golden_fixture_parses_as_serde_writes_it():
    text = open(GOLDEN).read()
    g = CGraph.from_json(text)
    out, _ = g.to_json()
    _same(out, text)
    doc = json.loads(out)
    assert doc["nodes"]["1"]["op"] == {"linear": {"in_features": 4, "out_features": 3, "bias": True}}
    assert doc["nodes"]["2"]["op"] == "relu"
    assert doc["nodes"]["1"]["params"]["b"]["data"] == [0.5, -1.25, 2.0]


def test_round_trip_matches_the_python_writer():
    w = configs.config1(batch=4)
    py, _ = to_serde_json(w.graph)
    c = CGraph.from_ir(w.graph)
    out, blob = c.to_json()
    assert blob.size == 0
    _same(out, py)
    again, _ = CGraph.from_json(out).to_json()
    assert again == out


def test_blob_carries_the_parameters():
    w = configs.config3(batch=1, seq=8, d=32, heads=2, ffn=64)
    py_inline, _ = to_serde_json(w.graph)
    py_lean, blob = to_serde_json(w.graph, inline=False)
    assert blob.size == sum(t.data.size for n in w.graph.nodes.values() for t in n.params.values())
    g = CGraph.from_json(py_lean, blob)
    out, _ = g.to_json(inline=True)
    _same(out, py_inline)
    lean, blob2 = g.to_json(inline=False)
    assert np.array_equal(blob2, blob)
    _same(lean, py_lean)


def test_every_variant_round_trips():
    ty = TensorType.f32([2, 4])
    ops = [OpenOp("identity"), OpenOp.linear(4, 4, False), OpenOp.relu(), OpenOp.gelu(), OpenOp.softmax(-1),
           OpenOp.layer_norm(3), OpenOp.add(), OpenOp.mul(), OpenOp.matmul(), OpenOp.transpose(0, 1),
           OpenOp.reshape([4, 2]), OpenOp.attention(2, 4, 2, causal=True), OpenOp.residual_add(),
           OpenOp("embedding", (100, 4)), OpenOp("rms_norm", (5,)),
           OpenOp("gqa_attention", (4, 2, 8, 32, 4096, 1000000)), OpenOp("swiglu", (4, 8)),
           OpenOp("router", (8, 2)), OpenOp.moe(8, 2, 4, 8), OpenOp("lm_head", (4, 100)),
           OpenOp("mla", (2, 3, 4, 5, 6, 7, 10000)), OpenOp("deepseek_moe", (8, 1, 2, 4, 2, 4, 8, 2500)),
           OpenOp("mix")]
    g = IrGraph("all_ops")
    for i, op in enumerate(ops):
        g.add_node(IrNode(i, f"n{i}", op, ty))
    py, _ = to_serde_json(g)
    out, _ = CGraph.from_json(py).to_json()
    _same(out, py)
    doc = json.loads(out)
    assert doc["nodes"]["8"]["op"] == "mat_mul" and doc["nodes"]["18"]["op"]["mo_e"]["top_k"] == 2
    assert doc["nodes"]["11"]["op"]["attention"]["causal"] is True
    assert doc["nodes"]["16"]["op"] == {"swi_glu": {"hidden": 4, "intermediate": 8}}
    # Option::None of the sliding window is null, as serde writes it.
    none = py.replace('"sliding_window":4096', '"sliding_window":null')
    assert json.loads(CGraph.from_json(none).to_json()[0])["nodes"]["15"]["op"]["gqa_attention"][
        "sliding_window"] is None


def test_non_finite_parameters_are_null():
    g = IrGraph("nf")
    ty = TensorType.f32([1, 3])
    g.add_node(IrNode(0, "lin", OpenOp.linear(3, 3, True), ty,
                      {"w": Tensor(TensorType.f32([3, 3]), np.eye(3)),
                       "b": Tensor(TensorType.f32([3]), [np.nan, np.inf, 1.0])}))
    py, _ = to_serde_json(g)
    assert '"data":[null,null,1.0]' in py
    out, _ = CGraph.from_json(py).to_json()
    assert json.loads(out)["nodes"]["0"]["params"]["b"]["data"][:2] == [None, None]


@pytest.mark.parametrize("text,kind", [
    ('{"name": "x", "nodes": {', "Parse"),
    ('{"name": "x", "nodes": {"0": {"id": 0, "name": "a", "op": "warp", "output_ty": '
     '{"shape": {"dims": [1]}, "dtype": "f32"}, "params": {}}}, "edges": [], "inputs": [], "outputs": []}',
     "Parse"),
    ('{"name": "x", "nodes": {"0": {"id": 0, "name": "a", "op": "identity", "output_ty": '
     '{"shape": {"dims": [1]}, "dtype": "f99"}, "params": {}}}, "edges": [], "inputs": [], "outputs": []}',
     "Parse"),
    ('{"name": "x", "nodes": {"0": {"id": 0, "name": "a", "op": "identity", "output_ty": '
     '{"shape": {"dims": [2]}, "dtype": "f32"}, "params": {"w": {"ty": {"shape": {"dims": [2]}, '
     '"dtype": "f32"}, "data": [1.0]}}}}, "edges": [], "inputs": [], "outputs": []}', "ShapeMismatch"),
])
def test_malformed_graphs_are_rejected(text, kind):
    with pytest.raises(CatError) as e:
        CGraph.from_json(text)
    assert e.value.kind == kind


def test_blob_length_must_match():
    w = configs.config1(batch=2)
    lean, blob = to_serde_json(w.graph, inline=False)
    with pytest.raises(CatError) as e:
        CGraph.from_json(lean, blob[:-1])
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(CatError) as e:
        CGraph.from_json(lean, np.concatenate([blob, [0.0]]))
    assert e.value.kind == "ShapeMismatch"
