"""Host-side checks that need no GPU: the C-ABI library loads and exports
every function include/catnn_hip.h declares, and the host logic behind it
(graph order, arena planning, spec lowering, Tensor helpers) matches the
oracle and the reference's own tests."""
import ctypes
import os
import re

import numpy as np
import pytest

import catnn_amd
import oracle
from catnn_amd import (BufferReq, CatError, IrGraph, IrNode, OpenOp, Tensor, TensorType,
                       place_arena, arena_conflict)
from catnn_amd._lib import SIGNATURES

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "catnn_hip.h")
GOLDEN = os.path.join(ROOT, "tests", "golden")
RNG = np.random.default_rng(7)


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(catnn_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(catnn_amd.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    assert sorted(SIGNATURES) == declared_functions()


def test_open_without_gpu_fails_loudly():
    if catnn_amd.Device.count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(CatError) as e:
        catnn_amd.Device(0)
    assert e.value.kind == "Device"
    assert "no CPU fallback" in str(e.value)


@pytest.mark.parametrize("seed", [0, 1, 42, 1009 * 3 + 17])
def test_tensor_lcg_and_checksum_match_oracle(seed):
    t = Tensor.lcg(TensorType.f32([3, 37]), seed)
    assert np.array_equal(t.data, oracle.lcg(111, seed))
    assert t.checksum() == oracle.checksum(t.data)


def _graph(edges, n):
    g = IrGraph("g")
    for i in range(n):
        g.add_node(IrNode(i, f"n{i}", OpenOp.relu(), TensorType.f32([1])))
    for s, d in edges:
        g.add_edge(s, d)
    return g


def test_topo_reference_chain_and_random_dags_match_oracle():
    assert _graph([(0, 1)], 2).topo() == [0, 1]
    for _ in range(50):
        n = int(RNG.integers(2, 12))
        edges = [(int(a), int(b)) for a in range(n) for b in range(a + 1, n) if RNG.random() < 0.3]
        perm = RNG.permutation(n)  # ids not in topological order
        edges = [(int(perm[a]), int(perm[b])) for a, b in edges]
        g = _graph(edges, n)
        order = g.topo()
        assert order == oracle.topo(g)
        pos = {v: i for i, v in enumerate(order)}
        assert all(pos[s] < pos[d] for s, d in edges)


def test_topo_rejects_cycles():
    with pytest.raises(CatError) as e:
        _graph([(0, 1), (1, 0)], 2).topo()
    assert e.value.kind == "Wiring"


def test_place_arena_reference_cases():
    a = place_arena([BufferReq("a", 8, 0, 1), BufferReq("b", 8, 2, 3)], 8)
    assert [x.offset for x in a] == [0, 0]
    assert arena_conflict(a) is None
    with pytest.raises(CatError) as e:
        place_arena([BufferReq("x", 8, 0, 2), BufferReq("y", 8, 1, 3)], 8)
    assert e.value.kind == "Fibration" and "y" in str(e.value)
    bad = [catnn_amd.ArenaAlloc("a", 8, 0, 0, 2), catnn_amd.ArenaAlloc("b", 8, 4, 1, 3)]
    assert arena_conflict(bad) == ("a", "b")


def test_place_arena_matches_oracle_on_random_requests():
    for _ in range(200):
        n = int(RNG.integers(1, 30))
        reqs = []
        for i in range(n):
            a = int(RNG.integers(0, 12))
            reqs.append(BufferReq(f"b{i}", int(RNG.integers(1, 1 << 20)), a, a + int(RNG.integers(0, 6))))
        got = place_arena(reqs, 1 << 40)
        off, order = oracle.place_arena([(r.bytes, r.live_from, r.live_to) for r in reqs], 1 << 40)
        assert [x.id for x in got] == [reqs[i].id for i in order]
        by_id = {x.id: x.offset for x in got}
        assert [by_id[r.id] for r in reqs] == off.tolist()
        assert arena_conflict(got) is None


def test_parse_catnn_example_and_lowering():
    # examples/mlp.catnn, the fixture of crates/catnn-rt/tests/e2e.rs:8-17
    src = open(os.path.join(GOLDEN, "mlp.catnn")).read()
    spec = catnn_amd.parse_catnn(src)
    assert (spec.name, spec.batch, len(spec.layers)) == ("mlp", 4, 3)
    g = catnn_amd.lower_architecture(catnn_amd.to_architecture(spec))
    assert list(g.nodes) == [0, 1, 2, 3] and g.inputs == [0] and g.outputs == [3]
    assert g.nodes[0].output_ty == TensorType.f32([4, 16])
    # params materialised with Tensor::lcg at seed id*1009 + 17 + port index
    assert np.array_equal(g.nodes[1].params["w"].data, oracle.lcg(16 * 32, 1 * 1009 + 17))
    assert np.array_equal(g.nodes[3].params["b"].data, oracle.lcg(8, 3 * 1009 + 18))
    fus = catnn_amd.propose_fusions(g)
    assert [f.ops for f in fus] == [["fc1", "act"]]


def test_parse_catnn_errors():
    with pytest.raises(CatError) as e:
        catnn_amd.parse_catnn("network x\nfrobnicate y\n")
    assert e.value.kind == "Parse"
    with pytest.raises(CatError) as e:
        catnn_amd.to_architecture(catnn_amd.parse_catnn("network x batch 2\nlinear a 4 8\nlinear b 3 3\n"))
    assert e.value.kind == "ShapeMismatch"


def test_transformer_example_lowers():
    src = open(os.path.join(GOLDEN, "transformer.catnn")).read()
    g = catnn_amd.lower_architecture(catnn_amd.to_architecture(catnn_amd.parse_catnn(src)))
    kinds = [n.op.kind for n in g.nodes.values()]
    assert kinds == ["identity", "attention", "layer_norm", "linear", "gelu", "linear", "layer_norm"]
    assert g.nodes[1].op.fields == (4, 16, 4)
    assert g.nodes[2].op.fields == (1,)


def test_config_builders_flops_match_the_survey():
    from catnn_amd import configs

    assert configs.config1().flops == 342_360_064
    assert configs.attention_flops(8, 1024, 16, 64, True) == 2 * 8_598_323_200
    # config 2 and 4 full sizes are large: check the formulas on the shapes.
    assert 2 * 8192 * 4096 * 16384 * 2 == 2_199_023_255_552
    assert 2 * 16384 * 1024 * 8 + 16384 * 2 * 2 * 3 * 1024 * 3584 == 721_822_941_184
