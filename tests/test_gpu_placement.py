"""A placed graph on two devices of a cluster: the HIP stage
(catnn_hip_install_placed) on the MI355X and, for the nodes placed on the
host CPU, the oracle's eval_node standing in for the reference's CpuRust
handler.  A driver runs forward waves on both, as coord.rs:592-686 does,
shipping each value a stage's output port produces to the "#recv" port of
the device that reads it, until both are quiescent; the graph output must
match the oracle's eval_graph of the whole graph (rel L2 1e-4)."""
import numpy as np
import pytest

import oracle
from catnn_amd import CatError, PlacedProgram, Placement, Tensor, TensorType, configs, device_memory
from conftest import rel_l2

pytestmark = pytest.mark.gpu

GPU, CPU = "node0.mi355x", "node0.cpu"


class CpuStage:
    """The nodes placed on the CPU device, evaluated by the oracle."""

    def __init__(self, graph, placement, default):
        self.g = graph
        self.ids = [i for i in oracle.topo(graph) if placement.get(graph.nodes[i].name, default) == CPU]
        self.vals = {}

    def wave(self, inbox):
        fired = 0
        self.vals.update(inbox)
        for i in self.ids:
            if i in self.vals:
                continue
            preds = [e.src for e in self.g.edges if e.dst == i]
            if not all(p in self.vals for p in preds):
                continue
            self.vals[i] = oracle.eval_node(self.g.nodes[i], [self.vals[p] for p in preds])
            fired += 1
        return fired


def _run_placed(device, g, assign, default, x):
    pl = Placement(assign)
    names = {n.name: i for i, n in g.nodes.items()}
    home = lambda name: pl.get(name) or default
    stage = PlacedProgram(device, g, pl, GPU, default)
    cpu = CpuStage(g, {k: v for k, v in pl.assign.items()}, default)
    stage.new_pass()
    inp = g.nodes[g.inputs[0]]
    cpu_inbox = {}
    if home(inp.name) == GPU:
        stage.set_value(inp.name, x)
    else:
        cpu_inbox[g.inputs[0]] = x.numpy().reshape(inp.output_ty.shape)
    shipped, waves = set(), 0
    while True:
        waves += 1
        fired = stage.wave() + cpu.wave(cpu_inbox)
        cpu_inbox = {}
        # fanout: GPU output ports to the CPU, CPU values to GPU "#recv" ports
        for name in stage.outputs:
            i = names[name]
            if name in shipped:
                continue
            try:
                v = stage.get_value(name, g.nodes[i].output_ty)
            except CatError as e:
                assert e.kind == "Wiring"  # not computed yet in this pass
                continue
            shipped.add(name)
            cpu_inbox[i] = v.numpy().reshape(g.nodes[i].output_ty.shape)
            fired += 1
        for port in stage.inputs:
            if port in shipped or not port.endswith("#recv"):
                continue
            i = names[port[: -len("#recv")]]
            if i in cpu.vals:
                stage.set_value(port, Tensor.from_numpy(np.ascontiguousarray(cpu.vals[i], np.float32)))
                shipped.add(port)
                fired += 1
        if not fired:
            break
        assert waves < 50
    out = g.outputs[-1]
    name = g.nodes[out].name
    if home(name) == GPU:
        got = stage.get_value(name, g.nodes[out].output_ty).numpy()
    else:
        got = cpu.vals[out]
    stage.free()
    return np.asarray(got).reshape(g.nodes[out].output_ty.shape), stage, waves


def test_mlp_split_across_gpu_and_cpu(device):
    # fc1+act1 (fused) and fc3 on the MI355X, fc2+act2 on the CPU: the GPU
    # stage reads act2 back through its "act2#recv" port in a later wave.
    w = configs.config1(batch=64)
    g = w.graph
    assign = {"mlp.in": GPU, "fc1": GPU, "act1": GPU, "fc2": CPU, "act2": CPU, "fc3": GPU}
    got, stage, waves = _run_placed(device, g, assign, CPU, w.x)
    assert stage.inputs == ["mlp.in", "act2#recv"] and stage.outputs == ["act1", "fc3"]
    want = oracle.eval_graph(g, w.x.numpy())
    print(f"  mlp placed: {waves} waves, rel_l2 {rel_l2(got, want):.2e}")
    assert rel_l2(got, want) < 1e-4


def test_block_with_attention_on_the_gpu(device):
    # Only the attention node on the MI355X: LayerNorm's output arrives as
    # "ln1#recv"; the residual adds on the CPU read the GPU's output.
    w = configs.config3(batch=2, seq=64, d=128, heads=2, ffn=256)
    g = w.graph
    got, stage, waves = _run_placed(device, g, {"attn": GPU}, CPU, w.x)
    assert stage.inputs == ["ln1#recv"] and stage.outputs == ["attn"]
    want = oracle.eval_graph(g, w.x.numpy())
    assert rel_l2(got, want) < 1e-4
    # and the converse: everything but the LayerNorms on the GPU
    got2, stage2, _ = _run_placed(device, g, {"ln1": CPU, "ln2": CPU}, GPU, w.x)
    assert "ln1#recv" in stage2.inputs and "ln2#recv" in stage2.inputs
    assert rel_l2(got2, want) < 1e-4


def test_placed_stage_errors_and_device_profile(device):
    g = configs.config1(batch=4).graph
    with pytest.raises(CatError) as e:
        PlacedProgram(device, g, Placement(), GPU, CPU)  # nothing placed on the GPU
    assert e.value.kind == "UnknownRealization"
    st = PlacedProgram(device, g, Placement({"fc1": GPU}), GPU, CPU)
    assert st.inputs == ["mlp.in#recv"] and st.outputs == ["fc1"]
    st.new_pass()
    with pytest.raises(CatError) as e:
        st.set_value("nope", Tensor.zeros(TensorType.f32([4, 784])))
    assert e.value.kind == "UnknownPort"
    with pytest.raises(CatError) as e:
        st.get_value("fc1", TensorType.f32([4, 512]))
    assert e.value.kind == "Wiring"
    assert st.wave() == 0  # its input has not arrived
    st.set_value("mlp.in#recv", Tensor.zeros(TensorType.f32([4, 784])))
    assert st.wave() == 1 and st.wave() == 0
    assert not st.get_value("fc1", TensorType.f32([4, 512])).data.any()  # zero input, zero bias
    st.free()
    m = device_memory(device)
    assert m["buffer"].bytes > 250 * 2**30 and m["buffer"].provenance.startswith("measured")
