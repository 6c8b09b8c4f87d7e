"""The placement target on the host (no GPU): kernels_for with the HIP arm
(place.rs:152-166 plus KernelBackend::Hip for gfx950 devices) and the
MI355X region profile of H without a device."""
import numpy as np

from catnn_amd import ClusterDevice, Placement, configs, device_memory, kernel_table, kernels_for

DEVICES = [ClusterDevice("node0.cpu", "cpu"), ClusterDevice("node0.mi355x", "gpu", "gfx950"),
           ClusterDevice("node1.gpu", "gpu"), ClusterDevice("node1.npu", "accel")]


def test_kernels_for_maps_each_node_to_its_devices_backend():
    g = configs.config1(batch=4).graph
    pl = Placement({"mlp.in": "node0.cpu", "fc1": "node0.mi355x", "act1": "node0.mi355x", "fc2": "node1.gpu",
                    "act2": "node1.npu", "fc3": "nowhere"})
    got = kernels_for(g, pl, DEVICES)
    assert got == [("mlp.in", "cpu_rust"), ("fc1", "hip"), ("act1", "hip"), ("fc2", "wgsl"), ("act2", "wgsl"),
                   ("fc3", "cpu_rust")]
    # an unplaced node falls back to the CPU backend, as kind None does in the reference
    assert kernels_for(g, Placement(), DEVICES)[1] == ("fc1", "cpu_rust")
    # a later entry for the same op replaces the earlier one (IndexMap::insert)
    pl.put("fc1", "node0.cpu")
    assert kernels_for(g, pl, DEVICES)[1] == ("fc1", "cpu_rust")


def test_mi355x_region_profile_without_a_device():
    m = device_memory()
    assert m["buffer"].bytes == 288 * 10**9 and m["buffer"].bandwidth_bps == 8e12
    assert m["scratch"].bytes == 160 * 1024
    assert m["code"].bytes == sum(k.code_bytes for k in kernel_table()) > 0
    assert m["code"].provenance.startswith("measured") and m["buffer"].provenance.startswith("cited")
