"""The MI355X as a placement target of H (the hardware category).

`Placement` is `Placement { assign: IndexMap<String, String> }`
(crates/catnn-core/src/architecture/realization.rs:13-31); `kernels_for`
is place.rs:152-166 with the HIP arm (a Gpu device of architecture gfx950
gets KernelBackend::Hip); `device_memory` is the MI355X region profile
(the counterpart of DeviceMemory::dgx_spark, memory.rs:136-175); and
`PlacedProgram` is the stage of a placed graph that runs on this device,
driven in forward waves as crates/catnn-rt/src/coord.rs:592-686 drives a
device: values from other devices arrive on "{producer}#recv" ports, each
wave runs every local node whose inputs are present, and local values that
other devices read leave through output ports.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np

from ._lib import (CClusterDevice, CDeviceMemory, CKernelChoice, CPlacementEntry, CTensor, ID_CAP, check, lib)
from .device import Device, graph_handle
from .ir import IrGraph, Tensor, TensorType, ctensor

KERNEL_BACKENDS = ["cpu_rust", "wgsl", "reference", "cuda_sm121", "hip"]  # KernelBackend + Hip
DEVICE_KINDS = {"cpu": 0, "gpu": 1, "accel": 2}


class Placement:
    """Where each IR node lives: op name → device id, in insertion order."""

    def __init__(self, assign: Optional[Dict[str, str]] = None):
        self.assign: Dict[str, str] = dict(assign or {})

    def put(self, op: str, device: str):
        self.assign[op] = device

    def get(self, op: str) -> Optional[str]:
        return self.assign.get(op)

    def to_c(self):
        keep = [(k.encode(), v.encode()) for k, v in self.assign.items()]
        arr = (CPlacementEntry * max(len(keep), 1))(*[CPlacementEntry(k, v) for k, v in keep])
        return arr, len(keep), keep


@dataclass
class ClusterDevice:
    """A cluster device (hardware.rs:39-49): id, kind ("cpu", "gpu",
    "accel") and the GPU architecture it reports ("gfx950" for MI355X)."""
    id: str
    kind: str
    arch: str = ""


def kernels_for(graph: IrGraph, placement: Placement, devices: List[ClusterDevice]) -> List[Tuple[str, str]]:
    """`KernelChoice { op, backend }` per node in IndexMap order."""
    h, owned = graph_handle(graph)
    pa, npl, keep = placement.to_c()
    keep_dev = [(d.id.encode(), d.arch.encode()) for d in devices]
    darr = (CClusterDevice * max(len(devices), 1))(
        *[CClusterDevice(i, DEVICE_KINDS[d.kind], a) for d, (i, a) in zip(devices, keep_dev)])
    n = ctypes.c_int32()
    try:
        check(lib.catnn_hip_kernels_for(h, pa, npl, darr, len(devices), None, 0, ctypes.byref(n)))
        out = (CKernelChoice * max(n.value, 1))()
        check(lib.catnn_hip_kernels_for(h, pa, npl, darr, len(devices), out, n.value, ctypes.byref(n)))
    finally:
        if owned:
            lib.catnn_graph_free(h)
    return [(c.op.decode(), KERNEL_BACKENDS[c.backend]) for c in out[: n.value]]


@dataclass
class MemoryRegion:
    bytes: int
    bandwidth_bps: float
    latency_s: float
    provenance: str


def device_memory(device: Optional[Device] = None) -> Dict[str, MemoryRegion]:
    """The MI355X `DeviceMemory { code, buffer, scratch }`."""
    m = CDeviceMemory()
    check(lib.catnn_hip_device_memory(device.handle if device else None, ctypes.byref(m)))
    conv = lambda r: MemoryRegion(int(r.bytes), float(r.bandwidth_bps), float(r.latency_s), r.provenance.decode())
    return {"code": conv(m.code), "buffer": conv(m.buffer), "scratch": conv(m.scratch)}


class PlacedProgram:
    """This device's stage of a placed graph (catnn_hip_install_placed)."""

    def __init__(self, device: Device, graph: IrGraph, placement: Placement, device_id: str,
                 default_device: str):
        self.device = device
        self.graph = graph
        h, owned = graph_handle(graph)
        pa, npl, keep = placement.to_c()
        self.handle = ctypes.c_void_p()
        try:
            check(lib.catnn_hip_install_placed(device.handle, h, pa, npl, device_id.encode(),
                                               default_device.encode(), ctypes.byref(self.handle)))
        finally:
            if owned:
                lib.catnn_graph_free(h)
        device._adopt(self)
        ni, no = ctypes.c_int32(), ctypes.c_int32()
        check(lib.catnn_hip_program_ports(self.handle, None, 0, ctypes.byref(ni), None, 0, ctypes.byref(no)))
        ins = (ctypes.c_char * ID_CAP * max(ni.value, 1))()
        outs = (ctypes.c_char * ID_CAP * max(no.value, 1))()
        check(lib.catnn_hip_program_ports(self.handle, ins, ni.value, ctypes.byref(ni), outs, no.value,
                                          ctypes.byref(no)))
        self.inputs = [bytes(ins[i]).split(b"\0", 1)[0].decode() for i in range(ni.value)]
        self.outputs = [bytes(outs[i]).split(b"\0", 1)[0].decode() for i in range(no.value)]

    def new_pass(self):
        check(lib.catnn_hip_program_new_pass(self.handle))

    def set_value(self, name: str, value: Tensor):
        c = ctensor(value)
        check(lib.catnn_hip_program_set_value(self.handle, name.encode(), ctypes.byref(c)))

    def wave(self) -> int:
        """One forward wave; returns the number of nodes fired."""
        n = ctypes.c_int32()
        check(lib.catnn_hip_forward_wave(self.handle, ctypes.byref(n)))
        return n.value

    def get_value(self, name: str, ty: TensorType) -> Tensor:
        buf = np.empty(max(ty.numel(), 1), np.float32)
        c = ctensor(ty=ty, buf=buf)
        check(lib.catnn_hip_program_get_value(self.handle, name.encode(), ctypes.byref(c)))
        shape = tuple(c.dims[i] for i in range(c.rank))
        return Tensor(TensorType(shape, "f32"), buf[: int(np.prod(shape)) if shape else 1].copy())

    def free(self):
        if self.handle:
            check(lib.catnn_hip_program_free(self.handle))
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
