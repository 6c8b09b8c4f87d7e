"""catnn_amd — host-side API of the MI355X execution backend for catnn IR.

Mirrors the reference's names for the path it replaces (IrGraph execution
through DeviceHandler::run_kernel, crates/catnn-rt/src/handler.rs:34).
All compute goes through lib/libcatnn_hip.so; importing without the built
library raises ImportError.
"""
from ._lib import CatError, LIB_PATH, STATUS_NAMES, lib
from .arena import ArenaAlloc, BufferReq, arena_conflict, place_arena
from .device import (Device, DeviceBuffer, DeviceHandler, Program, eval_graph_hip)
from .ir import (FLAG_CAUSAL, FusionGroup, IrEdge, IrGraph, IrNode, OpenOp, Tensor, TensorType)
from .train import Trainer
from .irjson import CGraph, to_serde_json
from .describe import KernelLaunch, KernelResource, describe, kernel_table
from .placement import ClusterDevice, PlacedProgram, Placement, device_memory, kernels_for
from .spec import (Architecture, NetworkSpec, lower_architecture, mlp_spec, parse_catnn,
                   propose_fusions, to_architecture, transformer_block_spec)

__all__ = [
    "ArenaAlloc", "Architecture", "BufferReq", "CGraph", "CatError", "ClusterDevice", "Device", "DeviceBuffer",
    "DeviceHandler", "FLAG_CAUSAL", "FusionGroup", "IrEdge", "IrGraph", "IrNode", "LIB_PATH",
    "NetworkSpec", "OpenOp", "PlacedProgram", "Placement", "Program", "STATUS_NAMES", "Tensor", "TensorType",
    "Trainer", "device_memory", "kernels_for",
    "arena_conflict", "eval_graph_hip", "lib", "lower_architecture", "mlp_spec", "parse_catnn",
    "place_arena", "propose_fusions", "to_architecture", "to_serde_json", "transformer_block_spec",
]
