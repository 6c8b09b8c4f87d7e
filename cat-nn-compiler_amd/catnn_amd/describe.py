"""describe(): the kernels a node runs on gfx950 and their resources.

The counterpart of `kernel::resource::describe`
(crates/catnn-compile/src/kernel/resource.rs:155-186) for the HIP backend.
The reference estimates CUDA code sizes and registers when nvcc is absent;
here every figure comes from this build's gfx950 code objects (read at
build time by kernel_table.py), and the launch geometry is the one the
backend's launchers choose for the given input types.  Host-only: no GPU.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Sequence, Tuple

from ._lib import CKernelLaunch, CKernelResource, CTensor, check, lib
from .ir import IrNode, TensorType, ctensor


@dataclass
class KernelLaunch:
    kernel: str
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    dynamic_lds_bytes: int
    code_bytes: int
    vgprs: int
    agprs: int
    sgprs: int
    static_lds_bytes: int
    kernarg_bytes: int
    scratch_bytes_per_lane: int


@dataclass
class KernelResource:
    """KernelResource (resource.rs:28-45) of one node; `launches` lists every
    kernel launch it makes, in order."""
    name: str
    backend: str
    code_bytes: int
    code_estimated: bool
    code_note: str
    registers_per_thread: int
    static_smem_bytes: int
    dynamic_smem_bytes: int
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    launch_arg_bytes: int
    temp_bytes: int
    launches: List[KernelLaunch] = field(default_factory=list)

    def scratch_bytes(self) -> int:
        """KernelResource::scratch_bytes (resource.rs:49-55): LDS plus the
        register file of one workgroup."""
        threads = self.block[0] * self.block[1] * self.block[2]
        return self.static_smem_bytes + self.dynamic_smem_bytes + self.registers_per_thread * 4 * threads

    def code_footprint(self) -> int:
        return self.code_bytes + self.launch_arg_bytes


def _launch(c: CKernelLaunch) -> KernelLaunch:
    return KernelLaunch(c.kernel.decode(), tuple(c.grid), tuple(c.block), c.dynamic_lds_bytes, c.code_bytes,
                        c.vgprs, c.agprs, c.sgprs, c.static_lds_bytes, c.kernarg_bytes, c.scratch_bytes_per_lane)


def describe(node: IrNode, in_types: Sequence[TensorType]) -> KernelResource:
    cnode, keep = node.to_c(with_data=False)
    cins = (CTensor * max(len(in_types), 1))(*[ctensor(ty=t) for t in in_types])
    out = CKernelResource()
    cap = 16
    launches = (CKernelLaunch * cap)()
    check(lib.catnn_hip_describe(ctypes.byref(cnode), cins, len(in_types), ctypes.byref(out), launches, cap))
    n = out.n_launches
    if n > cap:
        launches = (CKernelLaunch * n)()
        check(lib.catnn_hip_describe(ctypes.byref(cnode), cins, len(in_types), ctypes.byref(out), launches, n))
    del keep
    return KernelResource(
        node.name, "hip_gfx950", out.code_bytes, bool(out.code_estimated),
        f"read from this build's gfx950 code objects: {n} launch(es)", out.registers_per_thread,
        out.static_smem_bytes, out.dynamic_smem_bytes, tuple(out.grid), tuple(out.block), out.launch_arg_bytes,
        out.temp_bytes, [_launch(launches[i]) for i in range(n)])


def kernel_table() -> List[KernelLaunch]:
    """Every kernel of the build with its resources (block[0]: the largest
    workgroup it accepts)."""
    n = ctypes.c_int32()
    check(lib.catnn_hip_kernel_table_size(ctypes.byref(n)))
    rows = []
    for i in range(n.value):
        c = CKernelLaunch()
        check(lib.catnn_hip_kernel_table_entry(i, ctypes.byref(c)))
        rows.append(_launch(c))
    return rows
