"""The GPU device, the handler seam and installed programs.

  * `Device`        — one HIP device and its stream (catnn_hip_open).
  * `DeviceBuffer`  — device memory owned by a Device (plumbing for tests
                      and benchmarks).
  * `DeviceHandler` — mirror of crates/catnn-rt/src/handler.rs:14-92:
                      `run_kernel(node, inputs) -> Tensor` executes the node
                      on the GPU and records the same KernelStart/KernelEnd
                      events (with the output checksum) the reference
                      appends to its sheaf section.
  * `Program`       — an IrGraph installed on a device: arena planned with
                      place_arena, one hipMalloc, params uploaded once;
                      `forward` replaces eval_graph_cpu (crates/catnn-compile/src/lib.rs:48-68).
"""
from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from ._lib import CArenaAlloc, CEvent, CStepTiming, CTensor, check, lib
from .arena import ArenaAlloc
from .ir import IrGraph, IrNode, OP_KINDS, Tensor, TensorType, ctensor

VP = ctypes.c_void_p


class Device:
    def __init__(self, ordinal: int = 0):
        self.handle = VP()
        check(lib.catnn_hip_open(ordinal, ctypes.byref(self.handle)))
        self.ordinal = ordinal
        # Programs, trainers and buffers hold the device handle: close() frees
        # them first so none outlives it.
        self._owned = weakref.WeakSet()

    def _adopt(self, obj):
        self._owned.add(obj)

    @staticmethod
    def count() -> int:
        n = ctypes.c_int32()
        check(lib.catnn_hip_device_count(ctypes.byref(n)))
        return n.value

    def info(self) -> Tuple[str, int, int]:
        name = ctypes.create_string_buffer(256)
        hbm = ctypes.c_uint64()
        cus = ctypes.c_int32()
        check(lib.catnn_hip_device_info(self.handle, name, 256, ctypes.byref(hbm), ctypes.byref(cus)))
        return name.value.decode(), hbm.value, cus.value

    def sync(self):
        check(lib.catnn_hip_sync(self.handle))

    def close(self):
        if self.handle:
            for obj in list(self._owned):
                obj.free()
            check(lib.catnn_hip_close(self.handle))
            self.handle = VP()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- memory -------------------------------------------------------------
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def put(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, arr.nbytes)
        b.upload(arr)
        return b

    # -- timing (hipEvents on the device's stream) --------------------------
    def timer_start(self):
        check(lib.catnn_hip_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        check(lib.catnn_hip_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    # -- sheaf events ---------------------------------------------------------
    def events(self) -> List[Tuple[int, str, int, int]]:
        n = ctypes.c_int32()
        check(lib.catnn_hip_events(self.handle, None, 0, ctypes.byref(n)))
        buf = (CEvent * max(n.value, 1))()
        check(lib.catnn_hip_events(self.handle, buf, n.value, ctypes.byref(n)))
        return [(e.t_ns, e.op.decode(), e.kind, e.checksum) for e in buf[: n.value]]

    def clear_events(self):
        check(lib.catnn_hip_clear_events(self.handle))

    def trace_checksums(self, enable: bool):
        """Whether run_node's KernelEnd event carries the output's FNV-1a
        checksum (a device-to-host copy and a sync per node; on by default)."""
        check(lib.catnn_hip_trace_checksums(self.handle, int(bool(enable))))

    # -- the device arena (buffer-id API) -------------------------------------
    def arena_reserve(self, nbytes: int):
        check(lib.catnn_hip_arena_reserve(self.handle, nbytes))

    def bind(self, buffer_id: str, offset: int, nbytes: int):
        check(lib.catnn_hip_bind(self.handle, buffer_id.encode(), offset, nbytes))

    def upload(self, buffer_id: str, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        check(lib.catnn_hip_upload(self.handle, buffer_id.encode(), arr.ctypes.data_as(VP), arr.nbytes))

    def download(self, buffer_id: str, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(lib.catnn_hip_download(self.handle, buffer_id.encode(), out.ctypes.data_as(VP), out.nbytes))
        return out

    def buffer_ptr(self, buffer_id: str) -> Tuple[int, int]:
        p = VP()
        n = ctypes.c_uint64()
        check(lib.catnn_hip_buffer_ptr(self.handle, buffer_id.encode(), ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value


class DeviceBuffer:
    """hipMalloc'd memory freed with its owner or by `free()`."""

    def __init__(self, dev: Device, nbytes: int):
        self.dev = dev
        self.nbytes = int(nbytes)
        self.ptr = VP()
        check(lib.catnn_hip_alloc(dev.handle, max(self.nbytes, 4), ctypes.byref(self.ptr)))
        dev._adopt(self)

    def upload(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, "upload larger than the buffer"
        check(lib.catnn_hip_h2d(self.dev.handle, self.ptr, arr.ctypes.data_as(VP), arr.nbytes))

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes, "download larger than the buffer"
        check(lib.catnn_hip_d2h(self.dev.handle, out.ctypes.data_as(VP), self.ptr, out.nbytes))
        return out

    def zero(self):
        check(lib.catnn_hip_memset(self.dev.handle, self.ptr, 0, self.nbytes))

    def free(self):
        if self.ptr:
            check(lib.catnn_hip_free(self.dev.handle, self.ptr))
            self.ptr = VP()

    @property
    def p(self):
        return self.ptr


def _ptr(b) -> Optional[VP]:
    if b is None:
        return None
    if isinstance(b, DeviceBuffer):
        return b.ptr
    return VP(int(b))


class DeviceHandler:
    """handler.rs:14-92 on the GPU: one per device."""

    def __init__(self, device: Device):
        self.device = device

    def run_kernel(self, node: IrNode, inputs: Sequence[Tensor]) -> Tensor:
        cnode, keep = node.to_c()
        cins = (CTensor * max(len(inputs), 1))(*[ctensor(t) for t in inputs])
        # The output buffer: sized by the node's declared type, or by the
        # first input when larger (pass-through ops keep their input's type).
        cap = max([node.output_ty.numel()] + [t.ty.numel() for t in inputs] + [1])
        buf = np.empty(cap, np.float32)
        out = CTensor()
        out.data = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        out.dims[0] = cap
        out.rank = 1
        check(lib.catnn_hip_run_kernel(self.device.handle, ctypes.byref(cnode), cins, len(inputs),
                                       ctypes.byref(out)))
        shape = tuple(out.dims[i] for i in range(out.rank))
        ty = TensorType(shape, "f32")
        return Tensor(ty, buf[: ty.numel()].copy())

    def adjoint_of(self, node: IrNode, inputs: Sequence[Tensor], output: Optional[Tensor],
                   dy: Tensor) -> Tuple[List[Tensor], Dict[str, Tensor]]:
        """adjoint_of (crates/catnn-compile/src/kernel/adjoint.rs:762-951) on
        the GPU: (cotangent per input, {port: parameter cotangent}) in the
        node's param order.  `output` is recomputed on the device and may be
        None.  GEMMs on bf16 MFMA with fp32 accumulation, as the training step."""
        cnode, keep = node.to_c()
        cins = (CTensor * max(len(inputs), 1))(*[ctensor(t) for t in inputs])
        dxs = [np.empty(max(t.ty.numel(), 1), np.float32) for t in inputs]
        cdx = (CTensor * max(len(inputs), 1))(*[ctensor(ty=t.ty, buf=b) for t, b in zip(inputs, dxs)])
        ports = list(node.params)
        dps = [np.empty(max(node.params[p].ty.numel(), 1), np.float32) for p in ports]
        cdp = (CTensor * max(len(ports), 1))(*[ctensor(ty=node.params[p].ty, buf=b) for p, b in zip(ports, dps)])
        cdy = ctensor(dy)
        check(lib.catnn_hip_run_adjoint(self.device.handle, ctypes.byref(cnode), cins, len(inputs), None,
                                        ctypes.byref(cdy), cdx, cdp, len(ports)))
        dx = [Tensor(t.ty, b[: t.ty.numel()].copy()) for t, b in zip(inputs, dxs)]
        dp = {p: Tensor(node.params[p].ty, b[: node.params[p].ty.numel()].copy()) for p, b in zip(ports, dps)}
        return dx, dp

    def events(self):
        return self.device.events()


def graph_handle(graph):
    """(catnn_graph handle, whether the caller frees it) for an IrGraph or
    a backend-held graph (irjson.CGraph)."""
    if hasattr(graph, "handle") and not isinstance(graph, IrGraph):
        return graph.handle, False
    return graph.to_c(), True


@dataclass
class ProgramIO:
    in_ptr: int
    in_bytes: int
    out_ptr: int
    out_bytes: int


class Program:
    """An IrGraph installed on a device (catnn_hip_install)."""

    def __init__(self, device: Device, graph: IrGraph):
        self.device = device
        self.graph = graph
        self.out_ty: Optional[TensorType] = None
        h, owned = graph_handle(graph)
        self.handle = VP()
        try:
            check(lib.catnn_hip_install(device.handle, h, ctypes.byref(self.handle)))
        finally:
            if owned:
                lib.catnn_graph_free(h)
        device._adopt(self)

    def forward(self, x: Optional[Tensor]) -> Tensor:
        io = self.io()
        buf = np.empty(max(io.out_bytes // 4, 1), np.float32)
        out = CTensor()
        out.data = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        out.dims[0] = buf.size
        out.rank = 1
        cin = ctensor(x) if x is not None else None
        check(lib.catnn_hip_forward(self.handle, ctypes.byref(cin) if cin is not None else None,
                                    ctypes.byref(out)))
        shape = tuple(out.dims[i] for i in range(out.rank))
        ty = TensorType(shape, "f32")
        return Tensor(ty, buf[: ty.numel()].copy())

    def forward_resident(self):
        check(lib.catnn_hip_forward_resident(self.handle))

    def check(self):
        """Wait for the enqueued forwards; ShapeMismatch if one met a token
        id ≥ vocab (catnn_hip_program_check)."""
        check(lib.catnn_hip_program_check(self.handle))

    def io(self) -> ProgramIO:
        ip, op = VP(), VP()
        ib, ob = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib.catnn_hip_program_io(self.handle, ctypes.byref(ip), ctypes.byref(ib),
                                       ctypes.byref(op), ctypes.byref(ob)))
        return ProgramIO(ip.value or 0, ib.value, op.value or 0, ob.value)

    def arena(self) -> Tuple[List[ArenaAlloc], int]:
        n = ctypes.c_int32()
        reserved = ctypes.c_uint64()
        check(lib.catnn_hip_program_arena(self.handle, None, 0, ctypes.byref(n), ctypes.byref(reserved)))
        buf = (CArenaAlloc * max(n.value, 1))()
        check(lib.catnn_hip_program_arena(self.handle, buf, n.value, ctypes.byref(n), ctypes.byref(reserved)))
        return ([ArenaAlloc(a.id.decode(), a.bytes, a.offset, a.live_from, a.live_to)
                 for a in buf[: n.value]], reserved.value)

    def profile(self, enable: bool = True):
        """Record device time per executed step on later forwards."""
        check(lib.catnn_hip_program_profile(self.handle, int(enable)))

    def timings(self) -> List[Tuple[str, str, int, float]]:
        """(node name, op kind, timed calls, summed device ms) per step."""
        n = ctypes.c_int32()
        check(lib.catnn_hip_program_timings(self.handle, None, 0, ctypes.byref(n)))
        buf = (CStepTiming * max(n.value, 1))()
        check(lib.catnn_hip_program_timings(self.handle, buf, n.value, ctypes.byref(n)))
        return [(t.name.decode(), OP_KINDS[t.kind], t.calls, t.total_ms) for t in buf[: n.value]]

    def free(self):
        if self.handle:
            check(lib.catnn_hip_program_free(self.handle))
            self.handle = VP()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def eval_graph_hip(graph: IrGraph, x: Tensor, device: Device) -> Tensor:
    """`eval_graph_cpu` (lib.rs:48-68) executed on the GPU: `x` is bound to
    every graph input; returns the last output."""
    prog = Program(device, graph)
    try:
        return prog.forward(x)
    finally:
        prog.free()


# -------------------------------------------------------- raw kernels
# Thin wrappers over the device-pointer entry points; buffers are
# DeviceBuffer or raw device addresses.  They launch on the device stream
# and return without synchronising.

def linear(dev: Device, x, w, b, r, y, m: int, k: int, n: int, act: int = 0):
    check(lib.catnn_hip_linear_f32(dev.handle, _ptr(x), _ptr(w), _ptr(b), _ptr(r), _ptr(y),
                                   m, k, n, act))


def gemm_bf16_nt(dev: Device, a, lda: int, b, ldb: int, c, ldc: int, m: int, n: int, k: int,
                 accumulate: bool = False, tile_cfg: int = -1):
    """c (+)= a·bᵀ with a [m, k], b [n, k] bf16 bit patterns (uint16)."""
    check(lib.catnn_hip_gemm_bf16_nt(dev.handle, _ptr(a), lda, _ptr(b), ldb, _ptr(c), ldc, m, n, k,
                                     int(accumulate), tile_cfg))


def sgd(dev: Device, p, g, n: int, lr: float):
    """Sgd::put in place on n values (apply_update, pipeline.rs:455-472)."""
    check(lib.catnn_hip_sgd_f32(dev.handle, _ptr(p), _ptr(g), n, lr))


def adam(dev: Device, p, g, m, v, n: int, t: int, lr: float):
    """Adam::put in place on n values; `t` is AdamState.t before the step."""
    check(lib.catnn_hip_adam_f32(dev.handle, _ptr(p), _ptr(g), _ptr(m), _ptr(v), n, t, lr))


def act(dev: Device, x, y, n: int, kind: int):
    check(lib.catnn_hip_act_f32(dev.handle, _ptr(x), _ptr(y), n, kind))


def add(dev: Device, a, b, y, na: int, nb: int):
    check(lib.catnn_hip_add_f32(dev.handle, _ptr(a), _ptr(b), _ptr(y), na, nb))


def layer_norm(dev: Device, x, g, b, y, rows: int, cols: int, eps: float):
    check(lib.catnn_hip_layer_norm_f32(dev.handle, _ptr(x), _ptr(g), _ptr(b), _ptr(y), rows, cols, eps))


def softmax(dev: Device, x, y, rows: int, cols: int):
    check(lib.catnn_hip_softmax_f32(dev.handle, _ptr(x), _ptr(y), rows, cols))


def attention_core(dev: Device, q, k, v, ctx, batch: int, seq: int, d_model: int, n_heads: int,
                   d_head: int, causal: bool):
    check(lib.catnn_hip_attention_core_f32(dev.handle, _ptr(q), _ptr(k), _ptr(v), _ptr(ctx), batch,
                                           seq, d_model, n_heads, d_head, int(causal)))


def moe_route(dev: Device, x, gate, tokens: int, hidden: int, n_experts: int, top_k: int,
              idx=None, w=None, logits=None):
    check(lib.catnn_hip_moe_route_f32(dev.handle, _ptr(x), _ptr(gate), tokens, hidden, n_experts,
                                      top_k, _ptr(idx), _ptr(w), _ptr(logits)))


def moe_permute(dev: Device, idx, tokens: int, top_k: int, n_experts: int, counts, offsets,
                slot_of_pos, pos_of_slot):
    check(lib.catnn_hip_moe_permute(dev.handle, _ptr(idx), tokens, top_k, n_experts, _ptr(counts),
                                    _ptr(offsets), _ptr(slot_of_pos), _ptr(pos_of_slot)))


def moe(dev: Device, x, gate, w1s, w3s, w2s, tokens: int, hidden: int, intermediate: int,
        n_experts: int, top_k: int, out, idx=None, w=None, counts=None):
    arr = lambda bs: (VP * len(bs))(*[_ptr(b) for b in bs])
    check(lib.catnn_hip_moe_f32(dev.handle, _ptr(x), _ptr(gate), arr(w1s), arr(w3s), arr(w2s),
                                tokens, hidden, intermediate, n_experts, top_k, _ptr(out),
                                _ptr(idx), _ptr(w), _ptr(counts)))


# Size of the fixed device scratch behind moe_noalloc (CATNN_MOE_NOALLOC_SCRATCH_BYTES).
MOE_NOALLOC_SCRATCH_BYTES = 128 << 20


def moe_noalloc(dev: Device, x, gate, w1s, w3s, w2s, tokens: int, hidden: int, intermediate: int,
                n_experts: int, top_k: int, out, idx=None, w=None, counts=None):
    """`moe` without any device allocation: the workspace is the library's
    fixed per-GPU scratch (catnn_hip_moe_f32_noalloc).  Calls that overlap
    on one GPU race on that scratch."""
    arr = lambda bs: (VP * len(bs))(*[_ptr(b) for b in bs])
    check(lib.catnn_hip_moe_f32_noalloc(dev.handle, _ptr(x), _ptr(gate), arr(w1s), arr(w3s),
                                        arr(w2s), tokens, hidden, intermediate, n_experts, top_k,
                                        _ptr(out), _ptr(idx), _ptr(w), _ptr(counts)))
