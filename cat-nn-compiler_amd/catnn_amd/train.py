"""One training step of an IrGraph on the GPU (catnn_hip_train_*).

`Trainer.step()` replaces one step of pipeline::reference_train
(crates/catnn-compile/src/pipeline.rs:476-547) with MSE and the optimizer
TrainOptions.opt names (OptimizerKind, crates/catnn-core/src/lens/optim.rs:
142-145): forward, loss, reverse-topo adjoints, then Sgd::put or Adam::put
on the fp32 master weights.  GEMM operands are
bf16 (bf16 MFMA, fp32 accumulation) at precision "bf16", six-part split
(fp32-accurate) at precision "fp32"; masters, residual stream, norms, router
and gradient accumulation are fp32.
"""
from __future__ import annotations

import ctypes
from typing import List, Tuple

import numpy as np

from ._lib import CArenaAlloc, CTrainOptions, ID_CAP, check, lib
from .arena import ArenaAlloc
from .device import Device, graph_handle
from .ir import IrGraph, Tensor, ctensor

_FP = ctypes.POINTER(ctypes.c_float)

OPTIMIZERS = {"sgd": 0, "adam": 1}  # CATNN_OPT_SGD, CATNN_OPT_ADAM
PRECISIONS = {"bf16": 0, "fp32": 1}  # CATNN_PREC_BF16, CATNN_PREC_FP32


class Trainer:
    def __init__(self, device: Device, graph: IrGraph, lr: float = 0.05, opt: str = "sgd",
                 precision: str = "bf16", arena_cap: int = 0):
        """`opt` is OptimizerKind::parse's spelling: "sgd" or "adam".
        `precision` "bf16": bf16 MFMA GEMM operands (mixed precision);
        "fp32": every GEMM on six-part split operands, fp32-accurate.
        `arena_cap` (bytes, 0: the device's memory): activations are
        checkpointed and recomputed when the plan misses it."""
        if opt not in OPTIMIZERS:
            raise ValueError(f"unknown optimizer {opt!r} (expected sgd or adam)")
        if precision not in PRECISIONS:
            raise ValueError(f"unknown precision {precision!r} (expected bf16 or fp32)")
        self.device = device
        self.graph = graph
        self.lr = lr
        self.opt = opt
        self.precision = precision
        h, owned = graph_handle(graph)
        self.handle = ctypes.c_void_p()
        try:
            o = CTrainOptions(OPTIMIZERS[opt], lr, PRECISIONS[precision], int(arena_cap))
            check(lib.catnn_hip_train_install_ex(device.handle, h, ctypes.byref(o), ctypes.byref(self.handle)))
        finally:
            if owned:
                lib.catnn_graph_free(h)
        device._adopt(self)

    def set_batch(self, x: Tensor, target: Tensor):
        cx, ct = ctensor(x), ctensor(target)
        check(lib.catnn_hip_train_set_batch(self.handle, ctypes.byref(cx), ctypes.byref(ct)))

    def set_batch_classes(self, x: Tensor, ids):
        """The batch of a graph whose output is an LmHead: one class id per
        output row (TrainTarget::Classes, pipeline.rs:430-441)."""
        cx = ctensor(x)
        a = np.ascontiguousarray(np.asarray(ids).reshape(-1), np.uint32)
        check(lib.catnn_hip_train_set_batch_classes(self.handle, ctypes.byref(cx),
                                                    a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), a.size))

    def step(self, sync: bool = True):
        """One step; returns the loss (before the update) when `sync`."""
        if not sync:
            check(lib.catnn_hip_train_step(self.handle, None))
            return None
        loss = ctypes.c_float()
        check(lib.catnn_hip_train_step(self.handle, ctypes.byref(loss)))
        return float(loss.value)

    def reset(self):
        """Restore every parameter to its installed value (asynchronous)."""
        check(lib.catnn_hip_train_reset(self.handle))

    def _read(self, fn, node_id: int, port: str, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        check(fn(self.handle, node_id, port.encode(), out.ctypes.data_as(_FP), out.size))
        return out

    def param(self, node_id: int, port: str, shape) -> np.ndarray:
        return self._read(lib.catnn_hip_train_read_param, node_id, port, shape)

    def grad(self, node_id: int, port: str, shape) -> np.ndarray:
        return self._read(lib.catnn_hip_train_read_grad, node_id, port, shape)

    def moment(self, node_id: int, port: str, which: str, shape) -> np.ndarray:
        """Adam's first ("m") or second ("v") moment of a parameter."""
        out = np.empty(shape, np.float32)
        check(lib.catnn_hip_train_read_moment(self.handle, node_id, port.encode(), {"m": 0, "v": 1}[which],
                                              out.ctypes.data_as(_FP), out.size))
        return out

    def adam_step(self) -> int:
        """AdamState.t: Adam steps taken since install or reset."""
        t = ctypes.c_uint64()
        check(lib.catnn_hip_train_adam_step(self.handle, ctypes.byref(t)))
        return int(t.value)

    def value(self, node_id: int, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        check(lib.catnn_hip_train_read_value(self.handle, node_id, out.ctypes.data_as(_FP), out.size))
        return out

    def routing(self, node_id: int, tokens: int, top_k: int) -> np.ndarray:
        out = np.empty((tokens, top_k), np.int32)
        check(lib.catnn_hip_train_read_routing(self.handle, node_id,
                                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                               out.size))
        return out

    def arena(self) -> Tuple[List[ArenaAlloc], int]:
        n = ctypes.c_int32()
        reserved = ctypes.c_uint64()
        check(lib.catnn_hip_train_arena(self.handle, None, 0, ctypes.byref(n), ctypes.byref(reserved)))
        buf = (CArenaAlloc * max(n.value, 1))()
        check(lib.catnn_hip_train_arena(self.handle, buf, n.value, ctypes.byref(n), ctypes.byref(reserved)))
        return ([ArenaAlloc(a.id.decode(), a.bytes, a.offset, a.live_from, a.live_to)
                 for a in buf[: n.value]], reserved.value)

    def checkpointed(self) -> List[str]:
        """The activations the plan checkpoints ("act:{node id}")."""
        n = ctypes.c_int32()
        check(lib.catnn_hip_train_checkpointed(self.handle, None, 0, ctypes.byref(n)))
        buf = (ctypes.c_char * ID_CAP * max(n.value, 1))()
        check(lib.catnn_hip_train_checkpointed(self.handle, buf, n.value, ctypes.byref(n)))
        return [bytes(buf[i]).split(b"\0", 1)[0].decode() for i in range(n.value)]

    def free(self):
        if self.handle:
            check(lib.catnn_hip_train_free(self.handle))
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
