"""ctypes binding of include/catnn_hip.h (the backend's C ABI).

The shared library is built in-tree by `make -C cat-nn-compiler_amd` (or
`__graft_entry__.build()`).  There is no fallback: importing this module
without the built library raises, and every compute call goes to the GPU.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libcatnn_hip.so")

MAX_RANK = 8
ID_CAP = 128

# Status codes (catnn_status), mapped 1:1 to CatError variants
# (crates/catnn-core/src/error.rs:9-54).
STATUS_NAMES = {
    0: "Ok", 1: "InterfaceMismatch", 2: "ShapeMismatch", 3: "DTypeMismatch",
    4: "UnknownPort", 5: "UnknownComponent", 6: "UnknownArchitecture",
    7: "UnknownRealization", 8: "Wiring", 9: "Parse", 10: "Fibration",
    11: "Witness", 12: "Descent", 13: "Interval", 14: "Unlawful", 15: "Io",
    100: "Device", 101: "Unsupported", 102: "InvalidArgument",
}


class CatError(Exception):
    """A failed backend call; `kind` names the CatError variant."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = STATUS_NAMES.get(code, f"Status{code}")
        super().__init__(f"{self.kind}: {message}")


class CTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.POINTER(ctypes.c_float)),
                ("dims", ctypes.c_int64 * MAX_RANK),
                ("rank", ctypes.c_int32),
                ("dtype", ctypes.c_int32)]


class COp(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("a", ctypes.c_int64 * 8)]


class CParam(ctypes.Structure):
    _fields_ = [("port", ctypes.c_char_p), ("value", CTensor)]


class CNode(ctypes.Structure):
    _fields_ = [("id", ctypes.c_uint32), ("name", ctypes.c_char_p), ("op", COp),
                ("output_ty", CTensor), ("params", ctypes.POINTER(CParam)),
                ("n_params", ctypes.c_int32)]


class CBufferReq(ctypes.Structure):
    _fields_ = [("id", ctypes.c_char_p), ("bytes", ctypes.c_uint64),
                ("live_from", ctypes.c_uint64), ("live_to", ctypes.c_uint64),
                ("checkpoint", ctypes.c_int32)]


class CArenaAlloc(ctypes.Structure):
    _fields_ = [("id", ctypes.c_char * ID_CAP), ("bytes", ctypes.c_uint64),
                ("offset", ctypes.c_uint64), ("live_from", ctypes.c_uint64),
                ("live_to", ctypes.c_uint64)]


class CStepTiming(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * ID_CAP), ("kind", ctypes.c_int32),
                ("calls", ctypes.c_int32), ("total_ms", ctypes.c_double)]


class CPlacementEntry(ctypes.Structure):
    _fields_ = [("op", ctypes.c_char_p), ("device", ctypes.c_char_p)]


class CClusterDevice(ctypes.Structure):
    _fields_ = [("id", ctypes.c_char_p), ("kind", ctypes.c_int32), ("arch", ctypes.c_char_p)]


class CKernelChoice(ctypes.Structure):
    _fields_ = [("op", ctypes.c_char * ID_CAP), ("backend", ctypes.c_int32)]


class CMemoryRegion(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_uint64), ("bandwidth_bps", ctypes.c_double), ("latency_s", ctypes.c_double),
                ("provenance", ctypes.c_char * 256)]


class CDeviceMemory(ctypes.Structure):
    _fields_ = [("code", CMemoryRegion), ("buffer", CMemoryRegion), ("scratch", CMemoryRegion)]


class CTrainOptions(ctypes.Structure):
    _fields_ = [("optimizer", ctypes.c_int32), ("lr", ctypes.c_float), ("precision", ctypes.c_int32),
                ("arena_cap", ctypes.c_uint64)]


class CEvent(ctypes.Structure):
    _fields_ = [("t_ns", ctypes.c_uint64), ("op", ctypes.c_char * ID_CAP),
                ("kind", ctypes.c_int32), ("checksum", ctypes.c_uint64)]


class CKernelLaunch(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 256), ("grid", ctypes.c_uint32 * 3),
                ("block", ctypes.c_uint32 * 3), ("dynamic_lds_bytes", ctypes.c_uint64),
                ("code_bytes", ctypes.c_uint64), ("vgprs", ctypes.c_uint32), ("agprs", ctypes.c_uint32),
                ("sgprs", ctypes.c_uint32), ("static_lds_bytes", ctypes.c_uint64),
                ("kernarg_bytes", ctypes.c_uint64), ("scratch_bytes_per_lane", ctypes.c_uint64)]


class CKernelResource(ctypes.Structure):
    _fields_ = [("code_bytes", ctypes.c_uint64), ("code_estimated", ctypes.c_int32),
                ("registers_per_thread", ctypes.c_uint32), ("static_smem_bytes", ctypes.c_uint64),
                ("dynamic_smem_bytes", ctypes.c_uint64), ("grid", ctypes.c_uint32 * 3),
                ("block", ctypes.c_uint32 * 3), ("launch_arg_bytes", ctypes.c_uint64),
                ("temp_bytes", ctypes.c_uint64), ("n_launches", ctypes.c_int32)]


_VP = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_PI32 = ctypes.POINTER(ctypes.c_int32)
_PU64 = ctypes.POINTER(ctypes.c_uint64)

# name → argtypes (every function returns int unless listed in _RESTYPE)
SIGNATURES = {
    "catnn_hip_last_error": [],
    "catnn_place_arena": [ctypes.POINTER(CBufferReq), _I32, _U64, ctypes.POINTER(CArenaAlloc)],
    "catnn_arena_conflict": [ctypes.POINTER(CArenaAlloc), _I32, _PI32, _PI32, _PI32],
    "catnn_graph_new": [ctypes.c_char_p, ctypes.POINTER(_VP)],
    "catnn_graph_free": [_VP],
    "catnn_graph_add_node": [_VP, ctypes.POINTER(CNode)],
    "catnn_graph_add_edge": [_VP, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_char_p, ctypes.c_char_p],
    "catnn_graph_add_input": [_VP, ctypes.c_uint32],
    "catnn_graph_add_output": [_VP, ctypes.c_uint32],
    "catnn_graph_add_fusion": [_VP, ctypes.POINTER(ctypes.c_char_p), _I32],
    "catnn_graph_topo": [_VP, ctypes.POINTER(ctypes.c_uint32), _I32, _PI32],
    "catnn_graph_from_json": [ctypes.c_char_p, _U64, ctypes.POINTER(_F), _U64, ctypes.POINTER(_VP)],
    "catnn_graph_to_json": [_VP, _I32, ctypes.c_char_p, _U64, _PU64, ctypes.POINTER(_F), _U64, _PU64],
    "catnn_tensor_lcg": [_U64, ctypes.POINTER(ctypes.c_float), _I64],
    "catnn_tensor_checksum": [ctypes.POINTER(ctypes.c_float), _I64, _PU64],
    "catnn_hip_device_count": [_PI32],
    "catnn_hip_open": [_I32, ctypes.POINTER(_VP)],
    "catnn_hip_close": [_VP],
    "catnn_hip_sync": [_VP],
    "catnn_hip_device_info": [_VP, ctypes.c_char_p, _I32, _PU64, _PI32],
    "catnn_hip_arena_reserve": [_VP, _U64],
    "catnn_hip_bind": [_VP, ctypes.c_char_p, _U64, _U64],
    "catnn_hip_buffer_ptr": [_VP, ctypes.c_char_p, ctypes.POINTER(_VP), _PU64],
    "catnn_hip_upload": [_VP, ctypes.c_char_p, _VP, _U64],
    "catnn_hip_download": [_VP, ctypes.c_char_p, _VP, _U64],
    "catnn_hip_alloc": [_VP, _U64, ctypes.POINTER(_VP)],
    "catnn_hip_free": [_VP, _VP],
    "catnn_hip_h2d": [_VP, _VP, _VP, _U64],
    "catnn_hip_d2h": [_VP, _VP, _VP, _U64],
    "catnn_hip_memset": [_VP, _VP, _I32, _U64],
    "catnn_hip_timer_start": [_VP],
    "catnn_hip_timer_stop": [_VP, ctypes.POINTER(_F)],
    "catnn_hip_describe": [ctypes.POINTER(CNode), ctypes.POINTER(CTensor), _I32, ctypes.POINTER(CKernelResource),
                           ctypes.POINTER(CKernelLaunch), _I32],
    "catnn_hip_kernel_table_size": [_PI32],
    "catnn_hip_kernel_table_entry": [_I32, ctypes.POINTER(CKernelLaunch)],
    "catnn_hip_run_kernel": [_VP, ctypes.POINTER(CNode), ctypes.POINTER(CTensor), _I32,
                             ctypes.POINTER(CTensor)],
    "catnn_hip_run_node": [_VP, ctypes.POINTER(CNode), ctypes.POINTER(ctypes.c_char_p),
                           ctypes.POINTER(CTensor), _I32, ctypes.c_char_p, _I32, ctypes.c_char_p],
    "catnn_hip_install": [_VP, _VP, ctypes.POINTER(_VP)],
    "catnn_hip_program_free": [_VP],
    "catnn_hip_forward": [_VP, ctypes.POINTER(CTensor), ctypes.POINTER(CTensor)],
    "catnn_hip_forward_resident": [_VP],
    "catnn_hip_program_check": [_VP],
    "catnn_hip_program_io": [_VP, ctypes.POINTER(_VP), _PU64, ctypes.POINTER(_VP), _PU64],
    "catnn_hip_program_arena": [_VP, ctypes.POINTER(CArenaAlloc), _I32, _PI32, _PU64],
    "catnn_hip_program_profile": [_VP, _I32],
    "catnn_hip_program_timings": [_VP, ctypes.POINTER(CStepTiming), _I32, _PI32],
    "catnn_hip_train_install": [_VP, _VP, _F, ctypes.POINTER(_VP)],
    "catnn_hip_train_install_opt": [_VP, _VP, _I32, _F, ctypes.POINTER(_VP)],
    "catnn_hip_train_install_ex": [_VP, _VP, ctypes.POINTER(CTrainOptions), ctypes.POINTER(_VP)],
    "catnn_hip_train_checkpointed": [_VP, _VP, _I32, _PI32],
    "catnn_hip_train_set_batch_classes": [_VP, ctypes.POINTER(CTensor), ctypes.POINTER(ctypes.c_uint32), _I64],
    "catnn_hip_train_read_moment": [_VP, ctypes.c_uint32, ctypes.c_char_p, _I32, ctypes.POINTER(_F), _I64],
    "catnn_hip_train_adam_step": [_VP, _PU64],
    "catnn_hip_sgd_f32": [_VP, _VP, _VP, _I64, _F],
    "catnn_hip_run_adjoint": [_VP, _VP, ctypes.POINTER(CTensor), _I32, ctypes.POINTER(CTensor),
                              ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), _I32],
    "catnn_hip_adam_f32": [_VP, _VP, _VP, _VP, _VP, _I64, ctypes.c_uint64, _F],
    "catnn_hip_train_free": [_VP],
    "catnn_hip_train_set_batch": [_VP, ctypes.POINTER(CTensor), ctypes.POINTER(CTensor)],
    "catnn_hip_train_step": [_VP, ctypes.POINTER(_F)],
    "catnn_hip_train_reset": [_VP],
    "catnn_hip_train_read_param": [_VP, ctypes.c_uint32, ctypes.c_char_p, ctypes.POINTER(_F), _I64],
    "catnn_hip_train_read_grad": [_VP, ctypes.c_uint32, ctypes.c_char_p, ctypes.POINTER(_F), _I64],
    "catnn_hip_train_read_value": [_VP, ctypes.c_uint32, ctypes.POINTER(_F), _I64],
    "catnn_hip_train_read_routing": [_VP, ctypes.c_uint32, _PI32, _I64],
    "catnn_hip_train_arena": [_VP, ctypes.POINTER(CArenaAlloc), _I32, _PI32, _PU64],
    "catnn_hip_events": [_VP, ctypes.POINTER(CEvent), _I32, _PI32],
    "catnn_hip_clear_events": [_VP],
    "catnn_hip_trace_checksums": [_VP, _I32],
    "catnn_hip_kernels_for": [_VP, ctypes.POINTER(CPlacementEntry), _I32, ctypes.POINTER(CClusterDevice), _I32,
                              ctypes.POINTER(CKernelChoice), _I32, _PI32],
    "catnn_hip_device_memory": [_VP, ctypes.POINTER(CDeviceMemory)],
    "catnn_hip_install_placed": [_VP, _VP, ctypes.POINTER(CPlacementEntry), _I32, ctypes.c_char_p, ctypes.c_char_p,
                                 ctypes.POINTER(_VP)],
    "catnn_hip_program_ports": [_VP, _VP, _I32, _PI32, _VP, _I32, _PI32],
    "catnn_hip_program_new_pass": [_VP],
    "catnn_hip_program_set_value": [_VP, ctypes.c_char_p, ctypes.POINTER(CTensor)],
    "catnn_hip_forward_wave": [_VP, _PI32],
    "catnn_hip_program_get_value": [_VP, ctypes.c_char_p, ctypes.POINTER(CTensor)],
    "catnn_hip_linear_f32": [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32],
    "catnn_hip_gemm_bf16_nt": [_VP, _VP, _I64, _VP, _I64, _VP, _I64, _I64, _I64, _I64, _I32, _I32],
    "catnn_hip_act_f32": [_VP, _VP, _VP, _I64, _I32],
    "catnn_hip_add_f32": [_VP, _VP, _VP, _VP, _I64, _I64],
    "catnn_hip_mul_f32": [_VP, _VP, _VP, _VP, _I64],
    "catnn_hip_layer_norm_f32": [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _F],
    "catnn_hip_softmax_f32": [_VP, _VP, _VP, _I64, _I64],
    "catnn_hip_attention_core_f32": [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I32],
    "catnn_hip_moe_route_f32": [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP, _VP, _VP],
    "catnn_hip_moe_permute": [_VP, _VP, _I64, _I64, _I64, _VP, _VP, _VP, _VP],
    "catnn_hip_moe_f32": [_VP, _VP, _VP, ctypes.POINTER(_VP), ctypes.POINTER(_VP),
                          ctypes.POINTER(_VP), _I64, _I64, _I64, _I64, _I64, _VP, _VP, _VP, _VP],
    "catnn_hip_moe_f32_noalloc": [_VP, _VP, _VP, ctypes.POINTER(_VP), ctypes.POINTER(_VP),
                                  ctypes.POINTER(_VP), _I64, _I64, _I64, _I64, _I64, _VP, _VP, _VP,
                                  _VP],
}

_RESTYPE = {"catnn_hip_last_error": ctypes.c_char_p}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `make -C cat-nn-compiler_amd` "
            "(or __graft_entry__.build()). There is no CPU fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    return lib


lib = _load()


def check(rc: int) -> None:
    if rc != 0:
        raise CatError(rc, lib.catnn_hip_last_error().decode(errors="replace"))
