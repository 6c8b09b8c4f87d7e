"""describe()'s kernel table against the HIP runtime's own view of each
kernel.  The table (kernel_table(), compiled into the library) is read at
build time from this build's gfx950 code objects; the build also writes each
HIP source's code object to lib/co/.  Here those code objects are loaded with
hipModuleLoad and, for every kernel of the table, hipFuncGetAttribute must
report the same register count (the unified VGPR count, AGPRs included),
scratch bytes per lane, static LDS bytes and largest workgroup — the figures
KernelResource (crates/catnn-compile/src/kernel/resource.rs:28-45) carries.
"""
import ctypes
import glob
import os
import re

import pytest

import catnn_amd

pytestmark = pytest.mark.gpu

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "cat-nn-compiler_amd")
CO_DIR = os.path.join(PKG, "lib", "co")


def _hip_runtime():
    # The HIP runtime the library is bound to, opened by the soname it
    # needs: the dynamic loader returns the copy already in the process (a
    # process that imported torch first may hold torch's copy, and loading
    # another by path would give an uninitialised second runtime).
    with open(os.path.join(PKG, "lib", "libcatnn_hip.so"), "rb") as f:
        m = re.search(rb"libamdhip64\.so\.[0-9]+", f.read())
    return ctypes.CDLL(m.group(0).decode() if m else "libamdhip64.so")

# hipFunction_attribute (hip/driver_types.h)
MAX_THREADS_PER_BLOCK, SHARED_SIZE_BYTES, LOCAL_SIZE_BYTES, NUM_REGS = 0, 1, 3, 4


def test_kernel_table_matches_hip_func_attributes(device):
    paths = sorted(glob.glob(os.path.join(CO_DIR, "*.co")))
    assert paths, f"no code objects under {CO_DIR}: build the library (make -C cat-nn-compiler_amd)"
    hip = _hip_runtime()
    mods = []
    try:
        for p in paths:
            m = ctypes.c_void_p()
            assert hip.hipModuleLoad(ctypes.byref(m), p.encode()) == 0, p
            mods.append(m)
        rows = catnn_amd.kernel_table()
        assert len(rows) > 50
        for r in rows:
            found = []
            for m in mods:
                f = ctypes.c_void_p()
                if hip.hipModuleGetFunction(ctypes.byref(f), m, r.kernel.encode()) == 0:
                    found.append(f)
                else:
                    hip.hipGetLastError()  # a miss in this module: clear it, later launches check the error state
            assert len(found) == 1, (r.kernel, len(found))

            def attr(a):
                v = ctypes.c_int()
                assert hip.hipFuncGetAttribute(ctypes.byref(v), a, found[0]) == 0, (r.kernel, a)
                return v.value

            got = (attr(NUM_REGS), attr(LOCAL_SIZE_BYTES), attr(SHARED_SIZE_BYTES), attr(MAX_THREADS_PER_BLOCK))
            want = (r.vgprs, r.scratch_bytes_per_lane, r.static_lds_bytes, r.block[0])
            assert got == want, (r.kernel, got, want)
    finally:
        for m in mods:
            hip.hipModuleUnload(m)
        hip.hipGetLastError()
