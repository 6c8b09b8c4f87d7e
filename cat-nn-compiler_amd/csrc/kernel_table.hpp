// Resources of every gfx950 kernel in this build, read from the code
// objects by kernel_table.py at build time (generated kernel_table.cpp).
#pragma once

#include <cstdint>

namespace catnn {

struct KernelInfo {
    const char *symbol;         // mangled kernel name
    uint64_t code_bytes;        // size of the kernel's function symbol
    uint32_t vgprs;             // unified VGPR + AGPR allocation per lane (.vgpr_count)
    uint32_t agprs, sgprs;      // the AGPR part of it; SGPRs
    uint64_t lds_static;        // group segment bytes
    uint64_t kernarg_bytes;     // kernel-argument segment bytes
    uint64_t scratch_per_lane;  // private segment bytes
    uint32_t max_workgroup;
};

extern const KernelInfo kKernelTable[];
extern const int kKernelTableSize;

}  // namespace catnn
