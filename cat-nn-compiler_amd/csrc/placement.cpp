// The MI355X as a placement target of H: the HIP arm of kernels_for
// (crates/catnn-compile/src/place.rs:152-166) and the device's region
// profile (the counterpart of DeviceMemory::dgx_spark,
// crates/catnn-core/src/architecture/memory.rs:136-175).  The stage of a
// placed graph that runs here is built in graph.cpp
// (catnn_hip_install_placed).
#include <hip/hip_runtime_api.h>

#include <cstring>
#include <map>
#include <string>

#include "common.hpp"
#include "graph.hpp"
#include "kernel_table.hpp"

namespace catnn {
namespace {

// Published gfx950 / MI355X figures.
constexpr uint64_t kHbmBytes = 288ull * 1000 * 1000 * 1000;  // 288 GB HBM3E
constexpr double kHbmBandwidth = 8.0e12;                      // 8 TB/s
constexpr uint64_t kLdsPerCu = 160 * 1024;                    // LDS per CU

void set_region(catnn_memory_region &r, uint64_t bytes, double bw, double lat, const std::string &prov) {
    r.bytes = bytes;
    r.bandwidth_bps = bw;
    r.latency_s = lat;
    std::memset(r.provenance, 0, sizeof(r.provenance));
    std::strncpy(r.provenance, prov.c_str(), sizeof(r.provenance) - 1);
}

}  // namespace
}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_hip_kernels_for(const catnn_graph *g, const catnn_placement_entry *assign, int32_t n_assign,
                          const catnn_cluster_device *devices, int32_t n_devices, catnn_kernel_choice *out,
                          int32_t cap, int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(g && n && (assign || n_assign == 0) && (devices || n_devices == 0),
                      CATNN_ERR_INVALID_ARGUMENT, "null argument");
        std::map<std::string, std::string> where;
        for (int32_t i = 0; i < n_assign; ++i) {
            CATNN_REQUIRE(assign[i].op && assign[i].device, CATNN_ERR_INVALID_ARGUMENT, "null placement entry");
            where[assign[i].op] = assign[i].device;
        }
        int32_t k = 0;
        for (uint32_t id : g->node_order) {
            const Node &node = g->node(id);
            int32_t backend = CATNN_BACKEND_CPU_RUST;
            auto it = where.find(node.name);
            if (it != where.end()) {
                for (int32_t d = 0; d < n_devices; ++d) {
                    if (!devices[d].id || it->second != devices[d].id) continue;
                    const int32_t kind = devices[d].kind;
                    if (kind == CATNN_DEVICE_GPU && devices[d].arch && std::strcmp(devices[d].arch, "gfx950") == 0)
                        backend = CATNN_BACKEND_HIP;
                    else if (kind == CATNN_DEVICE_GPU || kind == CATNN_DEVICE_ACCELERATOR)
                        backend = CATNN_BACKEND_WGSL;
                    break;  // Cluster::find_device: the first device with the id
                }
            }
            if (out && k < cap) {
                std::memset(out[k].op, 0, CATNN_ID_CAP);
                std::strncpy(out[k].op, node.name.c_str(), CATNN_ID_CAP - 1);
                out[k].backend = backend;
            }
            ++k;
        }
        *n = k;
    });
}

int catnn_hip_device_memory(catnn_hip_device *dev, catnn_device_memory *out) {
    return guard([&] {
        CATNN_REQUIRE(out, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        uint64_t code = 0;
        for (int i = 0; i < kKernelTableSize; ++i) code += kKernelTable[i].code_bytes;
        set_region(out->code, code, kHbmBandwidth, 1e-6,
                   "measured: the gfx950 kernels of this library (" + std::to_string(kKernelTableSize) +
                       " code objects' function symbols), fetched from HBM3E");
        uint64_t hbm = kHbmBytes;
        std::string prov = "cited: AMD Instinct MI355X, 288 GB HBM3E at 8 TB/s";
        if (dev) {
            require_device(dev);
            hipDeviceProp_t prop;
            CATNN_HIP(hipGetDeviceProperties(&prop, dev->ordinal));
            hbm = prop.totalGlobalMem;
            prov = "measured: the device's reported HBM3E size; 8 TB/s cited (AMD Instinct MI355X)";
        }
        set_region(out->buffer, hbm, kHbmBandwidth, 1e-6, prov);
        set_region(out->scratch, kLdsPerCu, 128.0 * 2.4e9, 1e-8,
                   "cited: 160 KiB LDS per CU on gfx950 (the workgroup-shared scratch of a kernel); bandwidth "
                   "128 B/clk per CU at 2.4 GHz");
    });
}

}  // extern "C"
