// Internal plumbing shared by the runtime translation units: error
// propagation across the C ABI, HIP status checks, and the device handle.
#pragma once

#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "catnn_hip.h"

namespace catnn {

// Internal failure carrying a catnn_status code; converted to a return code
// and a thread-local message at the C boundary (see guard()).
struct Failure {
    int code;
    std::string msg;
};

[[noreturn]] void fail(int code, const std::string &msg);
void set_last_error(const std::string &msg);

#define CATNN_HIP(expr)                                                            \
    do {                                                                           \
        hipError_t catnn_e_ = (expr);                                              \
        if (catnn_e_ != hipSuccess)                                                \
            ::catnn::fail(CATNN_ERR_DEVICE,                                        \
                          std::string(#expr) + ": " + hipGetErrorString(catnn_e_)); \
    } while (0)

#define CATNN_REQUIRE(cond, code, msg)                   \
    do {                                                 \
        if (!(cond)) ::catnn::fail((code), (msg));       \
    } while (0)

// Run `f` and translate a Failure (or any exception) into a status code.
template <class F>
int guard(F &&f) {
    try {
        f();
        set_last_error("");
        return CATNN_OK;
    } catch (const Failure &e) {
        set_last_error(e.msg);
        return e.code;
    } catch (const std::exception &e) {
        set_last_error(std::string("internal: ") + e.what());
        return CATNN_ERR_INVALID_ARGUMENT;
    }
}

struct Binding {
    uint64_t offset;
    uint64_t bytes;
};

// Growable device scratch owned by a device (MoE permutation buffers,
// per-slot expert outputs).  Grown with hipMalloc, never shrunk.
struct Workspace {
    void *ptr = nullptr;
    uint64_t bytes = 0;
};

}  // namespace catnn

struct catnn_adjoint_cache;  // one-node trainers kept by catnn_hip_run_adjoint (train.cpp)

struct catnn_hip_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t_start = nullptr, t_stop = nullptr;
    // Sheaf events are stamped on the device: each kernel event records a
    // hipEvent on the stream; its time is resolved when the events are read
    // (catnn_hip_events), as the previous stamp plus the device time between
    // them, starting from ev_epoch (recorded at open, host time `epoch`).
    hipEvent_t ev_epoch = nullptr, ev_last = nullptr;
    double last_ns = 0.0;
    std::vector<std::pair<size_t, hipEvent_t>> ev_pending;  // (index in events, stamp)
    std::vector<hipEvent_t> ev_pool;
    bool trace_checksums = true;  // run_node: FNV-1a of the output on KernelEnd
    catnn_adjoint_cache *adj_cache = nullptr;
    void *arena = nullptr;
    uint64_t arena_bytes = 0;
    std::unordered_map<std::string, catnn::Binding> bindings;
    std::vector<void *> allocations;
    std::vector<catnn_event> events;
    std::chrono::steady_clock::time_point epoch;
    catnn::Workspace moe_ws;
    void *noalloc_scratch = nullptr;  // device address of the fixed MoE scratch
    // Partial tiles of the bf16 GEMM's stream-K remainder (gemm_bf16.hip
    // configuration 12): one 256 × 256 fp32 tile per CU, allocated once on
    // first use and shared by every GEMM on this device's stream.
    catnn::Workspace sk_ws;
    std::string noalloc_error;
    int cu_count = 0;
};

namespace catnn {

void require_device(catnn_hip_device *dev);
// Resolve a bound arena buffer; fails with UNKNOWN_PORT naming the id.
void *buffer(catnn_hip_device *dev, const std::string &id, uint64_t *bytes = nullptr);
// Make sure dev->moe_ws holds at least `bytes`.
void *workspace(catnn_hip_device *dev, Workspace &ws, uint64_t bytes);
// Appends a sheaf event stamped by a hipEvent recorded on dev's stream now
// (the time of the work enqueued before it); returns its index in
// dev->events so that the checksum can be filled in afterwards.
size_t push_device_event(catnn_hip_device *dev, const std::string &op, int kind, uint64_t checksum);
// Waits for the pending stamps and turns them into nanoseconds.
void resolve_events(catnn_hip_device *dev);
// The one-node trainers of catnn_hip_run_adjoint, freed with the device.
void free_adjoint_cache(catnn_hip_device *dev);
uint64_t fnv1a_f32(const float *data, uint64_t n);

}  // namespace catnn
