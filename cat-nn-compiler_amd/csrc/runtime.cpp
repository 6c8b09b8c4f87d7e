// Device lifecycle, the HBM arena, host↔device transfers, timing and the
// per-device event log.  This is the device side of the handler that
// crates/catnn-rt/src/handler.rs:14-92 models on the host: one handle per
// device, one in-order stream, events timestamped in ns from open.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace catnn {

namespace {
thread_local std::string g_last_error;
}

void fail(int code, const std::string &msg) { throw Failure{code, msg}; }

void set_last_error(const std::string &msg) { g_last_error = msg; }

void require_device(catnn_hip_device *dev) {
    CATNN_REQUIRE(dev != nullptr, CATNN_ERR_INVALID_ARGUMENT, "null device handle");
    CATNN_HIP(hipSetDevice(dev->ordinal));
}

void *buffer(catnn_hip_device *dev, const std::string &id, uint64_t *bytes) {
    auto it = dev->bindings.find(id);
    if (it == dev->bindings.end())
        fail(CATNN_ERR_UNKNOWN_PORT, "unknown port " + id + " on interface arena");
    if (bytes) *bytes = it->second.bytes;
    return static_cast<char *>(dev->arena) + it->second.offset;
}

void *workspace(catnn_hip_device *dev, Workspace &ws, uint64_t bytes) {
    if (ws.bytes >= bytes && ws.ptr) return ws.ptr;
    if (ws.ptr) {
        CATNN_HIP(hipStreamSynchronize(dev->stream));
        CATNN_HIP(hipFree(ws.ptr));
        ws.ptr = nullptr;
        ws.bytes = 0;
    }
    CATNN_HIP(hipMalloc(&ws.ptr, bytes));
    ws.bytes = bytes;
    return ws.ptr;
}

size_t push_device_event(catnn_hip_device *dev, const std::string &op, int kind, uint64_t checksum) {
    hipEvent_t ev = nullptr;
    if (!dev->ev_pool.empty()) {
        ev = dev->ev_pool.back();
        dev->ev_pool.pop_back();
    } else {
        CATNN_HIP(hipEventCreate(&ev));
    }
    hipError_t e = hipEventRecord(ev, dev->stream);
    if (e != hipSuccess) {
        dev->ev_pool.push_back(ev);
        fail(CATNN_ERR_DEVICE, std::string("hipEventRecord: ") + hipGetErrorString(e));
    }
    catnn_event rec{};
    std::strncpy(rec.op, op.c_str(), CATNN_ID_CAP - 1);
    rec.kind = kind;
    rec.checksum = checksum;
    dev->events.push_back(rec);
    dev->ev_pending.emplace_back(dev->events.size() - 1, ev);
    return dev->events.size() - 1;
}

void resolve_events(catnn_hip_device *dev) {
    // Stamps complete in stream order; each adds the device time since the
    // previous one, so long runs keep sub-microsecond spacing.
    for (auto &pe : dev->ev_pending) {
        CATNN_HIP(hipEventSynchronize(pe.second));
        float ms = 0.f;
        CATNN_HIP(hipEventElapsedTime(&ms, dev->ev_last ? dev->ev_last : dev->ev_epoch, pe.second));
        dev->last_ns += (double)ms * 1e6;
        if (dev->ev_last) dev->ev_pool.push_back(dev->ev_last);
        dev->ev_last = pe.second;
        uint64_t t = (uint64_t)std::llround(std::max(0.0, dev->last_ns));
        const size_t i = pe.first;
        if (i > 0 && t <= dev->events[i - 1].t_ns) t = dev->events[i - 1].t_ns + 1;  // handler.rs:47
        dev->events[i].t_ns = t;
    }
    dev->ev_pending.clear();
}

// FNV-1a over the f32 bit patterns, one 32-bit word per step, as
// Tensor::checksum (crates/catnn-core/src/tensor.rs:279-288).
uint64_t fnv1a_f32(const float *data, uint64_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t bits;
        std::memcpy(&bits, data + i, 4);
        h ^= (uint64_t)bits;
        h *= 0x100000001b3ull;
    }
    return h;
}

}  // namespace catnn

using namespace catnn;

extern "C" {

const char *catnn_hip_last_error(void) { return g_last_error.c_str(); }

// Tensor::lcg, crates/catnn-core/src/tensor.rs:259-268: state = max(seed, 1);
// per element state = state·6364136223846793005 + 1 (mod 2^64), value =
// f32(u32(state >> 33)) / f32(u32::MAX) · 2 − 1.
int catnn_tensor_lcg(uint64_t seed, float *out, int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(n >= 0 && (out || n == 0), CATNN_ERR_INVALID_ARGUMENT, "lcg: null output");
        uint64_t state = seed < 1 ? 1 : seed;
        for (int64_t i = 0; i < n; ++i) {
            state = state * 6364136223846793005ull + 1ull;
            const float unit = (float)(uint32_t)(state >> 33) / (float)UINT32_MAX;
            out[i] = unit * 2.0f - 1.0f;
        }
    });
}

int catnn_tensor_checksum(const float *data, int64_t n, uint64_t *out) {
    return guard([&] {
        CATNN_REQUIRE(out && n >= 0 && (data || n == 0), CATNN_ERR_INVALID_ARGUMENT,
                      "checksum: null argument");
        *out = fnv1a_f32(data, (uint64_t)n);
    });
}

int catnn_hip_device_count(int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(n, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        int c = 0;
        hipError_t e = hipGetDeviceCount(&c);
        *n = (e == hipSuccess) ? c : 0;
    });
}

int catnn_hip_open(int32_t ordinal, catnn_hip_device **out) {
    return guard([&] {
        CATNN_REQUIRE(out, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        *out = nullptr;
        int count = 0;
        hipError_t e = hipGetDeviceCount(&count);
        if (e != hipSuccess || count == 0)
            fail(CATNN_ERR_DEVICE, "no HIP device available (hipGetDeviceCount: " +
                                       std::string(hipGetErrorString(e)) +
                                       "); this backend has no CPU fallback");
        CATNN_REQUIRE(ordinal >= 0 && ordinal < count, CATNN_ERR_DEVICE,
                      "device ordinal " + std::to_string(ordinal) + " out of range");
        auto *dev = new catnn_hip_device();
        dev->ordinal = ordinal;
        dev->epoch = std::chrono::steady_clock::now();
        try {
            CATNN_HIP(hipSetDevice(ordinal));
            CATNN_HIP(hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking));
            CATNN_HIP(hipEventCreate(&dev->t_start));
            CATNN_HIP(hipEventCreate(&dev->t_stop));
            hipDeviceProp_t prop;
            CATNN_HIP(hipGetDeviceProperties(&prop, ordinal));
            dev->cu_count = prop.multiProcessorCount;
            dev->noalloc_scratch = k::moe_noalloc_scratch(ordinal, &dev->noalloc_error);
            CATNN_HIP(hipEventCreate(&dev->ev_epoch));
            CATNN_HIP(hipEventRecord(dev->ev_epoch, dev->stream));
            CATNN_HIP(hipEventSynchronize(dev->ev_epoch));
            dev->epoch = std::chrono::steady_clock::now();
        } catch (...) {
            delete dev;
            throw;
        }
        *out = dev;
    });
}

int catnn_hip_close(catnn_hip_device *dev) {
    return guard([&] {
        if (!dev) return;
        // Best effort: a failure here leaves nothing the caller can retry.
        (void)hipSetDevice(dev->ordinal);
        if (dev->stream) (void)hipStreamSynchronize(dev->stream);
        free_adjoint_cache(dev);
        for (auto &pe : dev->ev_pending) (void)hipEventDestroy(pe.second);
        for (hipEvent_t ev : dev->ev_pool) (void)hipEventDestroy(ev);
        if (dev->ev_last) (void)hipEventDestroy(dev->ev_last);
        if (dev->ev_epoch) (void)hipEventDestroy(dev->ev_epoch);
        for (void *p : dev->allocations) (void)hipFree(p);
        if (dev->arena) (void)hipFree(dev->arena);
        if (dev->moe_ws.ptr) (void)hipFree(dev->moe_ws.ptr);
        if (dev->sk_ws.ptr) (void)hipFree(dev->sk_ws.ptr);
        if (dev->t_start) (void)hipEventDestroy(dev->t_start);
        if (dev->t_stop) (void)hipEventDestroy(dev->t_stop);
        if (dev->stream) (void)hipStreamDestroy(dev->stream);
        delete dev;
    });
}

int catnn_hip_sync(catnn_hip_device *dev) {
    return guard([&] {
        require_device(dev);
        CATNN_HIP(hipStreamSynchronize(dev->stream));
    });
}

int catnn_hip_device_info(catnn_hip_device *dev, char *name, int32_t cap, uint64_t *hbm_bytes,
                          int32_t *cu_count) {
    return guard([&] {
        require_device(dev);
        hipDeviceProp_t prop;
        CATNN_HIP(hipGetDeviceProperties(&prop, dev->ordinal));
        if (name && cap > 0) {
            std::string s = std::string(prop.name) + " (" + prop.gcnArchName + ")";
            std::strncpy(name, s.c_str(), (size_t)cap - 1);
            name[cap - 1] = 0;
        }
        if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
        if (cu_count) *cu_count = prop.multiProcessorCount;
    });
}

int catnn_hip_arena_reserve(catnn_hip_device *dev, uint64_t bytes) {
    return guard([&] {
        require_device(dev);
        CATNN_HIP(hipStreamSynchronize(dev->stream));
        if (dev->arena) {
            CATNN_HIP(hipFree(dev->arena));
            dev->arena = nullptr;
            dev->arena_bytes = 0;
        }
        dev->bindings.clear();
        if (bytes == 0) return;
        hipError_t e = hipMalloc(&dev->arena, bytes);
        if (e != hipSuccess) {
            dev->arena = nullptr;
            fail(CATNN_ERR_FIBRATION, "buffer arena: hipMalloc of " + std::to_string(bytes) +
                                          " B failed (" + hipGetErrorString(e) + ")");
        }
        dev->arena_bytes = bytes;
    });
}

int catnn_hip_bind(catnn_hip_device *dev, const char *buffer_id, uint64_t offset, uint64_t bytes) {
    return guard([&] {
        CATNN_REQUIRE(dev && buffer_id, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        CATNN_REQUIRE(dev->arena, CATNN_ERR_FIBRATION, "bind before arena_reserve");
        CATNN_REQUIRE(offset + bytes <= dev->arena_bytes && offset + bytes >= offset,
                      CATNN_ERR_FIBRATION,
                      std::string("buffer arena overflow: ") + buffer_id + " at " +
                          std::to_string(offset) + "+" + std::to_string(bytes) + " (cap " +
                          std::to_string(dev->arena_bytes) + ")");
        dev->bindings[buffer_id] = Binding{offset, bytes};
    });
}

int catnn_hip_buffer_ptr(catnn_hip_device *dev, const char *buffer_id, void **dptr,
                         uint64_t *bytes) {
    return guard([&] {
        CATNN_REQUIRE(dev && buffer_id && dptr, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *dptr = buffer(dev, buffer_id, bytes);
    });
}

int catnn_hip_upload(catnn_hip_device *dev, const char *buffer_id, const void *host,
                     uint64_t bytes) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(buffer_id && (host || bytes == 0), CATNN_ERR_INVALID_ARGUMENT,
                      "null argument");
        uint64_t cap = 0;
        void *d = buffer(dev, buffer_id, &cap);
        CATNN_REQUIRE(bytes <= cap, CATNN_ERR_SHAPE_MISMATCH,
                      std::string("upload of ") + std::to_string(bytes) + " B into " + buffer_id +
                          " of " + std::to_string(cap) + " B");
        if (bytes == 0) return;
        CATNN_HIP(hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
    });
}

int catnn_hip_download(catnn_hip_device *dev, const char *buffer_id, void *host, uint64_t bytes) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(buffer_id && (host || bytes == 0), CATNN_ERR_INVALID_ARGUMENT,
                      "null argument");
        uint64_t cap = 0;
        void *d = buffer(dev, buffer_id, &cap);
        CATNN_REQUIRE(bytes <= cap, CATNN_ERR_SHAPE_MISMATCH,
                      std::string("download of ") + std::to_string(bytes) + " B from " +
                          buffer_id + " of " + std::to_string(cap) + " B");
        if (bytes == 0) return;
        CATNN_HIP(hipMemcpyAsync(host, d, bytes, hipMemcpyDeviceToHost, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
    });
}

int catnn_hip_alloc(catnn_hip_device *dev, uint64_t bytes, void **dptr) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(dptr, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        *dptr = nullptr;
        void *p = nullptr;
        CATNN_HIP(hipMalloc(&p, bytes ? bytes : 1));
        dev->allocations.push_back(p);
        *dptr = p;
    });
}

int catnn_hip_free(catnn_hip_device *dev, void *dptr) {
    return guard([&] {
        require_device(dev);
        for (size_t i = 0; i < dev->allocations.size(); ++i) {
            if (dev->allocations[i] == dptr) {
                CATNN_HIP(hipStreamSynchronize(dev->stream));
                CATNN_HIP(hipFree(dptr));
                dev->allocations.erase(dev->allocations.begin() + (long)i);
                return;
            }
        }
        fail(CATNN_ERR_INVALID_ARGUMENT, "pointer was not allocated by catnn_hip_alloc");
    });
}

int catnn_hip_h2d(catnn_hip_device *dev, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        require_device(dev);
        if (bytes == 0) return;
        CATNN_REQUIRE(dst && src, CATNN_ERR_INVALID_ARGUMENT, "null pointer");
        CATNN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
    });
}

int catnn_hip_d2h(catnn_hip_device *dev, void *dst, const void *src, uint64_t bytes) {
    return guard([&] {
        require_device(dev);
        if (bytes == 0) return;
        CATNN_REQUIRE(dst && src, CATNN_ERR_INVALID_ARGUMENT, "null pointer");
        CATNN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
    });
}

int catnn_hip_memset(catnn_hip_device *dev, void *dst, int32_t value, uint64_t bytes) {
    return guard([&] {
        require_device(dev);
        if (bytes == 0) return;
        CATNN_REQUIRE(dst, CATNN_ERR_INVALID_ARGUMENT, "null pointer");
        CATNN_HIP(hipMemsetAsync(dst, value, bytes, dev->stream));
    });
}

int catnn_hip_timer_start(catnn_hip_device *dev) {
    return guard([&] {
        require_device(dev);
        CATNN_HIP(hipEventRecord(dev->t_start, dev->stream));
    });
}

int catnn_hip_timer_stop(catnn_hip_device *dev, float *ms) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(ms, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        CATNN_HIP(hipEventRecord(dev->t_stop, dev->stream));
        CATNN_HIP(hipEventSynchronize(dev->t_stop));
        CATNN_HIP(hipEventElapsedTime(ms, dev->t_start, dev->t_stop));
    });
}

int catnn_hip_events(catnn_hip_device *dev, catnn_event *buf, int32_t cap, int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(dev && n, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(dev);
        resolve_events(dev);
        const int32_t total = (int32_t)dev->events.size();
        *n = total;
        if (!buf) return;
        for (int32_t i = 0; i < total && i < cap; ++i) buf[i] = dev->events[(size_t)i];
    });
}

int catnn_hip_clear_events(catnn_hip_device *dev) {
    return guard([&] {
        CATNN_REQUIRE(dev, CATNN_ERR_INVALID_ARGUMENT, "null device handle");
        require_device(dev);
        resolve_events(dev);  // keeps the chain of stamps for the next events
        dev->events.clear();
    });
}

int catnn_hip_trace_checksums(catnn_hip_device *dev, int32_t enable) {
    return guard([&] {
        CATNN_REQUIRE(dev, CATNN_ERR_INVALID_ARGUMENT, "null device handle");
        dev->trace_checksums = enable != 0;
    });
}

// ---------------------------------------------------------------- kernels

int catnn_hip_linear_f32(catnn_hip_device *dev, const float *x, const float *w, const float *b,
                         const float *r, float *y, int64_t m, int64_t k, int64_t n, int32_t act) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(m >= 0 && k >= 0 && n >= 0, CATNN_ERR_SHAPE_MISMATCH, "linear: negative dims");
        CATNN_REQUIRE((x && w && y) || m * n == 0, CATNN_ERR_INVALID_ARGUMENT,
                      "linear: null operand");
        k::linear_f32(dev->stream, x, k, w, n, b, r, n, y, n, m, k, n, act);
    });
}

int catnn_hip_act_f32(catnn_hip_device *dev, const float *x, float *y, int64_t n, int32_t act) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((x && y) || n == 0, CATNN_ERR_INVALID_ARGUMENT, "act: null operand");
        k::act_f32(dev->stream, x, y, n, act);
    });
}

int catnn_hip_add_f32(catnn_hip_device *dev, const float *a, const float *b, float *y, int64_t na,
                      int64_t nb) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((a && b && y) || na == 0, CATNN_ERR_INVALID_ARGUMENT, "add: null operand");
        CATNN_REQUIRE(nb == na || (nb > 0 && na % nb == 0), CATNN_ERR_SHAPE_MISMATCH,
                      "add " + std::to_string(na) + " vs " + std::to_string(nb));
        k::add_f32(dev->stream, a, b, y, na, nb);
    });
}

int catnn_hip_mul_f32(catnn_hip_device *dev, const float *a, const float *b, float *y, int64_t n) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((a && b && y) || n == 0, CATNN_ERR_INVALID_ARGUMENT, "mul: null operand");
        k::mul_f32(dev->stream, a, b, y, n);
    });
}

int catnn_hip_layer_norm_f32(catnn_hip_device *dev, const float *x, const float *gamma,
                             const float *beta, float *y, int64_t rows, int64_t cols, float eps) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((x && gamma && beta && y) || rows == 0, CATNN_ERR_INVALID_ARGUMENT,
                      "layer_norm: null operand");
        k::layer_norm_f32(dev->stream, x, gamma, beta, y, rows, cols, eps);
    });
}

int catnn_hip_softmax_f32(catnn_hip_device *dev, const float *x, float *y, int64_t rows,
                          int64_t cols) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((x && y) || rows == 0, CATNN_ERR_INVALID_ARGUMENT, "softmax: null operand");
        k::softmax_f32(dev->stream, x, y, rows, cols);
    });
}

}  // extern "C"
