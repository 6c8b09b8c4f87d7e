// Memory-bound kernels: elementwise activations and adds, LayerNorm and
// softmax over the last axis.  Each streams its operands once through HBM
// with 16-byte accesses; the row kernels keep a row in registers (one
// wavefront per row) so a row costs one read and one write.
//
// Replaces cpu::relu / cpu::gelu (crates/catnn-compile/src/kernel/cpu.rs:14-29),
// cpu::softmax_last (cpu.rs:31-52), cpu::layer_norm (cpu.rs:54-78),
// cpu::add (cpu.rs:80-98) and cpu::mul (cpu.rs:100-109).
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "devmath.hpp"
#include "kernels.hpp"

namespace catnn {
namespace k {

namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n, int64_t per_thread) {
    int64_t blocks = (n + kThreads * per_thread - 1) / (kThreads * per_thread);
    if (blocks < 1) blocks = 1;
    if (blocks > (1 << 20)) blocks = 1 << 20;  // grid-stride beyond this
    return (unsigned)blocks;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__global__ void act_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t n, int act) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t n4 = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 v = reinterpret_cast<const float4 *>(x)[i];
        v.x = apply_act(v.x, act);
        v.y = apply_act(v.y, act);
        v.z = apply_act(v.z, act);
        v.w = apply_act(v.w, act);
        reinterpret_cast<float4 *>(y)[i] = v;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = apply_act(x[i], act);
}

__global__ void act_scalar_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                  int act) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = apply_act(x[i], act);
}

// y[i] = a[i] + b[i % nb]; nb == na is the same-length case.
__global__ void add_kernel(const float *__restrict__ a, const float *__restrict__ b,
                           float *__restrict__ y, int64_t na, int64_t nb) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (nb == na) {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < na; i += stride)
            y[i] = a[i] + b[i];
    } else {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < na; i += stride)
            y[i] = a[i] + b[i % nb];
    }
}

__global__ void add4_kernel(const float4 *__restrict__ a, const float4 *__restrict__ b,
                            float4 *__restrict__ y, int64_t n4) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const float4 u = a[i], v = b[i];
        y[i] = make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
    }
}

__global__ void mul_kernel(const float *__restrict__ a, const float *__restrict__ b,
                           float *__restrict__ y, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = a[i] * b[i];
}

// One wavefront per row, the row held in registers as NV float4 per lane
// (cols == 256·NV·… is not required: lanes past the end hold zeros and are
// excluded from the statistics).  (Measured against this kernel with its
// inputs read from HBM: DPP row sums with unchecked loads, 4 % slower;
// γ/β staged once per block in LDS, 8 % slower.  Both were faster only on
// inputs held in the last-level cache.  Nontemporal loads of x and stores
// of y: 11.4 -> 12.7 us in the config-3 forward, not kept.)
template <int NV>
__global__ __launch_bounds__(256) void layer_norm_reg_kernel(
    const float *__restrict__ x, const float *__restrict__ gamma, const float *__restrict__ beta,
    float *__restrict__ y, int64_t rows, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float4 *xr = reinterpret_cast<const float4 *>(x + row * cols);
    const int c4 = cols / 4;
    float4 v[NV];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        v[i] = c < c4 ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const float n = (float)cols;
    const float mean = wave_sum(s) / n;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        if (c < c4) {
            const float d0 = v[i].x - mean, d1 = v[i].y - mean, d2 = v[i].z - mean,
                        d3 = v[i].w - mean;
            q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
    }
    const float var = wave_sum(q) / n;
    const float inv = 1.0f / sqrtf(var + eps);
    const float4 *g4 = reinterpret_cast<const float4 *>(gamma);
    const float4 *b4 = reinterpret_cast<const float4 *>(beta);
    float4 *yr = reinterpret_cast<float4 *>(y + row * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        if (c < c4) {
            const float4 g = g4[c], b = b4[c];
            float4 o;
            o.x = (v[i].x - mean) * inv * g.x + b.x;
            o.y = (v[i].y - mean) * inv * g.y + b.y;
            o.z = (v[i].z - mean) * inv * g.z + b.z;
            o.w = (v[i].w - mean) * inv * g.w + b.w;
            yr[c] = o;
        }
    }
}

// Any width: one wavefront per row, three passes over the row (L2-resident
// for the row sizes that reach this path).
__global__ __launch_bounds__(256) void layer_norm_any_kernel(
    const float *__restrict__ x, const float *__restrict__ gamma, const float *__restrict__ beta,
    float *__restrict__ y, int64_t rows, int64_t cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * cols;
    float s = 0.f;
    for (int64_t c = lane; c < cols; c += 64) s += xr[c];
    const float n = (float)cols;
    const float mean = wave_sum(s) / n;
    float q = 0.f;
    for (int64_t c = lane; c < cols; c += 64) {
        const float d = xr[c] - mean;
        q += d * d;
    }
    const float var = wave_sum(q) / n;
    const float inv = 1.0f / sqrtf(var + eps);
    float *yr = y + row * cols;
    for (int64_t c = lane; c < cols; c += 64) yr[c] = (xr[c] - mean) * inv * gamma[c] + beta[c];
}

template <int NV>
__global__ __launch_bounds__(256) void softmax_reg_kernel(const float *__restrict__ x,
                                                          float *__restrict__ y, int64_t rows,
                                                          int cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float4 *xr = reinterpret_cast<const float4 *>(x + row * cols);
    const int c4 = cols / 4;
    float4 v[NV];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        v[i] = c < c4 ? xr[c] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    }
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        if (c < c4) {
            v[i].x = expf(v[i].x - m);
            v[i].y = expf(v[i].y - m);
            v[i].z = expf(v[i].z - m);
            v[i].w = expf(v[i].w - m);
            s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        }
    }
    s = wave_sum(s);
    const float inv = 1.0f / fmaxf(s, 1e-30f);
    float4 *yr = reinterpret_cast<float4 *>(y + row * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        if (c < c4) yr[c] = make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
    }
}

__global__ __launch_bounds__(256) void softmax_any_kernel(const float *__restrict__ x,
                                                          float *__restrict__ y, int64_t rows,
                                                          int64_t cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * cols;
    float *yr = y + row * cols;
    float m = -INFINITY;
    for (int64_t c = lane; c < cols; c += 64) m = fmaxf(m, xr[c]);
    m = wave_max(m);
    float s = 0.f;
    for (int64_t c = lane; c < cols; c += 64) {
        const float e = expf(xr[c] - m);
        yr[c] = e;
        s += e;
    }
    s = wave_sum(s);
    const float inv = 1.0f / fmaxf(s, 1e-30f);
    for (int64_t c = lane; c < cols; c += 64) yr[c] *= inv;
}

unsigned row_grid(int64_t rows) {
    const int64_t b = (rows + 3) / 4;
    CATNN_REQUIRE(b < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "row kernel: too many rows");
    return (unsigned)b;
}

}  // namespace

void act_f32(hipStream_t s, const float *x, float *y, int64_t n, int act) {
    CATNN_REQUIRE(act == ACT_NONE || act == ACT_RELU || act == ACT_GELU,
                  CATNN_ERR_INVALID_ARGUMENT, "act must be 0, 2 or 3");
    if (n <= 0) return;
    if (aligned16(x) && aligned16(y))
        act_kernel<<<grid_for(n, 4), kThreads, 0, s>>>(x, y, n, act);
    else
        act_scalar_kernel<<<grid_for(n, 1), kThreads, 0, s>>>(x, y, n, act);
    CATNN_HIP(hipGetLastError());
}

void add_f32(hipStream_t s, const float *a, const float *b, float *y, int64_t na, int64_t nb) {
    if (na <= 0) return;
    CATNN_REQUIRE(nb > 0, CATNN_ERR_SHAPE_MISMATCH, "add: empty rhs");
    if (nb == na && na % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(y))
        add4_kernel<<<grid_for(na, 4), kThreads, 0, s>>>(
            reinterpret_cast<const float4 *>(a), reinterpret_cast<const float4 *>(b),
            reinterpret_cast<float4 *>(y), na / 4);
    else
        add_kernel<<<grid_for(na, 1), kThreads, 0, s>>>(a, b, y, na, nb);
    CATNN_HIP(hipGetLastError());
}

void mul_f32(hipStream_t s, const float *a, const float *b, float *y, int64_t n) {
    if (n <= 0) return;
    mul_kernel<<<grid_for(n, 1), kThreads, 0, s>>>(a, b, y, n);
    CATNN_HIP(hipGetLastError());
}

void copy_f32(hipStream_t s, const float *x, float *y, int64_t n) {
    if (n <= 0 || x == y) return;
    CATNN_HIP(hipMemcpyAsync(y, x, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
}

void layer_norm_f32(hipStream_t s, const float *x, const float *gamma, const float *beta, float *y,
                    int64_t rows, int64_t cols, float eps) {
    if (rows <= 0) return;
    CATNN_REQUIRE(cols > 0, CATNN_ERR_SHAPE_MISMATCH, "layer_norm: empty rows");
    const unsigned g = row_grid(rows);
    const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y) && aligned16(gamma) &&
                     aligned16(beta);
    const int64_t nv = (cols / 4 + 63) / 64;  // float4 per lane
    if (vec && nv <= 1)
        layer_norm_reg_kernel<1><<<g, 256, 0, s>>>(x, gamma, beta, y, rows, (int)cols, eps);
    else if (vec && nv <= 2)
        layer_norm_reg_kernel<2><<<g, 256, 0, s>>>(x, gamma, beta, y, rows, (int)cols, eps);
    else if (vec && nv <= 4)
        layer_norm_reg_kernel<4><<<g, 256, 0, s>>>(x, gamma, beta, y, rows, (int)cols, eps);
    else if (vec && nv <= 8)
        layer_norm_reg_kernel<8><<<g, 256, 0, s>>>(x, gamma, beta, y, rows, (int)cols, eps);
    else if (vec && nv <= 16)
        layer_norm_reg_kernel<16><<<g, 256, 0, s>>>(x, gamma, beta, y, rows, (int)cols, eps);
    else
        layer_norm_any_kernel<<<g, 256, 0, s>>>(x, gamma, beta, y, rows, cols, eps);
    CATNN_HIP(hipGetLastError());
}

void softmax_f32(hipStream_t s, const float *x, float *y, int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0) return;
    const unsigned g = row_grid(rows);
    const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y);
    const int64_t nv = (cols / 4 + 63) / 64;
    if (vec && nv <= 1)
        softmax_reg_kernel<1><<<g, 256, 0, s>>>(x, y, rows, (int)cols);
    else if (vec && nv <= 2)
        softmax_reg_kernel<2><<<g, 256, 0, s>>>(x, y, rows, (int)cols);
    else if (vec && nv <= 4)
        softmax_reg_kernel<4><<<g, 256, 0, s>>>(x, y, rows, (int)cols);
    else if (vec && nv <= 8)
        softmax_reg_kernel<8><<<g, 256, 0, s>>>(x, y, rows, (int)cols);
    else if (vec && nv <= 16)
        softmax_reg_kernel<16><<<g, 256, 0, s>>>(x, y, rows, (int)cols);
    else
        softmax_any_kernel<<<g, 256, 0, s>>>(x, y, rows, cols);
    CATNN_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace catnn
