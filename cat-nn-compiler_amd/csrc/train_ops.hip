// Memory-bound kernels of the training step: casts and transposes for the
// bf16 GEMM operands, LayerNorm with saved statistics and its adjoint,
// activation adjoints, bias-gradient column sums, MSE, SGD with the bf16
// weight refresh, and the MoE/router adjoint pieces.  All reductions are
// two-stage with a fixed order (no floating-point atomics), so a training
// step is run-to-run identical.
//
// Adjoints restate crates/catnn-compile/src/kernel/adjoint.rs:
// relu_backward :63-74, gelu_backward :76-90, mse_loss :106-119,
// layer_norm_backward :530-577, router_backward_ste :255-284, the token
// loop of moe_backward :471-526; SGD is Sgd::put (lens/optim.rs:32-42).
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "devmath.hpp"
#include "kernels.hpp"
#include "train_ops.hpp"

namespace catnn {
namespace k {

namespace {

__device__ __forceinline__ bf16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
    return (bf16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

unsigned blocks_for(int64_t n, int per_block) {
    int64_t b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > (1 << 20)) b = 1 << 20;
    return (unsigned)b;
}

__global__ void fill_kernel(float *__restrict__ y, float v, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = v;
}

__global__ void fill_bf16_kernel(bf16_t *__restrict__ y, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = 0;
}

__global__ void cast_kernel(const float *__restrict__ x, bf16_t *__restrict__ y, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = f2bf(x[i]);
}

__device__ __forceinline__ uint2 pack4(bf16_t a, bf16_t b, bf16_t c, bf16_t d) {
    return make_uint2(a | (uint32_t)b << 16, c | (uint32_t)d << 16);
}

// The same four elements a thread: 16-byte loads, 8-byte stores.
__global__ void cast4_kernel(const float4 *__restrict__ x, uint2 *__restrict__ y, int64_t n4) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const float4 v = x[i];
        y[i] = pack4(f2bf(v.x), f2bf(v.y), f2bf(v.z), f2bf(v.w));
    }
}

// dst[c][r] = src[map(r)][c] for r < rows (map(r) = rows_map[r] / div when
// given; a negative map entry is a padding row and yields 0), c < cols.
// 64×64 tiles through LDS so both the read and the write are coalesced.
template <typename TS>
__global__ __launch_bounds__(256) void transpose_kernel(const TS *__restrict__ src, int64_t lds,
                                                        const int32_t *__restrict__ rows_map,
                                                        int div, int rows, int cols,
                                                        bf16_t *__restrict__ dst, int64_t ldd) {
    __shared__ bf16_t t[64][66];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int r = r0 + i, c = c0 + tx;
        bf16_t v = 0;
        if (r < rows && c < cols) {
            int sr = r;
            if (rows_map) {
                const int m = rows_map[r];
                sr = m < 0 ? -1 : m / div;
            }
            if (sr >= 0) {
                if constexpr (sizeof(TS) == 4) v = f2bf(src[(int64_t)sr * lds + c]);
                else v = src[(int64_t)sr * lds + c];
            }
        }
        t[i][tx] = v;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) dst[(int64_t)c * ldd + r] = t[tx][i];
    }
}

// The same transpose for full 64×64 tiles with 16-byte global accesses.
// Each thread reads 16-byte runs of source rows (8 bf16 or 4 f32) into an
// LDS tile of 64-element rows whose 16-byte chunk c of row i sits at
// position c ^ (i/8 mod 8).  Then 8 lanes gather the 8 chunks of one
// destination row: lane k takes source rows 8k … 8k+7 of column oc (chunk
// (oc/8) ^ k of each, so a wavefront's reads fall on distinct banks) and
// the 8 lanes store one contiguous 128-byte run.  Launched only where the
// host has checked alignment; edge tiles take the element path.  (128-row
// tiles, 256-byte destination runs with every load issued before the LDS
// writes, measured the same in the config-5 step: 279 against 277 us for
// its 12 transposes; not kept.)
template <typename TS>
__global__ __launch_bounds__(256) void transpose_vec_kernel(const TS *__restrict__ src, int64_t lds,
                                                            const int32_t *__restrict__ rows_map, int div,
                                                            int rows, int cols, bf16_t *__restrict__ dst,
                                                            int64_t ldd) {
    constexpr int VPL = 16 / sizeof(TS);  // source values per 16-byte load
    __shared__ __align__(16) bf16_t t[64 * 66];  // swizzled 64 × 64, or 64 rows of 66 on edge tiles
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tid = threadIdx.x;
    if (r0 + 64 > rows || c0 + 64 > cols) {
        // edge tile: element path
        const int tx = tid & 63, ty = tid >> 6;
        for (int i = ty; i < 64; i += 4) {
            const int r = r0 + i, c = c0 + tx;
            bf16_t v = 0;
            if (r < rows && c < cols) {
                const int sr = rows_map ? (rows_map[r] < 0 ? -1 : rows_map[r] / div) : r;
                if (sr >= 0) {
                    if constexpr (sizeof(TS) == 4) v = f2bf(src[(int64_t)sr * lds + c]);
                    else v = src[(int64_t)sr * lds + c];
                }
            }
            t[i * 66 + tx] = v;
        }
        __syncthreads();
        for (int i = ty; i < 64; i += 4) {
            const int c = c0 + i, r = r0 + tx;
            if (c < cols && r < rows) dst[(int64_t)c * ldd + r] = t[tx * 66 + i];
        }
        return;
    }
    // element (i, c) of the tile
    auto at = [](int i, int c) { return i * 64 + ((((c >> 3) ^ (i >> 3)) & 7) << 3) + (c & 7); };
    constexpr int PER_ROW = 64 / VPL;
#pragma unroll
    for (int j = 0; j < 64 * PER_ROW / 256; ++j) {
        const int idx = tid + 256 * j, i = idx / PER_ROW, cc = (idx % PER_ROW) * VPL;
        const int r = r0 + i;
        const int sr = rows_map ? (rows_map[r] < 0 ? -1 : rows_map[r] / div) : r;
        uint4 w = make_uint4(0, 0, 0, 0);
        if (sr >= 0) w = *reinterpret_cast<const uint4 *>(src + (int64_t)sr * lds + c0 + cc);
        if constexpr (sizeof(TS) == 4) {
            const uint32_t lo = (uint32_t)f2bf(__uint_as_float(w.x)) | ((uint32_t)f2bf(__uint_as_float(w.y)) << 16);
            const uint32_t hi = (uint32_t)f2bf(__uint_as_float(w.z)) | ((uint32_t)f2bf(__uint_as_float(w.w)) << 16);
            *reinterpret_cast<uint2 *>(&t[at(i, cc)]) = make_uint2(lo, hi);
        } else {
            *reinterpret_cast<uint4 *>(&t[at(i, cc)]) = w;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int item = tid + 256 * j, k = item & 7, oc = item >> 3;  // source rows 8k … 8k+7, column oc
        uint32_t u[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
            u[m] = (uint32_t)t[at(8 * k + 2 * m, oc)] | ((uint32_t)t[at(8 * k + 2 * m + 1, oc)] << 16);
        *reinterpret_cast<uint4 *>(dst + (int64_t)(c0 + oc) * ldd + r0 + 8 * k) = make_uint4(u[0], u[1], u[2], u[3]);
    }
}

// A cotangent's uses in a weight product's backward in one pass over the
// fp32 rows: the bf16 transposed copy (the weight gradient's operand), and
// optionally the row-major bf16 copy (the input gradient's operand) and the
// bias gradient's per-64-row column partial sums.  One 64 × 64 tile a
// block: the fp32 tile goes to LDS (rows of 65 floats), the row-major copy
// straight from registers; 64 threads each add one column over the tile's
// rows in order from zero (the order and grouping of col_partials_kernel,
// so reduce_partials gives the same bits); eight lanes per destination row
// gather eight source rows each and store the rounded values as one
// 128-byte run.  Full tiles, 16-byte rows only.
__global__ __launch_bounds__(256) void transpose_colsum_kernel(const float *__restrict__ src, int64_t lds,
                                                               int cols, bf16_t *__restrict__ dst,
                                                               int64_t ldd, float *__restrict__ part,
                                                               bf16_t *__restrict__ rowb) {
    __shared__ float f[64][65];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tid = threadIdx.x;
    float4 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = tid + 256 * j, i = idx >> 4, cc = (idx & 15) * 4;
        w[j] = *reinterpret_cast<const float4 *>(src + (int64_t)(r0 + i) * lds + c0 + cc);
    }
    if (rowb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = tid + 256 * j, i = idx >> 4, cc = (idx & 15) * 4;
            *reinterpret_cast<uint2 *>(rowb + (int64_t)(r0 + i) * lds + c0 + cc) =
                pack4(f2bf(w[j].x), f2bf(w[j].y), f2bf(w[j].z), f2bf(w[j].w));
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int idx = tid + 256 * j, i = idx >> 4, cc = (idx & 15) * 4;
        f[i][cc + 0] = w[j].x;
        f[i][cc + 1] = w[j].y;
        f[i][cc + 2] = w[j].z;
        f[i][cc + 3] = w[j].w;
    }
    __syncthreads();
    if (part && tid < 64) {
        float sa = 0.f;
#pragma unroll 16
        for (int i = 0; i < 64; ++i) sa += f[i][tid];
        part[(int64_t)blockIdx.y * cols + c0 + tid] = sa;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int item = tid + 256 * j, k = item & 7, oc = item >> 3;  // source rows 8k … 8k+7, column oc
        uint32_t u[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
            u[m] = (uint32_t)f2bf(f[8 * k + 2 * m][oc]) | ((uint32_t)f2bf(f[8 * k + 2 * m + 1][oc]) << 16);
        *reinterpret_cast<uint4 *>(dst + (int64_t)(c0 + oc) * ldd + r0 + 8 * k) = make_uint4(u[0], u[1], u[2], u[3]);
    }
}

// Split-bf16 operands.  v = hi + lo + O(2⁻¹⁷|v|) with hi = bf16(v) and
// lo = bf16(v − hi).  A row of A' = [hi | lo | hi] against a row of
// B' = [hi | hi | lo] sums to hi·hi + lo·hi + hi·lo over 3K: an fp32 product
// to ~2⁻¹⁶ relative on the bf16 matrix cores (the dropped lo·lo term).  The
// first 2K alone, [hi | lo] against [hi | hi], give (hi + lo)·hi: A at split
// precision against B rounded once to bf16.
__device__ __forceinline__ void split_bf16(float v, bf16_t &hi, bf16_t &lo) {
    hi = f2bf(v);
    lo = f2bf(v - __uint_as_float((uint32_t)hi << 16));
}

// out[r] = [hi(x[r]) | lo(x[r]) | hi(x[r])], rows of K.
__global__ void split3_rows_kernel(const float *__restrict__ x, int64_t ldx, int64_t rows, int K,
                                   bf16_t *__restrict__ out, int64_t ldo) {
    const int64_t n = rows * K;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / K;
        const int c = (int)(i - r * K);
        bf16_t hi, lo;
        split_bf16(x[r * ldx + c], hi, lo);
        bf16_t *o = out + r * ldo;
        o[c] = hi;
        o[K + c] = lo;
        o[2 * K + c] = hi;
    }
}

// split3_rows_kernel four columns a thread: block row y (and every
// gridDim.y-th after it), column quad x·256 + t; 16-byte loads, 8-byte
// stores, no 64-bit division.
__global__ __launch_bounds__(256) void split3_rows4_kernel(const float4 *__restrict__ x, int64_t ldx4, int64_t rows,
                                                           int K4, uint2 *__restrict__ out, int64_t ldo4) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= K4) return;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float4 v = x[r * ldx4 + c];
        bf16_t h[4], l[4];
        split_bf16(v.x, h[0], l[0]);
        split_bf16(v.y, h[1], l[1]);
        split_bf16(v.z, h[2], l[2]);
        split_bf16(v.w, h[3], l[3]);
        const uint2 hv = pack4(h[0], h[1], h[2], h[3]);
        uint2 *o = out + r * ldo4;
        o[c] = hv;
        o[K4 + c] = pack4(l[0], l[1], l[2], l[3]);
        o[2 * K4 + c] = hv;
    }
}

// w [K, N] row-major → out [N, 3K] with out[n] = [hi(w[:,n]) | hi(w[:,n]) | lo(w[:,n])].
__global__ __launch_bounds__(256) void transpose_split3_kernel(const float *__restrict__ w, int64_t ldw,
                                                               int K, int N, bf16_t *__restrict__ out,
                                                               int64_t ldo) {
    __shared__ bf16_t th[64][66], tl[64][66];
    const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int k = k0 + i, n = n0 + tx;
        bf16_t hi = 0, lo = 0;
        if (k < K && n < N) split_bf16(w[(int64_t)k * ldw + n], hi, lo);
        th[i][tx] = hi;
        tl[i][tx] = lo;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int n = n0 + i, k = k0 + tx;
        if (n < N && k < K) {
            bf16_t *o = out + (int64_t)n * ldo;
            o[k] = th[tx][i];
            o[K + k] = th[tx][i];
            o[2 * K + k] = tl[tx][i];
        }
    }
}

// Six-part split for fp32-accurate products on the bf16 matrix cores:
// v = h + m + l + O(2⁻²⁶|v|) with h = bf16(v), m = bf16(v − h),
// l = bf16(v − h − m) (each difference exact in fp32).  Element k of a row
// becomes six consecutive bf16 values, interleaved along K so that any K
// range [k0, k1) of the original is the range [6k0, 6k1) of the split; the
// A role lays them out (h, m, h, l, h, m), the B role (h, h, m, h, l, m), so
// a GEMM over 6K sums hh + mh + hm + lh + hl + mm: every product term above
// 2⁻²⁴ relative.
__device__ __forceinline__ void split6_parts(float v, int role_b, bf16_t o[6]) {
    const bf16_t h = f2bf(v);
    const float r1 = v - __uint_as_float((uint32_t)h << 16);
    const bf16_t m = f2bf(r1);
    const bf16_t l = f2bf(r1 - __uint_as_float((uint32_t)m << 16));
    if (role_b) {
        o[0] = h; o[1] = h; o[2] = m; o[3] = h; o[4] = l; o[5] = m;
    } else {
        o[0] = h; o[1] = m; o[2] = h; o[3] = l; o[4] = h; o[5] = m;
    }
}

__device__ __forceinline__ void store6(bf16_t *dst, const bf16_t o[6]) {
    // dst is 4-byte aligned (6 bf16 per element, even element offsets).
    uint32_t *d = reinterpret_cast<uint32_t *>(dst);
    d[0] = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
    d[1] = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
    d[2] = (uint32_t)o[4] | ((uint32_t)o[5] << 16);
}

// out[r][6c .. 6c+5] = split6(x[r][c]).
__global__ void split6_rows_kernel(const float *__restrict__ x, int64_t ldx, int64_t rows, int K, int role_b,
                                   bf16_t *__restrict__ out, int64_t ldo) {
    const int64_t n = rows * K;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / K;
        const int c = (int)(i - r * K);
        bf16_t o[6];
        split6_parts(x[r * ldx + c], role_b, o);
        store6(out + r * ldo + 6 * (int64_t)c, o);
    }
}

// out[c][6r .. 6r+5] = split6(x[map(r)][c]) with map(r) = rows_map[r] / div
// (negative: a zero row; no map: r): a 64×64 fp32 tile through LDS.
__global__ __launch_bounds__(256) void split6_transpose_kernel(const float *__restrict__ x, int64_t ldx,
                                                               const int32_t *__restrict__ rows_map, int div,
                                                               int rows, int cols, int role_b,
                                                               bf16_t *__restrict__ out, int64_t ldo) {
    __shared__ float t[64][65];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int r = r0 + i, c = c0 + tx;
        float v = 0.f;
        if (r < rows && c < cols) {
            const int sr = rows_map ? (rows_map[r] < 0 ? -1 : rows_map[r] / div) : r;
            if (sr >= 0) v = x[(int64_t)sr * ldx + c];
        }
        t[i][tx] = v;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) {
            bf16_t o[6];
            split6_parts(t[tx][i], role_b, o);
            store6(out + (int64_t)c * ldo + 6 * (int64_t)r, o);
        }
    }
}

__global__ void scale_i32_kernel(const int32_t *__restrict__ src, int n, int factor, int32_t *__restrict__ dst) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i] * factor;
}

__global__ void swiglu_dadc_f32_kernel(const float *__restrict__ dh, const float *__restrict__ a,
                                       const float *__restrict__ c, float *__restrict__ da, float *__restrict__ dc,
                                       int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float z = a[i], sg = 1.0f / (1.0f + expf(-z));
        da[i] = dh[i] * c[i] * (sg + z * sg * (1.0f - sg));
        dc[i] = dh[i] * (z / (1.0f + expf(-z)));
    }
}

// LayerNorm forward for training: y (fp32 and/or bf16), mean and rstd per
// row.  One wavefront per row; any width.  NV4 > 0 (rows of 256·NV4
// floats): a lane's NV4 float4 runs of x are loaded once, into registers,
// and the three passes read them there, in the same order (same bits).
template <bool VEC, int NV4 = 0>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float *__restrict__ x,
                                                     const float *__restrict__ g,
                                                     const float *__restrict__ b,
                                                     float *__restrict__ y, bf16_t *__restrict__ yb,
                                                     bf16_t *__restrict__ y3, float *__restrict__ mean,
                                                     float *__restrict__ rstd, int64_t rows,
                                                     int cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * cols;
    if (VEC) {  // four consecutive columns a lane per step: 16-byte x, γ, β, y and 8-byte yb accesses
        const int c4n = cols / 4;
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        float4 xv[NV4 > 0 ? NV4 : 1];
        if constexpr (NV4 > 0) {
#pragma unroll
            for (int j = 0; j < NV4; ++j) xv[j] = x4[lane + 64 * j];
        }
        // f(c, x4[c]) for the lane's runs c = lane, lane + 64, … in order
        auto each = [&](auto &&f) {
            if constexpr (NV4 > 0) {
#pragma unroll
                for (int j = 0; j < NV4; ++j) f(lane + 64 * j, xv[j]);
            } else {
                for (int c = lane; c < c4n; c += 64) f(c, x4[c]);
            }
        };
        float s = 0.f;
        each([&](int, const float4 &v) {
            s += v.x;
            s += v.y;
            s += v.z;
            s += v.w;
        });
        const float n = (float)cols;
        const float mu = wave_sum_dpp(s) / n;
        float q = 0.f;
        each([&](int, const float4 &v) {
            const float d0 = v.x - mu, d1 = v.y - mu, d2 = v.z - mu, d3 = v.w - mu;
            q += d0 * d0;
            q += d1 * d1;
            q += d2 * d2;
            q += d3 * d3;
        });
        const float inv = 1.0f / sqrtf(wave_sum_dpp(q) / n + eps);
        const float4 *g4 = reinterpret_cast<const float4 *>(g), *b4 = reinterpret_cast<const float4 *>(b);
        each([&](int c, const float4 &v) {
            const float4 gv = g4[c], bv = b4[c];
            const float4 o = make_float4((v.x - mu) * inv * gv.x + bv.x, (v.y - mu) * inv * gv.y + bv.y,
                                         (v.z - mu) * inv * gv.z + bv.z, (v.w - mu) * inv * gv.w + bv.w);
            if (y) reinterpret_cast<float4 *>(y + row * cols)[c] = o;
            if (yb) reinterpret_cast<uint2 *>(yb + row * cols)[c] = pack4(f2bf(o.x), f2bf(o.y), f2bf(o.z), f2bf(o.w));
            if (y3) {  // [hi | lo | hi], as split3_rows
                bf16_t h[4], l[4];
                split_bf16(o.x, h[0], l[0]);
                split_bf16(o.y, h[1], l[1]);
                split_bf16(o.z, h[2], l[2]);
                split_bf16(o.w, h[3], l[3]);
                uint2 *r3 = reinterpret_cast<uint2 *>(y3 + row * 3 * cols);
                r3[c] = pack4(h[0], h[1], h[2], h[3]);
                r3[c4n + c] = pack4(l[0], l[1], l[2], l[3]);
                r3[2 * c4n + c] = pack4(h[0], h[1], h[2], h[3]);
            }
        });
        if (lane == 0) {
            mean[row] = mu;
            rstd[row] = inv;
        }
        return;
    }
    float s = 0.f;
    for (int c = lane; c < cols; c += 64) s += xr[c];
    const float n = (float)cols;
    const float mu = wave_sum_dpp(s) / n;
    float q = 0.f;
    for (int c = lane; c < cols; c += 64) {
        const float d = xr[c] - mu;
        q += d * d;
    }
    const float inv = 1.0f / sqrtf(wave_sum_dpp(q) / n + eps);
    for (int c = lane; c < cols; c += 64) {
        const float v = (xr[c] - mu) * inv * g[c] + b[c];
        if (y) y[row * cols + c] = v;
        if (yb) yb[row * cols + c] = f2bf(v);
        if (y3) {
            bf16_t h, l;
            split_bf16(v, h, l);
            y3[row * 3 * cols + c] = h;
            y3[row * 3 * cols + cols + c] = l;
            y3[row * 3 * cols + 2 * cols + c] = h;
        }
    }
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = inv;
    }
}

// Column sums of [rows, cols] tensors (bias and LayerNorm parameter
// gradients, the router's gate gradient) in two fixed-order stages, no
// atomics: col_partials sums groups of kColRows rows per column (threads
// along columns, so every row read is coalesced), reduce_partials adds the
// groups with four wavefronts per 64 columns.
constexpr int kColRows = 64;

// part_a[g][c] = Σ_r dy[r][c] and, for LayerNorm (LN), part_a = Σ_r dy·x̂,
// part_b = Σ_r dy with x̂ = (x − mean)·rstd, over the rows r of group g.
template <bool LN>
__global__ __launch_bounds__(256) void col_partials_kernel(const float *__restrict__ dy,
                                                           const float *__restrict__ x,
                                                           const float *__restrict__ mean,
                                                           const float *__restrict__ rstd, int64_t rows,
                                                           int cols, float *__restrict__ part_a,
                                                           float *__restrict__ part_b) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    const int64_t r0 = (int64_t)blockIdx.y * kColRows;
    const int64_t r1 = r0 + kColRows < rows ? r0 + kColRows : rows;
    float sa = 0.f, sb = 0.f;
    // Unrolled so that several rows' loads are in flight; the sums still
    // run row by row in order.  (All 64 of a group's loads issued before the
    // first sum, with LayerNorm's row statistics from LDS, measured the same
    // in the config-5 step: 67.6 against 69.2 us for its four launches.)
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) {
        const float d = dy[r * cols + c];
        if (LN) {
            const float xh = (x[r * cols + c] - mean[r]) * rstd[r];
            sa += d * xh;
            sb += d;
        } else {
            sa += d;
        }
    }
    part_a[(int64_t)blockIdx.y * cols + c] = sa;
    if (LN) part_b[(int64_t)blockIdx.y * cols + c] = sb;
}

// out[c] (+)= Σ_g part[g][c]: wavefront w sums groups w, w+4, …; the four
// sums are added in a fixed order.
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float *__restrict__ part, int ng,
                                                              int cols, float *__restrict__ out,
                                                              int accumulate) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (c < cols) {
#pragma unroll 8
        for (int g = w; g < ng; g += 4) s += part[(int64_t)g * cols + c];
    }
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && c < cols) {
        const float t = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
        out[c] = accumulate ? out[c] + t : t;
    }
}

// out[i] (+)= part[0][i] + part[1][i] + … in that order, four floats a
// thread per step (the split-K partial sums of one GEMM).
__global__ __launch_bounds__(256) void sum_parts_kernel(const float4 *__restrict__ part, int np, int64_t n4,
                                                        float4 *__restrict__ out, int accumulate) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        float4 t = part[i];
        for (int e = 1; e < np; ++e) {
            const float4 u = part[(int64_t)e * n4 + i];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        if (accumulate) {
            const float4 o = out[i];
            t.x = o.x + t.x;
            t.y = o.y + t.y;
            t.z = o.z + t.z;
            t.w = o.w + t.w;
        }
        out[i] = t;
    }
}

// LayerNorm adjoint, dx (+)= (rstd/n)(n·g − Σg − x̂·Σ(g·x̂)) with g = dy·γ:
// one wavefront per row, the row held in registers (NV values per lane,
// cols ≤ 64·NV), so x and dy are read once.
template <int NV>
__global__ __launch_bounds__(256) void ln_bwd_dx_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ gam,
                                                        const float *__restrict__ mean,
                                                        const float *__restrict__ rstd,
                                                        const float *__restrict__ dy,
                                                        float *__restrict__ dx, int accumulate,
                                                        int64_t rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float mu = mean[row], inv = rstd[row];
    const float *xr = x + row * cols, *gr = dy + row * cols;
    float xh[NV], gd[NV];
    float sd = 0.f, sdx = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + 64 * j;
        xh[j] = 0.f;
        gd[j] = 0.f;
        if (c < cols) {
            xh[j] = (xr[c] - mu) * inv;
            gd[j] = gr[c] * gam[c];
            sd += gd[j];
            sdx += gd[j] * xh[j];
        }
    }
    sd = wave_sum_dpp(sd);
    sdx = wave_sum_dpp(sdx);
    const float n = (float)cols;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + 64 * j;
        if (c < cols) {
            const float v = (inv / n) * (n * gd[j] - sd - xh[j] * sdx);
            float *o = dx + row * cols + c;
            *o = accumulate ? *o + v : v;
        }
    }
}

// Rows of 256·NV4 floats, 16-byte aligned: the same arithmetic with lane l
// holding the float4 runs l, l + 64, …, all of a lane's loads (x, dy, γ and,
// accumulating, the old dx) issued before the first product.
template <int NV4>
__global__ __launch_bounds__(256) void ln_bwd_dx4_kernel(const float *__restrict__ x,
                                                         const float *__restrict__ gam,
                                                         const float *__restrict__ mean,
                                                         const float *__restrict__ rstd,
                                                         const float *__restrict__ dy,
                                                         float *__restrict__ dx, int accumulate,
                                                         int64_t rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float mu = mean[row], inv = rstd[row];
    const float4 *xr = reinterpret_cast<const float4 *>(x + row * cols);
    const float4 *gr = reinterpret_cast<const float4 *>(dy + row * cols);
    const float4 *g4 = reinterpret_cast<const float4 *>(gam);
    float4 *o4 = reinterpret_cast<float4 *>(dx + row * cols);
    float4 xv[NV4], dv[NV4], gv[NV4], ov[NV4];
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        const int c = lane + 64 * j;
        xv[j] = xr[c];
        dv[j] = gr[c];
        gv[j] = g4[c];
        ov[j] = accumulate ? o4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float xh[NV4][4], gd[NV4][4];
    float sd = 0.f, sdx = 0.f;
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w}, ds[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w},
                    gs[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xh[j][q] = (xs[q] - mu) * inv;
            gd[j][q] = ds[q] * gs[q];
            sd += gd[j][q];
            sdx += gd[j][q] * xh[j][q];
        }
    }
    sd = wave_sum_dpp(sd);
    sdx = wave_sum_dpp(sdx);
    const float n = (float)cols;
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = (inv / n) * (n * gd[j][q] - sd - xh[j][q] * sdx);
        const float4 o = ov[j];
        o4[lane + 64 * j] = accumulate ? make_float4(o.x + v[0], o.y + v[1], o.z + v[2], o.w + v[3])
                                       : make_float4(v[0], v[1], v[2], v[3]);
    }
}

// Any width: the same with two passes over the row in memory.
__global__ __launch_bounds__(256) void ln_bwd_dx_any_kernel(const float *__restrict__ x,
                                                            const float *__restrict__ gam,
                                                            const float *__restrict__ mean,
                                                            const float *__restrict__ rstd,
                                                            const float *__restrict__ dy,
                                                            float *__restrict__ dx, int accumulate,
                                                            int64_t rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float mu = mean[row], inv = rstd[row];
    const float *xr = x + row * cols, *gr = dy + row * cols;
    float sd = 0.f, sdx = 0.f;
    for (int c = lane; c < cols; c += 64) {
        const float xh = (xr[c] - mu) * inv;
        const float d = gr[c] * gam[c];
        sd += d;
        sdx += d * xh;
    }
    sd = wave_sum_dpp(sd);
    sdx = wave_sum_dpp(sdx);
    const float n = (float)cols;
    for (int c = lane; c < cols; c += 64) {
        const float xh = (xr[c] - mu) * inv;
        const float d = gr[c] * gam[c];
        const float v = (inv / n) * (n * d - sd - xh * sdx);
        float *o = dx + row * cols + c;
        *o = accumulate ? *o + v : v;
    }
}

__global__ void act_bwd_kernel(const float *__restrict__ z, const float *__restrict__ dy,
                               float *__restrict__ dx, int64_t n, int act, int accumulate) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float zz = z[i];
        float d;
        if (act == ACT_RELU) {
            d = zz <= 0.f ? 0.f : dy[i];
        } else {
            const float C = 0.044715f, kk = 0.797884523868560791f;
            const float u = kk * (zz + C * zz * zz * zz);
            const float t = tanhf(u);
            const float du = kk * (1.0f + 3.0f * C * zz * zz);
            d = dy[i] * (0.5f * (1.0f + t) + 0.5f * zz * (1.0f - t * t) * du);
        }
        dx[i] = accumulate ? dx[i] + d : d;
    }
}

// MSE: d = 2e/n and per-block partial Σe² (float4 runs where the rows
// allow: 29.4 -> 18.3 us on config 5's 8192 x 1024 output).
__global__ __launch_bounds__(256) void mse_kernel(const float *__restrict__ pred,
                                                  const float *__restrict__ tgt,
                                                  float *__restrict__ d, int64_t n,
                                                  float *__restrict__ part, int vec) {
    __shared__ float ws[4];
    const float nf = (float)n;
    float s = 0.f;
    if (vec) {
        // float4 runs, four of them in flight per operand before the first
        // sum; the same per-element arithmetic
        const int64_t n4 = n / 4;
        const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
        const int64_t lo = (int64_t)blockIdx.x * per, hi = min(n4, lo + per);
        const float4 *p4 = reinterpret_cast<const float4 *>(pred), *t4 = reinterpret_cast<const float4 *>(tgt);
        float4 *d4 = reinterpret_cast<float4 *>(d);
        for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += 4 * 256) {
            float4 a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t i = i0 + 256 * u;
                if (i < hi) {
                    a[u] = p4[i];
                    b[u] = t4[i];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t i = i0 + 256 * u;
                if (i < hi) {
                    const float e0 = a[u].x - b[u].x, e1 = a[u].y - b[u].y, e2 = a[u].z - b[u].z,
                                e3 = a[u].w - b[u].w;
                    s += e0 * e0;
                    s += e1 * e1;
                    s += e2 * e2;
                    s += e3 * e3;
                    d4[i] = make_float4(2.0f * e0 / nf, 2.0f * e1 / nf, 2.0f * e2 / nf, 2.0f * e3 / nf);
                }
            }
        }
    } else {
        const int64_t per = (n + gridDim.x - 1) / gridDim.x;
        const int64_t lo = (int64_t)blockIdx.x * per, hi = min(n, lo + per);
        for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
            const float e = pred[i] - tgt[i];
            s += e * e;
            d[i] = 2.0f * e / nf;
        }
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = (ws[0] + ws[1]) + (ws[2] + ws[3]);
}

__global__ __launch_bounds__(256) void mse_finish_kernel(const float *__restrict__ part, int nb,
                                                         int64_t n, float *__restrict__ loss) {
    __shared__ float ws[4];
    float s = 0.f;
    for (int b = threadIdx.x; b < nb; b += 256) s += part[b];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) *loss = ((ws[0] + ws[1]) + (ws[2] + ws[3])) / (float)n;
}

// cross_entropy (adjoint.rs:123-145), one block per row of logits
// [rows, V]: softmax_last (row max, e = exp(x − max), inv = 1/max(Σe, 1e-30),
// p = e·inv; cpu.rs:31-52), then d = p/rows with 1/rows subtracted at the
// row's class id, and the row's loss term −ln(max(p_t, 1e-30)).  Ids are
// checked against V on the host.
__global__ __launch_bounds__(256) void ce_rows_kernel(const float *__restrict__ logits,
                                                      const uint32_t *__restrict__ ids, int64_t rows, int V,
                                                      float *__restrict__ d, float *__restrict__ row_loss) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const float *x = logits + r * V;
    float *o = d + r * V;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float m = -INFINITY;
    for (int j = threadIdx.x; j < V; j += 256) m = fmaxf(m, x[j]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (int j = threadIdx.x; j < V; j += 256) sum += expf(x[j] - m);
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    const float inv = 1.0f / fmaxf((red[0] + red[1]) + (red[2] + red[3]), 1e-30f);
    const float rf = (float)rows, sub = 1.0f / rf;
    const int t = (int)ids[r];
    for (int j = threadIdx.x; j < V; j += 256) {
        const float p = expf(x[j] - m) * inv;
        float v = p / rf;
        if (j == t) {
            v = v - sub;
            row_loss[r] = -logf(fmaxf(p, 1e-30f));
        }
        o[j] = v;
    }
}

// rmsnorm_backward (adjoint.rs:147-198), one wavefront per row: ms and
// dinv = Σ dy·x·w by wave reductions, inv = 1/√(ms+eps), dms =
// dinv·(−0.5)·(ms+eps)^(−1.5); dx = dy·inv·w + dms·(2x/n) (stored, or added
// to what dx holds), and the row's dw terms dy·x·inv into prod [rows, cols]
// for the column sum.
__global__ __launch_bounds__(256) void rms_bwd_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ dy, float *__restrict__ dx,
                                                      int acc_dx, float *__restrict__ prod, int64_t rows, int cols,
                                                      float eps) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * cols, *yr = dy + row * cols;
    float ss = 0.f, dinv = 0.f;
    for (int c = lane; c < cols; c += 64) {
        const float xv = xr[c];
        ss += xv * xv;
        dinv += yr[c] * xv * w[c];
    }
    ss = wave_sum(ss);
    dinv = wave_sum(dinv);
    const float n = (float)cols, ms = ss / n, inv = 1.0f / sqrtf(ms + eps);
    const float dms = dinv * (-0.5f) * powf(ms + eps, -1.5f);
    for (int c = lane; c < cols; c += 64) {
        const float xv = xr[c], d = yr[c];
        const float o = d * inv * w[c] + dms * (2.0f * xv / n);
        const int64_t e = row * cols + c;
        if (dx) dx[e] = acc_dx ? dx[e] + o : o;
        prod[e] = d * xv * inv;
    }
}

// mix_backward (deepseek.rs:241-258) with σ = σ(gate[0]) (gate null: 0):
// da = dy·σ and db = dy·(1 − σ), each stored or added (null: skipped), and
// per-block partial sums of (a − b)·dy for the gate.
__global__ __launch_bounds__(256) void mix_bwd_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                                      const float *__restrict__ gate, const float *__restrict__ dy,
                                                      float *da, int acc_a, float *db, int acc_b, int64_t n,
                                                      float *__restrict__ parts) {
#pragma clang fp contract(off)
    __shared__ float ws[4];
    const float g = gate ? gate[0] : 0.f;
    const float sg = 1.0f / (1.0f + expf(-g)), rs = 1.0f - sg;
    float acc = 0.f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float d = dy[i];
        if (da) da[i] = acc_a ? da[i] + d * sg : d * sg;
        if (db) db[i] = acc_b ? db[i] + d * rs : d * rs;
        acc += (a[i] - b[i]) * d;
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) parts[blockIdx.x] = (ws[0] + ws[1]) + (ws[2] + ws[3]);
}

// dg = σ(1 − σ)·Σ parts, the parts added in a fixed order.
__global__ __launch_bounds__(256) void mix_bwd_finish_kernel(const float *__restrict__ parts, int nb,
                                                             const float *__restrict__ gate, float *__restrict__ dg) {
#pragma clang fp contract(off)
    __shared__ float ws[4];
    float s = 0.f;
    for (int i = threadIdx.x; i < nb; i += 256) s += parts[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float g = gate ? gate[0] : 0.f;
        const float sg = 1.0f / (1.0f + expf(-g));
        dg[0] = ((ws[0] + ws[1]) + (ws[2] + ws[3])) * (sg * (1.0f - sg));
    }
}

// softmax_backward (adjoint.rs:92-104), one wavefront per row of the
// forward output y: dot = Σ y·dy, dx = y·(dy − dot), stored or added.
__global__ __launch_bounds__(256) void softmax_bwd_kernel(const float *__restrict__ y, const float *__restrict__ dy,
                                                          float *__restrict__ dx, int acc, int64_t rows, int cols) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *yr = y + row * cols, *gr = dy + row * cols;
    float dot = 0.f;
    for (int c = lane; c < cols; c += 64) dot += yr[c] * gr[c];
    dot = wave_sum(dot);
    for (int c = lane; c < cols; c += 64) {
        const int64_t e = row * cols + c;
        const float o = yr[c] * (gr[c] - dot);
        dx[e] = acc ? dx[e] + o : o;
    }
}

// The dense SwiGLU's hidden activation h = silu(a)·c (moe.rs:159-174).
__global__ void swiglu_h_kernel(const float *__restrict__ a, const float *__restrict__ c, float *__restrict__ h,
                                int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        h[i] = a[i] / (1.0f + expf(-a[i])) * c[i];
}

// swiglu_backward's elementwise step (adjoint.rs:238-242): da = dh·c·silu'(a),
// dc = dh·silu(a) with silu'(z) = s + z·s·(1 − s), s = 1/(1 + e^(−z)); both
// written as bf16 GEMM operands.
__global__ void swiglu_dadc_kernel(const float *__restrict__ dh, const float *__restrict__ a,
                                   const float *__restrict__ c, bf16_t *__restrict__ da, bf16_t *__restrict__ dc,
                                   int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float z = a[i], sg = 1.0f / (1.0f + expf(-z));
        da[i] = f2bf(dh[i] * c[i] * (sg + z * sg * (1.0f - sg)));
        dc[i] = f2bf(dh[i] * (z / (1.0f + expf(-z))));
    }
}

// Mul's adjoint (adjoint.rs:787-800) for one input: dx = dy·other, stored or
// added.
__global__ void mul_bwd_kernel(const float *__restrict__ dy, const float *__restrict__ other, float *dx, int acc,
                               int64_t n) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float o = dy[i] * other[i];
        dx[i] = acc ? dx[i] + o : o;
    }
}

// p −= lr·g; pb = bf16(p) when given.  g may have a row stride (packed
// gradients): element (r, c) of p [rows, cols] reads g[r·ldg + c].  The
// product and the difference are rounded separately, as Sgd::put does, so
// the update is bit-identical to the reference's for the same gradient.
__global__ void sgd_kernel(float *__restrict__ p, const float *__restrict__ g, int64_t ldg,
                           int64_t rows, int cols, float lr, bf16_t *__restrict__ pb) {
#pragma clang fp contract(off)
    const int64_t n = rows * cols;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / cols, c = i - r * cols;
        const float v = p[i] - lr * g[r * ldg + c];
        p[i] = v;
        if (pb) pb[i] = f2bf(v);
    }
}

// One parameter value under the update rule: Sgd::put (optim.rs:38-40),
// p − lr·g, or Adam::put (optim.rs:104-115) with moments m, v updated in
// place.  Every product, quotient, square root and sum is rounded on its
// own, in the reference's order ((1−β₂)·g·g is ((1−β₂)·g)·g, and lr·m̂/(…)
// is (lr·m̂)/(…)); division and sqrtf are correctly rounded in this build,
// so the new value is bit-identical to the reference's for the same inputs.
__device__ __forceinline__ float update_value(const UpdateRule &u, float p, float g, float &m, float &v) {
#pragma clang fp contract(off)
    if (!u.adam) return p - u.lr * g;
    const float mi = u.beta1 * m + (1.f - u.beta1) * g;
    const float vi = u.beta2 * v + (1.f - u.beta2) * g * g;
    m = mi;
    v = vi;
    const float mhat = mi / fmaxf(u.b1t, 1e-30f);
    const float vhat = vi / fmaxf(u.b2t, 1e-30f);
    return p - u.lr * mhat / (sqrtf(vhat) + u.eps);
}

// The update rule over n values: four a thread with 16-byte accesses when
// every buffer allows it, the same arithmetic either way.
__global__ void apply_update_kernel(UpdateRule u, float *__restrict__ p, const float *__restrict__ g,
                                    float *__restrict__ m, float *__restrict__ v, int64_t n, int vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int64_t nq = n / 4;
        for (int64_t q = i0; q < nq; q += stride) {
            float4 pv = reinterpret_cast<const float4 *>(p)[q];
            const float4 gv = reinterpret_cast<const float4 *>(g)[q];
            float4 mv = make_float4(0.f, 0.f, 0.f, 0.f), vv = mv;
            if (u.adam) {
                mv = reinterpret_cast<const float4 *>(m)[q];
                vv = reinterpret_cast<const float4 *>(v)[q];
            }
            pv.x = update_value(u, pv.x, gv.x, mv.x, vv.x);
            pv.y = update_value(u, pv.y, gv.y, mv.y, vv.y);
            pv.z = update_value(u, pv.z, gv.z, mv.z, vv.z);
            pv.w = update_value(u, pv.w, gv.w, mv.w, vv.w);
            reinterpret_cast<float4 *>(p)[q] = pv;
            if (u.adam) {
                reinterpret_cast<float4 *>(m)[q] = mv;
                reinterpret_cast<float4 *>(v)[q] = vv;
            }
        }
        for (int64_t i = nq * 4 + i0; i < n; i += stride) {
            float mi = u.adam ? m[i] : 0.f, vi = u.adam ? v[i] : 0.f;
            p[i] = update_value(u, p[i], g[i], mi, vi);
            if (u.adam) {
                m[i] = mi;
                v[i] = vi;
            }
        }
    } else {
        for (int64_t i = i0; i < n; i += stride) {
            float mi = u.adam ? m[i] : 0.f, vi = u.adam ? v[i] : 0.f;
            p[i] = update_value(u, p[i], g[i], mi, vi);
            if (u.adam) {
                m[i] = mi;
                v[i] = vi;
            }
        }
    }
}

// Multi-tensor update: block b updates one 64×64 tile of the parameter whose
// tile range holds b (binary search of the table), writes the master (and
// Adam's moments) and the row-major bf16 copy, and through LDS the
// transposed copies.  Every value is read and written once a step: the
// 16-byte loads and stores of the row-major streams carry the nontemporal
// hint (measured on config 5: SGD step 296 -> 283 us, Adam step 636 -> 605
// us).  The transposed copies' 8-byte stores, 16 threads to a 128-byte
// run, stay ordinary: with the hint they measured 10 % slower.
__global__ __launch_bounds__(256) void sgd_multi_kernel(const SgdParam *__restrict__ tab, int n,
                                                        UpdateRule u, int use_grad) {
#pragma clang fp contract(off)
    __shared__ bf16_t th[64][66], tl[64][66];
    const int b = blockIdx.x;
    int lo = 0, hi = n - 1;
    while (lo < hi) {  // last entry with tile0 <= b
        const int mid = (lo + hi + 1) >> 1;
        if (tab[mid].tile0 <= b) lo = mid;
        else hi = mid - 1;
    }
    const SgdParam P = tab[lo];
    const int t = b - P.tile0;
    const int r0 = (t / P.tiles_c) * 64, c0 = (t % P.tiles_c) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const bool grad = use_grad && P.g;
    auto al = [](const void *q, int a) { return (reinterpret_cast<uintptr_t>(q) & (a - 1)) == 0; };
    // One element: update, split into hi/lo bf16, row-major copy.
    auto one = [&](int64_t e, bf16_t &h, bf16_t &l) {
        float v = P.p[e];
        if (grad) {
            float mo = u.adam ? P.m[e] : 0.f, ve = u.adam ? P.v[e] : 0.f;
            v = update_value(u, v, P.g[e], mo, ve);
            P.p[e] = v;
            if (u.adam) {
                P.m[e] = mo;
                P.v[e] = ve;
            }
        }
        h = f2bf(v);
        l = f2bf(v - __uint_as_float((uint32_t)h << 16));
    };
    // Four consecutive columns a thread (16-byte master and gradient, 8-byte
    // bf16 rows) when the rows allow it; the same arithmetic either way.
    const bool vec = P.cols % 4 == 0 && al(P.p, 16) && (!grad || al(P.g, 16)) &&
                     (!P.b || (al(P.b, 8) && P.ldb % 4 == 0)) &&
                     (!grad || !u.adam || (al(P.m, 16) && al(P.v, 16)));
    if (vec) {
        // A thread's four rows (rq, rq+16, rq+32, rq+48): every load of the
        // four is issued before the first update and store.
        const int cq = 4 * (threadIdx.x & 15), rq = threadIdx.x >> 4;
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 pv[4], gv[4], mo[4], ve[4];
        bool in[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = r0 + rq + 16 * j, c = c0 + cq;
            in[j] = r < P.rows && c < P.cols;  // c + 3 < cols: cols and c0 are multiples of 4
            pv[j] = gv[j] = mo[j] = ve[j] = z4;
            if (in[j]) {
                const int64_t e = (int64_t)r * P.cols + c;
                pv[j] = load_stream(P.p + e);
                if (grad) {
                    gv[j] = load_stream(P.g + e);
                    if (u.adam) {
                        mo[j] = load_stream(P.m + e);
                        ve[j] = load_stream(P.v + e);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = rq + 16 * j;
            bf16_t h[4] = {0, 0, 0, 0}, l[4] = {0, 0, 0, 0};
            if (in[j]) {
                const int64_t e = (int64_t)(r0 + i) * P.cols + c0 + cq;
                float v[4] = {pv[j].x, pv[j].y, pv[j].z, pv[j].w};
                if (grad) {
                    v[0] = update_value(u, v[0], gv[j].x, mo[j].x, ve[j].x);
                    v[1] = update_value(u, v[1], gv[j].y, mo[j].y, ve[j].y);
                    v[2] = update_value(u, v[2], gv[j].z, mo[j].z, ve[j].z);
                    v[3] = update_value(u, v[3], gv[j].w, mo[j].w, ve[j].w);
                    store_stream(P.p + e, make_float4(v[0], v[1], v[2], v[3]));
                    if (u.adam) {
                        store_stream(P.m + e, mo[j]);
                        store_stream(P.v + e, ve[j]);
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    h[q] = f2bf(v[q]);
                    l[q] = f2bf(v[q] - __uint_as_float((uint32_t)h[q] << 16));
                }
                if (P.b)
                    store_stream(P.b + (int64_t)(r0 + i) * P.ldb + c0 + cq, h[0] | (uint32_t)h[1] << 16,
                                 h[2] | (uint32_t)h[3] << 16);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                th[i][cq + q] = h[q];
                tl[i][cq + q] = l[q];
            }
        }
    } else {
        for (int i = ty; i < 64; i += 4) {
            const int r = r0 + i, c = c0 + tx;
            bf16_t h = 0, l = 0;
            if (r < P.rows && c < P.cols) {
                one((int64_t)r * P.cols + c, h, l);
                if (P.b) P.b[(int64_t)r * P.ldb + c] = h;
            }
            th[i][tx] = h;
            tl[i][tx] = l;
        }
    }
    if (!P.bt && !P.bt3) return;  // uniform per block
    __syncthreads();
    // Transposed copies: four consecutive rows a thread (8-byte stores) when
    // every destination row starts on 8 bytes.  (Eight rows a thread with
    // 16-byte stores measured the same: 271 against 273 us a SGD step.)
    const bool tvec = P.rows % 4 == 0 && (!P.bt || al(P.bt, 8)) && (!P.bt3 || al(P.bt3, 8));
    if (tvec) {
        const int rq = 4 * (threadIdx.x & 15), cq = threadIdx.x >> 4;
        for (int i = cq; i < 64; i += 16) {
            const int c = c0 + i, r = r0 + rq;
            if (c < P.cols && r < P.rows) {  // r + 3 < rows
                const uint2 hv = make_uint2(th[rq][i] | (uint32_t)th[rq + 1][i] << 16,
                                            th[rq + 2][i] | (uint32_t)th[rq + 3][i] << 16);
                if (P.bt) *reinterpret_cast<uint2 *>(P.bt + (int64_t)c * P.rows + r) = hv;
                if (P.bt3) {
                    const uint2 lv = make_uint2(tl[rq][i] | (uint32_t)tl[rq + 1][i] << 16,
                                                tl[rq + 2][i] | (uint32_t)tl[rq + 3][i] << 16);
                    bf16_t *o = P.bt3 + (int64_t)c * 3 * P.rows;
                    *reinterpret_cast<uint2 *>(o + r) = hv;
                    *reinterpret_cast<uint2 *>(o + P.rows + r) = hv;
                    *reinterpret_cast<uint2 *>(o + 2 * P.rows + r) = lv;
                }
            }
        }
    } else {
        for (int i = ty; i < 64; i += 4) {
            const int c = c0 + i, r = r0 + tx;
            if (c < P.cols && r < P.rows) {
                if (P.bt) P.bt[(int64_t)c * P.rows + r] = th[tx][i];
                if (P.bt3) {
                    bf16_t *o = P.bt3 + (int64_t)c * 3 * P.rows;
                    o[r] = th[tx][i];
                    o[P.rows + r] = th[tx][i];
                    o[2 * P.rows + r] = tl[tx][i];
                }
            }
        }
    }
}

// Router STE, per token: dlogits[t, idx_k] = w_k (dw_k − Σ_j w_j dw_j).
__global__ void router_dlogits_kernel(const int32_t *__restrict__ idx, const float *__restrict__ w,
                                      const float *__restrict__ dw, int T, int E, int K,
                                      float *__restrict__ dl) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    float dot = 0.f;
    for (int j = 0; j < K; ++j) dot += w[(int64_t)t * K + j] * dw[(int64_t)t * K + j];
    for (int e = 0; e < E; ++e) dl[(int64_t)t * E + e] = 0.f;
    for (int j = 0; j < K; ++j) {
        const int e = idx[(int64_t)t * K + j];
        dl[(int64_t)t * E + e] += w[(int64_t)t * K + j] * (dw[(int64_t)t * K + j] - dot);
    }
}

// The same partials with thread h owning the E entries of row h: x[t][h] is
// read once (coalesced across h) and dl[t][·] is the same for every lane.
// EM ≥ E accumulators in registers; each entry still sums its tokens in
// order, so the result equals router_dgate_parts_kernel's.
template <int EM>
__global__ __launch_bounds__(256) void router_dgate_rows_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ dl, int T, int H,
                                                                int E, float *__restrict__ part) {
    __shared__ float dls[kColRows * EM];
    const int h = blockIdx.x * 256 + threadIdx.x;
    const int t0 = blockIdx.y * kColRows;
    const int t1 = t0 + kColRows < T ? t0 + kColRows : T;
    float acc[EM];
#pragma unroll
    for (int e = 0; e < EM; ++e) acc[e] = 0.f;
    if (t1 - t0 == kColRows && E == EM && (int)(blockIdx.x + 1) * 256 <= H) {
        // A whole group of exactly EM experts in a block whose columns are
        // all in range (block-uniform, so the barrier below is reached by
        // every thread).  Every x load of the group is issued first, then
        // the group's dl rows go to LDS (read back as broadcasts), so a
        // wavefront waits for memory once rather than once per token: with
        // a per-entry guard or per-token scalar loads of dl the compiler
        // kept eight loads in flight and waited on each scalar load.
        float xv[kColRows];
#pragma unroll
        for (int i = 0; i < kColRows; ++i) xv[i] = x[(int64_t)(t0 + i) * H + h];
        for (int j = threadIdx.x; j < kColRows * EM; j += 256) dls[j] = dl[(int64_t)t0 * EM + j];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kColRows; ++i)
#pragma unroll
            for (int e = 0; e < EM; ++e) acc[e] += xv[i] * dls[i * EM + e];
    } else {
        if (h >= H) return;
#pragma unroll 8
        for (int t = t0; t < t1; ++t) {  // unrolled: several tokens' loads in flight
            const float xv = x[(int64_t)t * H + h];
            const float *d = dl + (int64_t)t * E;
#pragma unroll
            for (int e = 0; e < EM; ++e)
                if (e < E) acc[e] += xv * d[e];
        }
    }
    float *o = part + (int64_t)blockIdx.y * H * E + (int64_t)h * E;
#pragma unroll
    for (int e = 0; e < EM; ++e)
        if (e < E) o[e] = acc[e];
}

// Partials of dgate[h][e] = Σ_t x[t][h]·dl[t][e] over groups of kColRows
// tokens; thread j owns entry j = h·E + e of the [H, E] gradient.
__global__ __launch_bounds__(256) void router_dgate_parts_kernel(const float *__restrict__ x,
                                                                 const float *__restrict__ dl, int T,
                                                                 int H, int E,
                                                                 float *__restrict__ part) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= H * E) return;
    const int h = j / E, e = j - h * E;
    const int t0 = blockIdx.y * kColRows;
    const int t1 = t0 + kColRows < T ? t0 + kColRows : T;
    float s = 0.f;
    for (int t = t0; t < t1; ++t) s += x[(int64_t)t * H + h] * dl[(int64_t)t * E + e];
    part[(int64_t)blockIdx.y * H * E + j] = s;
}

// Per permuted position: dys[pos] = bf16(w[slot]·dout[tok]) and
// dw[slot] = Σ_h y[pos][h]·dout[tok][h]; padding positions get zeros.
__device__ __forceinline__ void put_out(bf16_t *p, float v) { *p = f2bf(v); }
__device__ __forceinline__ void put_out(float *p, float v) { *p = v; }

template <typename OUT>
__global__ __launch_bounds__(256) void moe_slot_grad_kernel(
    const int32_t *__restrict__ slot_of_pos, const float *__restrict__ w,
    const float *__restrict__ y, const float *__restrict__ dout, int K, int H, int n_pos,
    OUT *__restrict__ dys, float *__restrict__ dw) {
    __shared__ float ws[4];
    const int pos = blockIdx.x;
    if (pos >= n_pos) return;
    const int slot = slot_of_pos[pos];
    if (slot < 0) {
        for (int h = threadIdx.x; h < H; h += 256) dys[(int64_t)pos * H + h] = 0;
        return;
    }
    const int t = slot / K;
    const float wt = w[slot];
    float s = 0.f;
    for (int h = threadIdx.x; h < H; h += 256) {
        const float g = dout[(int64_t)t * H + h];
        s += y[(int64_t)pos * H + h] * g;
        put_out(&dys[(int64_t)pos * H + h], wt * g);
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) dw[slot] = (ws[0] + ws[1]) + (ws[2] + ws[3]);
}

// The same for bf16 dys and rows of 256·NV4 floats (16-byte aligned): one
// wavefront per position, four positions a block, each lane holding NV4
// float4 runs of y and dout (all loaded before the first product), dw summed
// over the lane's runs and then across the wavefront by DPP.
template <int NV4>
__global__ __launch_bounds__(256) void moe_slot_grad4_kernel(const int32_t *__restrict__ slot_of_pos,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ y,
                                                             const float *__restrict__ dout, int K, int H,
                                                             int n_pos, bf16_t *__restrict__ dys,
                                                             float *__restrict__ dw) {
    const int lane = threadIdx.x & 63;
    const int pos = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (pos >= n_pos) return;
    const int slot = slot_of_pos[pos];
    uint2 *o = reinterpret_cast<uint2 *>(dys + (int64_t)pos * H);
    if (slot < 0) {
#pragma unroll
        for (int j = 0; j < NV4; ++j) o[lane + 64 * j] = make_uint2(0u, 0u);
        return;
    }
    const int t = slot / K;
    const float wt = w[slot];
    const float4 *g4 = reinterpret_cast<const float4 *>(dout + (int64_t)t * H);
    const float4 *y4 = reinterpret_cast<const float4 *>(y + (int64_t)pos * H);
    float4 gv[NV4], yv[NV4];
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        gv[j] = g4[lane + 64 * j];
        yv[j] = y4[lane + 64 * j];
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV4; ++j) {
        s += yv[j].x * gv[j].x;
        s += yv[j].y * gv[j].y;
        s += yv[j].z * gv[j].z;
        s += yv[j].w * gv[j].w;
        o[lane + 64 * j] = pack4(f2bf(wt * gv[j].x), f2bf(wt * gv[j].y), f2bf(wt * gv[j].z), f2bf(wt * gv[j].w));
    }
    s = wave_sum_dpp(s);
    if (lane == 0) dw[slot] = s;
}

// dx[t][h] (+)= Σ_k dxs[pos(t,k)][h] + Σ_e dl[t][e]·gate[h][e].  A thread
// owns one h for kMoeDxTokens tokens, so gate[h][·] is read once per
// thread and dl[t][·] is uniform across the block.
// KT > 0 (top-k known at compile time, a whole group of tokens): every
// slot row and every old dx value of the group is loaded before the first
// sum, so the gathers are in flight together; the sums keep the order and
// form of the general path (s = 0, then + each slot in k order, + the
// router term, then the old value first), so both give the same bits.
constexpr int kMoeDxTokens = 16;

template <int KT>
__global__ __launch_bounds__(256) void moe_dx_kernel(const float *__restrict__ dxs,
                                                     const int32_t *__restrict__ pos_of_slot,
                                                     const float *__restrict__ dl,
                                                     const float *__restrict__ gate, int T, int K,
                                                     int H, int E, float *__restrict__ dx,
                                                     int accumulate) {
    const int h = blockIdx.x * 256 + threadIdx.x;
    const int t0 = blockIdx.y * kMoeDxTokens;
    if (h >= H) return;
    float r[kMoeDxTokens];
#pragma unroll
    for (int i = 0; i < kMoeDxTokens; ++i) r[i] = 0.f;
    if (KT > 0 && t0 + kMoeDxTokens <= T) {
        constexpr int KK = KT > 0 ? KT : 1;
        float g[kMoeDxTokens][KK], old[kMoeDxTokens];
#pragma unroll
        for (int i = 0; i < kMoeDxTokens; ++i)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk)
                g[i][kk] = dxs[(int64_t)pos_of_slot[(int64_t)(t0 + i) * KK + kk] * H + h];
        if (accumulate) {
#pragma unroll
            for (int i = 0; i < kMoeDxTokens; ++i) old[i] = dx[(int64_t)(t0 + i) * H + h];
        }
        for (int e = 0; e < E; ++e) {
            const float gv = gate[(int64_t)h * E + e];
#pragma unroll
            for (int i = 0; i < kMoeDxTokens; ++i) r[i] += dl[(int64_t)(t0 + i) * E + e] * gv;
        }
#pragma unroll
        for (int i = 0; i < kMoeDxTokens; ++i) {
            float s = 0.f;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) s += g[i][kk];
            s += r[i];
            dx[(int64_t)(t0 + i) * H + h] = accumulate ? old[i] + s : s;
        }
        return;
    }
    for (int e = 0; e < E; ++e) {
        const float g = gate[(int64_t)h * E + e];
#pragma unroll
        for (int i = 0; i < kMoeDxTokens; ++i)
            if (t0 + i < T) r[i] += dl[(int64_t)(t0 + i) * E + e] * g;
    }
#pragma unroll
    for (int i = 0; i < kMoeDxTokens; ++i) {
        const int t = t0 + i;
        if (t >= T) break;
        float s = 0.f;
        for (int kk = 0; kk < K; ++kk) s += dxs[(int64_t)pos_of_slot[(int64_t)t * K + kk] * H + h];
        s += r[i];
        float *o = dx + (int64_t)t * H + h;
        *o = accumulate ? *o + s : s;
    }
}

}  // namespace

void fill_f32(hipStream_t s, float *y, float v, int64_t n) {
    if (n <= 0) return;
    fill_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(y, v, n);
    CATNN_HIP(hipGetLastError());
}

void fill_bf16_zero(hipStream_t s, bf16_t *y, int64_t n) {
    if (n <= 0) return;
    fill_bf16_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(y, n);
    CATNN_HIP(hipGetLastError());
}

void cast_f32_bf16(hipStream_t s, const float *x, bf16_t *y, int64_t n) {
    if (n <= 0) return;
    if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0)
        cast4_kernel<<<blocks_for(n / 4, 256 * 2), 256, 0, s>>>(reinterpret_cast<const float4 *>(x),
                                                                 reinterpret_cast<uint2 *>(y), n / 4);
    else
        cast_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(x, y, n);
    CATNN_HIP(hipGetLastError());
}

static bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

static dim3 tgrid(int rows, int cols) {
    return dim3((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
}

// The 16-byte path needs 16-byte aligned source and destination rows.
template <typename TS>
static void transpose_any(hipStream_t s, const TS *src, int64_t lds, const int32_t *rows_map, int div, int rows,
                          int cols, bf16_t *dst, int64_t ldd) {
    if (rows <= 0 || cols <= 0) return;
    CATNN_REQUIRE((rows + 63) / 64 < 65536, CATNN_ERR_SHAPE_MISMATCH, "transpose: too many rows");
    const bool vec = al16(src) && al16(dst) && (lds * (int64_t)sizeof(TS)) % 16 == 0 && ldd % 8 == 0;
    if (vec)
        transpose_vec_kernel<TS><<<tgrid(rows, cols), 256, 0, s>>>(src, lds, rows_map, div, rows, cols, dst, ldd);
    else
        transpose_kernel<TS><<<tgrid(rows, cols), 256, 0, s>>>(src, lds, rows_map, div, rows, cols, dst, ldd);
    CATNN_HIP(hipGetLastError());
}

void transpose_bf16(hipStream_t s, const bf16_t *src, int64_t lds, const int32_t *rows_map, int div,
                    int rows, int cols, bf16_t *dst, int64_t ldd) {
    transpose_any<bf16_t>(s, src, lds, rows_map, div, rows, cols, dst, ldd);
}

void transpose_f32_bf16(hipStream_t s, const float *src, int64_t lds, const int32_t *rows_map,
                        int div, int rows, int cols, bf16_t *dst, int64_t ldd) {
    transpose_any<float>(s, src, lds, rows_map, div, rows, cols, dst, ldd);
}

void split3_rows(hipStream_t s, const float *x, int64_t ldx, int64_t rows, int K, bf16_t *out,
                 int64_t ldo) {
    if (rows <= 0 || K <= 0) return;
    if (K % 4 == 0 && ldx % 4 == 0 && ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(out) & 7) == 0) {
        const dim3 grid((unsigned)((K / 4 + 255) / 256), (unsigned)std::min<int64_t>(rows, 65535));
        split3_rows4_kernel<<<grid, 256, 0, s>>>(reinterpret_cast<const float4 *>(x), ldx / 4, rows, K / 4,
                                                 reinterpret_cast<uint2 *>(out), ldo / 4);
    } else {
        split3_rows_kernel<<<blocks_for(rows * K, 256 * 4), 256, 0, s>>>(x, ldx, rows, K, out, ldo);
    }
    CATNN_HIP(hipGetLastError());
}

void transpose_split3(hipStream_t s, const float *w, int64_t ldw, int K, int N, bf16_t *out,
                      int64_t ldo) {
    if (K <= 0 || N <= 0) return;
    CATNN_REQUIRE((K + 63) / 64 < 65536, CATNN_ERR_SHAPE_MISMATCH, "transpose_split3: too many rows");
    transpose_split3_kernel<<<tgrid(K, N), 256, 0, s>>>(w, ldw, K, N, out, ldo);
    CATNN_HIP(hipGetLastError());
}

void ln_forward_train(hipStream_t s, const float *x, const float *g, const float *b, float *y,
                      bf16_t *yb, bf16_t *y3, float *mean, float *rstd, int64_t rows, int cols, float eps) {
    if (rows <= 0) return;
    auto al = [](const void *q, uintptr_t a) { return (reinterpret_cast<uintptr_t>(q) & (a - 1)) == 0; };
    const bool vec = cols % 4 == 0 && al(x, 16) && al(g, 16) && al(b, 16) && (!y || al(y, 16)) &&
                     (!yb || al(yb, 8)) && (!y3 || al(y3, 8));
    const unsigned blocks = (unsigned)((rows + 3) / 4);
    if (vec && cols == 1024) ln_fwd_kernel<true, 4><<<blocks, 256, 0, s>>>(x, g, b, y, yb, y3, mean, rstd, rows, cols, eps);
    else if (vec) ln_fwd_kernel<true><<<blocks, 256, 0, s>>>(x, g, b, y, yb, y3, mean, rstd, rows, cols, eps);
    else ln_fwd_kernel<false><<<blocks, 256, 0, s>>>(x, g, b, y, yb, y3, mean, rstd, rows, cols, eps);
    CATNN_HIP(hipGetLastError());
}

uint64_t ln_backward_scratch_bytes(int64_t rows, int cols) {
    const int64_t ng = (rows + kColRows - 1) / kColRows;
    return (uint64_t)ng * cols * 4 * 2;
}

void sum_parts(hipStream_t s, const float *parts, int np, int64_t n, float *out, bool accumulate) {
    CATNN_REQUIRE(np >= 1 && n % 4 == 0 && (reinterpret_cast<uintptr_t>(parts) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(out) & 15) == 0,
                  CATNN_ERR_SHAPE_MISMATCH, "sum_parts: needs 16-byte aligned rows of floats");
    if (n == 0) return;
    const int64_t n4 = n / 4;
    const unsigned blocks = (unsigned)std::min<int64_t>((n4 + 255) / 256, 4096);
    sum_parts_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<const float4 *>(parts), np, n4,
                                            reinterpret_cast<float4 *>(out), accumulate ? 1 : 0);
    CATNN_HIP(hipGetLastError());
}

static void reduce_partials(hipStream_t s, const float *part, int64_t ng, int cols, float *out,
                            bool accumulate) {
    reduce_partials_kernel<<<(unsigned)((cols + 63) / 64), 256, 0, s>>>(part, (int)ng, cols, out,
                                                                        accumulate ? 1 : 0);
    CATNN_HIP(hipGetLastError());
}

void ln_backward(hipStream_t s, const float *x, const float *g, const float *mean, const float *rstd,
                 const float *dy, float *dx, bool accumulate, float *dg, float *db, bool acc_params,
                 int64_t rows, int cols, float *scratch) {
    if (rows <= 0) return;
    const int64_t ng = (rows + kColRows - 1) / kColRows;
    CATNN_REQUIRE(ng < 65536, CATNN_ERR_SHAPE_MISMATCH, "layer_norm backward: too many rows");
    if (dx) {
        const unsigned blocks = (unsigned)((rows + 3) / 4);
        const int acc = accumulate ? 1 : 0;
        const bool v4 = al16(x) && al16(g) && al16(dy) && al16(dx);
        if (v4 && cols == 1024) ln_bwd_dx4_kernel<4><<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        else if (v4 && cols == 2048)
            ln_bwd_dx4_kernel<8><<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        else if (cols <= 256) ln_bwd_dx_kernel<4><<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        else if (cols <= 512) ln_bwd_dx_kernel<8><<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        else if (cols <= 1024) ln_bwd_dx_kernel<16><<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        else if (cols <= 2048) ln_bwd_dx_kernel<32><<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        else ln_bwd_dx_any_kernel<<<blocks, 256, 0, s>>>(x, g, mean, rstd, dy, dx, acc, rows, cols);
        CATNN_HIP(hipGetLastError());
    }
    float *pg = scratch, *pb = scratch + ng * cols;
    col_partials_kernel<true><<<dim3((cols + 255) / 256, (unsigned)ng), 256, 0, s>>>(dy, x, mean, rstd, rows,
                                                                                    cols, pg, pb);
    CATNN_HIP(hipGetLastError());
    reduce_partials(s, pg, ng, cols, dg, acc_params);
    reduce_partials(s, pb, ng, cols, db, acc_params);
}

uint64_t colsum_scratch_bytes(int64_t rows, int cols) {
    return (uint64_t)((rows + kColRows - 1) / kColRows) * cols * 4;
}

void colsum(hipStream_t s, const float *y, int64_t rows, int cols, float *out, bool accumulate,
            float *scratch) {
    if (rows <= 0 || cols <= 0) return;
    const int64_t ng = (rows + kColRows - 1) / kColRows;
    CATNN_REQUIRE(ng < 65536, CATNN_ERR_SHAPE_MISMATCH, "colsum: too many rows");
    col_partials_kernel<false><<<dim3((cols + 255) / 256, (unsigned)ng), 256, 0, s>>>(
        y, nullptr, nullptr, nullptr, rows, cols, scratch, nullptr);
    CATNN_HIP(hipGetLastError());
    reduce_partials(s, scratch, ng, cols, out, accumulate);
}

bool transpose_colsum(hipStream_t s, const float *y, int64_t rows, int cols, bf16_t *yt, int64_t ldt,
                      float *out, bool accumulate, float *scratch, bf16_t *yb) {
    if (rows <= 0 || cols <= 0) return true;
    if (rows % 64 != 0 || cols % 64 != 0 || !al16(y) || !al16(yt) || (yb && (reinterpret_cast<uintptr_t>(yb) & 7)) ||
        ldt % 8 != 0 || ldt < rows || rows / 64 >= 65536)
        return false;
    transpose_colsum_kernel<<<dim3((unsigned)(cols / 64), (unsigned)(rows / 64)), 256, 0, s>>>(
        y, cols, cols, yt, ldt, out ? scratch : nullptr, yb);
    CATNN_HIP(hipGetLastError());
    if (out) reduce_partials(s, scratch, rows / 64, cols, out, accumulate);
    return true;
}

void act_backward(hipStream_t s, const float *z, const float *dy, float *dx, int64_t n, int act,
                  bool accumulate) {
    if (n <= 0) return;
    act_bwd_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(z, dy, dx, n, act, accumulate ? 1 : 0);
    CATNN_HIP(hipGetLastError());
}

constexpr int kMseBlocks = 1024;

uint64_t mse_scratch_bytes() { return kMseBlocks * 4; }

void mse(hipStream_t s, const float *pred, const float *tgt, float *d, int64_t n, float *loss,
         float *scratch) {
    CATNN_REQUIRE(n > 0, CATNN_ERR_SHAPE_MISMATCH, "mse on empty tensors");
    auto al16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const int vec = n % 4 == 0 && al16(pred) && al16(tgt) && al16(d) ? 1 : 0;
    mse_kernel<<<kMseBlocks, 256, 0, s>>>(pred, tgt, d, n, scratch, vec);
    mse_finish_kernel<<<1, 256, 0, s>>>(scratch, kMseBlocks, n, loss);
    CATNN_HIP(hipGetLastError());
}

void rms_backward(hipStream_t s, const float *x, const float *w, const float *dy, float *dx, bool accumulate,
                  float *dw, int64_t rows, int cols, float eps, float *prod, float *colsum_scratch) {
    if (rows <= 0 || cols <= 0) return;
    CATNN_REQUIRE((rows + 3) / 4 < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "rmsnorm backward: too many rows");
    rms_bwd_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(x, w, dy, dx, accumulate ? 1 : 0, prod, rows, cols,
                                                                eps);
    CATNN_HIP(hipGetLastError());
    colsum(s, prod, rows, cols, dw, false, colsum_scratch);
}

uint64_t mix_scratch_bytes() { return (uint64_t)kMseBlocks * 4; }

void softmax_backward(hipStream_t s, const float *y, const float *dy, float *dx, bool accumulate, int64_t rows,
                      int cols) {
    if (rows <= 0 || cols <= 0) return;
    CATNN_REQUIRE((rows + 3) / 4 < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "softmax backward: too many rows");
    softmax_bwd_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(y, dy, dx, accumulate ? 1 : 0, rows, cols);
    CATNN_HIP(hipGetLastError());
}

void swiglu_h(hipStream_t s, const float *a, const float *c, float *h, int64_t n) {
    if (n <= 0) return;
    swiglu_h_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(a, c, h, n);
    CATNN_HIP(hipGetLastError());
}

void swiglu_dadc(hipStream_t s, const float *dh, const float *a, const float *c, bf16_t *da, bf16_t *dc, int64_t n) {
    if (n <= 0) return;
    swiglu_dadc_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(dh, a, c, da, dc, n);
    CATNN_HIP(hipGetLastError());
}

void mul_backward(hipStream_t s, const float *dy, const float *other, float *dx, bool accumulate, int64_t n) {
    if (n <= 0) return;
    mul_bwd_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(dy, other, dx, accumulate ? 1 : 0, n);
    CATNN_HIP(hipGetLastError());
}

void mix_backward(hipStream_t s, const float *a, const float *b, const float *gate, const float *dy, float *da,
                  bool acc_a, float *db, bool acc_b, int64_t n, float *dgate, float *parts) {
    if (n <= 0) return;
    mix_bwd_kernel<<<kMseBlocks, 256, 0, s>>>(a, b, gate, dy, da, acc_a ? 1 : 0, db, acc_b ? 1 : 0, n, parts);
    if (dgate) mix_bwd_finish_kernel<<<1, 256, 0, s>>>(parts, kMseBlocks, gate, dgate);
    CATNN_HIP(hipGetLastError());
}

void cross_entropy(hipStream_t s, const float *logits, const uint32_t *ids, int64_t rows, int V, float *d,
                   float *loss, float *row_loss) {
    CATNN_REQUIRE(rows > 0 && V > 0, CATNN_ERR_SHAPE_MISMATCH, "cross entropy on empty logits");
    CATNN_REQUIRE(rows < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "cross entropy: too many rows");
    ce_rows_kernel<<<(unsigned)rows, 256, 0, s>>>(logits, ids, rows, V, d, row_loss);
    // Σ of the row terms in a fixed order, divided by rows.
    mse_finish_kernel<<<1, 256, 0, s>>>(row_loss, (int)rows, rows, loss);
    CATNN_HIP(hipGetLastError());
}

void sgd(hipStream_t s, float *p, const float *g, int64_t ldg, int64_t rows, int cols, float lr,
         bf16_t *pb) {
    if (rows * cols <= 0) return;
    sgd_kernel<<<blocks_for(rows * cols, 256 * 4), 256, 0, s>>>(p, g, ldg, rows, cols, lr, pb);
    CATNN_HIP(hipGetLastError());
}

void sgd_multi(hipStream_t s, const SgdParam *table, int n, int tiles, const UpdateRule &u, bool use_grad) {
    if (n <= 0 || tiles <= 0) return;
    sgd_multi_kernel<<<(unsigned)tiles, 256, 0, s>>>(table, n, u, use_grad ? 1 : 0);
    CATNN_HIP(hipGetLastError());
}

float powi_f32(float b, int32_t t) {
#pragma clang fp contract(off)
    const bool recip = t < 0;
    uint32_t e = recip ? 0u - (uint32_t)t : (uint32_t)t;
    float r = 1.f;
    for (;;) {
        if (e & 1u) r *= b;
        e >>= 1;
        if (e == 0) break;
        b *= b;
    }
    return recip ? 1.f / r : r;
}

UpdateRule sgd_rule(float lr) {
    UpdateRule u{};
    u.adam = 0;
    u.lr = lr;
    return u;
}

// Adam::default (optim.rs:86-90) with the given lr; the step counter is
// AdamState.t saturating_add(1) and powi takes it `as i32` (optim.rs:98-103).
UpdateRule adam_rule(float lr, uint64_t t) {
#pragma clang fp contract(off)
    UpdateRule u{};
    u.adam = 1;
    u.lr = lr;
    u.beta1 = 0.9f;
    u.beta2 = 0.999f;
    u.eps = 1e-8f;
    u.b1t = 1.f - powi_f32(u.beta1, (int32_t)t);
    u.b2t = 1.f - powi_f32(u.beta2, (int32_t)t);
    return u;
}

void apply_update(hipStream_t s, const UpdateRule &u, float *p, const float *g, float *m, float *v,
                  int64_t n) {
    if (n <= 0) return;
    auto al = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const int vec = al(p) && al(g) && (!u.adam || (al(m) && al(v))) ? 1 : 0;
    apply_update_kernel<<<blocks_for(vec ? (n + 3) / 4 : n, 256), 256, 0, s>>>(u, p, g, m, v, n, vec);
    CATNN_HIP(hipGetLastError());
}

void router_backward(hipStream_t s, const int32_t *idx, const float *w, const float *dw,
                     const float *x, int T, int H, int E, int K, float *dl, float *dgate,
                     float *scratch) {
    CATNN_REQUIRE(E <= 64, CATNN_ERR_SHAPE_MISMATCH, "router backward: more than 64 experts");
    if (T <= 0) return;
    router_dlogits_kernel<<<(T + 255) / 256, 256, 0, s>>>(idx, w, dw, T, E, K, dl);
    const int ng = (T + kColRows - 1) / kColRows;
    CATNN_REQUIRE(ng < 65536, CATNN_ERR_SHAPE_MISMATCH, "router backward: too many tokens");
    const dim3 rgrid((unsigned)((H + 255) / 256), (unsigned)ng);
    if (E <= 4) router_dgate_rows_kernel<4><<<rgrid, 256, 0, s>>>(x, dl, T, H, E, scratch);
    else if (E <= 8) router_dgate_rows_kernel<8><<<rgrid, 256, 0, s>>>(x, dl, T, H, E, scratch);
    else if (E <= 16) router_dgate_rows_kernel<16><<<rgrid, 256, 0, s>>>(x, dl, T, H, E, scratch);
    else router_dgate_parts_kernel<<<dim3((unsigned)((H * E + 255) / 256), (unsigned)ng), 256, 0, s>>>(x, dl, T, H, E,
                                                                                                  scratch);
    CATNN_HIP(hipGetLastError());
    reduce_partials(s, scratch, ng, H * E, dgate, false);
}

uint64_t router_backward_scratch_bytes(int T, int H, int E) {
    return (uint64_t)((T + kColRows - 1) / kColRows) * H * E * 4;
}

void moe_slot_grads(hipStream_t s, const int32_t *slot_of_pos, const float *w, const float *y,
                    const float *dout, int K, int H, int n_pos, bf16_t *dys, float *dw) {
    if (n_pos <= 0) return;
    const bool v4 = (reinterpret_cast<uintptr_t>(y) & 15) == 0 && (reinterpret_cast<uintptr_t>(dout) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(dys) & 7) == 0;
    if (v4 && H == 1024)
        moe_slot_grad4_kernel<4><<<(unsigned)((n_pos + 3) / 4), 256, 0, s>>>(slot_of_pos, w, y, dout, K, H, n_pos,
                                                                            dys, dw);
    else
        moe_slot_grad_kernel<bf16_t><<<(unsigned)n_pos, 256, 0, s>>>(slot_of_pos, w, y, dout, K, H, n_pos, dys, dw);
    CATNN_HIP(hipGetLastError());
}

void moe_slot_grads_f32(hipStream_t s, const int32_t *slot_of_pos, const float *w, const float *y,
                        const float *dout, int K, int H, int n_pos, float *dys, float *dw) {
    if (n_pos <= 0) return;
    moe_slot_grad_kernel<float><<<(unsigned)n_pos, 256, 0, s>>>(slot_of_pos, w, y, dout, K, H, n_pos, dys, dw);
    CATNN_HIP(hipGetLastError());
}

void split6_rows(hipStream_t s, const float *x, int64_t ldx, int64_t rows, int K, bool role_b, bf16_t *out,
                 int64_t ldo) {
    if (rows <= 0 || K <= 0) return;
    CATNN_REQUIRE(ldo >= 6 * (int64_t)K && ldo % 2 == 0 && (reinterpret_cast<uintptr_t>(out) & 3) == 0,
                  CATNN_ERR_SHAPE_MISMATCH, "split6: output rows");
    split6_rows_kernel<<<blocks_for(rows * K, 256 * 4), 256, 0, s>>>(x, ldx, rows, K, role_b ? 1 : 0, out, ldo);
    CATNN_HIP(hipGetLastError());
}

void split6_transpose(hipStream_t s, const float *x, int64_t ldx, const int32_t *rows_map, int div, int rows,
                      int cols, bool role_b, bf16_t *out, int64_t ldo) {
    if (rows <= 0 || cols <= 0) return;
    CATNN_REQUIRE((rows + 63) / 64 < 65536, CATNN_ERR_SHAPE_MISMATCH, "split6 transpose: too many rows");
    CATNN_REQUIRE(ldo >= 6 * (int64_t)rows && ldo % 2 == 0 && (reinterpret_cast<uintptr_t>(out) & 3) == 0,
                  CATNN_ERR_SHAPE_MISMATCH, "split6 transpose: output rows");
    split6_transpose_kernel<<<tgrid(rows, cols), 256, 0, s>>>(x, ldx, rows_map, div, rows, cols, role_b ? 1 : 0,
                                                              out, ldo);
    CATNN_HIP(hipGetLastError());
}

void scale_i32(hipStream_t s, const int32_t *src, int n, int factor, int32_t *dst) {
    if (n <= 0) return;
    scale_i32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(src, n, factor, dst);
    CATNN_HIP(hipGetLastError());
}

void swiglu_dadc_f32(hipStream_t s, const float *dh, const float *a, const float *c, float *da, float *dc,
                     int64_t n) {
    if (n <= 0) return;
    swiglu_dadc_f32_kernel<<<blocks_for(n, 256 * 4), 256, 0, s>>>(dh, a, c, da, dc, n);
    CATNN_HIP(hipGetLastError());
}

void moe_dx(hipStream_t s, const float *dxs, const int32_t *pos_of_slot, const float *dl,
            const float *gate, int T, int K, int H, int E, float *dx, bool accumulate) {
    if (T <= 0) return;
    CATNN_REQUIRE((T + kMoeDxTokens - 1) / kMoeDxTokens < 65536, CATNN_ERR_SHAPE_MISMATCH, "moe dx: too many tokens");
    const dim3 grid((unsigned)((H + 255) / 256), (unsigned)((T + kMoeDxTokens - 1) / kMoeDxTokens));
    const int acc = accumulate ? 1 : 0;
    if (K == 2) moe_dx_kernel<2><<<grid, 256, 0, s>>>(dxs, pos_of_slot, dl, gate, T, K, H, E, dx, acc);
    else if (K == 1) moe_dx_kernel<1><<<grid, 256, 0, s>>>(dxs, pos_of_slot, dl, gate, T, K, H, E, dx, acc);
    else moe_dx_kernel<0><<<grid, 256, 0, s>>>(dxs, pos_of_slot, dl, gate, T, K, H, E, dx, acc);
    CATNN_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace catnn
