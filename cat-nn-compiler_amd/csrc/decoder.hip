// The decoder ops of Mixtral-style graphs: RMSNorm, the token-embedding
// gather, rotary position embedding, GQA attention, dense SwiGLU, the LM head
// and the sigmoid-gated mix.  The row and elementwise kernels stream their
// operands once with 16-byte accesses where the layout allows; the matrix
// work runs on the fp32 MFMA GEMM (gemm_f32.hip) and the flash attention core
// (attention.hip).
//
// Replaces moe::rmsnorm (crates/catnn-compile/src/kernel/moe.rs:17-32), the
// Embedding arm of eval_cpu (kernel/mod.rs:81-96) over moe::embedding
// (moe.rs:34-45), moe::gqa with apply_rope (moe.rs:47-136), moe::swiglu
// (moe.rs:159-174), moe::lm_head (moe.rs:325-333) and deepseek::mix
// (deepseek.rs:229-239).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.hpp"
#include "devmath.hpp"
#include "gemm_f32.hpp"
#include "kernels.hpp"
#include "train_ops.hpp"

namespace catnn {
namespace k {

namespace {

constexpr int kThreads = 256;

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

unsigned blocks_for(int64_t n, int64_t per_block) {
    const int64_t b = (n + per_block - 1) / per_block;
    CATNN_REQUIRE(b < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "decoder op: grid too large");
    return (unsigned)std::max<int64_t>(b, 1);
}

// One wavefront per row, the row held in registers as NV float4 per lane.
// y = x · (1 / sqrt(mean(x²) + eps)) · w, multiplied in that order.  FULL:
// cols == 256·NV, so the w loads of all chunks go out before the first
// store; the row sum uses the DPP reduction.
template <int NV, bool FULL>
__global__ __launch_bounds__(256) void rms_norm_reg_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ w,
                                                           float *__restrict__ y, int64_t rows,
                                                           int cols, float eps) {
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
        v[i] = (FULL || c < c4) ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        s += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
    }
    const float inv = 1.0f / sqrtf(wave_sum_dpp(s) / (float)cols + eps);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 *yr = reinterpret_cast<float4 *>(y + row * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + i * 64;
        if (FULL || c < c4) {
            const float4 g = w4[c];
            yr[c] = make_float4(v[i].x * inv * g.x, v[i].y * inv * g.y, v[i].z * inv * g.z,
                                v[i].w * inv * g.w);
        }
    }
}

// Any width or alignment: one wavefront per row, two passes over the row.
__global__ __launch_bounds__(256) void rms_norm_any_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ w,
                                                           float *__restrict__ y, int64_t rows,
                                                           int64_t cols, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * cols;
    float s = 0.f;
    for (int64_t c = lane; c < cols; c += 64) s += xr[c] * xr[c];
    const float inv = 1.0f / sqrtf(wave_sum(s) / (float)cols + eps);
    float *yr = y + row * cols;
    for (int64_t c = lane; c < cols; c += 64) yr[c] = xr[c] * inv * w[c];
}

// Token id of an f32 id value as the reference converts it: rounded half
// away from zero, clamped to [0, u32::MAX] (NaN → 0), saturating.
__device__ __forceinline__ int64_t token_id(float v) {
    v = roundf(v);
    if (!(v >= 0.f)) return 0;
    if (v >= 4294967296.0f) return 4294967295ll;
    return (int64_t)v;
}

// One wavefront per token copies its table row.  An id ≥ vocab sets *bad and
// writes zeros (the table is never read out of range).  Rows of 1024 floats
// take embedding_pair_kernel instead.
template <bool VEC>
__global__ __launch_bounds__(256) void embedding_kernel(const float *__restrict__ ids, int64_t n,
                                                        const float *__restrict__ table,
                                                        int64_t vocab, int64_t hidden,
                                                        float *__restrict__ y, int *__restrict__ bad) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const int64_t id = token_id(ids[t]);
    float *yr = y + t * hidden;
    if (id >= vocab) {
        if (lane == 0) *bad = 1;
        for (int64_t c = lane; c < hidden; c += 64) yr[c] = 0.f;
        return;
    }
    const float *src = table + id * hidden;
    if (VEC) {
        // Four 16-byte loads in flight per lane before their stores.
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        float4 *y4 = reinterpret_cast<float4 *>(yr);
        const int64_t nq = hidden / 4;
        int64_t c = lane;
        for (; c + 192 < nq; c += 256) {
            const float4 a = s4[c], b = s4[c + 64], d = s4[c + 128], e = s4[c + 192];
            y4[c] = a;
            y4[c + 64] = b;
            y4[c + 128] = d;
            y4[c + 192] = e;
        }
        for (; c < nq; c += 64) y4[c] = s4[c];
    } else {
        for (int64_t c = lane; c < hidden; c += 64) yr[c] = src[c];
    }
}

// Rows of exactly 1024 floats (16-byte aligned): one wavefront copies two
// tokens' rows, all eight of a lane's 16-byte loads issued before its
// stores.  Same id conversion and bad-id handling as embedding_kernel.
// (A variant with the token index made wavefront-uniform — ids through the
// scalar cache, row loads under uniform branches — ran the same or slower
// with the table and ids read from HBM; nontemporal table loads ran 14 %
// slower in the decoder forward; loads always from a valid row (row 0 for
// a bad id, zeroed after), which removes the pick between the table and a
// zero vector in scratch, averaged 15.0 against 14.0 us; none kept.)
__global__ __launch_bounds__(256) void embedding_pair_kernel(const float *__restrict__ ids, int64_t n,
                                                             const float4 *__restrict__ table, int64_t vocab,
                                                             float4 *__restrict__ y, int *__restrict__ bad) {
    constexpr int kQ = 256;  // float4 per row
    const int lane = threadIdx.x & 63;
    const int64_t t0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    if (t0 >= n) return;
    const bool two = t0 + 1 < n;
    const int64_t id0 = token_id(ids[t0]);
    const int64_t id1 = two ? token_id(ids[t0 + 1]) : 0;
    const bool ok0 = id0 < vocab, ok1 = two && id1 < vocab;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a[j] = ok0 ? table[id0 * kQ + lane + 64 * j] : z;
        b[j] = ok1 ? table[id1 * kQ + lane + 64 * j] : z;
    }
    if (lane == 0 && (!ok0 || (two && !ok1))) *bad = 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) y[t0 * kQ + lane + 64 * j] = a[j];
    if (two) {
#pragma unroll
        for (int j = 0; j < 4; ++j) y[(t0 + 1) * kQ + lane + 64 * j] = b[j];
    }
}

// embedding_backward (adjoint.rs:187-197): dW [vocab, hidden] gets, in row
// id_t, Σ_t dy[t] in token order.  First the ids as integers (the forward's
// conversion; an id ≥ vocab, which the forward refuses, becomes −1) and a
// mark per vocabulary row that occurs; then one block per row: unmarked
// rows are zeroed, marked rows add their tokens' cotangent rows in token
// order from zero — the reference's order, bit for bit, with no atomics.
__global__ void fill_int_kernel(int *__restrict__ p, int v, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ void embedding_bwd_ids_kernel(const float *__restrict__ ids, int64_t n, int64_t vocab,
                                         int *__restrict__ idi, int *__restrict__ hit) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const int64_t id = token_id(ids[t]);
    if (id < vocab) {
        idi[t] = (int)id;
        hit[id] = 1;
    } else {
        idi[t] = -1;
    }
}

__global__ __launch_bounds__(256) void embedding_bwd_rows_kernel(const int *__restrict__ idi, int64_t n,
                                                                 const float *__restrict__ dy, int64_t hidden,
                                                                 int64_t vocab, const int *__restrict__ hit,
                                                                 float *__restrict__ dw) {
#pragma clang fp contract(off)
    for (int64_t v = blockIdx.x; v < vocab; v += gridDim.x) {
        float *o = dw + v * hidden;
        if (!hit[v]) {
            for (int64_t c = threadIdx.x; c < hidden; c += 256) o[c] = 0.f;
            continue;
        }
        for (int64_t c0 = 0; c0 < hidden; c0 += 1024) {
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int64_t t = 0; t < n; ++t) {
                if (idi[t] != (int)v) continue;  // the same t for every thread of the block
                const float *d = dy + t * hidden;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t c = c0 + threadIdx.x + 256 * j;
                    if (c < hidden) acc[j] += d[c];
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t c = c0 + threadIdx.x + 256 * j;
                if (c < hidden) o[c] = acc[j];
            }
        }
    }
}

// RoPE table [S, hd/2] of (cos, sin): angle pos · θ^(−2i/hd) in f64, the
// sine and cosine rounded to f32 (moe.rs:47-53).
__global__ void rope_table_kernel(float2 *__restrict__ tab, int64_t n, int half, int hd, double theta) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int64_t pos = idx / half;
    const int i = (int)(idx % half);
    const double freq = 1.0 / pow(theta, 2.0 * (double)i / (double)hd);
    const double ang = (double)pos * freq;
    tab[idx] = make_float2((float)cos(ang), (float)sin(ang));
}

// Rotates the pairs (2i, 2i+1) of `heads` consecutive heads of width hd at
// the start of each row (row r is position r mod S), in place.
// `sign` −1 rotates by −angle (sin negated after rounding).
__global__ void rope_apply_kernel(float *__restrict__ qk, int64_t ld, int64_t rows, int S, int heads,
                                  int hd, const float2 *__restrict__ tab, float sign) {
#pragma clang fp contract(off)
    const int half = hd / 2;
    const int64_t per_row = (int64_t)heads * half;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * per_row) return;
    const int64_t r = idx / per_row;
    const int p = (int)(idx - r * per_row);
    const int head = p / half, i = p - head * half;
    const float2 cs = tab[(r % S) * half + i];
    const float sn = sign * cs.y;
    float *q = qk + r * ld + (int64_t)head * hd + 2 * i;
    const float a = q[0], b = q[1];
    q[0] = a * cs.x - b * sn;
    q[1] = a * sn + b * cs.x;
}

// The same rotation, two pairs a thread with 16-byte accesses (hd a multiple
// of 4, rows and the table 16-byte aligned): (cos, sin) of pairs i and i+1
// come as one float4.
__global__ void rope_apply2_kernel(float *__restrict__ qk, int64_t ld, int64_t rows, int S, int heads,
                                   int hd, const float4 *__restrict__ tab, float sign) {
#pragma clang fp contract(off)
    const int half = hd / 2;
    const int64_t per_row = (int64_t)heads * (half / 2);
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * per_row) return;
    const int64_t r = idx / per_row;
    const int p = 2 * (int)(idx - r * per_row);
    const int head = p / half, i = p - head * half;
    const float4 cs = tab[((r % S) * half + i) / 2];
    const float s0 = sign * cs.y, s1 = sign * cs.w;
    float4 *q = reinterpret_cast<float4 *>(qk + r * ld + (int64_t)head * hd + 2 * i);
    const float4 v = *q;
    float4 o;
    o.x = v.x * cs.x - v.y * s0;
    o.y = v.x * s0 + v.y * cs.x;
    o.z = v.z * cs.z - v.w * s1;
    o.w = v.z * s1 + v.w * cs.z;
    *q = o;
}

// y = σ(g)·a + (1 − σ(g))·b with σ(g) = 1 / (1 + e^(−g)), g = gate[0].
__global__ void mix_kernel(const float *__restrict__ a, const float *__restrict__ b,
                           const float *__restrict__ gate, float *__restrict__ y, int64_t n) {
#pragma clang fp contract(off)
    const float g = gate ? gate[0] : 0.f;
    const float s = 1.0f / (1.0f + expf(-g));
    const float r = 1.0f - s;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = s * a[i] + r * b[i];
}

// dst [C, R] = srcᵀ for src [R, C]: 32×32 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float *__restrict__ src, int64_t R,
                                                            int64_t C, float *__restrict__ dst,
                                                            int64_t tiles_c) {
    __shared__ float t[32][33];
    const int64_t tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int k = ty; k < 32; k += 8) {
        const int64_t r = tr * 32 + k, c = tc * 32 + tx;
        if (r < R && c < C) t[k][tx] = src[r * C + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int64_t c = tc * 32 + k, r = tr * 32 + tx;
        if (r < R && c < C) dst[c * R + r] = t[tx][k];
    }
}

}  // namespace

void rms_norm_f32(hipStream_t s, const float *x, const float *w, float *y, int64_t rows, int64_t cols,
                  float eps) {
    if (rows <= 0 || cols <= 0) return;
    const unsigned grid = blocks_for(rows, 4);
    const int64_t c4 = cols / 4;
    if (cols % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(y) && c4 <= 64 * 16) {
        const int c = (int)cols;
        auto launch = [&](auto nv_c) {
            constexpr int NV = decltype(nv_c)::value;
            if (c4 == 64 * NV) rms_norm_reg_kernel<NV, true><<<grid, kThreads, 0, s>>>(x, w, y, rows, c, eps);
            else rms_norm_reg_kernel<NV, false><<<grid, kThreads, 0, s>>>(x, w, y, rows, c, eps);
        };
        if (c4 <= 64) launch(std::integral_constant<int, 1>{});
        else if (c4 <= 128) launch(std::integral_constant<int, 2>{});
        else if (c4 <= 256) launch(std::integral_constant<int, 4>{});
        else if (c4 <= 512) launch(std::integral_constant<int, 8>{});
        else launch(std::integral_constant<int, 16>{});
    } else {
        rms_norm_any_kernel<<<grid, kThreads, 0, s>>>(x, w, y, rows, cols, eps);
    }
    CATNN_HIP(hipGetLastError());
}

void embedding_f32(hipStream_t s, const float *ids, int64_t n, const float *table, int64_t vocab,
                   int64_t hidden, float *y, int *bad) {
    if (n <= 0 || hidden <= 0) return;
    if (hidden == 1024 && aligned16(table) && aligned16(y)) {
        embedding_pair_kernel<<<blocks_for((n + 1) / 2, 4), kThreads, 0, s>>>(
            ids, n, reinterpret_cast<const float4 *>(table), vocab, reinterpret_cast<float4 *>(y), bad);
        CATNN_HIP(hipGetLastError());
        return;
    }
    const unsigned grid = blocks_for(n, 4);
    if (hidden % 4 == 0 && aligned16(table) && aligned16(y))
        embedding_kernel<true><<<grid, kThreads, 0, s>>>(ids, n, table, vocab, hidden, y, bad);
    else
        embedding_kernel<false><<<grid, kThreads, 0, s>>>(ids, n, table, vocab, hidden, y, bad);
    CATNN_HIP(hipGetLastError());
}

void embedding_backward(hipStream_t s, const float *ids, int64_t n, const float *dy, int64_t vocab, int64_t hidden,
                        float *dw, int *idi, int *hit) {
    if (vocab <= 0 || hidden <= 0) return;
    CATNN_REQUIRE(vocab < (1ll << 31) && n < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "embedding backward: size");
    fill_int_kernel<<<std::min<unsigned>(blocks_for(vocab, kThreads), 4096u), kThreads, 0, s>>>(hit, 0, vocab);
    if (n > 0) embedding_bwd_ids_kernel<<<blocks_for(n, kThreads), kThreads, 0, s>>>(ids, n, vocab, idi, hit);
    embedding_bwd_rows_kernel<<<(unsigned)std::min<int64_t>(vocab, 65536), kThreads, 0, s>>>(idi, n, dy, hidden, vocab,
                                                                                            hit, dw);
    CATNN_HIP(hipGetLastError());
}

void mix_f32(hipStream_t s, const float *a, const float *b, const float *gate, float *y, int64_t n) {
    if (n <= 0) return;
    mix_kernel<<<std::min<unsigned>(blocks_for(n, kThreads * 4), 1u << 20), kThreads, 0, s>>>(a, b, gate,
                                                                                              y, n);
    CATNN_HIP(hipGetLastError());
}

void transpose_f32(hipStream_t s, const float *src, int64_t rows, int64_t cols, float *dst) {
    if (rows <= 0 || cols <= 0) return;
    const int64_t tr = (rows + 31) / 32, tc = (cols + 31) / 32;
    transpose_f32_kernel<<<blocks_for(tr * tc, 1), kThreads, 0, s>>>(src, rows, cols, dst, tc);
    CATNN_HIP(hipGetLastError());
}

static int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

void rope_table(hipStream_t s, float *tab, int64_t S, int64_t hd, double theta) {
    const int half = (int)(hd / 2);
    const int64_t nt = S * half;
    if (nt <= 0) return;
    rope_table_kernel<<<blocks_for(nt, kThreads), kThreads, 0, s>>>(reinterpret_cast<float2 *>(tab), nt, half,
                                                                      (int)hd, theta);
    CATNN_HIP(hipGetLastError());
}

void rope_apply(hipStream_t s, float *qk, int64_t ld, int64_t rows, int64_t S, int64_t heads, int64_t hd,
                const float *tab, float sign) {
    const int half = (int)(hd / 2);
    const int64_t np = rows * heads * half;
    if (np <= 0) return;
    CATNN_REQUIRE(S > 0 && heads * hd <= ld, CATNN_ERR_SHAPE_MISMATCH, "rope: heads exceed the row");
    if (half % 2 == 0 && ld % 4 == 0 && aligned16(qk) && aligned16(tab))
        rope_apply2_kernel<<<blocks_for(np / 2, kThreads), kThreads, 0, s>>>(
            qk, ld, rows, (int)S, (int)heads, (int)hd, reinterpret_cast<const float4 *>(tab), sign);
    else
        rope_apply_kernel<<<blocks_for(np, kThreads), kThreads, 0, s>>>(
            qk, ld, rows, (int)S, (int)heads, (int)hd, reinterpret_cast<const float2 *>(tab), sign);
    CATNN_HIP(hipGetLastError());
}

GqaLayout gqa_layout(int64_t tokens, int64_t seq, int64_t n_heads, int64_t n_kv, int64_t head_dim) {
    GqaLayout L;
    L.qkv_ld = (n_heads + 2 * n_kv) * head_dim;
    L.qkv = 0;
    L.ctx = round_up(tokens * L.qkv_ld, 64);
    L.rope = L.ctx + round_up(tokens * n_heads * head_dim, 64);
    L.floats = L.rope + round_up(seq * (head_dim / 2) * 2, 64);
    return L;
}

void gqa_f32(hipStream_t s, const float *x, const float *wqkv, const float *wq, const float *wk,
             const float *wv, const float *wo, int64_t B, int64_t S, int64_t D, int64_t n_heads,
             int64_t n_kv, int64_t head_dim, double theta, int64_t window, const float *residual,
             float *y, float *scratch, const GqaLayout &L) {
    CATNN_REQUIRE(n_heads > 0 && n_kv > 0 && head_dim > 0 && n_heads % n_kv == 0,
                  CATNN_ERR_SHAPE_MISMATCH, "gqa: n_heads must be a positive multiple of n_kv_heads");
    const int64_t T = B * S;
    if (T == 0) return;
    const int64_t QW = n_heads * head_dim, KW = n_kv * head_dim, LD = L.qkv_ld;
    float *qkv = scratch + L.qkv, *ctx = scratch + L.ctx;
    float2 *tab = reinterpret_cast<float2 *>(scratch + L.rope);
    if (wqkv) {
        linear_f32(s, x, D, wqkv, LD, nullptr, nullptr, 0, qkv, LD, T, D, LD, ACT_NONE);
    } else {
        linear_f32(s, x, D, wq, QW, nullptr, nullptr, 0, qkv, LD, T, D, QW, ACT_NONE);
        linear_f32(s, x, D, wk, KW, nullptr, nullptr, 0, qkv + QW, LD, T, D, KW, ACT_NONE);
        linear_f32(s, x, D, wv, KW, nullptr, nullptr, 0, qkv + QW + KW, LD, T, D, KW, ACT_NONE);
    }
    rope_table(s, reinterpret_cast<float *>(tab), S, head_dim, theta);
    rope_apply(s, qkv, LD, T, S, n_heads + n_kv, head_dim, reinterpret_cast<const float *>(tab), 1.0f);
    attention_core_gqa_f32(s, qkv, qkv + QW, qkv + QW + KW, LD, LD, n_heads / n_kv, window, ctx, QW, B,
                           S, n_heads, head_dim);
    linear_f32(s, ctx, QW, wo, D, nullptr, residual, D, y, D, T, QW, D, ACT_NONE);
}

void swiglu_f32(hipStream_t s, const float *x, const float *w1, const float *w3, const float *w2,
                int64_t T, int64_t H, int64_t I, const float *residual, float *y, float *h) {
    if (T <= 0) return;
    CATNN_REQUIRE(T < (1ll << 31) && H < (1ll << 31) && I < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH,
                  "swiglu: dimension exceeds 2^31");
    GemmParams p{};
    p.A = x;
    p.lda = H;
    p.a_row_div = 1;
    p.B = w1;
    p.B2 = w3;
    p.ldb = I;
    p.C = h;
    p.ldc = I;
    p.M = (int)T;
    p.N = (int)I;
    p.K = (int)H;
    gemm_launch(s, p, true);  // h = silu(x·w1) · (x·w3)
    linear_f32(s, h, I, w2, H, nullptr, residual, H, y, H, T, I, H, ACT_NONE);
}

}  // namespace k
}  // namespace catnn
