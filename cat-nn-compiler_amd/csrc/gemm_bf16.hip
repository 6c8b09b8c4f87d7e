// bf16 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x16_bf16), fp32
// accumulation, for the training step (forward and backward of Linear,
// the attention projections and the MoE experts).
//
// C[M,N] = Σ_k A[m][k]·B[n][k] with A [M,K] and B [N,K] both k-contiguous.
// MFMA 32x32x16 bf16 operand layout (checked on the device): lane l
// supplies A[l%32][8(l/32) + j] and B[8(l/32) + j][l%32] for j = 0..7 —
// eight consecutive k values, one 16-byte LDS read per operand — and
// accumulator r of lane l is C[8(r/4) + 4(l/32) + r%4][l%32].
//
// Block: 256 threads, 2×2 wavefronts of 64×64 (2×2 MFMA blocks), BK = 32
// (two k16 steps), A and B tiles staged in LDS (row stride BK+8 bf16, so
// eight lanes' 16-byte reads hit distinct banks), double-buffered behind
// register prefetch.  Epilogues and grids are listed in gemm_bf16.hpp.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "devmath.hpp"
#include "gemm_bf16.hpp"

namespace catnn {
namespace k {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BM = 128, BN = 128, BK = 32, LDT = BK + 8;

struct Smem {
    bf16_t a[2][BM][LDT];
    bf16_t b[2][BN][LDT];
};

__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float((uint32_t)v << 16); }

// Round to nearest even; NaN stays NaN.
__device__ __forceinline__ bf16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
    return (bf16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float gelu_grad(float z) {
    const float C = 0.044715f, kk = 0.797884523868560791f;
    const float u = kk * (z + C * z * z * z);
    const float t = tanhf(u);
    const float du = kk * (1.0f + 3.0f * C * z * z);
    return 0.5f * (1.0f + t) + 0.5f * z * (1.0f - t * t) * du;
}

__device__ __forceinline__ float silu_grad(float x) {
    const float s = 1.0f / (1.0f + expf(-x));
    return s + x * s * (1.0f - s);
}

template <bool VEC, bool DUAL>
__device__ __forceinline__ void tile(Smem &sm, const GemmBf16Params &p, const bf16_t *__restrict__ B,
                                     const bf16_t *__restrict__ B2, int row0, int row_end, int col0,
                                     int k_lo, int k_hi, float *__restrict__ C32) {
    constexpr int FM = 2, FN = 2;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lg = lane >> 5;
    const int N = p.N;

    // Load assignments: 2 × 16 B of A and of B per thread per chunk.
    const bf16_t *a_src[2];
    bool a_ok[2];
    int a_r[2], a_c[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = tid + it * 256;
        a_r[it] = idx >> 2;
        a_c[it] = (idx & 3) * 8;
        const int gr = row0 + a_r[it];
        a_ok[it] = gr < row_end;
        int src = gr;
        if (a_ok[it] && p.a_rows) src = p.a_rows[gr] / p.a_row_div;
        a_src[it] = p.A + (int64_t)(a_ok[it] ? src : 0) * p.lda;
    }
    const bf16_t *b_src[2];
    bool b_ok[2];
    int b_r[2], b_c[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = tid + it * 256;
        b_r[it] = idx >> 2;
        b_c[it] = (idx & 3) * 8;
        int n;
        const bf16_t *base;
        if (DUAL) {
            const bool second = b_r[it] >= BN / 2;
            n = col0 + b_r[it] - (second ? BN / 2 : 0);
            base = second ? B2 : B;
        } else {
            n = col0 + b_r[it];
            base = B;
        }
        b_ok[it] = n < N;
        b_src[it] = base + (int64_t)(b_ok[it] ? n : 0) * p.ldb;
    }

    // 8 consecutive k values of one row: one 16-byte load when all 8 are in
    // range and aligned, element loads (zero past k_hi) otherwise.
    auto load8 = [&](const bf16_t *src, bool ok, int kk) -> uint4 {
        if (!ok || kk >= k_hi) return make_uint4(0, 0, 0, 0);
        if (VEC && kk + 8 <= k_hi) return *reinterpret_cast<const uint4 *>(src + kk);
        uint16_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = kk + j < k_hi ? src[kk + j] : 0;
        return make_uint4(v[0] | (uint32_t)v[1] << 16, v[2] | (uint32_t)v[3] << 16,
                          v[4] | (uint32_t)v[5] << 16, v[6] | (uint32_t)v[7] << 16);
    };
    uint4 ra[2], rb[2];
    auto gload = [&](int k0) {
#pragma unroll
        for (int it = 0; it < 2; ++it) ra[it] = load8(a_src[it], a_ok[it], k0 + a_c[it]);
#pragma unroll
        for (int it = 0; it < 2; ++it) rb[it] = load8(b_src[it], b_ok[it], k0 + b_c[it]);
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            *reinterpret_cast<uint4 *>(&sm.a[buf][a_r[it]][a_c[it]]) = ra[it];
            *reinterpret_cast<uint4 *>(&sm.b[buf][b_r[it]][b_c[it]]) = rb[it];
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

    auto compute = [&](int buf) {
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
                af[mi] = *reinterpret_cast<const bf16x8 *>(&sm.a[buf][wm * 64 + mi * 32 + lr][s * 16 + 8 * lg]);
#pragma unroll
            for (int ni = 0; ni < FN; ++ni) {
                const int row = DUAL ? (ni * (BN / 2) + wn * 32 + lr) : (wn * 64 + ni * 32 + lr);
                bfr[ni] = *reinterpret_cast<const bf16x8 *>(&sm.b[buf][row][s * 16 + 8 * lg]);
            }
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
        }
    };

    const int nk = (k_hi - k_lo + BK - 1) / BK;
    if (nk > 0) {
        gload(k_lo);
        sstore(0);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            const int buf = kt & 1;
            const bool more = kt + 1 < nk;
            if (more) gload(k_lo + (kt + 1) * BK);
            compute(buf);
            if (more) sstore(buf ^ 1);
            __syncthreads();
        }
    }

#pragma unroll
    for (int mi = 0; mi < FM; ++mi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
            if (row >= row_end) continue;
            if (DUAL) {
                const int col = col0 + wn * 32 + lr;
                if (col >= N) continue;
                const float a = acc[mi][0][r], c = acc[mi][1][r];
                const int64_t so = (int64_t)row * p.lds + col;
                if (p.S1) p.S1[so] = f2bf(a);
                if (p.S2) p.S2[so] = f2bf(c);
                p.Cb[(int64_t)row * p.ldcb + col] = f2bf(silu(a) * c);
                continue;
            }
#pragma unroll
            for (int ni = 0; ni < FN; ++ni) {
                const int col = col0 + wn * 64 + ni * 32 + lr;
                if (col >= N) continue;
                float v = acc[mi][ni][r];
                if (p.epi == EPI_LINEAR) {
                    if (p.bias) v += p.bias[col];
                    if (p.Z) p.Z[(int64_t)row * p.ldz + col] = v;
                    v = apply_act(v, p.act);
                    if (p.R) v = p.R[(int64_t)row * p.ldr + col] + v;
                } else if (p.epi == EPI_GELU_BWD) {
                    v *= gelu_grad(p.Z[(int64_t)row * p.ldz + col]);
                } else if (p.epi == EPI_SWIGLU_BWD) {
                    const int64_t so = (int64_t)row * p.lds + col;
                    const float a = bf2f(p.S1[so]), c = bf2f(p.S2[so]);
                    p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v * c * silu_grad(a));
                    p.Cb2[(int64_t)row * p.ldcb + col] = f2bf(v * silu(a));
                    continue;
                }
                if (C32) {
                    float *dst = C32 + (int64_t)row * p.ldc32 + col;
                    *dst = p.accumulate ? *dst + v : v;
                }
                if (p.Cb) p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v);
            }
        }
    }
}

template <bool VEC, bool DUAL>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(GemmBf16Params p) {
    __shared__ Smem sm;
    const int bn_out = DUAL ? BN / 2 : BN;
    const int tiles_n = (p.N + bn_out - 1) / bn_out;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    if (p.grid == GRID_PLAIN) {
        const int tiles_m = (p.M + BM - 1) / BM;
        int tm, tn;
        grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
        tile<VEC, DUAL>(sm, p, p.B, p.B2, tm * BM, p.M, tn * bn_out, 0, p.K, p.C32);
    } else if (p.grid == GRID_ROWS) {
        int tm, tn;
        grouped_tile(lid, p.max_tiles, tiles_n, 8, tm, tn);
        if (tm >= *p.n_tiles) return;
        const int e = p.tile_expert[tm];
        const int end = p.seg_counts ? p.seg_offsets[e] + p.seg_counts[e] : p.seg_offsets[e + 1];
        tile<VEC, DUAL>(sm, p, p.B_e[e], DUAL ? p.B2_e[e] : nullptr, p.tile_row0[tm], end,
                        tn * bn_out, 0, p.K, p.C32);
    } else {  // GRID_SEGK: expert e = blockIdx.y reduces over its own K segment
        const int tiles_m = (p.M + BM - 1) / BM;
        int tm, tn;
        grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
        const int e = blockIdx.y;
        const int lo = p.seg_offsets[e];
        const int hi = p.seg_counts ? lo + p.seg_counts[e] : p.seg_offsets[e + 1];
        tile<VEC, DUAL>(sm, p, p.B, nullptr, tm * BM, p.M, tn * bn_out, lo, hi, p.C_e[e]);
    }
}

bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

int gemm_bf16_tile_rows() { return BM; }

void gemm_bf16_launch(hipStream_t s, const GemmBf16Params &p) {
    CATNN_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, CATNN_ERR_SHAPE_MISMATCH, "bf16 gemm: dims");
    const bool dual = p.epi == EPI_SWIGLU_FWD;
    CATNN_REQUIRE(!dual || p.Cb, CATNN_ERR_INVALID_ARGUMENT, "swiglu epilogue needs Cb");
    CATNN_REQUIRE(p.epi != EPI_SWIGLU_BWD || (p.Cb && p.Cb2 && p.S1 && p.S2),
                  CATNN_ERR_INVALID_ARGUMENT, "swiglu backward epilogue operands");
    CATNN_REQUIRE(p.epi != EPI_GELU_BWD || p.Z, CATNN_ERR_INVALID_ARGUMENT, "gelu backward needs Z");
    if (p.N == 0) return;
    bool vec = p.K % 8 == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 && al16(p.A);
    const int bn_out = dual ? BN / 2 : BN;
    int64_t blocks;
    unsigned gy = 1;
    if (p.grid == GRID_PLAIN) {
        if (p.M == 0) return;
        vec = vec && al16(p.B) && (!p.B2 || al16(p.B2));
        blocks = (int64_t)((p.M + BM - 1) / BM) * ((p.N + bn_out - 1) / bn_out);
    } else {
        CATNN_REQUIRE(p.n_experts > 0 && p.n_experts <= kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                      "bf16 gemm: n_experts out of range");
        if (p.grid == GRID_ROWS) {
            for (int e = 0; e < p.n_experts; ++e)
                vec = vec && al16(p.B_e[e]) && (!dual || al16(p.B2_e[e]));
            blocks = (int64_t)p.max_tiles * ((p.N + bn_out - 1) / bn_out);
        } else {
            // K segments start on multiples of 8 only when the caller pads them.
            vec = vec && al16(p.B) && p.segk_aligned;
            blocks = (int64_t)((p.M + BM - 1) / BM) * ((p.N + bn_out - 1) / bn_out);
            gy = (unsigned)p.n_experts;
        }
    }
    if (blocks == 0) return;
    CATNN_REQUIRE(blocks < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "bf16 gemm: grid too large");
    dim3 grid((unsigned)blocks, gy), block(256);
    if (dual) {
        if (vec) gemm_bf16_kernel<true, true><<<grid, block, 0, s>>>(p);
        else gemm_bf16_kernel<false, true><<<grid, block, 0, s>>>(p);
    } else {
        if (vec) gemm_bf16_kernel<true, false><<<grid, block, 0, s>>>(p);
        else gemm_bf16_kernel<false, false><<<grid, block, 0, s>>>(p);
    }
    CATNN_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace catnn
