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
// Blocks of 2×2 or 4×2 wavefronts; tiles of 128×128, 256×128 or 128×256
// with BK = 32 or 64 (Cfg below), A and B tiles staged in LDS (row stride
// BK+8 bf16, so eight lanes' 16-byte reads hit distinct banks),
// double-buffered behind register prefetch; full k chunks load without
// branches so the next chunk's loads stay in flight behind the MFMAs.
// Epilogues and grids are listed in gemm_bf16.hpp.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "devmath.hpp"
#include "gemm_bf16.hpp"

namespace catnn {
namespace k {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// A block of WAVES_M × WAVES_N wavefronts computes a BM × BN tile; each
// wavefront owns (BM / WAVES_M) × (BN / WAVES_N) = FM × FN MFMA blocks of
// 32 × 32.  Per k16 step a wavefront reads (FM + FN) KB of LDS for FM·FN
// MFMAs, so wider wavefront tiles relieve the LDS port.
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int BK_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int BK = BK_, LDT = BK + 8;  // LDS row stride (bf16): conflict-free b128 reads
    static constexpr int LDS_BYTES = 2 * (BM + BN) * LDT * 2;
    static constexpr int NT = 64 * WAVES_M * WAVES_N;
    static constexpr int FM = BM / (32 * WAVES_M), FN = BN / (32 * WAVES_N);
    static constexpr int A_IT = BM * (BK / 8) / NT;  // 16-byte chunks per thread per k chunk
    static constexpr int B_IT = BN * (BK / 8) / NT;
    static_assert(FM >= 1 && FN >= 1 && FM * 32 * WAVES_M == BM && FN * 32 * WAVES_N == BN, "tile");
    static_assert(A_IT >= 1 && B_IT >= 1 && A_IT * NT == BM * (BK / 8) && B_IT * NT == BN * (BK / 8),
                  "load split");
};

// All with 64 × 64 per wavefront: wider wavefront tiles (64 × 128) ran
// slower on the training shapes (one wavefront per SIMD at 270+ registers).
using Cfg0 = Cfg<128, 128, 2, 2, 32>;
using Cfg2 = Cfg<128, 128, 2, 2, 64>;
using Cfg3 = Cfg<256, 128, 4, 2, 32>;  // 8 wavefronts
using Cfg4 = Cfg<256, 128, 4, 2, 64>;


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

// Epilogue of one wavefront's FM × FN accumulator blocks, one loop nest per
// kind (fully unrolled, so the accumulators stay in registers).  Entry r of
// block (mi, ni) is row wrow0 + 32·mi + 8(r/4) + r%4, column wcol0 + 32·ni.
template <class C, bool DUAL, int EPI>
__device__ __forceinline__ void epilogue(const GemmBf16Params &p, const f32x16 (&acc)[C::FM][C::FN],
                                         int wrow0, int wcol0, int row_end, float *__restrict__ C32) {
    constexpr int NF = DUAL ? C::FN / 2 : C::FN;
#pragma unroll
    for (int mi = 0; mi < C::FM; ++mi)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = wrow0 + mi * 32 + 8 * (r >> 2) + (r & 3);
            if (row >= row_end) continue;
#pragma unroll
            for (int ni = 0; ni < NF; ++ni) {
                const int col = wcol0 + ni * 32;
                if (col >= p.N) continue;
                float v = acc[mi][ni][r];
                if (EPI == EPI_SWIGLU_FWD) {
                    const float c = acc[mi][ni + NF][r];
                    const int64_t so = (int64_t)row * p.lds + col;
                    if (p.S1) p.S1[so] = f2bf(v);
                    if (p.S2) p.S2[so] = f2bf(c);
                    p.Cb[(int64_t)row * p.ldcb + col] = f2bf(silu(v) * c);
                    continue;
                }
                if (EPI == EPI_SWIGLU_BWD) {
                    const int64_t so = (int64_t)row * p.lds + col;
                    const float a = bf2f(p.S1[so]), c = bf2f(p.S2[so]);
                    p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v * c * silu_grad(a));
                    p.Cb2[(int64_t)row * p.ldcb + col] = f2bf(v * silu(a));
                    continue;
                }
                if (EPI == EPI_LINEAR) {
                    if (p.bias) v += p.bias[col];
                    if (p.Z) p.Z[(int64_t)row * p.ldz + col] = v;
                    v = apply_act(v, p.act);
                    if (p.R) v = p.R[(int64_t)row * p.ldr + col] + v;
                } else if (EPI == EPI_GELU_BWD) {
                    v *= gelu_grad(p.Z[(int64_t)row * p.ldz + col]);
                }
                if (C32) {
                    float *dst = C32 + (int64_t)row * p.ldc32 + col;
                    *dst = p.accumulate ? *dst + v : v;
                }
                if (p.Cb) p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v);
            }
        }
}

template <class C, bool VEC, bool DUAL, int GRID>
__device__ __forceinline__ void tile(bf16_t (*sa)[C::BM][C::LDT], bf16_t (*sb)[C::BN][C::LDT], const GemmBf16Params &p,
                                     const bf16_t *__restrict__ B, const bf16_t *__restrict__ B2, int row0,
                                     int row_end, int col0, int k_lo, int k_hi, float *__restrict__ C32) {
    constexpr int BM = C::BM, BN = C::BN, FM = C::FM, FN = C::FN, BK = C::BK;
    // DUAL: B rows [0, BN/2) come from B, [BN/2, BN) from B2; a wavefront's
    // fragment ni < FN/2 pairs with fragment ni + FN/2 (same output column).
    constexpr int WCOLS = DUAL ? BN / 2 / C::WAVES_N : BN / C::WAVES_N;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const int lr = lane & 31, lg = lane >> 5;
    const int N = p.N;

    const bf16_t *a_src[C::A_IT];
    bool a_ok[C::A_IT];
    int a_r[C::A_IT], a_c[C::A_IT];
#pragma unroll
    for (int it = 0; it < C::A_IT; ++it) {
        const int idx = tid + it * C::NT;
        a_r[it] = idx / (BK / 8);
        a_c[it] = (idx % (BK / 8)) * 8;
        const int gr = row0 + a_r[it];
        a_ok[it] = gr < row_end;
        int src = gr;
        if (a_ok[it] && p.a_rows) src = p.a_rows[gr] / p.a_row_div;
        a_src[it] = p.A + (int64_t)(a_ok[it] ? src : 0) * p.lda;
    }
    const bf16_t *b_src[C::B_IT];
    bool b_ok[C::B_IT];
    int b_r[C::B_IT], b_c[C::B_IT];
#pragma unroll
    for (int it = 0; it < C::B_IT; ++it) {
        const int idx = tid + it * C::NT;
        b_r[it] = idx / (BK / 8);
        b_c[it] = (idx % (BK / 8)) * 8;
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

    uint4 ra[C::A_IT], rb[C::B_IT];
    // Full chunks (VEC launches, all BK values inside [k_lo, k_hi)): one
    // unconditional 16-byte load per row piece — rows past the edge read row
    // 0 of the operand and are zeroed by a select — so nothing branches and
    // the loads stay in flight behind the MFMAs of the current chunk.
    auto gload_full = [&](int k0) {
#pragma unroll
        for (int it = 0; it < C::A_IT; ++it) {
            const uint4 v = *reinterpret_cast<const uint4 *>(a_src[it] + k0 + a_c[it]);
            ra[it] = a_ok[it] ? v : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int it = 0; it < C::B_IT; ++it) {
            const uint4 v = *reinterpret_cast<const uint4 *>(b_src[it] + k0 + b_c[it]);
            rb[it] = b_ok[it] ? v : make_uint4(0, 0, 0, 0);
        }
    };
    // The tail chunk and unaligned launches: 8 consecutive k values of one
    // row, one 16-byte load when all 8 are in range and aligned, element
    // loads (zero past k_hi) otherwise.
    auto load8 = [&](const bf16_t *src, bool ok, int kk) -> uint4 {
        if (!ok || kk >= k_hi) return make_uint4(0, 0, 0, 0);
        if (VEC && kk + 8 <= k_hi) return *reinterpret_cast<const uint4 *>(src + kk);
        uint16_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = kk + j < k_hi ? src[kk + j] : 0;
        return make_uint4(v[0] | (uint32_t)v[1] << 16, v[2] | (uint32_t)v[3] << 16,
                          v[4] | (uint32_t)v[5] << 16, v[6] | (uint32_t)v[7] << 16);
    };
    auto gload = [&](int k0) {
#pragma unroll
        for (int it = 0; it < C::A_IT; ++it) ra[it] = load8(a_src[it], a_ok[it], k0 + a_c[it]);
#pragma unroll
        for (int it = 0; it < C::B_IT; ++it) rb[it] = load8(b_src[it], b_ok[it], k0 + b_c[it]);
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int it = 0; it < C::A_IT; ++it) *reinterpret_cast<uint4 *>(&sa[buf][a_r[it]][a_c[it]]) = ra[it];
#pragma unroll
        for (int it = 0; it < C::B_IT; ++it) *reinterpret_cast<uint4 *>(&sb[buf][b_r[it]][b_c[it]]) = rb[it];
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

    auto brow = [&](int ni) {
        if (DUAL) return (ni < FN / 2 ? 0 : BN / 2) + wn * WCOLS + (ni % (FN / 2)) * 32 + lr;
        return wn * WCOLS + ni * 32 + lr;
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
                af[mi] = *reinterpret_cast<const bf16x8 *>(&sa[buf][wm * (BM / C::WAVES_M) + mi * 32 + lr][s * 16 + 8 * lg]);
#pragma unroll
            for (int ni = 0; ni < FN; ++ni)
                bfr[ni] = *reinterpret_cast<const bf16x8 *>(&sb[buf][brow(ni)][s * 16 + 8 * lg]);
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
        }
    };

    const int nk = (k_hi - k_lo + BK - 1) / BK;
    const int nfull = VEC ? (k_hi - k_lo) / BK : 0;
    if (nk > 0) {
        if (nfull > 0) gload_full(k_lo);
        else gload(k_lo);
        sstore(0);
        __syncthreads();
        int kt = 0;
        for (; kt + 1 < nfull; ++kt) {  // the next chunk is full
            gload_full(k_lo + (kt + 1) * BK);
            compute(kt & 1);
            sstore((kt & 1) ^ 1);
            __syncthreads();
        }
        for (; kt < nk; ++kt) {  // the last full chunk and the tail
            const bool more = kt + 1 < nk;
            if (more) gload(k_lo + (kt + 1) * BK);
            compute(kt & 1);
            if (more) sstore((kt & 1) ^ 1);
            __syncthreads();
        }
    }

    const int wrow0 = row0 + wm * (BM / C::WAVES_M) + 4 * lg;
    const int wcol0 = col0 + wn * WCOLS + lr;
    if (DUAL) {
        epilogue<C, true, EPI_SWIGLU_FWD>(p, acc, wrow0, wcol0, row_end, C32);
        return;
    }
    // Each grid is built only with the epilogues the training step uses on it.
    if constexpr (GRID == GRID_PLAIN) {
        switch (p.epi) {
            case EPI_LINEAR: epilogue<C, false, EPI_LINEAR>(p, acc, wrow0, wcol0, row_end, C32); break;
            case EPI_GELU_BWD: epilogue<C, false, EPI_GELU_BWD>(p, acc, wrow0, wcol0, row_end, C32); break;
            default: epilogue<C, false, EPI_STORE>(p, acc, wrow0, wcol0, row_end, C32);
        }
    } else if constexpr (GRID == GRID_ROWS) {
        if (p.epi == EPI_SWIGLU_BWD) epilogue<C, false, EPI_SWIGLU_BWD>(p, acc, wrow0, wcol0, row_end, C32);
        else epilogue<C, false, EPI_STORE>(p, acc, wrow0, wcol0, row_end, C32);
    } else {
        epilogue<C, false, EPI_STORE>(p, acc, wrow0, wcol0, row_end, C32);
    }
}

template <class C, bool VEC, bool DUAL, int GRID>
__global__ __launch_bounds__(C::NT) void gemm_bf16_kernel(GemmBf16Params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    auto sa = reinterpret_cast<bf16_t(*)[C::BM][C::LDT]>(smem);
    auto sb = reinterpret_cast<bf16_t(*)[C::BN][C::LDT]>(smem + 2 * C::BM * C::LDT * 2);
    const int bn_out = DUAL ? C::BN / 2 : C::BN;
    const int tiles_n = (p.N + bn_out - 1) / bn_out;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    if constexpr (GRID == GRID_PLAIN) {
        const int tiles_m = (p.M + C::BM - 1) / C::BM;
        int tm, tn;
        grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
        tile<C, VEC, DUAL, GRID>(sa, sb, p, p.B, p.B2, tm * C::BM, p.M, tn * bn_out, 0, p.K, p.C32);
    } else if constexpr (GRID == GRID_ROWS) {
        // Tiles of the table are kRowTile rows; C::BM equals it for this grid.
        int tm, tn;
        grouped_tile(lid, p.max_tiles, tiles_n, 8, tm, tn);
        if (tm >= *p.n_tiles) return;
        const int e = p.tile_expert[tm];
        const int end = p.seg_counts ? p.seg_offsets[e] + p.seg_counts[e] : p.seg_offsets[e + 1];
        tile<C, VEC, DUAL, GRID>(sa, sb, p, p.B_e[e], DUAL ? p.B2_e[e] : nullptr, p.tile_row0[tm], end,
                                 tn * bn_out, 0, p.K, p.C32);
    } else {  // GRID_SEGK: expert e = blockIdx.y reduces over its own K segment
        const int tiles_m = (p.M + C::BM - 1) / C::BM;
        int tm, tn;
        grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
        const int e = blockIdx.y;
        const int lo = p.seg_offsets[e];
        const int hi = p.seg_counts ? lo + p.seg_counts[e] : p.seg_offsets[e + 1];
        tile<C, VEC, DUAL, GRID>(sa, sb, p, p.B, nullptr, tm * C::BM, p.M, tn * bn_out, lo, hi, p.C_e[e]);
    }
}

bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

constexpr int kRowTile = 128;  // rows per tile of the grouped tile table (build_tiles)

template <class C, int GRID, bool DUAL>
void launch_kernel(hipStream_t s, const GemmBf16Params &p, bool vec, dim3 grid) {
    // Tiles above 64 KiB of LDS need the per-kernel opt-in (gfx950: 160 KiB per CU).
    static bool attr_set = false;
    if (!attr_set) {
        CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_bf16_kernel<C, true, DUAL, GRID>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES));
        CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_bf16_kernel<C, false, DUAL, GRID>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES));
        attr_set = true;
    }
    if (vec) gemm_bf16_kernel<C, true, DUAL, GRID><<<grid, dim3(C::NT), C::LDS_BYTES, s>>>(p);
    else gemm_bf16_kernel<C, false, DUAL, GRID><<<grid, dim3(C::NT), C::LDS_BYTES, s>>>(p);
    CATNN_HIP(hipGetLastError());
}

// Grids and epilogues each configuration is built with: plain (store,
// linear, GELU adjoint) and per-expert K segments (store) for all; grouped
// rows (store, SwiGLU adjoint, and with DUAL the SwiGLU forward) for the
// 128-row tiles.
template <class C, bool DUAL_OK>
void launch_cfg(hipStream_t s, const GemmBf16Params &p, bool vec, bool dual, unsigned gy) {
    CATNN_REQUIRE(DUAL_OK || !dual, CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: SwiGLU forward needs tile configuration 0");
    const bool ok_epi = p.grid == GRID_PLAIN ? (p.epi == EPI_STORE || p.epi == EPI_LINEAR || p.epi == EPI_GELU_BWD)
                        : p.grid == GRID_ROWS ? (p.epi == EPI_STORE || p.epi == EPI_SWIGLU_FWD || p.epi == EPI_SWIGLU_BWD)
                                              : p.epi == EPI_STORE;
    CATNN_REQUIRE(ok_epi, CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: epilogue not built for this grid");
    const int bn_out = dual ? C::BN / 2 : C::BN;
    int64_t blocks;
    if (p.grid == GRID_ROWS) blocks = (int64_t)p.max_tiles * ((p.N + bn_out - 1) / bn_out);
    else blocks = (int64_t)((p.M + C::BM - 1) / C::BM) * ((p.N + bn_out - 1) / bn_out);
    if (blocks == 0) return;
    CATNN_REQUIRE(blocks < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "bf16 gemm: grid too large");
    const dim3 grid((unsigned)blocks, gy);
    if (p.grid == GRID_PLAIN) {
        launch_kernel<C, GRID_PLAIN, false>(s, p, vec, grid);
    } else if (p.grid == GRID_SEGK) {
        launch_kernel<C, GRID_SEGK, false>(s, p, vec, grid);
    } else {
        if constexpr (C::BM == kRowTile) {
            if constexpr (DUAL_OK) {
                if (dual) {
                    launch_kernel<C, GRID_ROWS, true>(s, p, vec, grid);
                    return;
                }
            }
            launch_kernel<C, GRID_ROWS, false>(s, p, vec, grid);
        } else {
            fail(CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: grouped rows need 128-row tiles");
        }
    }
}

}  // namespace

int gemm_bf16_tile_rows() { return kRowTile; }

void gemm_bf16_launch_cfg(hipStream_t s, const GemmBf16Params &p, int cfg) {
    CATNN_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, CATNN_ERR_SHAPE_MISMATCH, "bf16 gemm: dims");
    const bool dual = p.epi == EPI_SWIGLU_FWD;
    CATNN_REQUIRE(!dual || p.Cb, CATNN_ERR_INVALID_ARGUMENT, "swiglu epilogue needs Cb");
    CATNN_REQUIRE(p.epi != EPI_SWIGLU_BWD || (p.Cb && p.Cb2 && p.S1 && p.S2),
                  CATNN_ERR_INVALID_ARGUMENT, "swiglu backward epilogue operands");
    CATNN_REQUIRE(p.epi != EPI_GELU_BWD || p.Z, CATNN_ERR_INVALID_ARGUMENT, "gelu backward needs Z");
    if (p.N == 0) return;
    bool vec = p.K % 8 == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 && al16(p.A);
    unsigned gy = 1;
    if (p.grid == GRID_PLAIN) {
        if (p.M == 0) return;
        vec = vec && al16(p.B) && (!p.B2 || al16(p.B2));
    } else {
        CATNN_REQUIRE(p.n_experts > 0 && p.n_experts <= kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                      "bf16 gemm: n_experts out of range");
        if (p.grid == GRID_ROWS) {
            for (int e = 0; e < p.n_experts; ++e)
                vec = vec && al16(p.B_e[e]) && (!dual || al16(p.B2_e[e]));
        } else {
            // K segments start on multiples of 8 only when the caller pads them.
            vec = vec && al16(p.B) && p.segk_aligned;
            gy = (unsigned)p.n_experts;
        }
    }
    switch (cfg) {
        case 0: launch_cfg<Cfg0, true>(s, p, vec, dual, gy); break;
        case 2: launch_cfg<Cfg2, false>(s, p, vec, dual, gy); break;
        case 3: launch_cfg<Cfg3, false>(s, p, vec, dual, gy); break;
        case 4: launch_cfg<Cfg4, false>(s, p, vec, dual, gy); break;
        default: fail(CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: unknown tile configuration");
    }
}

// Tile choice, from a sweep of the training step's shapes on MI355X
// (TFLOP/s of cfg 3 / 4 / 2): 256×128 tiles with BK 32 when there are at
// least four of them per CU (8192×4096×3072: 831/785/800), BK 64 when there
// are one to four (8192×1024×12288: 665/917/883), 128×128 with BK 64 below
// that (4096×1024×8192: 385/510/613).  Grouped-row grids need 128-row tiles.
void gemm_bf16_launch(hipStream_t s, const GemmBf16Params &p) {
    // The SwiGLU epilogues (two outputs per element) run best on the
    // 128×128×32 tile (config-5 expert GEMMs: 442 vs 545 µs forward).
    int cfg = p.epi == EPI_SWIGLU_FWD || p.epi == EPI_SWIGLU_BWD ? 0 : 2;
    if (p.grid != GRID_ROWS && p.epi != EPI_SWIGLU_FWD) {
        const int64_t t3 = (int64_t)((p.M + 255) / 256) * ((p.N + 127) / 128) *
                           (p.grid == GRID_SEGK ? p.n_experts : 1);
        cfg = t3 >= 1024 ? 3 : t3 >= 256 ? 4 : 2;
    }
    gemm_bf16_launch_cfg(s, p, cfg);
}

}  // namespace k
}  // namespace catnn
