// fp32 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x2_f32) with an
// LDS-staged, double-buffered K loop and a fused epilogue.
//
// Replaces the hot loop of cpu::linear → matmul_mk_kn → dot_row
// (crates/catnn-compile/src/kernel/cpu.rs:135-232), whose strided gathers of
// w[p·N+j] bound the reference by cache misses, and the separate bias pass
// (cpu.rs:173-182), activation passes (cpu.rs:14-29) and residual add
// (cpu.rs:80-98) that follow it in a graph.
//
// Layout: x [M,K], w [K,N] (the reference's [in_features, out_features],
// morphism.rs:249-256), y [M,N], all row-major f32.
//
// Tiling: a 256-thread block (4 wavefronts, 2×2) owns a BM×BN tile of C;
// each wavefront owns (BM/2)×(BN/2) as (BM/64)×(BN/64) MFMA 32×32 blocks
// held in accumulator registers.  Per K chunk of BK, the block stages
// A[BM×BK] (k contiguous) and B[BK×BN] (n contiguous) in LDS while the next
// chunk's global loads are in flight.
//
// MFMA 32x32x2 operand layout: lane l supplies A[i = l%32][kslot = l/32] and
// B[kslot = l/32][j = l%32]; accumulator r of lane l is C[8(r/4) + 4(l/32) +
// r%4][l%32].  Within a chunk, lane group g = l/32 feeds the k values
// g·BK/2 … g·BK/2 + BK/2-1 over BK/2 consecutive MFMAs, so each lane reads
// its A values as contiguous 16-byte LDS loads; A and B use the same k
// assignment, so every product A[i][k]·B[k][j] is accumulated exactly once.
//
// Two block-level modes share the tile body:
//  * plain: C = act(A·B + bias) + R;
//  * dual (SwiGLU gate/up, moe.rs:159-174): the B tile's first half comes
//    from W1 and its second half from W3 at the same columns, so each lane
//    holds a = x·w1 and c = x·w3 for the same (i, j) and writes silu(a)·c.
// and two grid-level modes: a plain M×N grid, and a grouped grid over
// per-expert row segments of a permuted token order (A rows optionally
// gathered through an index array) for the MoE expert GEMMs.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "devmath.hpp"
#include "kernels.hpp"
#include "gemm_f32.hpp"

namespace catnn {
namespace k {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int BM, int BN, int BK>
struct GemmSmem {
    float a[2][BM][BK + 4];
    float b[2][BK][BN + 4];
};

template <int BM, int BN, int BK, bool VEC, bool DUAL>
__device__ __forceinline__ void gemm_block(GemmSmem<BM, BN, BK> &sm, const float *__restrict__ A,
                                           int64_t lda, const int32_t *__restrict__ a_rows,
                                           int a_row_div, int row0, int row_end,
                                           const float *__restrict__ B,
                                           const float *__restrict__ B2, int64_t ldb, int col0,
                                           int N, int K, const float *__restrict__ bias,
                                           const float *__restrict__ R, int64_t ldr,
                                           float *__restrict__ C, int64_t ldc, int act) {
    static_assert(BM % 64 == 0 && BN % 64 == 0 && BK % 8 == 0, "tile shape");
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int KH = BK / 2;
    constexpr int A_IT = BM * BK / 4 / 256;
    constexpr int B_IT = BK * BN / 4 / 256;
    static_assert(A_IT >= 1 && B_IT >= 1, "tile too small for 256 threads");
    static_assert(!DUAL || FN == 2, "dual mode pairs one W1 and one W3 fragment");

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lg = lane >> 5;

    // Per-thread global load assignments.
    const float *a_src[A_IT];
    int a_r[A_IT], a_k[A_IT];
    bool a_ok[A_IT];
#pragma unroll
    for (int it = 0; it < A_IT; ++it) {
        const int idx = tid + it * 256;
        a_r[it] = idx / (BK / 4);
        a_k[it] = (idx % (BK / 4)) * 4;
        const int gr = row0 + a_r[it];
        a_ok[it] = gr < row_end;
        int src = gr;
        if (a_ok[it] && a_rows) src = a_rows[gr] / a_row_div;
        a_src[it] = A + (int64_t)(a_ok[it] ? src : 0) * lda;
    }
    const float *b_src[B_IT];
    int b_kr[B_IT], b_c[B_IT], b_ncol[B_IT];
#pragma unroll
    for (int it = 0; it < B_IT; ++it) {
        const int idx = tid + it * 256;
        b_kr[it] = idx / (BN / 4);
        b_c[it] = (idx % (BN / 4)) * 4;
        int lc;  // logical output column of the first of the 4 values
        const float *base;
        if (DUAL) {
            const bool second = b_c[it] >= BN / 2;
            lc = col0 + b_c[it] - (second ? BN / 2 : 0);
            base = second ? B2 : B;
        } else {
            lc = col0 + b_c[it];
            base = B;
        }
        b_ncol[it] = lc;
        b_src[it] = base + lc;
    }

    float4 ra[A_IT], rb[B_IT];
    auto gload = [&](int k0) {
#pragma unroll
        for (int it = 0; it < A_IT; ++it) {
            const int kk = k0 + a_k[it];
            if (VEC) {
                ra[it] = (a_ok[it] && kk < K) ? *reinterpret_cast<const float4 *>(a_src[it] + kk)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = (a_ok[it] && kk + j < K) ? a_src[it][kk + j] : 0.f;
                ra[it] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
#pragma unroll
        for (int it = 0; it < B_IT; ++it) {
            const int kk = k0 + b_kr[it];
            if (VEC) {
                rb[it] = (kk < K && b_ncol[it] < N)
                             ? *reinterpret_cast<const float4 *>(b_src[it] + (int64_t)kk * ldb)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[j] = (kk < K && b_ncol[it] + j < N) ? b_src[it][(int64_t)kk * ldb + j] : 0.f;
                rb[it] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int it = 0; it < A_IT; ++it)
            *reinterpret_cast<float4 *>(&sm.a[buf][a_r[it]][a_k[it]]) = ra[it];
#pragma unroll
        for (int it = 0; it < B_IT; ++it)
            *reinterpret_cast<float4 *>(&sm.b[buf][b_kr[it]][b_c[it]]) = rb[it];
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

    auto compute = [&](int buf) {
        float af[FM][KH], bf[FN][KH];
#pragma unroll
        for (int mi = 0; mi < FM; ++mi) {
            const float *src = &sm.a[buf][wm * WM + mi * 32 + lr][lg * KH];
#pragma unroll
            for (int q = 0; q < KH / 4; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(src + 4 * q);
                af[mi][4 * q + 0] = v.x;
                af[mi][4 * q + 1] = v.y;
                af[mi][4 * q + 2] = v.z;
                af[mi][4 * q + 3] = v.w;
            }
        }
#pragma unroll
        for (int ni = 0; ni < FN; ++ni) {
            const int col = DUAL ? (ni * (BN / 2) + wn * 32 + lr) : (wn * WN + ni * 32 + lr);
#pragma unroll
            for (int s = 0; s < KH; ++s) bf[ni][s] = sm.b[buf][lg * KH + s][col];
        }
#pragma unroll
        for (int s = 0; s < KH; ++s)
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[mi][s], bf[ni][s],
                                                                       acc[mi][ni], 0, 0, 0);
    };

    const int nk = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload((kt + 1) * BK);
        compute(buf);
        if (more) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue straight from the accumulators: for a fixed r, lanes 0-31
    // write 32 consecutive columns of one row and lanes 32-63 those of the
    // row 4 below, so each store is two 128-byte segments.
#pragma unroll
    for (int mi = 0; mi < FM; ++mi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + wm * WM + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
            if (row >= row_end) continue;
            if (DUAL) {
                const int col = col0 + wn * 32 + lr;
                if (col < N) C[(int64_t)row * ldc + col] = silu(acc[mi][0][r]) * acc[mi][1][r];
            } else {
#pragma unroll
                for (int ni = 0; ni < FN; ++ni) {
                    const int col = col0 + wn * WN + ni * 32 + lr;
                    if (col >= N) continue;
                    float v = acc[mi][ni][r];
                    if (bias) v += bias[col];
                    v = apply_act(v, act);
                    if (R) v = R[(int64_t)row * ldr + col] + v;
                    C[(int64_t)row * ldc + col] = v;
                }
            }
        }
    }
}

template <int BM, int BN, int BK, bool VEC, bool DUAL>
__global__ __launch_bounds__(256, 2) void gemm_plain_kernel(GemmParams p) {
    __shared__ GemmSmem<BM, BN, BK> sm;
    constexpr int BN_OUT = DUAL ? BN / 2 : BN;
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN_OUT - 1) / BN_OUT;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    int tm, tn;
    grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
    gemm_block<BM, BN, BK, VEC, DUAL>(sm, p.A, p.lda, p.a_rows, p.a_row_div, tm * BM, p.M, p.B,
                                      p.B2, p.ldb, tn * BN_OUT, p.N, p.K, p.bias, p.R, p.ldr,
                                      p.C, p.ldc, p.act);
}

template <int BM, int BN, int BK, bool VEC, bool DUAL>
__global__ __launch_bounds__(256, 2) void gemm_grouped_kernel(GemmParams p) {
    __shared__ GemmSmem<BM, BN, BK> sm;
    constexpr int BN_OUT = DUAL ? BN / 2 : BN;
    const int tiles_n = (p.N + BN_OUT - 1) / BN_OUT;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    int tm, tn;
    grouped_tile(lid, p.max_tiles, tiles_n, 8, tm, tn);
    if (tm >= *p.n_tiles) return;
    const int e = p.tile_expert[tm];
    const int r0 = p.tile_row0[tm];
    const int rend = p.seg_offsets[e + 1];
    gemm_block<BM, BN, BK, VEC, DUAL>(sm, p.A, p.lda, p.a_rows, p.a_row_div, r0, rend,
                                      p.B_e[e], DUAL ? p.B2_e[e] : nullptr, p.ldb, tn * BN_OUT,
                                      p.N, p.K, p.bias, p.R, p.ldr, p.C, p.ldc, p.act);
}

// Direct-to-LDS form of the 128 × 128 tile for 16-byte aligned launches, on
// the plain or the grouped grid, single or dual (SwiGLU gate/up) operand: k
// chunks of 16 go HBM → LDS by global_load_lds_dwordx4,
// STAGES deep, with no registers in between.  A rows (k-contiguous) are 64
// bytes, 4 chunks of 4 k values, chunk c of row r at position
// c ^ ((r / 2) mod 4), so the 8 rows a read touches sit on distinct banks;
// B rows (n-contiguous) are 512 bytes and need no swizzle.  A wave load
// fills 1 KiB: 16 A rows or 2 B rows.  The MFMA schedule, the k split across
// lane halves and the epilogue are those of gemm_block.
constexpr int kDmaLead = 2;  // k slots of MFMAs issued before each step's loads

template <int STAGES, bool DUAL, bool GROUPED>
__global__ __launch_bounds__(256, 2) void gemm_dma_kernel(GemmParams p) {
    constexpr int BM = 128, BN = 128, BK = 16, KH = BK / 2;
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    constexpr int BN_OUT = DUAL ? BN / 2 : BN;
    constexpr int A_BYTES = BM * BK * 4, STAGE = A_BYTES + BK * BN * 4;  // 8 KiB + 8 KiB
    constexpr int LPC = 4;  // wave loads per wavefront and chunk: 2 for A, 2 for B
    static_assert(STAGES >= 2 && STAGES <= 4, "the waits cover up to 3 chunks in flight");
    static_assert(!DUAL || FN == 2, "dual mode pairs one W1 and one W3 fragment");
    extern __shared__ __align__(16) unsigned char smem[];
    const int tiles_n = (p.N + BN_OUT - 1) / BN_OUT;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    int tm, tn, row0, M;  // M: the end of this tile's rows
    const float *B = p.B, *B2 = p.B2;
    if constexpr (GROUPED) {
        grouped_tile(lid, p.max_tiles, tiles_n, 8, tm, tn);
        if (tm >= *p.n_tiles) return;
        const int e = p.tile_expert[tm];
        row0 = p.tile_row0[tm];
        M = p.seg_offsets[e + 1];
        B = p.B_e[e];
        B2 = DUAL ? p.B2_e[e] : nullptr;
    } else {
        grouped_tile(lid, (p.M + BM - 1) / BM, tiles_n, 8, tm, tn);
        row0 = tm * BM;
        M = p.M;
    }
    const int col0 = tn * BN_OUT, N = p.N, K = p.K;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lg = lane >> 5;

    // A: wave load q of wavefront w fills rows 16(2w + q) … +15, lane l row
    // … + l/4 at position l mod 4 = chunk (l mod 4) ^ ((row / 2) mod 4).
    const float *a_src[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = (2 * wave + q) * 16 + (lane >> 2);
        const int gr = row0 + r < M ? row0 + r : row0;  // rows past the end read row0; never stored
        const int src = p.a_rows ? p.a_rows[gr] / p.a_row_div : gr;
        a_src[q] = p.A + (int64_t)src * p.lda + 4 * ((lane & 3) ^ ((r >> 1) & 3));
    }
    // B: wave load q fills k rows 2(2w + q), +1: lane l row l/32, tile
    // columns 4(l mod 32) … +3 — output columns col0 + those, or with DUAL
    // W1 for the first BN/2 and W3 for the rest at the same output columns
    // (past N: column col0, never stored).
    const float *b_src[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int kr = (2 * wave + q) * 2 + (lane >> 5);
        const int tc = 4 * (lane & 31);
        const bool second = DUAL && tc >= BN / 2;
        const int c = col0 + tc - (second ? BN / 2 : 0);
        b_src[q] = (second ? B2 : B) + (int64_t)kr * p.ldb + (c + 4 <= N ? c : col0);
    }
    const uint32_t lds0 = lds_addr(smem) + 2 * wave * 1024;  // this wavefront's first A load, stage 0
    auto issue = [&](int kt) {
        const uint32_t st = lds0 + (kt % STAGES) * STAGE;
        const int k0 = kt * BK;
#pragma unroll
        for (int q = 0; q < 2; ++q) load_lds16_at(a_src[q] + k0, st + q * 1024);
#pragma unroll
        for (int q = 0; q < 2; ++q) load_lds16_at(b_src[q] + (int64_t)k0 * p.ldb, st + A_BYTES + q * 1024);
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

    // Lane half g takes k values g·KH … g·KH + KH − 1: A chunks 2g and 2g + 1.
    struct Frags {
        float a[FM][KH], b[FN][KH];
    };
    auto load_frags = [&](const unsigned char *st, Frags &f) {
#pragma unroll
        for (int mi = 0; mi < FM; ++mi) {
            const int r = wm * WM + mi * 32 + lr;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(st + r * 64 + (((2 * lg + q) ^ ((r >> 1) & 3)) << 4));
                f.a[mi][4 * q + 0] = v.x;
                f.a[mi][4 * q + 1] = v.y;
                f.a[mi][4 * q + 2] = v.z;
                f.a[mi][4 * q + 3] = v.w;
            }
        }
        const float *bt = reinterpret_cast<const float *>(st + A_BYTES);
#pragma unroll
        for (int ni = 0; ni < FN; ++ni) {
            const int col = DUAL ? (ni * (BN / 2) + wn * 32 + lr) : (wn * WN + ni * 32 + lr);
#pragma unroll
            for (int s2 = 0; s2 < KH; ++s2) f.b[ni][s2] = bt[(lg * KH + s2) * BN + col];
        }
    };
    // MFMAs of k slots [lo, hi) of f (compile-time bounds).
    auto mma_part = [&](const Frags &f, auto lo, auto hi) {
#pragma unroll
        for (int s2 = decltype(lo)::value; s2 < decltype(hi)::value; ++s2)
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[mi][s2], f.b[ni][s2], acc[mi][ni], 0, 0, 0);
    };
    using K0 = std::integral_constant<int, 0>;
    using KS = std::integral_constant<int, kDmaLead>;
    using KE = std::integral_constant<int, KH>;
    auto mma = [&](const Frags &f) { mma_part(f, K0{}, KE{}); };

    // Software pipeline: the fragments of chunk kt + 1 are read from LDS
    // while the MFMAs of chunk kt (already in registers) run.  Chunk kt + S
    // goes into chunk kt's slot once every wavefront has read chunk kt (the
    // lgkmcnt(0) before the barrier of step kt).  The wait before that
    // barrier lets the loads of the chunks issued after kt + 1 stay in
    // flight: up to S − 2 of them.
    const int nfull = K / BK;
    Frags f0, f1;
#pragma unroll
    for (int j = 0; j < STAGES; ++j)
        if (j < nfull) issue(j);
    // Chunk c landed for every wavefront, with the loads of up to `most`
    // chunks issued after c still in flight (fewer near the end of K).
    auto wait_chunk = [&](int c, int most) {
        const int ahead = min(most, nfull - 1 - c);
        if (STAGES > 3 && ahead >= 3) dma_sync<3 * LPC>();
        else if (STAGES > 2 && ahead >= 2) dma_sync<2 * LPC>();
        else if (ahead >= 1) dma_sync<LPC>();
        else dma_sync<0>();
    };
    // Step kt for kt + 1 < nfull.  No LDS read is left pending on any path
    // into mma(cur), so the compiler's own wait there is for cur alone.
    // The first kDmaLead k slots of MFMAs go ahead of the load issue, so the
    // matrix pipe starts right after the barrier while the address work and
    // the loads issue behind it (the scheduler keeps this order).
    auto step = [&](int kt, Frags &cur, Frags &nxt) {
        wait_chunk(kt + 1, STAGES - 2);  // issued so far: chunks up to kt + S − 1
        mma_part(cur, K0{}, KS{});
        __builtin_amdgcn_sched_barrier(0);
        if (kt + STAGES < nfull) issue(kt + STAGES);
        load_frags(smem + ((kt + 1) % STAGES) * STAGE, nxt);
        __builtin_amdgcn_sched_barrier(0);
        mma_part(cur, KS{}, KE{});
    };
    if (nfull > 0) {
        wait_chunk(0, STAGES - 1);  // issued so far: chunks 0 … S − 1
        load_frags(smem, f0);
        int kt = 0;
        for (; kt + 2 < nfull; kt += 2) {
            step(kt, f0, f1);
            step(kt + 1, f1, f0);
        }
        if (kt + 1 < nfull) {  // two chunks left
            step(kt, f0, f1);
            mma(f1);
        } else {
            mma(f0);
        }
    }
    const int k0 = nfull * BK;
    if (k0 < K) {  // partial last chunk through registers, zero past K (K % 4 == 0 here)
        dma_sync<0>();
        for (int i = tid; i < BM * 4 + BK * (BN / 4); i += 256) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            unsigned char *dst;
            if (i < BM * 4) {
                const int r = i >> 2, c = i & 3, kk = k0 + 4 * c;
                if (row0 + r < M && kk < K) {
                    const int src = p.a_rows ? p.a_rows[row0 + r] / p.a_row_div : row0 + r;
                    v = *reinterpret_cast<const float4 *>(p.A + (int64_t)src * p.lda + kk);
                }
                dst = smem + r * 64 + ((c ^ ((r >> 1) & 3)) << 4);
            } else {
                const int j = i - BM * 4, kr = j / (BN / 4), tc = (j % (BN / 4)) * 4;
                const bool second = DUAL && tc >= BN / 2;
                const int c = col0 + tc - (second ? BN / 2 : 0);
                if (k0 + kr < K && c + 4 <= N)
                    v = *reinterpret_cast<const float4 *>((second ? B2 : B) + (int64_t)(k0 + kr) * p.ldb + c);
                dst = smem + A_BYTES + (kr * BN + tc) * 4;
            }
            *reinterpret_cast<float4 *>(dst) = v;
        }
        dma_sync<0>();
        load_frags(smem, f0);
        mma(f0);
    }

#pragma unroll
    for (int mi = 0; mi < FM; ++mi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = row0 + wm * WM + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
            if (row >= M) continue;
            if constexpr (DUAL) {
                const int col = col0 + wn * 32 + lr;
                if (col < N) p.C[(int64_t)row * p.ldc + col] = silu(acc[mi][0][r]) * acc[mi][1][r];
            } else {
#pragma unroll
                for (int ni = 0; ni < FN; ++ni) {
                    const int col = col0 + wn * WN + ni * 32 + lr;
                    if (col >= N) continue;
                    float v = acc[mi][ni][r];
                    if (p.bias) v += p.bias[col];
                    v = apply_act(v, p.act);
                    if (p.R) v = p.R[(int64_t)row * p.ldr + col] + v;
                    p.C[(int64_t)row * p.ldc + col] = v;
                }
            }
        }
    }
}

// Tile-table builder for the grouped grid: one entry per BM-row tile of each
// expert's segment, in expert order.  Single wavefront; n_experts is small.
__global__ void build_tiles_kernel(const int32_t *__restrict__ offsets, int n_experts, int bm,
                                   int32_t *__restrict__ tile_expert,
                                   int32_t *__restrict__ tile_row0, int32_t *__restrict__ n_tiles) {
    if (threadIdx.x != 0) return;
    int t = 0;
    for (int e = 0; e < n_experts; ++e) {
        for (int r = offsets[e]; r < offsets[e + 1]; r += bm) {
            tile_expert[t] = e;
            tile_row0[t] = r;
            ++t;
        }
    }
    *n_tiles = t;
}

constexpr int kBM = 128, kBN = 128, kBK = 16;
constexpr int kDmaStages = 4;  // gemm_dma_kernel chunks in LDS (16 KiB each)

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int gemm_tile_rows() { return kBM; }

void gemm_launch(hipStream_t s, const GemmParams &p, bool dual) {
    CATNN_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, CATNN_ERR_SHAPE_MISMATCH, "gemm: negative dims");
    if (p.M == 0 || p.N == 0) return;
    const bool vec = (p.K % 4 == 0) && (p.N % 4 == 0) && (p.lda % 4 == 0) && (p.ldb % 4 == 0) &&
                     aligned16(p.A) && aligned16(p.B) && (!p.B2 || aligned16(p.B2));
    const int bn_out = dual ? kBN / 2 : kBN;
    const int64_t tiles = (int64_t)((p.M + kBM - 1) / kBM) * ((p.N + bn_out - 1) / bn_out);
    CATNN_REQUIRE(tiles < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "gemm: grid too large");
    dim3 grid((unsigned)tiles), block(256);
    constexpr size_t dma_lds = kDmaStages * 16384;
    if (vec && dual) {
        gemm_dma_kernel<kDmaStages, true, false><<<grid, block, dma_lds, s>>>(p);
    } else if (vec) {
        gemm_dma_kernel<kDmaStages, false, false><<<grid, block, dma_lds, s>>>(p);
    } else if (dual) {
        gemm_plain_kernel<kBM, kBN, kBK, false, true><<<grid, block, 0, s>>>(p);
    } else {
        gemm_plain_kernel<kBM, kBN, kBK, false, false><<<grid, block, 0, s>>>(p);
    }
    CATNN_HIP(hipGetLastError());
}

void gemm_grouped_launch(hipStream_t s, const GemmParams &p, bool dual) {
    CATNN_REQUIRE(p.n_experts > 0 && p.n_experts <= kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                  "grouped gemm: n_experts out of range");
    bool vec = (p.K % 4 == 0) && (p.N % 4 == 0) && (p.lda % 4 == 0) && (p.ldb % 4 == 0) &&
               aligned16(p.A);
    for (int e = 0; e < p.n_experts; ++e)
        vec = vec && aligned16(p.B_e[e]) && (!dual || aligned16(p.B2_e[e]));
    const int bn_out = dual ? kBN / 2 : kBN;
    const int64_t tiles = (int64_t)p.max_tiles * ((p.N + bn_out - 1) / bn_out);
    if (tiles == 0) return;
    CATNN_REQUIRE(tiles < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "grouped gemm: grid too large");
    dim3 grid((unsigned)tiles), block(256);
    constexpr size_t dma_lds = kDmaStages * 16384;
    if (vec && dual) gemm_dma_kernel<kDmaStages, true, true><<<grid, block, dma_lds, s>>>(p);
    else if (vec) gemm_dma_kernel<kDmaStages, false, true><<<grid, block, dma_lds, s>>>(p);
    else if (dual) gemm_grouped_kernel<kBM, kBN, kBK, false, true><<<grid, block, 0, s>>>(p);
    else gemm_grouped_kernel<kBM, kBN, kBK, false, false><<<grid, block, 0, s>>>(p);
    CATNN_HIP(hipGetLastError());
}

void build_tiles(hipStream_t s, const int32_t *offsets, int n_experts, int32_t *tile_expert,
                 int32_t *tile_row0, int32_t *n_tiles) {
    build_tiles_kernel<<<1, 64, 0, s>>>(offsets, n_experts, kBM, tile_expert, tile_row0, n_tiles);
    CATNN_HIP(hipGetLastError());
}

void linear_f32(hipStream_t s, const float *x, int64_t lda, const float *w, int64_t ldb,
                const float *b, const float *r, int64_t ldr, float *y, int64_t ldc, int64_t m,
                int64_t k, int64_t n, int act) {
    CATNN_REQUIRE(m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH,
                  "linear: dimension exceeds 2^31");
    CATNN_REQUIRE(act == ACT_NONE || act == ACT_RELU || act == ACT_GELU,
                  CATNN_ERR_INVALID_ARGUMENT, "linear: act must be 0, 2 or 3");
    GemmParams p{};
    p.A = x;
    p.lda = lda;
    p.a_row_div = 1;
    p.B = w;
    p.ldb = ldb;
    p.bias = b;
    p.R = r;
    p.ldr = ldr;
    p.C = y;
    p.ldc = ldc;
    p.M = (int)m;
    p.N = (int)n;
    p.K = (int)k;
    p.act = act;
    gemm_launch(s, p, false);
}

}  // namespace k
}  // namespace catnn
