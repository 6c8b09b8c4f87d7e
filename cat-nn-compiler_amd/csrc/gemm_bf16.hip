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

#include <utility>

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
    static constexpr bool DMA = false, PP = false;
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

// Register-staged tiles of 64 × 64 per wavefront: the SwiGLU forward (two
// B operands) and launches without 16-byte aligned rows.
using Cfg0 = Cfg<128, 128, 2, 2, 32>;
using Cfg2 = Cfg<128, 128, 2, 2, 64>;

// Direct-to-LDS configurations: full k chunks (BK = 64) travel from HBM
// into LDS by global_load_lds_dwordx4 without passing through registers,
// STAGES chunks deep.  One such load fills 1 KiB of LDS contiguously, lane
// l at byte 16·l, so rows are 128 bytes (8 chunks of 8 k values) with no
// padding.  gfx950's LDS has 64 banks: a 16-byte operand read serves 16
// lanes per cycle from one 256-byte bank window, i.e. 16 consecutive rows
// of one chunk, two rows per window.  Chunk c of row r therefore sits at
// position c ^ ((r / 2) mod 8): the 8 even and the 8 odd rows of any 16
// each cover the 8 positions, so the 16 reads fall on distinct banks.
// (Swizzling by r mod 8 leaves rows r and r + 8 on the same banks.)
//
// With BK = 32 rows are 64 bytes (4 chunks, four rows per window) and a
// wave load fills 16 rows; chunk c of row r sits at c ^ ((r / 4) mod 4).
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int STAGES_, int BK_ = 64>
struct DCfg {
    static constexpr bool DMA = true, PP = false;
    static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, STAGES = STAGES_;
    static constexpr int BK = BK_;
    static constexpr int ROWB = BK * 2, CPR = BK / 8, RPL = 64 / CPR;  // row bytes, chunks a row, rows a wave load
    static constexpr int NT = 64 * WAVES_M * WAVES_N, NW = WAVES_M * WAVES_N;
    static constexpr int FM = BM / (32 * WAVES_M), FN = BN / (32 * WAVES_N);
    static constexpr int STAGE_BYTES = (BM + BN) * ROWB;
    static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
    // wave loads (RPL rows each) per wavefront and k chunk
    static constexpr int A_LD = BM / (RPL * NW), B_LD = BN / (RPL * NW), LPC = A_LD + B_LD;
    // chunk position swizzle of row r
    static __device__ __forceinline__ int sw(int r) { return CPR == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); }
    static_assert(BK == 64 || BK == 32, "k chunk");
    static_assert(FM >= 1 && FN >= 1 && FM * 32 * WAVES_M == BM && FN * 32 * WAVES_N == BN, "tile");
    static_assert(A_LD >= 1 && B_LD >= 1 && A_LD * RPL * NW == BM && B_LD * RPL * NW == BN, "load split");
    static_assert(STAGES >= 2 && LDS_BYTES <= 160 * 1024, "LDS");
    static_assert(STAGES <= 4 && LPC * (STAGES - 2) < 64, "vmcnt range (the main loop waits for up to 2 chunks ahead)");
};

// 128 × 128 tiles of four 64 × 64 wavefronts: two stages (64 KiB, two
// blocks per CU) or three (96 KiB).  Sweeps over the training shapes also
// tried 256 × 128 tiles of eight wavefronts (three stages), 256 × 128 of four
// 128 × 64 wavefronts and 256 × 256 of eight 128 × 64 wavefronts: those won
// only on 8192³ (1067 against 981 TFLOP/s) and lost on the rest.  With the
// 64-bank swizzle, 256 × 128 and 128 × 256 tiles of four or eight
// wavefronts in three 48 KiB stages, also with the fragments of the next k
// step read during the current step's MFMAs, stayed at 0.8–1.0× of this
// tile on every training shape.
using Cfg7 = DCfg<128, 128, 2, 2, 2>;
using Cfg9 = DCfg<128, 128, 2, 2, 3>;
using Cfg10 = DCfg<128, 128, 2, 2, 4, 32>;  // 32-deep chunks, four stages in the same 64 KiB

// Ping-pong tiles: 256 × 256 outputs, eight wavefronts in two groups of
// four (group g owns rows 128g … 128g+127, wavefront i of a group columns
// 64i … 64i+63), one block per CU.  A 128 × 128 tile at full MFMA rate asks
// 64 B/clk per CU of its operands from L2 (two blocks per CU); this one half
// that.  The two groups take turns: while one group's wavefronts issue their
// MFMAs, the other's read their next fragments from LDS, so each SIMD's
// matrix core always has one wavefront feeding it.  k chunks are 32 deep
// (64-byte rows, chunk c of row r at c ^ (r/4 mod 4)) in four 32 KiB stages;
// the loads of a chunk are issued by the wavefronts in their MFMA phase, one
// after every fourth MFMA (a burst of them stalls the issuing wavefront for
// as long as the CU's address unit takes to accept them, ~1000 cycles for a
// whole chunk).  Measured (plain grid, TFLOP/s) against the 128 × 128 tile:
// 8192³ 1278 vs 1011, 16384×7168×2048 1102 vs 894, 16384×1024×3584 1193
// vs 997, 8192×4096×1024 890 vs 677; with fewer than one tile per CU it
// loses (8192×1024×4096, 128 tiles: 812 vs 982).
// (A 256 × 128 tile of eight 64 × 64 wavefronts, twice the tiles for grids
// whose last round of 256 × 256 tiles leaves CUs idle, ran at 0.75–0.96× the
// 128 × 128 tile on the training shapes: 16-MFMA phases of 128 × 64
// wavefronts are what the ping-pong needs.)
template <int BN_, int WAVES_M_, int WAVES_N_>
struct PCfg {
    static constexpr bool DMA = true, PP = true;
    static constexpr int BM = 256, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, STAGES = 4;
    static constexpr int BK = 32, ROWB = 64, CPR = 4, RPL = 16;
    static constexpr int NT = 512, NW = 8, FM = BM / (32 * WAVES_M), FN = BN / (32 * WAVES_N);
    static constexpr int STAGE_BYTES = (BM + BN) * ROWB;
    static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
    static constexpr int LPW = (BM + BN) / (RPL * NW);  // wave loads per wavefront and chunk
    static __device__ __forceinline__ int sw(int r) { return (r >> 2) & 3; }
    static_assert(WAVES_M * WAVES_N == NW && WAVES_M % 2 == 0, "two groups of four wavefronts, whole rows each");
    static_assert(LPW * RPL * NW == BM + BN && BM % RPL == 0, "wave loads cover the A and B rows");
    static_assert((2 * FM * FN) / LPW >= 2, "one load after every second MFMA at most");
};
using Cfg11 = PCfg<256, 2, 4>;  // 256 × 256, wavefronts of 128 × 64


__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float((uint32_t)v << 16); }

// Round to nearest even; NaN stays NaN.
__device__ __forceinline__ bf16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
    return (bf16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Activation functions of the training epilogues on the hardware exp2 and
// reciprocal (about 1e-7 relative; every output they feed is rounded to
// bf16 or enters a bf16 product).
__device__ __forceinline__ float sigmoid_hw(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * x));
}

// tanh(u) = 1 − 2/(1 + e^{2u}); saturates to ±1 where e^{2u} overflows or
// vanishes.
__device__ __forceinline__ float tanh_hw(float u) {
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(2.88539008177792682f * u));
}

__device__ __forceinline__ float gelu_hw(float z) {
    const float c = 0.797884523868560791f;
    return 0.5f * z * (1.0f + tanh_hw(c * (z + 0.044715f * z * z * z)));
}

__device__ __forceinline__ float gelu_grad_hw(float z) {
    const float C = 0.044715f, kk = 0.797884523868560791f;
    const float t = tanh_hw(kk * (z + C * z * z * z));
    const float du = kk * (1.0f + 3.0f * C * z * z);
    return 0.5f * (1.0f + t) + 0.5f * z * (1.0f - t * t) * du;
}

// One output element of the epilogue kind EPI.
template <bool DUAL, int EPI>
__device__ __forceinline__ void epi_elem(const GemmBf16Params &p, float v, float c2, int row, int col,
                                         float *__restrict__ C32) {
    if constexpr (EPI == EPI_SWIGLU_FWD) {
        const int64_t so = (int64_t)row * p.lds + col;
        if (p.S1) p.S1[so] = f2bf(v);
        if (p.S2) p.S2[so] = f2bf(c2);
        p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v * sigmoid_hw(v) * c2);
        return;
    } else if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int64_t so = (int64_t)row * p.lds + col;
        const float a = bf2f(p.S1[so]), c = bf2f(p.S2[so]);
        const float sg = sigmoid_hw(a);
        // silu'(a) = σ(a)·(1 + a·(1 − σ(a)))
        p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v * c * (sg * (1.0f + a * (1.0f - sg))));
        p.Cb2[(int64_t)row * p.ldcb + col] = f2bf(v * (a * sg));
        return;
    } else {
        if constexpr (EPI == EPI_LINEAR) {
            if (p.bias) v += p.bias[col];
            if (p.Z) p.Z[(int64_t)row * p.ldz + col] = v;
            if (p.act == 2) v = fmaxf(v, 0.0f);
            else if (p.act == 3) v = gelu_hw(v);
            if (p.R) v = p.R[(int64_t)row * p.ldr + col] + v;
        } else if constexpr (EPI == EPI_GELU_BWD) {
            v *= gelu_grad_hw(p.Z[(int64_t)row * p.ldz + col]);
        }
        if (C32) {
            float *dst = C32 + (int64_t)row * p.ldc32 + col;
            *dst = p.accumulate ? *dst + v : v;
        }
        if (p.Cb) p.Cb[(int64_t)row * p.ldcb + col] = f2bf(v);
    }
}

// Epilogue of one wavefront's FM × FN accumulator blocks, one loop nest per
// kind (fully unrolled, so the accumulators stay in registers).  Entry r of
// block (mi, ni) is row wrow0 + 32·mi + 8(r/4) + r%4, column wcol0 + 32·ni.
// A wavefront whose whole tile lies inside the output takes the loop
// without bounds checks.
// f(integral_constant<int, i>) for i = 0 … N−1, expanded at compile time
// (a loop the compiler left rolled would index the accumulators at run time
// and move them to scratch memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_seq(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

template <class C, bool DUAL, int EPI, bool CHECK>
__device__ __forceinline__ void epilogue_loop(const GemmBf16Params &p, const f32x16 (&acc)[C::FM][C::FN],
                                              int wrow0, int wcol0, int row_end, float *__restrict__ C32) {
    constexpr int NF = DUAL ? C::FN / 2 : C::FN;
    static_for<C::FM>([&](auto mi_c) __attribute__((always_inline)) {
        constexpr int mi = decltype(mi_c)::value;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = wrow0 + mi * 32 + 8 * (r >> 2) + (r & 3);
            if (CHECK && row >= row_end) continue;
#pragma unroll
            for (int ni = 0; ni < NF; ++ni) {
                const int col = wcol0 + ni * 32;
                if (CHECK && col >= p.N) continue;
                epi_elem<DUAL, EPI>(p, acc[mi][ni][r], DUAL ? acc[mi][ni + NF][r] : 0.f, row, col, C32);
            }
        }
    });
}

template <class C, bool DUAL, int EPI>
__device__ __forceinline__ void epilogue(const GemmBf16Params &p, const f32x16 (&acc)[C::FM][C::FN], int wrow0,
                                         int wcol0, int row_end, float *__restrict__ C32) {
    constexpr int NF = DUAL ? C::FN / 2 : C::FN;
    const int lane = threadIdx.x & 63;
    // The wavefront's first row and column (lane 0's) and its extent.
    const int r0 = wrow0 - 4 * (lane >> 5), c0 = wcol0 - (lane & 31);
    const bool full = __builtin_amdgcn_readfirstlane(r0 + C::FM * 32 <= row_end && c0 + NF * 32 <= p.N);
    if (full) epilogue_loop<C, DUAL, EPI, false>(p, acc, wrow0, wcol0, row_end, C32);
    else epilogue_loop<C, DUAL, EPI, true>(p, acc, wrow0, wcol0, row_end, C32);
}

template <class C, bool DUAL, int GRID>
__device__ __forceinline__ void finish(const GemmBf16Params &p, const f32x16 (&acc)[C::FM][C::FN], int wrow0,
                                       int wcol0, int row_end, float *__restrict__ C32);

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

    finish<C, DUAL, GRID>(p, acc, row0 + wm * (BM / C::WAVES_M) + 4 * lg, col0 + wn * WCOLS + lr, row_end,
                          C32);
}

// Each grid is built only with the epilogues the training step uses on it.
template <class C, bool DUAL, int GRID>
__device__ __forceinline__ void finish(const GemmBf16Params &p, const f32x16 (&acc)[C::FM][C::FN], int wrow0,
                                       int wcol0, int row_end, float *__restrict__ C32) {
    if constexpr (DUAL) {
        epilogue<C, true, EPI_SWIGLU_FWD>(p, acc, wrow0, wcol0, row_end, C32);
        return;
    } else if constexpr (GRID == GRID_PLAIN) {
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


__device__ __forceinline__ void unpack8(uint4 w, float (&f)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(u[j] << 16);
        f[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
    }
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = (uint32_t)f2bf(f[2 * j]) | ((uint32_t)f2bf(f[2 * j + 1]) << 16);
    return make_uint4(u[0], u[1], u[2], u[3]);
}

__device__ __forceinline__ void load8f(const float *src, float (&f)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(src), b = *reinterpret_cast<const float4 *>(src + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

__device__ __forceinline__ void store8f(float *dst, const float (&f)[8]) {
    *reinterpret_cast<float4 *>(dst) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4 *>(dst + 4) = make_float4(f[4], f[5], f[6], f[7]);
}

// The epilogue's per-element operands at (row, col … col+7), loaded ahead:
// SwiGLU adjoint: a = S1 and c = S2 (bf16, one uint4 each); GELU adjoint:
// Z (fp32, two uint4 of float bits).
template <int EPI>
__device__ __forceinline__ void epi_preload(const GemmBf16Params &p, int row, int col, uint4 (&pre)[2]) {
    if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int64_t so = (int64_t)row * p.lds + col;
        pre[0] = *reinterpret_cast<const uint4 *>(p.S1 + so);
        pre[1] = *reinterpret_cast<const uint4 *>(p.S2 + so);
    } else if constexpr (EPI == EPI_GELU_BWD) {
        const uint4 *z = reinterpret_cast<const uint4 *>(p.Z + (int64_t)row * p.ldz + col);
        pre[0] = z[0];
        pre[1] = z[1];
    }
}

// Eight consecutive outputs (row, col … col+7) of epilogue kind EPI with
// 16-byte accesses; the same arithmetic per element as epi_elem.  `pre`
// (or null: loaded here) holds what epi_preload reads.
template <int EPI>
__device__ __forceinline__ void epi_vec8(const GemmBf16Params &p, float (&v)[8], int row, int col,
                                         float *__restrict__ C32, const uint4 *pre = nullptr) {
    if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int64_t so = (int64_t)row * p.lds + col;
        float a[8], c[8], d1[8], d2[8];
        unpack8(pre ? pre[0] : *reinterpret_cast<const uint4 *>(p.S1 + so), a);
        unpack8(pre ? pre[1] : *reinterpret_cast<const uint4 *>(p.S2 + so), c);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sg = sigmoid_hw(a[j]);
            d1[j] = v[j] * c[j] * (sg * (1.0f + a[j] * (1.0f - sg)));
            d2[j] = v[j] * (a[j] * sg);
        }
        *reinterpret_cast<uint4 *>(p.Cb + (int64_t)row * p.ldcb + col) = pack8(d1);
        *reinterpret_cast<uint4 *>(p.Cb2 + (int64_t)row * p.ldcb + col) = pack8(d2);
    } else {
        if constexpr (EPI == EPI_LINEAR) {
            if (p.bias) {
                float b[8];
                load8f(p.bias + col, b);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] += b[j];
            }
            if (p.Z) store8f(p.Z + (int64_t)row * p.ldz + col, v);
            if (p.act == 2) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = fmaxf(v[j], 0.0f);
            } else if (p.act == 3) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = gelu_hw(v[j]);
            }
            if (p.R) {
                float r[8];
                load8f(p.R + (int64_t)row * p.ldr + col, r);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = r[j] + v[j];
            }
        } else if constexpr (EPI == EPI_GELU_BWD) {
            float z[8];
            if (pre) {
                const uint32_t u[8] = {pre[0].x, pre[0].y, pre[0].z, pre[0].w, pre[1].x, pre[1].y, pre[1].z, pre[1].w};
#pragma unroll
                for (int j = 0; j < 8; ++j) z[j] = __uint_as_float(u[j]);
            } else {
                load8f(p.Z + (int64_t)row * p.ldz + col, z);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= gelu_grad_hw(z[j]);
        }
        if (C32) {
            float *dst = C32 + (int64_t)row * p.ldc32 + col;
            if (p.accumulate) {
                float o[8];
                load8f(dst, o);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = o[j] + v[j];
            }
            store8f(dst, v);
        }
        if (p.Cb) *reinterpret_cast<uint4 *>(p.Cb + (int64_t)row * p.ldcb + col) = pack8(v);
    }
}

// Epilogue of a block whose whole tile lies inside the output: the
// accumulators go through LDS (free once the last k chunk is consumed) so
// that each thread finishes runs of 8 consecutive columns with 16-byte
// loads and stores.
// DUAL (SwiGLU forward): the staged tile holds a = x·w1 in columns
// [0, BN/2) and c = x·w3 in [BN/2, BN) for the BN/2 output columns.
template <class C, bool DUAL>
__device__ __forceinline__ int staged_col(int wn, int ni, int lr) {
    if constexpr (DUAL) {
        constexpr int H = C::FN / 2, WCOLS = C::BN / 2 / C::WAVES_N;
        return (ni < H ? 0 : C::BN / 2) + wn * WCOLS + (ni % H) * 32 + lr;
    } else {
        return wn * (C::BN / C::WAVES_N) + ni * 32 + lr;
    }
}

template <class C, bool DUAL, int EPI>
__device__ __forceinline__ void epilogue_staged(unsigned char *smem, const GemmBf16Params &p,
                                                const f32x16 (&acc)[C::FM][C::FN], int row0, int col0,
                                                float *__restrict__ C32) {
    constexpr int BM = C::BM, BN = C::BN, WM = BM / C::WAVES_M, CH = (DUAL ? BN / 2 : BN) / 8;
    // A tile larger than the operand stages goes through LDS in slices of
    // SR rows (whole wavefront rows), one after the other.
    constexpr int SL = BM * BN * 4 <= C::LDS_BYTES ? 1 : 2, SR = BM / SL;
    static_assert(SR * BN * 4 <= C::LDS_BYTES && SR % WM == 0, "the staged slice must fit the operand stages");
    float *t = reinterpret_cast<float *>(smem);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N, lr = lane & 31, lg = lane >> 5;
    dma_sync<0>();  // every wavefront is done with the operand stages
    // Adjoint epilogues read an operand per output: issue all of this
    // thread's loads of the slice now, so that they are in flight while the
    // slice is staged (the barrier below waits for the LDS writes only).
    constexpr bool PRE = !DUAL && (EPI == EPI_SWIGLU_BWD || EPI == EPI_GELU_BWD) && (SR * CH) % C::NT == 0;
    constexpr int IT = PRE ? SR * CH / C::NT : 1;
    static_assert(2 * IT < 64, "preloads must fit the vmcnt counter");
#pragma unroll
    for (int sl = 0; sl < SL; ++sl) {
        const int srow0 = row0 + sl * SR;
        uint4 pre[IT][2];
        if constexpr (PRE) {
#pragma unroll
            for (int i = 0; i < IT; ++i) {
                const int idx = threadIdx.x + i * C::NT;
                epi_preload<EPI>(p, srow0 + idx / CH, col0 + (idx % CH) * 8, pre[i]);
            }
        }
        if (SL == 1 || wm * WM / SR == sl) {
#pragma unroll
            for (int mi = 0; mi < C::FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < C::FN; ++ni)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        t[(wm * WM - sl * SR + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3)) * BN +
                          staged_col<C, DUAL>(wn, ni, lr)] = acc[mi][ni][r];
        }
        if constexpr (PRE) {
            dma_sync<63>();  // LDS writes of every wavefront visible; preloads may still be in flight
#pragma unroll
            for (int i = 0; i < IT; ++i) {
                const int idx = threadIdx.x + i * C::NT;
                const int r = idx / CH, c = (idx % CH) * 8;
                float v[8];
                load8f(t + r * BN + c, v);
                epi_vec8<EPI>(p, v, srow0 + r, col0 + c, C32, pre[i]);
            }
        } else {
            dma_sync<0>();
            for (int idx = threadIdx.x; idx < SR * CH; idx += C::NT) {
                const int r = idx / CH, c = (idx % CH) * 8;
                float v[8];
                load8f(t + r * BN + c, v);
                if constexpr (DUAL) {
                    float cv[8], h[8];
                    load8f(t + r * BN + BN / 2 + c, cv);
                    const int64_t so = (int64_t)(srow0 + r) * p.lds + col0 + c;
                    if (p.S1) *reinterpret_cast<uint4 *>(p.S1 + so) = pack8(v);
                    if (p.S2) *reinterpret_cast<uint4 *>(p.S2 + so) = pack8(cv);
#pragma unroll
                    for (int j = 0; j < 8; ++j) h[j] = v[j] * sigmoid_hw(v[j]) * cv[j];
                    *reinterpret_cast<uint4 *>(p.Cb + (int64_t)(srow0 + r) * p.ldcb + col0 + c) = pack8(h);
                } else {
                    epi_vec8<EPI>(p, v, srow0 + r, col0 + c, C32);
                }
            }
        }
        // the next slice overwrites the staged rows: every read of them done
        if (sl + 1 < SL) dma_sync<63>();
    }
}

template <class C, bool DUAL, int GRID>
__device__ __forceinline__ void finish_staged(unsigned char *smem, const GemmBf16Params &p,
                                              const f32x16 (&acc)[C::FM][C::FN], int row0, int col0,
                                              float *__restrict__ C32) {
    if constexpr (DUAL) {
        epilogue_staged<C, true, EPI_SWIGLU_FWD>(smem, p, acc, row0, col0, C32);
    } else if constexpr (GRID == GRID_PLAIN) {
        switch (p.epi) {
            case EPI_LINEAR: epilogue_staged<C, false, EPI_LINEAR>(smem, p, acc, row0, col0, C32); break;
            case EPI_GELU_BWD: epilogue_staged<C, false, EPI_GELU_BWD>(smem, p, acc, row0, col0, C32); break;
            default: epilogue_staged<C, false, EPI_STORE>(smem, p, acc, row0, col0, C32);
        }
    } else if constexpr (GRID == GRID_ROWS) {
        if (p.epi == EPI_SWIGLU_BWD) epilogue_staged<C, false, EPI_SWIGLU_BWD>(smem, p, acc, row0, col0, C32);
        else epilogue_staged<C, false, EPI_STORE>(smem, p, acc, row0, col0, C32);
    } else {
        epilogue_staged<C, false, EPI_STORE>(smem, p, acc, row0, col0, C32);
    }
}

// The direct-to-LDS main loop (DCfg): chunk kt lands in stage kt mod STAGES;
// at the top of iteration kt a wavefront waits for its own loads of chunk kt
// (later chunks may stay in flight), the barrier makes every wavefront's
// loads visible and retires the reads of chunk kt−1, whose stage then takes
// chunk kt+STAGES−1.  A partial last chunk goes through registers (zero
// past k_hi).
// DUAL: B rows [0, BN/2) of the tile come from B (W1ᵀ) and [BN/2, BN) from
// B2 (W3ᵀ) at the same BN/2 output columns.
template <class C, bool DUAL, int GRID>
__device__ __forceinline__ void tile_dma(unsigned char *smem, const GemmBf16Params &p, const bf16_t *__restrict__ B,
                                         const bf16_t *__restrict__ B2, int row0, int row_end, int col0, int k_lo,
                                         int k_hi, float *__restrict__ C32) {
    constexpr int BM = C::BM, BN = C::BN, FM = C::FM, FN = C::FN, BK = C::BK;
    constexpr int BN_OUT = DUAL ? BN / 2 : BN, WCOLS = BN_OUT / C::WAVES_N;
    // B row r of the tile: operand and output column.
    auto b_row_src = [&](int r, int &n) -> const bf16_t * {
        if (DUAL && r >= BN / 2) {
            n = col0 + r - BN / 2;
            return B2;
        }
        n = col0 + r;
        return B;
    };
    // wave is uniform across the wavefront; readfirstlane lets the LDS
    // destinations (M0) come from a scalar register.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const int lr = lane & 31, lg = lane >> 5;

    // Wave load q of a wavefront fills tile rows RPL·(wave·LD + q) … +RPL−1:
    // lane l row … + l/CPR at position l mod CPR, i.e. k chunk
    // (l mod CPR) ^ sw(row).  Rows past the tile's end read row row0 (col0
    // for B): their outputs are never stored.  (B rows start at BM, a
    // multiple of 32, so their swizzle is that of their row within B.)
    constexpr int CPR = C::CPR, RPL = C::RPL, ROWB = C::ROWB;
    const int lrow = lane / CPR, lpos = lane % CPR;
    const bf16_t *a_src[C::A_LD];
#pragma unroll
    for (int q = 0; q < C::A_LD; ++q) {
        const int r = (wave * C::A_LD + q) * RPL + lrow;
        int gr = row0 + r;
        if (gr >= row_end) gr = row0;
        const int src = p.a_rows ? p.a_rows[gr] / p.a_row_div : gr;
        a_src[q] = p.A + (int64_t)src * p.lda + (lpos ^ C::sw(r)) * 8;
    }
    const bf16_t *b_src[C::B_LD];
#pragma unroll
    for (int q = 0; q < C::B_LD; ++q) {
        const int r = (wave * C::B_LD + q) * RPL + lrow;
        int n;
        const bf16_t *base = b_row_src(r, n);
        if (n >= p.N) n = col0;
        b_src[q] = base + (int64_t)n * p.ldb + (lpos ^ C::sw(r)) * 8;
    }
    const uint32_t lds0 = lds_addr(smem);
    const int kwrap = p.b_kwrap;
    auto issue = [&](int kt) {
        const uint32_t st = lds0 + (kt % C::STAGES) * C::STAGE_BYTES;
        const int k0 = k_lo + kt * BK;
        const int kb0 = kwrap ? k0 % kwrap : k0;  // whole chunks: kwrap is a multiple of BK
#pragma unroll
        for (int q = 0; q < C::A_LD; ++q)
            load_lds16_at(a_src[q] + k0, st + (wave * C::A_LD + q) * 1024);  // RPL rows × ROWB = 1 KiB
#pragma unroll
        for (int q = 0; q < C::B_LD; ++q)
            load_lds16_at(b_src[q] + kb0, st + BM * ROWB + (wave * C::B_LD + q) * 1024);
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

    // Lane l reads k values 16s + 8(l/32) … +7 of row l mod 32 of each block.
    const int a_off = (wm * (BM / C::WAVES_M) + lr) * ROWB;
    const int sw = C::sw(lr);  // fragment rows start on multiples of 32
    auto b_off = [&](int ni) { return (BM + staged_col<C, DUAL>(wn, ni, lr)) * ROWB; };
    // k steps [lo, hi) of the chunk in st (compile-time bounds).
    auto compute_part = [&](const unsigned char *st, auto lo, auto hi) {
#pragma unroll
        for (int s = decltype(lo)::value; s < decltype(hi)::value; ++s) {
            const int pos = ((2 * s + lg) ^ sw) << 4;
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
                af[mi] = *reinterpret_cast<const bf16x8 *>(st + a_off + mi * 32 * ROWB + pos);
#pragma unroll
            for (int ni = 0; ni < FN; ++ni)
                bfr[ni] = *reinterpret_cast<const bf16x8 *>(st + b_off(ni) + pos);
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using SE = std::integral_constant<int, BK / 16>;
    auto compute = [&](const unsigned char *st) { compute_part(st, S0{}, SE{}); };

    const int nfull = (k_hi - k_lo) / BK;
#pragma unroll
    for (int j = 0; j < C::STAGES - 1; ++j)
        if (j < nfull) issue(j);
    for (int kt = 0; kt < nfull; ++kt) {
        // Chunks issued after kt: min(STAGES − 2, nfull − 1 − kt); their loads may stay in flight.
        const int ahead = min(C::STAGES - 2, nfull - 1 - kt);
        if (C::STAGES > 3 && ahead >= 2) dma_sync<C::LPC * (C::STAGES > 3 ? 2 : 0)>();
        else if (C::STAGES > 2 && ahead >= 1) dma_sync<C::LPC>();
        else dma_sync<0>();
        // The first k step's MFMAs go ahead of the load issue (which fills
        // the slot chunk kt − 1 used), so the matrix pipe starts at once.
        const unsigned char *st = smem + (kt % C::STAGES) * C::STAGE_BYTES;
        compute_part(st, S0{}, S1{});
        __builtin_amdgcn_sched_barrier(0);
        if (kt + C::STAGES - 1 < nfull) issue(kt + C::STAGES - 1);
        __builtin_amdgcn_sched_barrier(0);
        compute_part(st, S1{}, SE{});
    }
    const int kt0 = k_lo + nfull * BK;
    if (kt0 < k_hi) {
        dma_sync<0>();
        for (int idx = tid; idx < (BM + C::BN) * CPR; idx += C::NT) {
            const int r = idx / CPR, c = idx % CPR, kk = kt0 + 8 * c;
            const bf16_t *src = nullptr;
            if (r < BM) {
                const int gr = row0 + r;
                if (gr < row_end) src = p.A + (int64_t)(p.a_rows ? p.a_rows[gr] / p.a_row_div : gr) * p.lda;
            } else {
                int n;
                const bf16_t *base = b_row_src(r - BM, n);
                if (n < p.N) src = base + (int64_t)n * p.ldb;
            }
            uint4 v = make_uint4(0, 0, 0, 0);
            const int ks = (r >= BM && kwrap) ? kk % kwrap : kk;  // B's column of k = kk
            if (src && kk < k_hi) {
                if (kk + 8 <= k_hi) {
                    v = *reinterpret_cast<const uint4 *>(src + ks);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) e[j] = kk + j < k_hi ? src[ks + j] : 0;
                    v = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                                   e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
                }
            }
            // B rows start at BM, a multiple of 32: the same swizzle as row r − BM
            *reinterpret_cast<uint4 *>(smem + r * ROWB + ((c ^ C::sw(r)) << 4)) = v;
        }
        dma_sync<0>();
        compute(smem);
    }
    if (p.vec_epi && row0 + BM <= row_end && col0 + BN_OUT <= p.N)
        finish_staged<C, DUAL, GRID>(smem, p, acc, row0, col0, C32);
    else
        finish<C, DUAL, GRID>(p, acc, row0 + wm * (BM / C::WAVES_M) + 4 * lg, col0 + wn * WCOLS + lr, row_end,
                              C32);
}

// s_waitcnt vmcnt ≤ N and lgkmcnt 0, without a barrier.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The ping-pong main loop (PCfg).  Chunk j lands in stage j mod 4.  Group
// 1 starts one barrier later than group 0, so between consecutive barriers
// one group is in its memory phase (read chunk j's fragments from LDS, then
// wait until chunk j+1 is in LDS) while the other is in its MFMA phase
// (2·FM·FN MFMAs on the fragments it read, with this wavefront's LPW
// loads of chunk j+3 issued among them).  Chunk j+3 goes to the stage chunk j−1
// used, which both groups finished reading before the MFMA phase of chunk
// j began; every wavefront waits for its own loads of chunk j+1 at the end
// of its memory phase of chunk j, and the barrier after that wait precedes
// the first read of chunk j+1 by either group.  After the loop group 0
// takes one more barrier, so both groups pass the same number.  A partial
// last chunk goes through registers, computed by all eight wavefronts.
template <class C, bool DUAL, int GRID, bool PIECE = false>
__device__ __forceinline__ void tile_pp(unsigned char *smem, const GemmBf16Params &p, const bf16_t *__restrict__ B,
                                        const bf16_t *__restrict__ B2, int row0, int row_end, int col0, int k_lo,
                                        int k_hi, float *__restrict__ C32, float *__restrict__ part = nullptr) {
    constexpr int BM = C::BM, BN = C::BN, FM = C::FM, FN = C::FN, BK = C::BK, ROWB = C::ROWB, S = C::STAGES;
    constexpr int LPW = C::LPW, CPR = C::CPR;
    constexpr int BN_OUT = DUAL ? BN / 2 : BN, WCOLS = BN_OUT / C::WAVES_N;
    auto b_row_src = [&](int r, int &n) -> const bf16_t * {
        if (DUAL && r >= BN / 2) {
            n = col0 + r - BN / 2;
            return B2;
        }
        n = col0 + r;
        return B;
    };
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = wave >> 2, wn = wave % C::WAVES_N;  // group g: wavefronts 4g … 4g+3
    const int lr = lane & 31, lg = lane >> 5;

    // Wave load L = LPW·w + q of wavefront w fills combined rows 16L … 16L+15
    // of [A tile; B tile] (A when 16L < BM; uniform per wave load): lane l
    // row … + l/4 at position l mod 4, i.e. k chunk (l mod 4) ^ sw(row).
    // Rows past the tile's end read row row0 (col0 for B): their outputs are
    // never stored.
    const int lrow = lane / CPR, lpos = lane % CPR;
    const bf16_t *src[LPW];
    bool is_b[LPW];
#pragma unroll
    for (int q = 0; q < LPW; ++q) {
        const int R = (wave * LPW + q) * C::RPL + lrow;  // row of [A; B]
        is_b[q] = (wave * LPW + q) * C::RPL >= BM;
        const int r = is_b[q] ? R - BM : R;  // row within the A or B tile
        const int off = (lpos ^ C::sw(r)) * 8;
        if (!is_b[q]) {
            int gr = row0 + r;
            if (gr >= row_end) gr = row0;
            const int srow = p.a_rows ? p.a_rows[gr] / p.a_row_div : gr;
            src[q] = p.A + (int64_t)srow * p.lda + off;
        } else {
            int n;
            const bf16_t *base = b_row_src(r, n);
            if (n >= p.N) n = col0;
            src[q] = base + (int64_t)n * p.ldb + off;
        }
    }
    const uint32_t lds_w = lds_addr(smem) + wave * LPW * 1024;
    // k offsets of chunk kt in A and in B (B's wraps: whole chunks, b_kwrap a multiple of BK)
    auto koff = [&](int kt, int &ka, int &kb) {
        ka = k_lo + kt * BK;
        kb = p.b_kwrap ? ka % p.b_kwrap : ka;
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

    // Lane l reads k values 16s + 8(l/32) … +7 of row l mod 32 of each block;
    // fragment rows start on multiples of 32, so their swizzle is sw(l mod 32).
    const int swl = C::sw(lr);
    const int wm = wave / C::WAVES_N;
    const int a_off = (wm * (BM / C::WAVES_M) + lr) * ROWB;
    int b_off[FN];
#pragma unroll
    for (int ni = 0; ni < FN; ++ni) b_off[ni] = (BM + staged_col<C, DUAL>(wn, ni, lr)) * ROWB;

    const int nfull = (k_hi - k_lo) / BK;
    for (int c = 0; c < S - 1 && c < nfull; ++c) {
        int ka, kb;
        koff(c, ka, kb);
#pragma unroll
        for (int q = 0; q < LPW; ++q)
            load_lds16_at(src[q] + (is_b[q] ? kb : ka), lds_w + c * C::STAGE_BYTES + q * 1024);
    }
    {  // chunk 0 in LDS; chunks 1 … min(nfull, S−1)−1 may stay in flight
        const int after = min(nfull - 1, S - 2);
        if (after >= 2) wait_vm_lgkm<2 * LPW>();
        else if (after == 1) wait_vm_lgkm<LPW>();
        else wait_vm_lgkm<0>();
    }
    block_barrier();
    if (g == 1) block_barrier();
    bf16x8 fa[2][FM], fb[2][FN];
    for (int j = 0; j < nfull; ++j) {
        // memory phase: chunk j's fragments
        __builtin_amdgcn_sched_barrier(0);
        const unsigned char *st = smem + (j % S) * C::STAGE_BYTES;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int pos = ((2 * s + lg) ^ swl) << 4;
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
                fa[s][mi] = *reinterpret_cast<const bf16x8 *>(st + a_off + mi * 32 * ROWB + pos);
#pragma unroll
            for (int ni = 0; ni < FN; ++ni) fb[s][ni] = *reinterpret_cast<const bf16x8 *>(st + b_off[ni] + pos);
        }
        {  // this wavefront's loads of chunk j+1 done; chunks j+2 … min(nfull−1, j+S−2) may stay in flight
            const int after = min(nfull - 1, j + S - 2) - (j + 1);
            if (after >= 1) wait_vm_lgkm<LPW>();
            else wait_vm_lgkm<0>();
        }
        block_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // MFMA phase, with the loads of chunk j+S−1: load q after MFMA q·SP+1
        constexpr int NM = 2 * FM * FN, SP = NM / LPW;
        const int kt = j + S - 1;
        const bool iss = kt < nfull;
        int ka = 0, kb = 0;
        if (iss) koff(kt, ka, kb);
        const uint32_t dst = lds_w + (kt % S) * C::STAGE_BYTES;
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            const int s = t / (FM * FN), mi = (t / FN) % FM, ni = t % FN;
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s][mi], fb[s][ni], acc[mi][ni], 0, 0, 0);
            if (t % SP == 1 && t / SP < LPW) {
                const int q = t / SP;
                if (iss) load_lds16_at(src[q] + (is_b[q] ? kb : ka), dst + q * 1024);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        block_barrier();
    }
    if (g == 0) block_barrier();
    const int kt0 = k_lo + nfull * BK;
    if (kt0 < k_hi) {
        // every wavefront is past its last read of the stages (the loop's barriers)
        for (int idx = tid; idx < (BM + BN) * CPR; idx += C::NT) {
            const int r = idx / CPR, c = idx % CPR, kk = kt0 + 8 * c;
            const bf16_t *src1 = nullptr;
            if (r < BM) {
                const int gr = row0 + r;
                if (gr < row_end) src1 = p.A + (int64_t)(p.a_rows ? p.a_rows[gr] / p.a_row_div : gr) * p.lda;
            } else {
                int n;
                const bf16_t *base = b_row_src(r - BM, n);
                if (n < p.N) src1 = base + (int64_t)n * p.ldb;
            }
            uint4 v = make_uint4(0, 0, 0, 0);
            const int ks = (r >= BM && p.b_kwrap) ? kk % p.b_kwrap : kk;  // B's column of k = kk
            if (src1 && kk < k_hi) {
                if (kk + 8 <= k_hi) {
                    v = *reinterpret_cast<const uint4 *>(src1 + ks);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) e[q] = kk + q < k_hi ? src1[ks + q] : 0;
                    v = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                                   e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
                }
            }
            // B rows start at BM, a multiple of 16: the same swizzle as row r − BM
            *reinterpret_cast<uint4 *>(smem + r * ROWB + ((c ^ C::sw(r)) << 4)) = v;
        }
        dma_sync<0>();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int pos = ((2 * s + lg) ^ swl) << 4;
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
                fa[0][mi] = *reinterpret_cast<const bf16x8 *>(smem + a_off + mi * 32 * ROWB + pos);
#pragma unroll
            for (int ni = 0; ni < FN; ++ni) fb[0][ni] = *reinterpret_cast<const bf16x8 *>(smem + b_off[ni] + pos);
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0][mi], fb[0][ni], acc[mi][ni], 0, 0, 0);
        }
    }
    if constexpr (PIECE) {  // stream-K piece: the raw fp32 tile, BM × BN row-major (the fixup adds the pieces)
        static_assert(!DUAL, "stream-K pieces take plain B");
#pragma unroll
        for (int mi = 0; mi < FM; ++mi)
#pragma unroll
            for (int ni = 0; ni < FN; ++ni)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    part[(wm * (BM / C::WAVES_M) + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3)) * BN +
                         wn * (BN / C::WAVES_N) + ni * 32 + lr] = acc[mi][ni][r];
    } else {
        // Plain fp32 stores go straight from the accumulators (each store
        // instruction writes whole 128-byte row runs); epilogues with bf16
        // outputs or per-output operands go through LDS in two 128-row slices.
        const bool staged = DUAL || p.epi != EPI_STORE || p.Cb;
        if (staged && p.vec_epi && row0 + BM <= row_end && col0 + BN_OUT <= p.N)
            finish_staged<C, DUAL, GRID>(smem, p, acc, row0, col0, C32);
        else
            finish<C, DUAL, GRID>(p, acc, row0 + wm * (BM / C::WAVES_M) + 4 * lg, col0 + wn * WCOLS + lr, row_end,
                                  C32);
    }
}

template <class C, bool VEC, bool DUAL, int GRID>
__device__ __forceinline__ void run_tile(unsigned char *smem, const GemmBf16Params &p, const bf16_t *B,
                                         const bf16_t *B2, int row0, int row_end, int col0, int k_lo, int k_hi,
                                         float *C32) {
    if constexpr (C::PP) {
        static_assert(VEC, "direct-to-LDS tiles take 16-byte aligned rows");
        tile_pp<C, DUAL, GRID>(smem, p, B, B2, row0, row_end, col0, k_lo, k_hi, C32);
    } else if constexpr (C::DMA) {
        static_assert(VEC, "direct-to-LDS tiles take 16-byte aligned rows");
        tile_dma<C, DUAL, GRID>(smem, p, B, B2, row0, row_end, col0, k_lo, k_hi, C32);
    } else {
        auto sa = reinterpret_cast<bf16_t(*)[C::BM][C::LDT]>(smem);
        auto sb = reinterpret_cast<bf16_t(*)[C::BN][C::LDT]>(smem + 2 * C::BM * C::LDT * 2);
        tile<C, VEC, DUAL, GRID>(sa, sb, p, B, B2, row0, row_end, col0, k_lo, k_hi, C32);
    }
}

// Tile t of a stream-K launch (plain or grouped-row grid, 256 × 256 tiles in
// the grouped order of the ordinary grid over the tiles that exist).
template <class C, int GRID>
__device__ __forceinline__ void sk_tile(const GemmBf16Params &p, int t, int tiles_mr, int tiles_n, int &row0,
                                        int &row_end, int &col0, const bf16_t *&B) {
    int tm, tn;
    grouped_tile(t, tiles_mr, tiles_n, 8, tm, tn);
    col0 = tn * C::BN;
    if constexpr (GRID == GRID_PLAIN) {
        row0 = tm * C::BM;
        row_end = p.M;
        B = p.B;
    } else {
        const int e = p.tile_expert[tm];
        row0 = p.tile_row0[tm];
        row_end = p.seg_counts ? p.seg_offsets[e] + p.seg_counts[e] : p.seg_offsets[e + 1];
        B = p.B_e[e];
    }
}

template <class C, int GRID>
__device__ __forceinline__ int sk_tiles_m(const GemmBf16Params &p) {
    if constexpr (GRID == GRID_PLAIN) return (p.M + C::BM - 1) / C::BM;
    else return *p.n_tiles;
}

template <class C, bool VEC, bool DUAL, int GRID>
__global__ __launch_bounds__(C::NT) void gemm_bf16_kernel(GemmBf16Params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int bn_out = DUAL ? C::BN / 2 : C::BN;
    const int tiles_n = (p.N + bn_out - 1) / bn_out;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    if constexpr (GRID == GRID_PLAIN || GRID == GRID_ROWS) {
        int row0, row_end, col0;
        const bf16_t *B, *B2 = nullptr;
        if (C::PP && !DUAL && p.sk_ctas) {
            // Stream-K launch (configuration 12): this grid runs the whole
            // rounds of tiles, t = lid < rounds·G in the enumeration of
            // sk_tile; gemm_bf16_sk_kernel and sk_fixup_kernel the rest.
            const int tiles_mr = sk_tiles_m<C, GRID>(p), G = p.sk_ctas;
            if (lid >= tiles_mr * tiles_n / G * G) return;
            sk_tile<C, GRID>(p, lid, tiles_mr, tiles_n, row0, row_end, col0, B);
        } else if constexpr (GRID == GRID_PLAIN) {
            const int tiles_m = (p.M + C::BM - 1) / C::BM;
            int tm, tn;
            grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
            row0 = tm * C::BM;
            row_end = p.M;
            col0 = tn * bn_out;
            B = p.B;
            B2 = p.B2;
        } else {
            // Tiles of the table are C::BM rows (the launcher passes the table built for C::BM).
            int tm, tn;
            grouped_tile(lid, p.max_tiles, tiles_n, 8, tm, tn);
            if (tm >= *p.n_tiles) return;
            const int e = p.tile_expert[tm];
            row_end = p.seg_counts ? p.seg_offsets[e] + p.seg_counts[e] : p.seg_offsets[e + 1];
            row0 = p.tile_row0[tm];
            col0 = tn * bn_out;
            B = p.B_e[e];
            B2 = DUAL ? p.B2_e[e] : nullptr;
        }
        run_tile<C, VEC, DUAL, GRID>(smem, p, B, B2, row0, row_end, col0, 0, p.K, p.C32);
    } else {  // GRID_SEGK: expert e = blockIdx.y reduces over its own K segment
        const int tiles_m = (p.M + C::BM - 1) / C::BM;
        int tm, tn;
        grouped_tile(lid, tiles_m, tiles_n, 8, tm, tn);
        const int e = blockIdx.y;
        int lo, hi;
        if (p.seg_offsets) {
            lo = p.seg_offsets[e];
            hi = p.seg_counts ? lo + p.seg_counts[e] : p.seg_offsets[e + 1];
        } else {  // split K: equal segments of ksplit
            lo = e * p.ksplit;
            hi = min(p.K, lo + p.ksplit);
        }
        run_tile<C, VEC, DUAL, GRID>(smem, p, p.B, nullptr, tm * C::BM, p.M, tn * bn_out, lo, hi, p.C_e[e]);
    }
}

// Stream-K remainder (configuration 12).  The ordinary kernel runs the
// whole rounds of tiles (rounds·G of them, G = one block per CU); the
// remaining rem < G tiles are each cut into S = G / rem k ranges of whole
// chunks, and this kernel (G blocks) computes piece lid = rt·S + s into
// sk_part[lid] as a raw fp32 tile; sk_fixup_kernel adds a tile's pieces in
// order s = 0 … S−1 and runs the epilogue.
template <class C, int GRID>
__global__ __launch_bounds__(C::NT) void gemm_bf16_sk_kernel(GemmBf16Params p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int G = p.sk_ctas;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int tiles_n = (p.N + C::BN - 1) / C::BN;
    const int tiles_mr = sk_tiles_m<C, GRID>(p);
    const int total = tiles_mr * tiles_n, rounds = total / G, rem = total - rounds * G;
    if (rem == 0) return;
    const int S = G / rem;
    if (lid >= rem * S) return;
    const int nk = (p.K + C::BK - 1) / C::BK, per = (nk + S - 1) / S;
    const int k_lo = min(p.K, (lid % S) * per * C::BK), k_hi = min(p.K, k_lo + per * C::BK);
    int row0, row_end, col0;
    const bf16_t *B;
    sk_tile<C, GRID>(p, rounds * G + lid / S, tiles_mr, tiles_n, row0, row_end, col0, B);
    tile_pp<C, false, GRID, true>(smem, p, B, nullptr, row0, row_end, col0, k_lo, k_hi, nullptr,
                                  p.sk_part + (int64_t)lid * (C::BM * C::BN));
}

// Stream-K fixup: the remainder tiles of a configuration-12 launch.  One
// thread per 8 consecutive outputs of a tile (32 blocks a tile): the tile's
// S partial pieces added in order s = 0 … S−1, then the launch's epilogue.
template <int GRID>
__global__ __launch_bounds__(256) void sk_fixup_kernel(GemmBf16Params p) {
    using C = Cfg11;
    constexpr int BM = C::BM, BN = C::BN, BPT = BM * BN / 8 / 256;
    const int G = p.sk_ctas;
    const int tiles_n = (p.N + BN - 1) / BN;
    const int tiles_mr = sk_tiles_m<C, GRID>(p);
    const int total = tiles_mr * tiles_n, full = total / G * G, rem = total - full;
    const int rt = blockIdx.x / BPT;
    if (rt >= rem) return;
    const int S = G / rem;
    int row0, row_end, col0;
    const bf16_t *B;
    sk_tile<C, GRID>(p, full + rt, tiles_mr, tiles_n, row0, row_end, col0, B);
    const int run = (blockIdx.x % BPT) * 256 + threadIdx.x;
    const int r = run / (BN / 8), c = (run % (BN / 8)) * 8;
    const int row = row0 + r, col = col0 + c;
    if (row >= row_end || col >= p.N) return;
    const float *src = p.sk_part + (int64_t)rt * S * (BM * BN) + r * BN + c;
    float v[8], w[8];
    load8f(src, v);
    for (int q = 1; q < S; ++q) {
        load8f(src + (int64_t)q * (BM * BN), w);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] += w[j];
    }
    auto finish8 = [&](auto epi_c) {
        constexpr int EPI = decltype(epi_c)::value;
        if (p.vec_epi && col + 8 <= p.N) {
            epi_vec8<EPI>(p, v, row, col, p.C32);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (col + j < p.N) epi_elem<false, EPI>(p, v[j], 0.f, row, col + j, p.C32);
        }
    };
    if constexpr (GRID == GRID_PLAIN) {
        switch (p.epi) {
            case EPI_LINEAR: finish8(std::integral_constant<int, EPI_LINEAR>{}); break;
            case EPI_GELU_BWD: finish8(std::integral_constant<int, EPI_GELU_BWD>{}); break;
            default: finish8(std::integral_constant<int, EPI_STORE>{});
        }
    } else {
        if (p.epi == EPI_SWIGLU_BWD) finish8(std::integral_constant<int, EPI_SWIGLU_BWD>{});
        else finish8(std::integral_constant<int, EPI_STORE>{});
    }
}

bool al16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

bool epi_rows_aligned(const GemmBf16Params &p) {
    auto ok = [](const void *ptr, int64_t ld) { return !ptr || (al16(ptr) && ld % 8 == 0); };
    bool a = ok(p.C32, p.ldc32) && ok(p.Cb, p.ldcb) && ok(p.Cb2, p.ldcb) && ok(p.S1, p.lds) && ok(p.S2, p.lds) &&
             ok(p.Z, p.ldz) && ok(p.R, p.ldr) && (!p.bias || al16(p.bias));
    if (p.grid == GRID_SEGK)
        for (int e = 0; e < p.n_experts; ++e) a = a && ok(p.C_e[e], p.ldc32);
    return a;
}

constexpr int kRowTile = 128;  // rows per tile of the grouped tile table (build_tiles)

template <class C, int GRID, bool DUAL>
void launch_kernel(hipStream_t s, const GemmBf16Params &p, bool vec, dim3 grid) {
    // Tiles above 64 KiB of LDS need the per-kernel opt-in (gfx950: 160 KiB per CU).
    static bool attr_set = false;
    if constexpr (C::DMA) {
        CATNN_REQUIRE(vec, CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: direct-to-LDS tiles need 16-byte aligned rows");
        if (!attr_set) {
            CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_bf16_kernel<C, true, DUAL, GRID>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES));
            attr_set = true;
        }
        gemm_bf16_kernel<C, true, DUAL, GRID><<<grid, dim3(C::NT), C::LDS_BYTES, s>>>(p);
    } else {
        if (!attr_set) {
            CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_bf16_kernel<C, true, DUAL, GRID>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES));
            CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_bf16_kernel<C, false, DUAL, GRID>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS_BYTES));
            attr_set = true;
        }
        if (vec) gemm_bf16_kernel<C, true, DUAL, GRID><<<grid, dim3(C::NT), C::LDS_BYTES, s>>>(p);
        else gemm_bf16_kernel<C, false, DUAL, GRID><<<grid, dim3(C::NT), C::LDS_BYTES, s>>>(p);
    }
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
        if constexpr (C::BM == kRowTile || C::BM == 256) {
            if constexpr (DUAL_OK) {
                if (dual) {
                    launch_kernel<C, GRID_ROWS, true>(s, p, vec, grid);
                    return;
                }
            }
            launch_kernel<C, GRID_ROWS, false>(s, p, vec, grid);
        } else {
            fail(CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: grouped rows need 128- or 256-row tiles");
        }
    }
}

// One wavefront lists the 128-row and the 256-row tiles of every segment
// (11 us as one thread's walk on config 5's eight experts).
__global__ void build_tiles2_kernel(const int32_t *__restrict__ offsets, int n_experts, int32_t *__restrict__ t1,
                                    int max1, int32_t *__restrict__ t2, int max2) {
    // One wavefront, lane e owning expert e (n_experts ≤ 64): the tiles of
    // expert e start at the exclusive prefix of the experts' tile counts,
    // so the table is the one an in-order walk over the experts writes,
    // cut at its capacity.
    const int e = threadIdx.x;
    for (int w = 0; w < 2; ++w) {
        int32_t *t = w ? t2 : t1;
        const int mx = w ? max2 : max1, bm = w ? 256 : kRowTile;
        int r0 = 0, cnt = 0;
        if (e < n_experts) {
            r0 = offsets[e];
            const int r1 = offsets[e + 1];
            cnt = r1 > r0 ? (r1 - r0 + bm - 1) / bm : 0;
        }
        int incl = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            if (e >= off) incl += o;
        }
        const int start = incl - cnt, total = __shfl(incl, 63, 64);
        for (int i = 0; i < cnt && start + i < mx; ++i) {
            t[start + i] = e;
            t[mx + start + i] = r0 + i * bm;
        }
        if (e == 0) t[2 * mx] = total < mx ? total : mx;
    }
}

int max_tiles_for(int64_t rows, int n_experts, int bm) { return (int)((rows + bm - 1) / bm + n_experts); }

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    CATNN_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) CATNN_HIP(hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cus[dev];
}

// Tile configuration of an automatic launch.  The grid runs in rounds of
// concurrent tiles: 256 × 256 tiles one per CU, 128 × 128 tiles two per CU.
// A 256 × 256 tile does the work of four 128 × 128 tiles in 4 / 1.2 of the
// time a CU takes for them (the measured plain-grid throughput ratio), so
// it wins when ⌈T256 / CUs⌉ · 4 / 1.2 < ⌈T128 / 2·CUs⌉ · 2: many tiles, or
// a grid that fills its last round.  A grouped grid's tile count is only
// known on the device; its bound (segments padded) is used.  k ranges
// under 256 stay on the 128 × 128 tile, and so does the SwiGLU adjoint
// under 2048: at one block per CU nothing overlaps a tile's epilogue, and
// that epilogue (two bf16 operands read, two written per output) outweighs
// the main loop's gain at short k (config 5, K = 1024: 324 against 296 µs).
int pick_cfg(const GemmBf16Params &p) {
    if (p.epi == EPI_SWIGLU_BWD && p.K < 2048) return 7;
    // Grouped rows with a single B: the MoE down and input-gradient GEMMs
    // (N = 1024, eight experts' B operands) ran slower per unit of work on
    // the 256 × 256 tile than on two 128 × 128 blocks per CU (config 5: one
    // round of 256 tiles 218 µs, against 203 µs for the whole down GEMM on the
    // 128 × 128 tile), so they stay there, stream-K remainder or not.
    if (p.grid == GRID_ROWS && p.epi != EPI_SWIGLU_FWD) return 7;
    const bool dual = p.epi == EPI_SWIGLU_FWD;
    const int64_t tn2 = (p.N + (dual ? 127 : 255)) / (dual ? 128 : 256);
    const int64_t tn1 = (p.N + (dual ? 63 : 127)) / (dual ? 64 : 128);
    int64_t t2, t1, klen;
    if (p.grid == GRID_PLAIN) {
        t2 = (p.M + 255) / 256 * tn2;
        t1 = (p.M + 127) / 128 * tn1;
        klen = p.K;
    } else if (p.grid == GRID_ROWS) {
        if (!p.tiles256) return 7;
        t2 = (int64_t)p.max_tiles256 * tn2;
        t1 = (int64_t)p.max_tiles * tn1;
        klen = p.K;
    } else {
        const int64_t e = p.n_experts > 0 ? p.n_experts : 1;
        t2 = (p.M + 255) / 256 * tn2 * e;
        t1 = (p.M + 127) / 128 * tn1 * e;
        klen = p.seg_offsets ? p.K / e : p.ksplit;
    }
    if (klen < 256) return 7;
    const int64_t cus = device_cus();
    const double pp = (double)((t2 + cus - 1) / cus) * 4.0 / 1.2;
    const double c7 = (double)((t1 + 2 * cus - 1) / (2 * cus)) * 2.0;
    // Configuration 12 (stream-K remainder, scratch given, at least one whole
    // round): the whole rounds, then the remainder's tiles cut in S = CUs /
    // rem k ranges, plus the fixup (reads S·rem partial tiles: about 0.15 of
    // a round, more when k is short).
    double sk = 1e30;
    if (p.sk_part && !dual && p.grid == GRID_PLAIN && t2 >= cus) {
        const int64_t full = t2 / cus, rem = t2 - full * cus;
        sk = (double)full * 4.0 / 1.2;
        if (rem > 0) sk += 4.0 / 1.2 / (double)(cus / rem) + 0.15 + 0.3 * 1024.0 / (double)klen;
    }
    if (sk < pp && sk < c7) return 12;
    return pp < c7 ? 11 : 7;
}

}  // namespace

int gemm_bf16_tile_rows() { return kRowTile; }

int64_t gemm_bf16_sk_floats() { return (int64_t)device_cus() * Cfg11::BM * Cfg11::BN; }

int64_t gemm_bf16_tiles_ints(int64_t rows, int n_experts) {
    return 2 * (int64_t)max_tiles_for(rows, n_experts, kRowTile) + 1 + 2 * (int64_t)max_tiles_for(rows, n_experts, 256) + 1;
}

void gemm_bf16_build_tiles(hipStream_t s, const int32_t *offsets, int n_experts, int64_t rows, int32_t *tiles) {
    CATNN_REQUIRE(n_experts > 0 && n_experts <= kMaxExperts, CATNN_ERR_SHAPE_MISMATCH, "tile table: expert count");
    const int m1 = max_tiles_for(rows, n_experts, kRowTile), m2 = max_tiles_for(rows, n_experts, 256);
    build_tiles2_kernel<<<1, 64, 0, s>>>(offsets, n_experts, tiles, m1, tiles + 2 * m1 + 1, m2);
    CATNN_HIP(hipGetLastError());
}

void gemm_bf16_use_tiles(GemmBf16Params &p, const int32_t *tiles, int64_t rows, int n_experts) {
    const int m1 = max_tiles_for(rows, n_experts, kRowTile), m2 = max_tiles_for(rows, n_experts, 256);
    p.tile_expert = tiles;
    p.tile_row0 = tiles + m1;
    p.n_tiles = tiles + 2 * m1;
    p.max_tiles = m1;
    p.tiles256 = tiles + 2 * m1 + 1;
    p.max_tiles256 = m2;
}

// Up to 8 splits while the split grid stays within 512 tiles (two per CU)
// and each segment keeps 1024 or more k values; only grids of at most 256
// tiles (one per CU) with 16-byte output rows are split.  The case is a
// weight gradient with few outputs and many tokens: config 5's wo gradient
// (1024 × 1024 × 8192, 64 tiles) took 89 µs unsplit, 193 TFLOP/s; its
// 192–256-tile gradients (QKV, fc1, fc2), one tile per CU unsplit, take
// 67–77 µs in two halves plus 7–9 µs of partial sums against 96–103 µs.
int gemm_bf16_splitk(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
    if (tiles > 256 || K < 2048 || N % 4 != 0) return 1;
    int s = 1;
    while (s < 8 && tiles * s * 2 <= 512 && K / (s * 2) >= 1024) s *= 2;
    return s;
}

// Segment length: whole 64-deep chunks (the last segment takes the rest).
int gemm_bf16_splitk_len(int64_t K, int splits) { return (int)((K / splits + 63) / 64 * 64); }

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
    if (cfg >= 7 && !vec) cfg = dual ? 0 : 2;  // direct-to-LDS tiles need 16-byte aligned rows
    CATNN_REQUIRE(!p.b_kwrap || (cfg >= 7 && p.b_kwrap % 64 == 0 && p.K % p.b_kwrap == 0 &&
                                 p.ldb >= p.b_kwrap),
                  CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: a wrapping B needs aligned rows and whole k chunks");
    // The staged epilogue moves 8 consecutive outputs per access: every
    // output, saved and residual row must start on a 16-byte boundary.
    GemmBf16Params q = p;
    q.vec_epi = epi_rows_aligned(p);
    q.sk_ctas = 0;  // set for configuration 12 only
    if (cfg == 12 && (dual || p.grid == GRID_SEGK || !p.sk_part || !vec)) cfg = 11;
    if ((cfg == 11 || cfg == 12) && p.grid == GRID_ROWS) {
        CATNN_REQUIRE(p.tiles256, CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: 256-row tiles need their tile table");
        q.tile_expert = p.tiles256;
        q.tile_row0 = p.tiles256 + p.max_tiles256;
        q.n_tiles = p.tiles256 + 2 * p.max_tiles256;
        q.max_tiles = p.max_tiles256;
    }
    switch (cfg) {
        case 0: launch_cfg<Cfg0, true>(s, q, vec, dual, gy); break;
        case 2: launch_cfg<Cfg2, false>(s, q, vec, dual, gy); break;
        case 7: launch_cfg<Cfg7, true>(s, q, vec, dual, gy); break;
        case 9: launch_cfg<Cfg9, false>(s, q, vec, dual, gy); break;
        case 10: launch_cfg<Cfg10, true>(s, q, vec, dual, gy); break;
        case 11: launch_cfg<Cfg11, true>(s, q, vec, dual, gy); break;
        case 12: {
            // One block per CU; the fixup finishes the remainder's tiles.
            const bool ok_epi = p.grid == GRID_PLAIN
                                    ? (p.epi == EPI_STORE || p.epi == EPI_LINEAR || p.epi == EPI_GELU_BWD)
                                    : (p.epi == EPI_STORE || p.epi == EPI_SWIGLU_BWD);
            CATNN_REQUIRE(ok_epi, CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: epilogue not built for this grid");
            if (p.grid == GRID_PLAIN && p.M == 0) return;
            q.sk_ctas = device_cus();
            const int64_t tiles_n = (p.N + Cfg11::BN - 1) / Cfg11::BN;
            // the ordinary grid: the plain grid's whole rounds, or the grouped grid's tile bound
            const int64_t g1 = p.grid == GRID_PLAIN
                                   ? ((p.M + Cfg11::BM - 1) / Cfg11::BM * tiles_n) / q.sk_ctas * q.sk_ctas
                                   : (int64_t)q.max_tiles * tiles_n;
            static bool attr_set[2] = {false, false};  // per grid: the opt-in for 128 KiB of LDS
            auto run = [&](int gi, auto pieces, auto fix) {
                if (!attr_set[gi]) {
                    CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(pieces),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, Cfg11::LDS_BYTES));
                    attr_set[gi] = true;
                }
                pieces<<<(unsigned)q.sk_ctas, Cfg11::NT, Cfg11::LDS_BYTES, s>>>(q);
                fix<<<(unsigned)q.sk_ctas * 32, 256, 0, s>>>(q);
            };
            if (p.grid == GRID_PLAIN) {
                if (g1 > 0) launch_kernel<Cfg11, GRID_PLAIN, false>(s, q, vec, dim3((unsigned)g1));
                run(0, gemm_bf16_sk_kernel<Cfg11, GRID_PLAIN>, sk_fixup_kernel<GRID_PLAIN>);
            } else {
                if (g1 > 0) launch_kernel<Cfg11, GRID_ROWS, false>(s, q, vec, dim3((unsigned)g1));
                run(1, gemm_bf16_sk_kernel<Cfg11, GRID_ROWS>, sk_fixup_kernel<GRID_ROWS>);
            }
            CATNN_HIP(hipGetLastError());
            break;
        }
        default: fail(CATNN_ERR_INVALID_ARGUMENT, "bf16 gemm: unknown tile configuration");
    }
}

// Tile choice, from sweeps of the training step's shapes on MI355X
// (TFLOP/s).  The direct-to-LDS 128×128 tile with two stages and two blocks
// per CU (configuration 7) leads on all of them once the epilogue is staged:
// 8192×4096×3072 839, 8192×1024×12288 898, 4096×1024×8192 732, against 603,
// 663 and 683 for three stages at one block per CU (configuration 9) and 749,
// 782 and 655 for four 32-deep stages (configuration 10); the register-staged
// tiles reached 742, 881 and 585.  Launches without 16-byte aligned rows run
// on the register-staged tiles (configuration 0 for the SwiGLU forward, 2
// otherwise).  The ping-pong tile (configuration 11) takes over when its
// grid fills the GPU (pick_cfg).
void gemm_bf16_launch(hipStream_t s, const GemmBf16Params &p) { gemm_bf16_launch_cfg(s, p, pick_cfg(p)); }

}  // namespace k
}  // namespace catnn
