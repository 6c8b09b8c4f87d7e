// Adjoint of the attention core (the score/softmax/PV part of
// attention_backward, crates/catnn-compile/src/kernel/adjoint.rs:582-722; the
// causal window as gqa_backward, adjoint.rs:372-405), fp32 MFMA, from the
// log-sum-exp the forward stored instead of the S×S probability matrix the
// reference keeps:
//   P  = exp2(S·log2e/√dh − lse),   D_i = Σ_d dO[i][d]·O[i][d],
//   dV = Pᵀ·dO,   dS = P ∘ (dO·Vᵀ − D),   dK = dSᵀ·Q/√dh,   dQ = dS·K/√dh.
// Two deterministic kernels, no atomics:
//  * dK/dV: a block owns 128 keys of one (b, h); with S = Q·Kᵀ computed as
//    A = Q (LDS), B = K (registers), lane l holds the scores of key l%32, so
//    dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS accumulate per key in registers and P, dS
//    sit exactly where the MFMA reads its B operand;
//  * dQ: a block owns 128 queries, the transposed frame of the forward
//    (Sᵀ = K·Qᵀ, dPᵀ = V·dOᵀ, dQᵀ += Kᵀ·dSᵀ), lane l owning query l%32.
// d_head 32, 64 and 128 take these kernels; other head sizes use
// one-wavefront-per-row kernels.
// Grouped K/V heads (gqa_backward, adjoint.rs:287-440): query head h reads
// K/V head h / group; a dK/dV block owns the keys of one K/V head and sums
// over the group's query heads in head order, so dK and dV need no atomics.
// A sliding window (window > 0, with causal) limits query i to keys
// [i − window + 1, i], as the forward.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "devmath.hpp"
#include "train_ops.hpp"

namespace catnn {
namespace k {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

// 2^x on the hardware exp unit (v_exp_f32; below 2^-126 flushes to zero).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// D[row·H + h] = Σ_d dO·O over head h.
__global__ __launch_bounds__(256) void attn_dot_kernel(const float *__restrict__ o,
                                                       const float *__restrict__ dout, int64_t ldo,
                                                       int64_t rows, int H, int DH,
                                                       float *__restrict__ D) {
    const int lane = threadIdx.x & 63;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= rows * H) return;
    const int64_t row = gw / H;
    const int h = (int)(gw % H);
    float s = 0.f;
    for (int d = lane; d < DH; d += 64)
        s += o[row * ldo + (int64_t)h * DH + d] * dout[row * ldo + (int64_t)h * DH + d];
    s = wave_sum(s);
    if (lane == 0) D[gw] = s;
}

// The same for d_head 64 on 16-byte aligned rows: 16 lanes per (row, head),
// one float4 of each operand a lane, a 16-lane butterfly sum.
__global__ __launch_bounds__(256) void attn_dot64_kernel(const float *__restrict__ o,
                                                         const float *__restrict__ dout, int64_t ldo,
                                                         int64_t rows, int H, float *__restrict__ D) {
    const int64_t pair = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int q = threadIdx.x & 15;
    float s = 0.f;
    if (pair < rows * H) {
        const int64_t off = (pair / H) * ldo + (pair % H) * 64 + 4 * q;
        const float4 a = *reinterpret_cast<const float4 *>(o + off);
        const float4 b = *reinterpret_cast<const float4 *>(dout + off);
        s = (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
    }
#pragma unroll
    for (int m = 8; m > 0; m >>= 1) s += __shfl_xor(s, m, 64);
    if (pair < rows * H && q == 0) D[pair] = s;
}

// Column swizzle of the transposed K tile of the dQ kernel (row d = head
// dimension): row d holds key j at j ^ tsw(d).  The transposing stores put
// 16 rows 4 apart into one wavefront store; with the swizzle those rows
// spread over the banks (2-way instead of 8-way conflicts), while a float4
// read of four consecutive keys stays contiguous (tsw is a multiple of 4).
// (The dK/dV kernel keeps its transposed tiles unswizzled: the swizzled
// reads lose their constant offsets and the kernel then spills.)
__device__ __forceinline__ int tsw(int d) { return ((d >> 3) & 7) << 2; }

template <int DH>
__global__ __launch_bounds__(256, DH == 128 ? 1 : 2) void attn_bwd_dkdv_kernel(
    const float *__restrict__ q, int64_t ldq, const float *__restrict__ k, const float *__restrict__ v,
    int64_t ldk, const float *__restrict__ dout, int64_t ldo, const float *__restrict__ lse,
    const float *__restrict__ Dv, float *__restrict__ dk, float *__restrict__ dv, int64_t ldd, int S,
    int H, int group, int window, float qscale, float scale, int causal, int n_kblocks) {
    static_assert(DH == 32 || DH == 64 || DH == 128, "d_head 32, 64 or 128");
    constexpr int BKEY = 128, BQ = 64, LDQ = DH + 4, LDT = BQ + 4;
    constexpr int IT = BQ * DH / 4 / 256;
    // Q and dO tiles row-major (the S and dP products read rows along d)
    // and transposed (dV and dK read four consecutive queries per float4).
    __shared__ float Qs[BQ][LDQ];
    __shared__ float Os[BQ][LDQ];
    __shared__ float Qt[DH][LDT];
    __shared__ float Ot[DH][LDT];
    __shared__ float Ls[BQ], Ds[BQ];

    // Low key blocks see the most queries: first, spread over the XCDs.
    int kb, bh;
    split_bh_block(blockIdx.x, n_kblocks, (int)(gridDim.x / n_kblocks), kb, bh);
    const int HK = H / group;
    const int b = bh / HK, hk = bh % HK;
    const int k0 = kb * BKEY;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, g = lane >> 5;
    const int kj = k0 + wave * 32 + lr;
    const int wave_kmin = k0 + wave * 32;
    const int64_t row_base = (int64_t)b * S;

    float kf[DH / 2], vf[DH / 2];
    if (kj < S) {
        const float4 *ks = reinterpret_cast<const float4 *>(k + (row_base + kj) * ldk + (int64_t)hk * DH + (DH / 2) * g);
        const float4 *vs = reinterpret_cast<const float4 *>(v + (row_base + kj) * ldk + (int64_t)hk * DH + (DH / 2) * g);
#pragma unroll
        for (int c = 0; c < DH / 8; ++c) {
            const float4 a = ks[c], bb = vs[c];
            kf[4 * c] = a.x; kf[4 * c + 1] = a.y; kf[4 * c + 2] = a.z; kf[4 * c + 3] = a.w;
            vf[4 * c] = bb.x; vf[4 * c + 1] = bb.y; vf[4 * c + 2] = bb.z; vf[4 * c + 3] = bb.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < DH / 2; ++s) kf[s] = vf[s] = 0.f;
    }
    f32x16 dka[DH / 32], dva[DH / 32];
#pragma unroll
    for (int db = 0; db < DH / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dka[db][r] = dva[db][r] = 0.f;

    // Query tiles of every query head of the group, head by head: tile t is
    // head hk·group + t / tiles_per_head at queries q_start + (t % tiles)·BQ.
    // The next Q/dO tile is loaded into registers while the current one is
    // consumed from LDS.
    const int q_start = causal ? (k0 / BQ) * BQ : 0;
    const int q_end = window > 0 ? min(S, k0 + BKEY - 1 + window) : S;
    const int tiles_per_head = q_end > q_start ? (q_end - q_start + BQ - 1) / BQ : 0;
    const int n_tiles = tiles_per_head * group;
    float4 pq[IT], po[IT];
    float pl = 0.f, pd = 0.f;
    auto gload = [&](int t) {
        const int h = hk * group + t / tiles_per_head;
        const int q0 = q_start + (t % tiles_per_head) * BQ;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int idx = tid + it * 256;
            const int r = idx / (DH / 4), c4 = idx % (DH / 4);
            const int qi = q0 + r;
            pq[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            po[it] = pq[it];
            if (qi < S) {
                pq[it] = *reinterpret_cast<const float4 *>(q + (row_base + qi) * ldq + (int64_t)h * DH + 4 * c4);
                po[it] = *reinterpret_cast<const float4 *>(dout + (row_base + qi) * ldo + (int64_t)h * DH + 4 * c4);
            }
        }
        if (tid < BQ) {
            const int qi = q0 + tid;
            pl = qi < S ? lse[(row_base + qi) * H + h] : 0.f;
            pd = qi < S ? Dv[(row_base + qi) * H + h] : 0.f;
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int idx = tid + it * 256;
            const int r = idx / (DH / 4), c4 = idx % (DH / 4);
            *reinterpret_cast<float4 *>(&Qs[r][4 * c4]) = pq[it];
            *reinterpret_cast<float4 *>(&Os[r][4 * c4]) = po[it];
            Qt[4 * c4 + 0][r] = pq[it].x; Qt[4 * c4 + 1][r] = pq[it].y;
            Qt[4 * c4 + 2][r] = pq[it].z; Qt[4 * c4 + 3][r] = pq[it].w;
            Ot[4 * c4 + 0][r] = po[it].x; Ot[4 * c4 + 1][r] = po[it].y;
            Ot[4 * c4 + 2][r] = po[it].z; Ot[4 * c4 + 3][r] = po[it].w;
        }
        if (tid < BQ) {
            Ls[tid] = pl;
            Ds[tid] = pd;
        }
    };

    if (n_tiles > 0) gload(0);
    for (int t = 0; t < n_tiles; ++t) {
        const int q0 = q_start + (t % tiles_per_head) * BQ;
        sstore();
        __syncthreads();
        if (t + 1 < n_tiles) gload(t + 1);
#pragma unroll
        for (int qb = 0; qb < BQ / 32; ++qb) {
            const int qs0 = q0 + qb * 32;
            const bool active = __builtin_amdgcn_readfirstlane(
                qs0 < S && (!causal || qs0 + 31 >= wave_kmin) && (window <= 0 || qs0 <= wave_kmin + 30 + window));
            if (!active) continue;
            // No mask needed: every query of the 32 and every key of the
            // wavefront in range, (causal) every key at or before every query,
            // and (window) every key within the window of every query.
            const bool full = __builtin_amdgcn_readfirstlane(
                qs0 + 31 < S && wave_kmin + 31 < S && (!causal || wave_kmin + 31 <= qs0) &&
                (window <= 0 || qs0 + 31 - wave_kmin <= window - 1));
            f32x16 sa, pa;
#pragma unroll
            for (int r = 0; r < 16; ++r) sa[r] = pa[r] = 0.f;
            const float *qrow = &Qs[qb * 32 + lr][(DH / 2) * g];
            const float *orow = &Os[qb * 32 + lr][(DH / 2) * g];
#pragma unroll
            for (int c = 0; c < DH / 8; ++c) {
                const float4 qv = *reinterpret_cast<const float4 *>(qrow + 4 * c);
                const float4 ov = *reinterpret_cast<const float4 *>(orow + 4 * c);
                sa = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.x, kf[4 * c + 0], sa, 0, 0, 0);
                sa = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.y, kf[4 * c + 1], sa, 0, 0, 0);
                sa = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.z, kf[4 * c + 2], sa, 0, 0, 0);
                sa = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.w, kf[4 * c + 3], sa, 0, 0, 0);
                pa = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.x, vf[4 * c + 0], pa, 0, 0, 0);
                pa = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.y, vf[4 * c + 1], pa, 0, 0, 0);
                pa = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.z, vf[4 * c + 2], pa, 0, 0, 0);
                pa = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.w, vf[4 * c + 3], pa, 0, 0, 0);
            }
            // Entry r holds query row qs0 + 8(r/4) + 4g + r%4 of key kj.
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int il = qb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                const int qi = q0 + il;
                const bool ok = full || (qi < S && kj < S && (!causal || kj <= qi) && (window <= 0 || qi - kj < window));
                const float p = ok ? fast_exp2(sa[r] * qscale - Ls[il]) : 0.f;
                pa[r] = p * (pa[r] - Ds[il]);
                sa[r] = p;
            }
            // dVᵀ[d][j] += Σ_i dO[i][d]·P[i][j];  dKᵀ[d][j] += Σ_i Q[i][d]·dS[i][j]
            // Step s uses query qb·32 + 8(s/4) + 4g + s%4: steps 4s4…4s4+3
            // read four consecutive queries of the transposed tiles.
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const int il0 = qb * 32 + 8 * s4 + 4 * g;
#pragma unroll
                for (int db = 0; db < DH / 32; ++db) {
                    const float4 ov = *reinterpret_cast<const float4 *>(&Ot[db * 32 + lr][il0]);
                    const float4 qv = *reinterpret_cast<const float4 *>(&Qt[db * 32 + lr][il0]);
                    dva[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.x, sa[4 * s4 + 0], dva[db], 0, 0, 0);
                    dka[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.x, pa[4 * s4 + 0], dka[db], 0, 0, 0);
                    dva[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.y, sa[4 * s4 + 1], dva[db], 0, 0, 0);
                    dka[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.y, pa[4 * s4 + 1], dka[db], 0, 0, 0);
                    dva[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.z, sa[4 * s4 + 2], dva[db], 0, 0, 0);
                    dka[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.z, pa[4 * s4 + 2], dka[db], 0, 0, 0);
                    dva[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(ov.w, sa[4 * s4 + 3], dva[db], 0, 0, 0);
                    dka[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(qv.w, pa[4 * s4 + 3], dka[db], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }
    if (kj < S) {
        float *dkr = dk + (row_base + kj) * ldd + (int64_t)hk * DH;
        float *dvr = dv + (row_base + kj) * ldd + (int64_t)hk * DH;
#pragma unroll
        for (int db = 0; db < DH / 32; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = db * 32 + 8 * r4 + 4 * g;
                *reinterpret_cast<float4 *>(dkr + d) =
                    make_float4(dka[db][4 * r4] * scale, dka[db][4 * r4 + 1] * scale,
                                dka[db][4 * r4 + 2] * scale, dka[db][4 * r4 + 3] * scale);
                *reinterpret_cast<float4 *>(dvr + d) =
                    make_float4(dva[db][4 * r4], dva[db][4 * r4 + 1], dva[db][4 * r4 + 2], dva[db][4 * r4 + 3]);
            }
    }
}

template <int DH>
__global__ __launch_bounds__(256, DH == 128 ? 1 : 2) void attn_bwd_dq_kernel(
    const float *__restrict__ q, int64_t ldq, const float *__restrict__ k, const float *__restrict__ v,
    int64_t ldk, const float *__restrict__ dout, int64_t ldo, const float *__restrict__ lse,
    const float *__restrict__ Dv, float *__restrict__ dq, int64_t ldd, int S, int H, int group, int window,
    float qscale, float scale, int causal, int n_qblocks) {
    static_assert(DH == 32 || DH == 64 || DH == 128, "d_head 32, 64 or 128");
    constexpr int BQ = 128, BKV = 64, LDK = DH + 4, LDT = BKV + 4;
    constexpr int KV_IT = BKV * DH / 4 / 256;
    // K and V row-major (Sᵀ and dPᵀ read rows along d); K also transposed,
    // so dQ reads four consecutive keys per float4.
    __shared__ float Ks[1][BKV][LDK];
    __shared__ float Vs[1][BKV][LDK];
    __shared__ float Kt[DH][LDT];

    int blk, bh;
    split_bh_block(blockIdx.x, n_qblocks, (int)(gridDim.x / n_qblocks), blk, bh);
    const int qb = n_qblocks - 1 - blk;
    const int b = bh / H, h = bh % H, hk = h / group;
    const int q0 = qb * BQ;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, g = lane >> 5;
    const int qi = q0 + wave * 32 + lr;
    const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
    const int64_t row_base = (int64_t)b * S;

    float qf[DH / 2], of[DH / 2];
    float lse_i = 0.f, D_i = 0.f;
    if (qi < S) {
        const float4 *qs = reinterpret_cast<const float4 *>(q + (row_base + qi) * ldq + (int64_t)h * DH + (DH / 2) * g);
        const float4 *os = reinterpret_cast<const float4 *>(dout + (row_base + qi) * ldo + (int64_t)h * DH + (DH / 2) * g);
#pragma unroll
        for (int c = 0; c < DH / 8; ++c) {
            const float4 a = qs[c], bb = os[c];
            qf[4 * c] = a.x * qscale; qf[4 * c + 1] = a.y * qscale;
            qf[4 * c + 2] = a.z * qscale; qf[4 * c + 3] = a.w * qscale;
            of[4 * c] = bb.x; of[4 * c + 1] = bb.y; of[4 * c + 2] = bb.z; of[4 * c + 3] = bb.w;
        }
        lse_i = lse[(row_base + qi) * H + h];
        D_i = Dv[(row_base + qi) * H + h];
    } else {
#pragma unroll
        for (int s = 0; s < DH / 2; ++s) qf[s] = of[s] = 0.f;
    }
    f32x16 dqa[DH / 32];
#pragma unroll
    for (int db = 0; db < DH / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqa[db][r] = 0.f;

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int t_first = window > 0 ? max(0, q0 - window + 1) / BKV : 0;  // tiles before the window are skipped
    const int ntiles = (kv_end + BKV - 1) / BKV;
    // The next K/V tile is loaded into registers while the current one is
    // consumed from LDS.
    float4 pk[KV_IT], pv[KV_IT];
    auto gload = [&](int t) {
#pragma unroll
        for (int it = 0; it < KV_IT; ++it) {
            const int idx = tid + it * 256;
            const int kr = idx / (DH / 4), c4 = idx % (DH / 4);
            const int key = t * BKV + kr;
            pk[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            pv[it] = pk[it];
            if (key < S) {
                const int64_t off = (row_base + key) * ldk + (int64_t)hk * DH + 4 * c4;
                pk[it] = *reinterpret_cast<const float4 *>(k + off);
                pv[it] = *reinterpret_cast<const float4 *>(v + off);
            }
        }
    };
    if (ntiles > t_first) gload(t_first);
    for (int t = t_first; t < ntiles; ++t) {
        const int buf = 0;
#pragma unroll
        for (int it = 0; it < KV_IT; ++it) {
            const int idx = tid + it * 256;
            const int kr = idx / (DH / 4), c4 = idx % (DH / 4);
            *reinterpret_cast<float4 *>(&Ks[buf][kr][4 * c4]) = pk[it];
            *reinterpret_cast<float4 *>(&Vs[buf][kr][4 * c4]) = pv[it];
            const int kc = kr ^ tsw(4 * c4);  // rows 4c4 … 4c4+3 share one swizzle
            Kt[4 * c4 + 0][kc] = pk[it].x; Kt[4 * c4 + 1][kc] = pk[it].y;
            Kt[4 * c4 + 2][kc] = pk[it].z; Kt[4 * c4 + 3][kc] = pk[it].w;
        }
        __syncthreads();
        if (t + 1 < ntiles) gload(t + 1);
        const int j0 = t * BKV;
        for (int kb = 0; kb < BKV / 32; ++kb) {
            const int jb = j0 + kb * 32;
            if (!__builtin_amdgcn_readfirstlane(jb < S && (!causal || jb <= wave_qmax) &&
                                                (window <= 0 || jb + 31 >= wave_qmin - window + 1)))
                continue;
            // No mask: all 32 keys in range, (causal) none after any query of
            // the wavefront and (window) none before any query's window.
            // Padded queries (≥ S) are never stored.
            const bool full = __builtin_amdgcn_readfirstlane(jb + 31 < S && (!causal || jb + 31 <= wave_qmin) &&
                                                             (window <= 0 || jb >= wave_qmax - window + 1));
            f32x16 sa, pa;
#pragma unroll
            for (int r = 0; r < 16; ++r) sa[r] = pa[r] = 0.f;
            {
                const float *krow = &Ks[buf][kb * 32 + lr][(DH / 2) * g];
                const float *vrow = &Vs[buf][kb * 32 + lr][(DH / 2) * g];
#pragma unroll
                for (int c = 0; c < DH / 8; ++c) {
                    const float4 kv = *reinterpret_cast<const float4 *>(krow + 4 * c);
                    const float4 vv = *reinterpret_cast<const float4 *>(vrow + 4 * c);
                    sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * c + 0], sa, 0, 0, 0);
                    sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * c + 1], sa, 0, 0, 0);
                    sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * c + 2], sa, 0, 0, 0);
                    sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * c + 3], sa, 0, 0, 0);
                    pa = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, of[4 * c + 0], pa, 0, 0, 0);
                    pa = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, of[4 * c + 1], pa, 0, 0, 0);
                    pa = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, of[4 * c + 2], pa, 0, 0, 0);
                    pa = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, of[4 * c + 3], pa, 0, 0, 0);
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = jb + 8 * (r >> 2) + 4 * g + (r & 3);
                const bool ok = full || (qi < S && j < S && (!causal || j <= qi) && (window <= 0 || j > qi - window));
                const float p = ok ? fast_exp2(sa[r] - lse_i) : 0.f;
                pa[r] = p * (pa[r] - D_i);  // dSᵀ entry
            }
            // dQᵀ[d][i] += Σ_j K[j][d]·dSᵀ[j][i]; steps 4s4…4s4+3 take keys
            // kb·32 + 8s4 + 4g + 0…3, one float4 of the transposed tile.
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int db = 0; db < DH / 32; ++db) {
                    const float4 kv = *reinterpret_cast<const float4 *>(
                        &Kt[db * 32 + lr][(kb * 32 + 8 * s4 + 4 * g) ^ tsw(db * 32 + lr)]);
                    dqa[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, pa[4 * s4 + 0], dqa[db], 0, 0, 0);
                    dqa[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, pa[4 * s4 + 1], dqa[db], 0, 0, 0);
                    dqa[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, pa[4 * s4 + 2], dqa[db], 0, 0, 0);
                    dqa[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, pa[4 * s4 + 3], dqa[db], 0, 0, 0);
                }
        }
        __syncthreads();
    }
    if (qi < S) {
        float *dst = dq + (row_base + qi) * ldd + (int64_t)h * DH;
#pragma unroll
        for (int db = 0; db < DH / 32; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = db * 32 + 8 * r4 + 4 * g;
                *reinterpret_cast<float4 *>(dst + d) =
                    make_float4(dqa[db][4 * r4] * scale, dqa[db][4 * r4 + 1] * scale,
                                dqa[db][4 * r4 + 2] * scale, dqa[db][4 * r4 + 3] * scale);
            }
    }
}

// Any head size ≤ 256: one wavefront per (b, h, query) for dQ ...
__global__ __launch_bounds__(256) void attn_bwd_dq_generic(
    const float *__restrict__ q, int64_t ldq, const float *__restrict__ k, const float *__restrict__ v,
    int64_t ldk, const float *__restrict__ dout, int64_t ldo, const float *__restrict__ lse,
    const float *__restrict__ Dv, float *__restrict__ dq, int64_t ldd, int B, int S, int H, int DH,
    int group, int window, float scale, int causal) {
    const int lane = threadIdx.x & 63;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= (int64_t)B * H * S) return;
    const int i = (int)(gw % S);
    const int64_t bh = gw / S;
    const int h = (int)(bh % H), b = (int)(bh / H), hk = h / group;
    const int64_t rb = (int64_t)b * S;
    float qv[4], ov[4], acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        qv[c] = d < DH ? q[(rb + i) * ldq + (int64_t)h * DH + d] : 0.f;
        ov[c] = d < DH ? dout[(rb + i) * ldo + (int64_t)h * DH + d] : 0.f;
        acc[c] = 0.f;
    }
    const float l2 = lse[(rb + i) * H + h], Di = Dv[(rb + i) * H + h];
    const int jend = causal ? i + 1 : S;
    for (int j = window > 0 ? max(0, i - window + 1) : 0; j < jend; ++j) {
        const float *kr = k + (rb + j) * ldk + (int64_t)hk * DH;
        const float *vr = v + (rb + j) * ldk + (int64_t)hk * DH;
        float sp = 0.f, dp = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = lane + 64 * c;
            if (d < DH) {
                sp += qv[c] * kr[d];
                dp += ov[c] * vr[d];
            }
        }
        const float p = exp2f(wave_sum(sp) * scale * kLog2e - l2);
        const float dsv = p * (wave_sum(dp) - Di);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = lane + 64 * c;
            if (d < DH) acc[c] += dsv * kr[d];
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        if (d < DH) dq[(rb + i) * ldd + (int64_t)h * DH + d] = acc[c] * scale;
    }
}

// ... and one wavefront per (b, h, key) for dK and dV.
__global__ __launch_bounds__(256) void attn_bwd_dkdv_generic(
    const float *__restrict__ q, int64_t ldq, const float *__restrict__ k, const float *__restrict__ v,
    int64_t ldk, const float *__restrict__ dout, int64_t ldo, const float *__restrict__ lse,
    const float *__restrict__ Dv, float *__restrict__ dk, float *__restrict__ dv, int64_t ldd, int B,
    int S, int H, int DH, int group, int window, float scale, int causal) {
    const int lane = threadIdx.x & 63;
    const int HK = H / group;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= (int64_t)B * HK * S) return;
    const int j = (int)(gw % S);
    const int64_t bh = gw / S;
    const int hk = (int)(bh % HK), b = (int)(bh / HK);
    const int64_t rb = (int64_t)b * S;
    float kv[4], vv[4], ak[4], av[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        kv[c] = d < DH ? k[(rb + j) * ldk + (int64_t)hk * DH + d] : 0.f;
        vv[c] = d < DH ? v[(rb + j) * ldk + (int64_t)hk * DH + d] : 0.f;
        ak[c] = av[c] = 0.f;
    }
    const int iend = window > 0 ? min(S, j + window) : S;
    for (int gi = 0; gi < group; ++gi)
    for (int i = causal ? j : 0; i < iend; ++i) {
        const int h = hk * group + gi;
        const float *qr = q + (rb + i) * ldq + (int64_t)h * DH;
        const float *orr = dout + (rb + i) * ldo + (int64_t)h * DH;
        float sp = 0.f, dp = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = lane + 64 * c;
            if (d < DH) {
                sp += qr[d] * kv[c];
                dp += orr[d] * vv[c];
            }
        }
        const float p = exp2f(wave_sum(sp) * scale * kLog2e - lse[(rb + i) * H + h]);
        const float dsv = p * (wave_sum(dp) - Dv[(rb + i) * H + h]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = lane + 64 * c;
            if (d < DH) {
                av[c] += p * orr[d];
                ak[c] += dsv * qr[d];
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        if (d < DH) {
            dk[(rb + j) * ldd + (int64_t)hk * DH + d] = ak[c] * scale;
            dv[(rb + j) * ldd + (int64_t)hk * DH + d] = av[c];
        }
    }
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void attention_rowdot(hipStream_t s, const float *o, const float *dout, int64_t ld, int64_t rows, int64_t n_heads,
                      int64_t d_head, float *D) {
    if (rows == 0) return;
    if (d_head == 64 && ld % 4 == 0 && al16(o) && al16(dout))
        attn_dot64_kernel<<<(unsigned)((rows * n_heads + 15) / 16), 256, 0, s>>>(o, dout, ld, rows, (int)n_heads, D);
    else
        attn_dot_kernel<<<(unsigned)((rows * n_heads + 3) / 4), 256, 0, s>>>(o, dout, ld, rows, (int)n_heads,
                                                                            (int)d_head, D);
    CATNN_HIP(hipGetLastError());
}

uint64_t attention_bwd_scratch_bytes(int64_t batch, int64_t seq, int64_t n_heads) {
    return (uint64_t)(batch * seq * n_heads) * 4;
}

void attention_core_bwd_gqa(hipStream_t s, const float *q, int64_t ldq, const float *k, const float *v,
                            int64_t ldk, int64_t group, int64_t window, const float *o, const float *dout,
                            int64_t ldo, const float *lse, float *dq, int64_t ld_dq, float *dk, float *dv,
                            int64_t ld_dkv, int64_t batch, int64_t seq, int64_t n_heads, int64_t d_head,
                            bool causal, float *scratch) {
    CATNN_REQUIRE(batch >= 0 && seq >= 0 && n_heads > 0 && d_head > 0 && d_head <= 256,
                  CATNN_ERR_SHAPE_MISMATCH, "attention backward: bad dims");
    CATNN_REQUIRE(group >= 1 && n_heads % group == 0, CATNN_ERR_SHAPE_MISMATCH,
                  "attention backward: n_heads not a multiple of the kv groups");
    CATNN_REQUIRE(n_heads * d_head <= ldq && n_heads * d_head <= ldo && n_heads * d_head <= ld_dq &&
                      (n_heads / group) * d_head <= ldk && (n_heads / group) * d_head <= ld_dkv,
                  CATNN_ERR_SHAPE_MISMATCH, "attention backward: row strides too small");
    CATNN_REQUIRE(window <= 0 || causal, CATNN_ERR_INVALID_ARGUMENT, "attention backward: a window needs causal");
    CATNN_REQUIRE(batch * seq * n_heads < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH,
                  "attention backward: too many rows");
    if (batch == 0 || seq == 0) return;
    const int win = (int)std::min<int64_t>(std::max<int64_t>(window, 0), seq);
    const int64_t rows = batch * seq;
    const int64_t HK = n_heads / group;
    float *D = scratch;
    attention_rowdot(s, o, dout, ldo, rows, n_heads, d_head, D);
    const float scale = 1.0f / sqrtf((float)d_head);
    const bool mfma = (d_head == 32 || d_head == 64 || d_head == 128) && ldq % 4 == 0 && ldk % 4 == 0 &&
                      ldo % 4 == 0 && ld_dq % 4 == 0 && ld_dkv % 4 == 0 && al16(q) && al16(k) && al16(v) &&
                      al16(dout) && al16(dq) && al16(dk) && al16(dv);
    if (mfma) {
        const int nkb = (int)((seq + 127) / 128);
        auto launch = [&](auto dkdv, auto dqk) {
            dkdv<<<(unsigned)(batch * HK * nkb), 256, 0, s>>>(q, ldq, k, v, ldk, dout, ldo, lse, D, dk, dv, ld_dkv,
                                                              (int)seq, (int)n_heads, (int)group, win,
                                                              scale * kLog2e, scale, causal ? 1 : 0, nkb);
            CATNN_HIP(hipGetLastError());
            dqk<<<(unsigned)(batch * n_heads * nkb), 256, 0, s>>>(q, ldq, k, v, ldk, dout, ldo, lse, D, dq, ld_dq,
                                                                  (int)seq, (int)n_heads, (int)group, win,
                                                                  scale * kLog2e, scale, causal ? 1 : 0, nkb);
            CATNN_HIP(hipGetLastError());
        };
        if (d_head == 32) launch(attn_bwd_dkdv_kernel<32>, attn_bwd_dq_kernel<32>);
        else if (d_head == 64) launch(attn_bwd_dkdv_kernel<64>, attn_bwd_dq_kernel<64>);
        else launch(attn_bwd_dkdv_kernel<128>, attn_bwd_dq_kernel<128>);
    } else {
        const unsigned qblocks = (unsigned)((batch * n_heads * seq + 3) / 4);
        const unsigned kblocks = (unsigned)((batch * HK * seq + 3) / 4);
        attn_bwd_dq_generic<<<qblocks, 256, 0, s>>>(q, ldq, k, v, ldk, dout, ldo, lse, D, dq, ld_dq, (int)batch,
                                                    (int)seq, (int)n_heads, (int)d_head, (int)group, win, scale,
                                                    causal ? 1 : 0);
        attn_bwd_dkdv_generic<<<kblocks, 256, 0, s>>>(q, ldq, k, v, ldk, dout, ldo, lse, D, dk, dv, ld_dkv,
                                                      (int)batch, (int)seq, (int)n_heads, (int)d_head, (int)group,
                                                      win, scale, causal ? 1 : 0);
        CATNN_HIP(hipGetLastError());
    }
}

void attention_core_bwd(hipStream_t s, const float *q, const float *k, const float *v, int64_t ld,
                        const float *o, const float *dout, int64_t ldo, const float *lse, float *dq,
                        float *dk, float *dv, int64_t ld_d, int64_t batch, int64_t seq,
                        int64_t n_heads, int64_t d_head, bool causal, float *scratch) {
    attention_core_bwd_gqa(s, q, ld, k, v, ld, 1, 0, o, dout, ldo, lse, dq, ld_d, dk, dv, ld_d, batch, seq,
                           n_heads, d_head, causal, scratch);
}

}  // namespace k
}  // namespace catnn
