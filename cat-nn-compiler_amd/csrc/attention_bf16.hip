// Attention core of the training step on bf16 MFMA (v_mfma_f32_32x32x16_bf16,
// fp32 accumulation), d_head = 64: the forward with its log-sum-exp and the
// two adjoint kernels, from bf16 copies of q, k, v and dO.  Same algorithm
// as the fp32 kernels of attention.hip / attention_bwd.hip (the score,
// softmax and PV part of attention_backward,
// crates/catnn-compile/src/kernel/adjoint.rs:582-722), with these rounding
// points, which the bf16 training step declares:
//   S = bf16(q)·bf16(k)ᵀ (fp32 accumulation), lse and the softmax in fp32;
//   O = bf16(P)·bf16(v) with P normalised (P = 2^(S·log2e/√dh − lse));
//   dV = bf16(P)ᵀ·bf16(dO), dP = bf16(dO)·bf16(v)ᵀ, dS = P∘(dP − D) in fp32,
//   dQ = bf16(dS)·bf16(k)/√dh, dK = bf16(dS)ᵀ·bf16(q)/√dh,
// with D_i = Σ_d dO[i][d]·O[i][d] from the fp32 forward output.  The forward
// takes two passes over the keys (the first for max and sum, the second for
// P·V), so that P is rounded after its normalisation, as the rounding model
// of the step rounds it.
//
// MFMA 32×32×16 operand layout: lane l supplies A[l%32][8(l/32) + j] and
// B[8(l/32) + j][l%32], j = 0..7; accumulator r of lane l is
// C[8(r/4) + 4(l/32) + r%4][l%32].  Products are arranged so that a lane's
// accumulators are one column: the scores of one query (forward, dQ) or of
// one key (dK/dV).  Such a column, converted to bf16, is directly the B
// operand of the next product when that product's reduction runs over the
// accumulator rows, with the rows taken in the order ρ(u, g, j) = 16u + 4g +
// j (j < 4), 16u + 8 + 4g + (j − 4) (j ≥ 4) for k step u; the other operand
// then comes from a transposed tile whose 16-byte chunks are stored in that
// order (TTile).  Every LDS tile row is 64 bf16 (128 bytes) with
// chunk c at position c ^ ((row / 2) mod 8): a 16-byte read serves 16 lanes
// per cycle from one 256-byte window of gfx950's 64 banks, and the 16
// consecutive rows of one chunk then fall on distinct banks.
//
// Transposed copies: xt[b][f][s] (transpose_bt) for f < F features of
// batch element b, s < Sp = S rounded up to 64, zero for s ≥ S, so that
// every 64-wide tile row is in bounds and 16-byte aligned.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "devmath.hpp"
#include "train_ops.hpp"

namespace catnn {
namespace k {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMasked = -1e30f;  // finite: a fully masked row never meets inf − inf
constexpr int DH = 64;
constexpr int ROWB = DH * 2;             // bytes per tile row
constexpr int TILE_BYTES = 64 * ROWB;    // one 64 × 64 bf16 tile

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int chunk_pos(int row, int c) { return row * ROWB + ((c ^ ((row >> 1) & 7)) << 4); }

__device__ __forceinline__ bf16x8 lds_frag(const unsigned char *tile, int row, int c) {
    return *reinterpret_cast<const bf16x8 *>(tile + chunk_pos(row, c));
}

// bf16x8 of accumulator entries base … base+7 (round to nearest even).
__device__ __forceinline__ bf16x8 pack8(const f32x16 &v, int base) {
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (__bf16)v[base + j];
    return r;
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.f;
    return z;
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// A row-major 64-row tile: rows r0 … r0+63 (rows ≥ nrows read as zero) of
// a bf16 matrix with row stride ld, columns col … col+63; two 16-byte chunks
// per thread of a 256-thread block.
struct RowTile {
    uint4 v[2];
    __device__ __forceinline__ void load(const bf16_t *base, int64_t ld, int r0, int nrows, int64_t col) {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int idx = threadIdx.x + 256 * it, row = idx >> 3, c = idx & 7;
            v[it] = r0 + row < nrows
                        ? *reinterpret_cast<const uint4 *>(base + (int64_t)(r0 + row) * ld + col + 8 * c)
                        : make_uint4(0, 0, 0, 0);
        }
    }
    __device__ __forceinline__ void store(unsigned char *tile) const {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int idx = threadIdx.x + 256 * it, row = idx >> 3, c = idx & 7;
            *reinterpret_cast<uint4 *>(tile + chunk_pos(row, c)) = v[it];
        }
    }
};

// A transposed tile: rows f0 … f0+63 of xt (row stride Sp), columns s0 …
// s0+63; thread t takes chunks 2p, 2p+1 (p = t mod 4) of row t / 4 and stores
// their halves in ρ order: chunk 2p holds columns 16p + {0..3, 8..11} and
// chunk 2p+1 columns 16p + {4..7, 12..15}.
struct TTile {
    uint4 a, b;
    __device__ __forceinline__ void load(const bf16_t *xt, int64_t row0, int64_t Sp, int s0) {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        const bf16_t *src = xt + (row0 + row) * Sp + s0 + 16 * p;
        a = *reinterpret_cast<const uint4 *>(src);
        b = *reinterpret_cast<const uint4 *>(src + 8);
    }
    __device__ __forceinline__ void store(unsigned char *tile) const {
        const int row = threadIdx.x >> 2, p = threadIdx.x & 3;
        *reinterpret_cast<uint4 *>(tile + chunk_pos(row, 2 * p)) = make_uint4(a.x, a.y, b.x, b.y);
        *reinterpret_cast<uint4 *>(tile + chunk_pos(row, 2 * p + 1)) = make_uint4(a.z, a.w, b.z, b.w);
    }
};

// ------------------------------------------------------------- forward
// Block: 4 wavefronts × 32 queries of one (b, h); key tiles of 64.  Lane l
// of wavefront w owns query q0 + 32w + l%32: Sᵀ = K·Qᵀ (A = K from LDS, B =
// the query's bf16 row in registers), Oᵀ += Vᵀ·Pᵀ (A = the transposed V
// tile, B = P from the score accumulators).
__global__ __launch_bounds__(256, 2) void attn_fwd_bf16_kernel(
    const bf16_t *__restrict__ qkv, int64_t ld, int64_t kcol, const bf16_t *__restrict__ xt, int64_t F,
    int64_t Sp, int64_t vrow, float *__restrict__ o, int64_t ldo, float *__restrict__ lse, int S, int H,
    float qscale, int causal, int n_qblocks) {
    constexpr int BQ = 128, BKV = 64;
    __shared__ __align__(16) unsigned char Ks[2][TILE_BYTES];
    __shared__ __align__(16) unsigned char Vt[2][TILE_BYTES];

    int blk, bh;
    split_bh_block(blockIdx.x, n_qblocks, (int)(gridDim.x / n_qblocks), blk, bh);
    const int qb = n_qblocks - 1 - blk;
    const int b = bh / H, h = bh % H;
    const int q0 = qb * BQ;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 31, g = lane >> 5;
    const int qi = q0 + wave * 32 + lr;
    const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
    const bf16_t *base = qkv + (int64_t)b * S * ld;
    const int64_t qcol = (int64_t)h * DH, kc = kcol + (int64_t)h * DH;
    const int64_t vt_row = (int64_t)b * F + vrow + (int64_t)h * DH;

    bf16x8 qf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (qi < S) qf[s] = *reinterpret_cast<const bf16x8 *>(base + (int64_t)qi * ld + qcol + 16 * s + 8 * g);
        else
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[s][j] = (__bf16)0.f;
    }

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kv_end + BKV - 1) / BKV;

    // Scores of tile t (buffer buf), scaled into the log2 domain and masked.
    auto scores = [&](const unsigned char *kt, int j0, f32x16 (&sacc)[2]) {
        bool active[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int jb = j0 + 32 * kb;
            active[kb] = __builtin_amdgcn_readfirstlane(jb < S && (!causal || jb <= wave_qmax));
            sacc[kb] = zero16();
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                if (active[kb]) sacc[kb] = mfma(lds_frag(kt, 32 * kb + lr, 2 * s + g), qf[s], sacc[kb]);
        const bool full = __builtin_amdgcn_readfirstlane(j0 + BKV <= S && (!causal || j0 + BKV - 1 <= wave_qmin));
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = j0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
                const bool ok = full || (active[kb] && j < S && (!causal || j <= qi));
                sacc[kb][r] = ok ? sacc[kb][r] * qscale : kMasked;
            }
    };

    // Pass 1: running max and sum over every key of the query's row.
    float m = -INFINITY, l = 0.f;
    {
        RowTile kr;
        kr.load(base, ld, 0, S, kc);
        kr.store(Ks[0]);
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const bool more = t + 1 < ntiles;
            if (more) kr.load(base, ld, (t + 1) * BKV, S, kc);
            f32x16 sacc[2];
            scores(Ks[buf], t * BKV, sacc);
            float mx = kMasked;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m, mx);
            float ps = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) ps += fast_exp2(sacc[kb][r] - m_new);
            ps += __shfl_xor(ps, 32, 64);
            l = l * fast_exp2(m - m_new) + ps;
            m = m_new;
            if (more) kr.store(Ks[buf ^ 1]);
            __syncthreads();
        }
    }
    const float row_lse = m + log2f(fmaxf(l, 1e-30f));

    // Pass 2: P = 2^(S − lse), rounded to bf16, into Oᵀ += Vᵀ·Pᵀ.
    f32x16 oacc[2] = {zero16(), zero16()};
    RowTile kr;
    TTile vr;
    kr.load(base, ld, 0, S, kc);
    vr.load(xt, vt_row, Sp, 0);
    kr.store(Ks[0]);
    vr.store(Vt[0]);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) {
            kr.load(base, ld, (t + 1) * BKV, S, kc);
            vr.load(xt, vt_row, Sp, (t + 1) * BKV);
        }
        f32x16 sacc[2];
        scores(Ks[buf], t * BKV, sacc);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = fast_exp2(sacc[kb][r] - row_lse);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bf16x8 pb = pack8(sacc[u >> 1], 8 * (u & 1));
#pragma unroll
            for (int db = 0; db < 2; ++db) oacc[db] = mfma(lds_frag(Vt[buf], 32 * db + lr, 2 * u + g), pb, oacc[db]);
        }
        if (more) {
            kr.store(Ks[buf ^ 1]);
            vr.store(Vt[buf ^ 1]);
        }
        __syncthreads();
    }

    if (qi < S) {
        lse[((int64_t)b * S + qi) * H + h] = row_lse;
        float *dst = o + ((int64_t)b * S + qi) * ldo + (int64_t)h * DH;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *reinterpret_cast<float4 *>(dst + 32 * db + 8 * r4 + 4 * g) =
                    make_float4(oacc[db][4 * r4], oacc[db][4 * r4 + 1], oacc[db][4 * r4 + 2], oacc[db][4 * r4 + 3]);
    }
}

// --------------------------------------------------------- dK and dV
// Block: 4 wavefronts × 32 keys of one (b, h); query tiles of 64.  Lane l of
// wavefront w owns key k0 + 32w + l%32: S = Q·Kᵀ and dP = dO·Vᵀ (A = the Q
// and dO tiles, B = the key's bf16 K and V rows in registers), then
// dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS (A = the transposed Q and dO tiles, B = P and
// dS from the accumulators).  Dynamic LDS: two stages of the four tiles,
// then lse and D of the stage's queries.
constexpr int DKDV_STAGE = 4 * TILE_BYTES + 2 * 64 * 4;
constexpr int DKDV_LDS = 2 * DKDV_STAGE;

__global__ __launch_bounds__(256, 2) void attn_bwd_dkdv_bf16_kernel(
    const bf16_t *__restrict__ qkv, int64_t ld, int64_t kcol, int64_t vcol, const bf16_t *__restrict__ xt,
    int64_t F, int64_t Sp, const bf16_t *__restrict__ dob, int64_t ldob, const bf16_t *__restrict__ dot,
    int64_t Fo, const float *__restrict__ lse, const float *__restrict__ Dv, float *__restrict__ dk,
    float *__restrict__ dv, int64_t ldd, int S, int H, float qscale, float scale, int causal, int n_kblocks) {
    constexpr int BKEY = 128, BQ = 64;
    extern __shared__ __align__(16) unsigned char smem[];

    int kb_, bh;
    split_bh_block(blockIdx.x, n_kblocks, (int)(gridDim.x / n_kblocks), kb_, bh);
    const int b = bh / H, h = bh % H;
    const int k0 = kb_ * BKEY;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 31, g = lane >> 5;
    const int kj = k0 + wave * 32 + lr;
    const int wave_kmin = k0 + wave * 32, wave_kmax = wave_kmin + 31;
    const int64_t row_base = (int64_t)b * S;
    const bf16_t *base = qkv + row_base * ld;
    const bf16_t *dbase = dob + row_base * ldob;
    const int64_t qcol = (int64_t)h * DH;
    const int64_t qt_row = (int64_t)b * F + (int64_t)h * DH, ot_row = (int64_t)b * Fo + (int64_t)h * DH;

    bf16x8 kf[4], vf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (kj < S) {
            kf[s] = *reinterpret_cast<const bf16x8 *>(base + (int64_t)kj * ld + kcol + qcol + 16 * s + 8 * g);
            vf[s] = *reinterpret_cast<const bf16x8 *>(base + (int64_t)kj * ld + vcol + qcol + 16 * s + 8 * g);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) kf[s][j] = vf[s][j] = (__bf16)0.f;
        }
    }
    f32x16 dka[2] = {zero16(), zero16()}, dva[2] = {zero16(), zero16()};

    const int q_start = causal ? (k0 / BQ) * BQ : 0;
    const int ntiles = S > q_start ? (S - q_start + BQ - 1) / BQ : 0;
    auto stage = [&](int t) { return smem + (t & 1) * DKDV_STAGE; };
    RowTile qr, orr;
    TTile qtr, otr;
    float ls = 0.f, ds = 0.f;
    auto load = [&](int t) {
        const int i0 = q_start + t * BQ;
        qr.load(base, ld, i0, S, qcol);
        orr.load(dbase, ldob, i0, S, qcol);
        qtr.load(xt, qt_row, Sp, i0);
        otr.load(dot, ot_row, Sp, i0);
        if (threadIdx.x < 64) {
            const int i = i0 + threadIdx.x;
            ls = i < S ? lse[(row_base + i) * H + h] : 0.f;
            ds = i < S ? Dv[(row_base + i) * H + h] : 0.f;
        }
    };
    auto store = [&](int t) {
        unsigned char *st = stage(t);
        qr.store(st);
        orr.store(st + TILE_BYTES);
        qtr.store(st + 2 * TILE_BYTES);
        otr.store(st + 3 * TILE_BYTES);
        if (threadIdx.x < 64) {
            reinterpret_cast<float *>(st + 4 * TILE_BYTES)[threadIdx.x] = ls;
            reinterpret_cast<float *>(st + 4 * TILE_BYTES)[64 + threadIdx.x] = ds;
        }
    };

    if (ntiles > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const bool more = t + 1 < ntiles;
        if (more) load(t + 1);
        const int i0 = q_start + t * BQ;
        // Under the mask no query of this tile reaches the wavefront's keys.
        const bool skip = __builtin_amdgcn_readfirstlane(causal && i0 + BQ - 1 < wave_kmin);
        if (!skip) {
            const unsigned char *st = stage(t);
            const float *Ls = reinterpret_cast<const float *>(st + 4 * TILE_BYTES), *Ds = Ls + 64;
            const bool full = __builtin_amdgcn_readfirstlane(i0 + BQ <= S && wave_kmax < S &&
                                                             (!causal || i0 >= wave_kmax));
            // One 32-query block at a time keeps two score accumulators live.
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                f32x16 sacc = zero16(), dpacc = zero16();
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    sacc = mfma(lds_frag(st, 32 * mb + lr, 2 * s + g), kf[s], sacc);
                    dpacc = mfma(lds_frag(st + TILE_BYTES, 32 * mb + lr, 2 * s + g), vf[s], dpacc);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int ir = 32 * mb + 8 * (r >> 2) + 4 * g + (r & 3), i = i0 + ir;
                    const bool ok = full || (i < S && kj < S && (!causal || i >= kj));
                    const float p = ok ? fast_exp2(sacc[r] * qscale - Ls[ir]) : 0.f;
                    sacc[r] = p;
                    dpacc[r] = p * (dpacc[r] - Ds[ir]);
                }
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int u = 2 * mb + tt;
                    const bf16x8 pb = pack8(sacc, 8 * tt);
                    const bf16x8 dsb = pack8(dpacc, 8 * tt);
#pragma unroll
                    for (int db = 0; db < 2; ++db) {
                        dva[db] = mfma(lds_frag(st + 3 * TILE_BYTES, 32 * db + lr, 2 * u + g), pb, dva[db]);
                        dka[db] = mfma(lds_frag(st + 2 * TILE_BYTES, 32 * db + lr, 2 * u + g), dsb, dka[db]);
                    }
                }
            }
        }
        if (more) store(t + 1);
        __syncthreads();
    }

    if (kj < S) {
        float *dkr = dk + (row_base + kj) * ldd + qcol, *dvr = dv + (row_base + kj) * ldd + qcol;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = 32 * db + 8 * r4 + 4 * g;
                *reinterpret_cast<float4 *>(dkr + d) =
                    make_float4(dka[db][4 * r4] * scale, dka[db][4 * r4 + 1] * scale, dka[db][4 * r4 + 2] * scale,
                                dka[db][4 * r4 + 3] * scale);
                *reinterpret_cast<float4 *>(dvr + d) =
                    make_float4(dva[db][4 * r4], dva[db][4 * r4 + 1], dva[db][4 * r4 + 2], dva[db][4 * r4 + 3]);
            }
    }
}

// --------------------------------------------------------------- dQ
// Block: 4 wavefronts × 32 queries of one (b, h); key tiles of 64.  Lane l
// owns query q0 + 32w + l%32: Sᵀ = K·Qᵀ and dPᵀ = V·dOᵀ (A = the K and V
// tiles, B = the query's bf16 q and dO rows), then dQᵀ += Kᵀ·dSᵀ (A = the
// transposed K tile, B = dS from the accumulators).
constexpr int DQ_STAGE = 3 * TILE_BYTES;
constexpr int DQ_LDS = 2 * DQ_STAGE;

__global__ __launch_bounds__(256, 2) void attn_bwd_dq_bf16_kernel(
    const bf16_t *__restrict__ qkv, int64_t ld, int64_t kcol, int64_t vcol, const bf16_t *__restrict__ xt,
    int64_t F, int64_t Sp, const bf16_t *__restrict__ dob, int64_t ldob, const float *__restrict__ lse,
    const float *__restrict__ Dv, float *__restrict__ dq, int64_t ldd, int S, int H, float qscale, float scale,
    int causal, int n_qblocks) {
    constexpr int BQ = 128, BKV = 64;
    extern __shared__ __align__(16) unsigned char smem[];

    int blk, bh;
    split_bh_block(blockIdx.x, n_qblocks, (int)(gridDim.x / n_qblocks), blk, bh);
    const int qb = n_qblocks - 1 - blk;
    const int b = bh / H, h = bh % H;
    const int q0 = qb * BQ;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 31, g = lane >> 5;
    const int qi = q0 + wave * 32 + lr;
    const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
    const int64_t row_base = (int64_t)b * S;
    const bf16_t *base = qkv + row_base * ld;
    const int64_t qcol = (int64_t)h * DH;
    const int64_t kt_row = (int64_t)b * F + kcol + (int64_t)h * DH;

    bf16x8 qf[4], of[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (qi < S) {
            qf[s] = *reinterpret_cast<const bf16x8 *>(base + (int64_t)qi * ld + qcol + 16 * s + 8 * g);
            of[s] = *reinterpret_cast<const bf16x8 *>(dob + (row_base + qi) * ldob + qcol + 16 * s + 8 * g);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[s][j] = of[s][j] = (__bf16)0.f;
        }
    }
    const float row_lse = qi < S ? lse[(row_base + qi) * H + h] : 0.f;
    const float row_d = qi < S ? Dv[(row_base + qi) * H + h] : 0.f;
    f32x16 dqa[2] = {zero16(), zero16()};

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kv_end + BKV - 1) / BKV;
    auto stage = [&](int t) { return smem + (t & 1) * DQ_STAGE; };
    RowTile kr, vr;
    TTile ktr;
    auto load = [&](int t) {
        kr.load(base, ld, t * BKV, S, kcol + qcol);
        vr.load(base, ld, t * BKV, S, vcol + qcol);
        ktr.load(xt, kt_row, Sp, t * BKV);
    };
    auto store = [&](int t) {
        unsigned char *st = stage(t);
        kr.store(st);
        vr.store(st + TILE_BYTES);
        ktr.store(st + 2 * TILE_BYTES);
    };

    load(0);
    store(0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const bool more = t + 1 < ntiles;
        if (more) load(t + 1);
        const unsigned char *st = stage(t);
        const int j0 = t * BKV;
        const bool full = __builtin_amdgcn_readfirstlane(j0 + BKV <= S && (!causal || j0 + BKV - 1 <= wave_qmin));
        // One 32-key block at a time keeps two score accumulators live.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int jb = j0 + 32 * kb;
            if (!__builtin_amdgcn_readfirstlane(jb < S && (!causal || jb <= wave_qmax))) continue;
            f32x16 sacc = zero16(), dpacc = zero16();
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                sacc = mfma(lds_frag(st, 32 * kb + lr, 2 * s + g), qf[s], sacc);
                dpacc = mfma(lds_frag(st + TILE_BYTES, 32 * kb + lr, 2 * s + g), of[s], dpacc);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = jb + 8 * (r >> 2) + 4 * g + (r & 3);
                const bool ok = full || (j < S && (!causal || j <= qi));
                const float p = ok ? fast_exp2(sacc[r] * qscale - row_lse) : 0.f;
                dpacc[r] = p * (dpacc[r] - row_d);
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const bf16x8 dsb = pack8(dpacc, 8 * tt);
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    dqa[db] = mfma(lds_frag(st + 2 * TILE_BYTES, 32 * db + lr, 2 * (2 * kb + tt) + g), dsb, dqa[db]);
            }
        }
        if (more) store(t + 1);
        __syncthreads();
    }

    if (qi < S) {
        float *dst = dq + (row_base + qi) * ldd + qcol;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *reinterpret_cast<float4 *>(dst + 32 * db + 8 * r4 + 4 * g) =
                    make_float4(dqa[db][4 * r4] * scale, dqa[db][4 * r4 + 1] * scale, dqa[db][4 * r4 + 2] * scale,
                                dqa[db][4 * r4 + 3] * scale);
    }
}

// ------------------------------------------------------------ transpose
// y[b][f][s] = x[b·S + s][f] for f < F, s < Sp (zero for s ≥ S): one 64 × 64
// tile per block through LDS (row stride 66 bf16 against bank conflicts).
__global__ __launch_bounds__(256) void transpose_bt_kernel(const bf16_t *__restrict__ x, int64_t ldx, int S,
                                                           int64_t F, int64_t Sp, bf16_t *__restrict__ y) {
    __shared__ bf16_t tile[64][66];
    const int s0 = blockIdx.x * 64, f0 = blockIdx.y * 64, b = blockIdx.z;
    const bf16_t *xb = x + (int64_t)b * S * ldx;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = threadIdx.x + 256 * it, r = idx >> 3, c = idx & 7;
        const int s = s0 + r;
        const int64_t f = f0 + 8 * c;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (s < S && f + 8 <= F) v = *reinterpret_cast<const uint4 *>(xb + (int64_t)s * ldx + f);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            tile[r][8 * c + 2 * j] = (bf16_t)(w[j] & 0xffffu);
            tile[r][8 * c + 2 * j + 1] = (bf16_t)(w[j] >> 16);
        }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int idx = threadIdx.x + 256 * it, fr = idx >> 3, c = idx & 7;
        const int64_t f = f0 + fr;
        if (f >= F) continue;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = (uint32_t)tile[8 * c + 2 * j][fr] | ((uint32_t)tile[8 * c + 2 * j + 1][fr] << 16);
        *reinterpret_cast<uint4 *>(y + ((int64_t)b * F + f) * Sp + s0 + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int64_t attention_bf16_seq_pad(int64_t seq) { return (seq + 63) / 64 * 64; }

void transpose_bt(hipStream_t s, const bf16_t *x, int64_t ldx, int64_t batch, int64_t seq, int64_t F, bf16_t *y) {
    CATNN_REQUIRE(F % 8 == 0 && ldx % 8 == 0 && al16(x) && al16(y), CATNN_ERR_INVALID_ARGUMENT,
                  "transpose_bt: 16-byte aligned rows of a multiple of 8 features");
    if (batch == 0 || seq == 0 || F == 0) return;
    const int64_t Sp = attention_bf16_seq_pad(seq);
    CATNN_REQUIRE(batch <= 65535 && (F + 63) / 64 <= 65535, CATNN_ERR_SHAPE_MISMATCH, "transpose_bt: grid");
    transpose_bt_kernel<<<dim3((unsigned)(Sp / 64), (unsigned)((F + 63) / 64), (unsigned)batch), 256, 0, s>>>(
        x, ldx, (int)seq, F, Sp, y);
    CATNN_HIP(hipGetLastError());
}

bool attention_bf16_supported(int64_t d_head, int64_t ld) { return d_head == DH && ld % 8 == 0; }

void attention_core_fwd_bf16(hipStream_t s, const bf16_t *qkv, int64_t ld, const bf16_t *qkvt, float *ctx,
                             int64_t ldo, float *lse, int64_t batch, int64_t seq, int64_t n_heads, bool causal) {
    const int64_t D = n_heads * DH;
    CATNN_REQUIRE(batch >= 0 && seq >= 0 && n_heads > 0 && 3 * D <= ld && D <= ldo, CATNN_ERR_SHAPE_MISMATCH,
                  "bf16 attention: bad dims");
    CATNN_REQUIRE(ld % 8 == 0 && ldo % 4 == 0 && al16(qkv) && al16(qkvt) && al16(ctx), CATNN_ERR_INVALID_ARGUMENT,
                  "bf16 attention: rows must be 16-byte aligned");
    CATNN_REQUIRE(batch * seq * n_heads < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "bf16 attention: too many rows");
    if (batch == 0 || seq == 0) return;
    const int nqb = (int)((seq + 127) / 128);
    const float qscale = kLog2e / sqrtf((float)DH);
    attn_fwd_bf16_kernel<<<(unsigned)(batch * n_heads * nqb), 256, 0, s>>>(
        qkv, ld, D, qkvt, 3 * D, attention_bf16_seq_pad(seq), 2 * D, ctx, ldo, lse, (int)seq, (int)n_heads,
        qscale, causal ? 1 : 0, nqb);
    CATNN_HIP(hipGetLastError());
}

void attention_core_bwd_bf16(hipStream_t s, const bf16_t *qkv, int64_t ld, const bf16_t *qkvt, const float *ctx,
                             const float *dctx, int64_t ldo, const bf16_t *dctxb, const bf16_t *dctxt,
                             const float *lse, float *dqkv, int64_t ldd, int64_t batch, int64_t seq,
                             int64_t n_heads, bool causal, float *scratch) {
    const int64_t D = n_heads * DH;
    CATNN_REQUIRE(batch >= 0 && seq >= 0 && n_heads > 0 && 3 * D <= ld && 3 * D <= ldd && D <= ldo,
                  CATNN_ERR_SHAPE_MISMATCH, "bf16 attention backward: bad dims");
    CATNN_REQUIRE(ld % 8 == 0 && ldo % 8 == 0 && ldd % 4 == 0 && al16(qkv) && al16(qkvt) && al16(dctxb) &&
                      al16(dctxt) && al16(dqkv),
                  CATNN_ERR_INVALID_ARGUMENT, "bf16 attention backward: rows must be 16-byte aligned");
    CATNN_REQUIRE(batch * seq * n_heads < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH,
                  "bf16 attention backward: too many rows");
    if (batch == 0 || seq == 0) return;
    static bool attr_set = false;
    if (!attr_set) {
        CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(attn_bwd_dkdv_bf16_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, DKDV_LDS));
        CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(attn_bwd_dq_bf16_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, DQ_LDS));
        attr_set = true;
    }
    float *Dv = scratch;
    attention_rowdot(s, ctx, dctx, ldo, batch * seq, n_heads, DH, Dv);
    const int64_t Sp = attention_bf16_seq_pad(seq);
    const float qscale = kLog2e / sqrtf((float)DH), scale = 1.0f / sqrtf((float)DH);
    const int nb = (int)((seq + 127) / 128);
    attn_bwd_dkdv_bf16_kernel<<<(unsigned)(batch * n_heads * nb), 256, DKDV_LDS, s>>>(
        qkv, ld, D, 2 * D, qkvt, 3 * D, Sp, dctxb, ldo, dctxt, D, lse, Dv, dqkv + D, dqkv + 2 * D, ldd, (int)seq,
        (int)n_heads, qscale, scale, causal ? 1 : 0, nb);
    CATNN_HIP(hipGetLastError());
    attn_bwd_dq_bf16_kernel<<<(unsigned)(batch * n_heads * nb), 256, DQ_LDS, s>>>(
        qkv, ld, D, 2 * D, qkvt, 3 * D, Sp, dctxb, ldo, lse, Dv, dqkv, ldd, (int)seq, (int)n_heads, qscale, scale,
        causal ? 1 : 0, nb);
    CATNN_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace catnn
