// Attention core on gfx950: ctx = softmax(q·kᵀ/√dh)·v per (batch, head),
// non-causal (the reference op, cpu.rs:252-295) or causal (the masking of
// moe::gqa, crates/catnn-compile/src/kernel/moe.rs:104-121: query i sees keys
// j ≤ i, masked scores are −∞, inv = 1/max(Σ, 1e-30)).  The reference
// materialises an S×S score matrix per (b,h) and walks it sequentially; here
// the scores never leave registers.
//
// d_head 32, 64 and 128 run on fp32 MFMA with an online softmax.  The kernel works
// in the transposed frame so that each lane owns one query:
//   Sᵀ[j][i] = Σ_d K[j][d]·Q[i][d]   (A = K from LDS, B = Q from registers)
//   Oᵀ[d][i] += Σ_j V[j][d]·P[i][j]  (A = V from LDS, B = P from registers)
// With the 32×32 accumulator layout (lane l holds column l%32), lane l holds
// Sᵀ and Oᵀ entries of query i = l%32 only: the row max / row sum need one
// exchange with lane l^32, and the rescale of O is lane-local.  The P values
// sit in exactly the registers the second MFMA reads as its B operand, so P
// never goes through LDS.
//
// Block: 4 wavefronts × 32 queries = 128 queries of one (b, h); K/V tiles of
// 64 keys are staged in LDS, double-buffered behind register prefetch.
// Other head sizes use a one-wavefront-per-query kernel (the reference's
// small demo blocks have d_head = 4, Mixtral-tiny's 8).
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "devmath.hpp"
#include "kernels.hpp"
#include "train_ops.hpp"

namespace catnn {
namespace k {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
// Masked scores: far below any real score but finite, so a row whose keys
// are all masked so far never produces inf − inf.
constexpr float kMasked = -1e30f;

// 2^x on the hardware exp unit (v_exp_f32); results below 2^-126 flush to
// zero, which no softmax weight in the fp32 tolerance can see.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K and V rows have their own stride ldk and hold H / group heads (grouped-
// query attention: head h reads K/V head h / group); window > 0 restricts
// query i to keys [i − window + 1, i] (with causal set).
template <int DH>
__global__ __launch_bounds__(256, DH == 128 ? 1 : 2) void attn_mfma_kernel(const float *__restrict__ q,
                                                           const float *__restrict__ k,
                                                           const float *__restrict__ v,
                                                           int64_t ld, int64_t ldk, int group, int window,
                                                           float *__restrict__ o,
                                                           int64_t ldo, float *__restrict__ lse,
                                                           int S, int H, float qscale, int causal,
                                                           int n_qblocks, int pair_halves) {
    static_assert(DH == 32 || DH == 64 || DH == 128, "MFMA attention: d_head 32, 64 or 128");
    constexpr int BQ = 128, BKV = 64, LDK = DH + 4, LDV = BKV + 4;
    constexpr int KV_IT = BKV * DH / 4 / 256;  // float4 per thread per tile, per operand
    // K row-major; V transposed (Vt[d][key]) so that the four keys a lane
    // feeds to four consecutive P·V MFMAs are one 16-byte LDS read.  Row d
    // of Vt holds key j at column j ^ vsw(d): rows 8 apart land on other
    // banks, so the transposing stores (16 rows 4 apart per wavefront) are
    // 2-way instead of 8-way conflicted, while a read's 8 rows share one
    // swizzle and stay conflict-free.
    __shared__ float Ks[2][BKV][LDK];
    __shared__ float Vt[2][DH][LDV];

    // Causal work grows with the query block: start the heavy ones first,
    // spread evenly over the XCDs.  pair_halves (a grid of exactly two
    // blocks per CU, all resident at once): the second half runs light to
    // heavy, so block i and block i + grid/2, which share a CU, hold query
    // blocks n−1−k and k and every CU gets the same number of key tiles.
    int blk, bh;
    split_bh_block(blockIdx.x, n_qblocks, (int)(gridDim.x / n_qblocks), blk, bh);
    const int half = n_qblocks / 2;
    const int qb = pair_halves && blk >= half ? blk - half : n_qblocks - 1 - blk;
    const int b = bh / H, h = bh % H, hk = h / group;
    const int q0 = qb * BQ;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 31, g = lane >> 5;
    const int qi = q0 + wave * 32 + lr;
    const int wave_qmin = q0 + wave * 32, wave_qmax = wave_qmin + 31;
    const int64_t row_base = (int64_t)b * S;

    // This lane's query, pre-scaled into the log2 domain: Q[i][(DH/2)·g + s].
    constexpr int HALF = DH / 2;
    float qf[HALF];
    if (qi < S) {
        const float4 *src =
            reinterpret_cast<const float4 *>(q + (row_base + qi) * ld + (int64_t)h * DH + HALF * g);
#pragma unroll
        for (int c = 0; c < HALF / 4; ++c) {
            const float4 t = src[c];
            qf[4 * c + 0] = t.x * qscale;
            qf[4 * c + 1] = t.y * qscale;
            qf[4 * c + 2] = t.z * qscale;
            qf[4 * c + 3] = t.w * qscale;
        }
    } else {
#pragma unroll
        for (int s = 0; s < HALF; ++s) qf[s] = 0.f;
    }

    f32x16 oacc[DH / 32];
#pragma unroll
    for (int db = 0; db < DH / 32; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
    float m = -INFINITY, l = 0.f;

    const int kv_end = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kv_end + BKV - 1) / BKV;
    // Sliding window: tiles before the first key of the block's first query are skipped.
    const int t_first = window > 0 ? max(0, q0 - window + 1) / BKV : 0;

    auto vsw = [](int d) { return ((d >> 3) & 7) << 2; };
    float4 pk[KV_IT], pv[KV_IT];
    auto gload = [&](int t) {
#pragma unroll
        for (int it = 0; it < KV_IT; ++it) {
            const int idx = tid + it * 256;
            const int key = t * BKV + idx / (DH / 4);
            const int c4 = idx % (DH / 4);
            if (key < S) {
                const int64_t off = (row_base + key) * ldk + (int64_t)hk * DH + 4 * c4;
                pk[it] = *reinterpret_cast<const float4 *>(k + off);
                pv[it] = *reinterpret_cast<const float4 *>(v + off);
            } else {
                pk[it] = make_float4(0.f, 0.f, 0.f, 0.f);
                pv[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int it = 0; it < KV_IT; ++it) {
            const int idx = tid + it * 256;
            const int key = idx / (DH / 4), c4 = idx % (DH / 4);
            *reinterpret_cast<float4 *>(&Ks[buf][key][4 * c4]) = pk[it];
            // rows 4c4 … 4c4+3 share d >> 3, hence one swizzle
            const int kc = key ^ vsw(4 * c4);
            Vt[buf][4 * c4 + 0][kc] = pv[it].x;
            Vt[buf][4 * c4 + 1][kc] = pv[it].y;
            Vt[buf][4 * c4 + 2][kc] = pv[it].z;
            Vt[buf][4 * c4 + 3][kc] = pv[it].w;
        }
    };

    gload(t_first);
    sstore(t_first & 1);
    __syncthreads();
    for (int t = t_first; t < ntiles; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) gload(t + 1);
        const int j0 = t * BKV;

        f32x16 sacc[BKV / 32];
        bool active[BKV / 32];
        // A tile with every key in range and (causal) at or below every query
        // of the wavefront needs no mask.  Queries ≥ S are padding: their
        // scores are computed but never stored.
        const bool full = __builtin_amdgcn_readfirstlane(
            j0 + BKV <= S && (!causal || j0 + BKV - 1 <= wave_qmin) &&
            (window <= 0 || j0 >= wave_qmax - window + 1));
#pragma unroll
        for (int kb = 0; kb < BKV / 32; ++kb) {
            const int jb = j0 + kb * 32;
            active[kb] = __builtin_amdgcn_readfirstlane(jb < S && (!causal || jb <= wave_qmax) &&
                                                        (window <= 0 || jb + 31 >= wave_qmin - window + 1));
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
        }
        static_assert(BKV == 64, "two 32-key blocks per tile");
        if (active[0] && active[1]) {
            // Both key blocks: alternate their accumulator chains so that
            // consecutive MFMAs are independent.
            const float *k0 = &Ks[buf][lr][HALF * g], *k1 = &Ks[buf][32 + lr][HALF * g];
#pragma unroll
            for (int c = 0; c < HALF / 4; ++c) {
                const float4 a = *reinterpret_cast<const float4 *>(k0 + 4 * c);
                const float4 b = *reinterpret_cast<const float4 *>(k1 + 4 * c);
                sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qf[4 * c + 0], sacc[0], 0, 0, 0);
                sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(b.x, qf[4 * c + 0], sacc[1], 0, 0, 0);
                sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qf[4 * c + 1], sacc[0], 0, 0, 0);
                sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(b.y, qf[4 * c + 1], sacc[1], 0, 0, 0);
                sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qf[4 * c + 2], sacc[0], 0, 0, 0);
                sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(b.z, qf[4 * c + 2], sacc[1], 0, 0, 0);
                sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qf[4 * c + 3], sacc[0], 0, 0, 0);
                sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(b.w, qf[4 * c + 3], sacc[1], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < BKV / 32; ++kb) {
                if (!active[kb]) continue;
                const float *krow = &Ks[buf][kb * 32 + lr][HALF * g];
                float4 kf[HALF / 4];
#pragma unroll
                for (int c = 0; c < HALF / 4; ++c) kf[c] = *reinterpret_cast<const float4 *>(krow + 4 * c);
#pragma unroll
                for (int c = 0; c < HALF / 4; ++c) {
                    const float4 kv = kf[c];
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * c + 0], sacc[kb], 0, 0, 0);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * c + 1], sacc[kb], 0, 0, 0);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * c + 2], sacc[kb], 0, 0, 0);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * c + 3], sacc[kb], 0, 0, 0);
                }
            }
        }

        // Mask (edge tiles only) and running max for this lane's query.
        // Entry r of block kb is key j0 + 32kb + 8(r/4) + 4g + r%4.
        float mx = kMasked;
        if (full) {
#pragma unroll
            for (int kb = 0; kb < BKV / 32; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
        } else {
#pragma unroll
            for (int kb = 0; kb < BKV / 32; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int j = j0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    const bool ok = active[kb] && j < S && (!causal || j <= qi) &&
                                    (window <= 0 || j >= qi - window + 1);
                    const float sv = ok ? sacc[kb][r] : kMasked;
                    sacc[kb][r] = sv;
                    mx = fmaxf(mx, sv);
                }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m, mx);  // finite from the first tile on
        const float factor = fast_exp2(m - m_new);
        float psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < BKV / 32; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(sacc[kb][r] - m_new);
                sacc[kb][r] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 32, 64);
        l = l * factor + psum;
        m = m_new;
#pragma unroll
        for (int db = 0; db < DH / 32; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[db][r] *= factor;

        // Oᵀ += Vᵀ·Pᵀ: step s feeds key 32kb + 8(s/4) + 4g + s%4 from lane
        // half g — the key whose probability this lane holds in sacc[kb][s];
        // steps 4s4 … 4s4+3 read their four V values as one float4.
#pragma unroll
        for (int kb = 0; kb < BKV / 32; ++kb) {
            if (!active[kb]) continue;
            float4 vf[4][DH / 32];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int db = 0; db < DH / 32; ++db)
                    vf[s4][db] = *reinterpret_cast<const float4 *>(
                        &Vt[buf][db * 32 + lr][(kb * 32 + 8 * s4 + 4 * g) ^ vsw(db * 32 + lr)]);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int db = 0; db < DH / 32; ++db) {
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s4][db].x, sacc[kb][4 * s4 + 0], oacc[db], 0, 0, 0);
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s4][db].y, sacc[kb][4 * s4 + 1], oacc[db], 0, 0, 0);
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s4][db].z, sacc[kb][4 * s4 + 2], oacc[db], 0, 0, 0);
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s4][db].w, sacc[kb][4 * s4 + 3], oacc[db], 0, 0, 0);
                }
        }
        if (more) sstore(buf ^ 1);
        __syncthreads();
    }

    if (qi < S) {
        const float inv = 1.0f / fmaxf(l, 1e-30f);
        if (lse) lse[(row_base + qi) * H + h] = m + log2f(fmaxf(l, 1e-30f));
        float *dst = o + (row_base + qi) * ldo + (int64_t)h * DH;
#pragma unroll
        for (int db = 0; db < DH / 32; ++db)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = db * 32 + 8 * r4 + 4 * g;
                *reinterpret_cast<float4 *>(dst + d) =
                    make_float4(oacc[db][4 * r4 + 0] * inv, oacc[db][4 * r4 + 1] * inv,
                                oacc[db][4 * r4 + 2] * inv, oacc[db][4 * r4 + 3] * inv);
            }
    }
}

// Any head size up to 256: one wavefront per (b, h, query), lanes over the
// head dimension, online softmax over the keys.
__global__ __launch_bounds__(256) void attn_generic_kernel(const float *__restrict__ q,
                                                           const float *__restrict__ k,
                                                           const float *__restrict__ v,
                                                           int64_t ld, int64_t ldk, int group, int window,
                                                           float *__restrict__ o,
                                                           int64_t ldo, float *__restrict__ lse,
                                                           int B, int S, int H, int DH, float scale,
                                                           int causal) {
    const int lane = threadIdx.x & 63;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t total = (int64_t)B * H * S;
    if (gw >= total) return;
    const int i = (int)(gw % S);
    const int64_t bh = gw / S;
    const int h = (int)(bh % H), b = (int)(bh / H), hk = h / group;
    const int64_t row_base = (int64_t)b * S;
    float qv[4], acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        qv[c] = d < DH ? q[(row_base + i) * ld + (int64_t)h * DH + d] : 0.f;
        acc[c] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    const int jend = causal ? i + 1 : S;
    const int jstart = window > 0 ? max(0, i - window + 1) : 0;
    for (int j = jstart; j < jend; ++j) {
        const float *kr = k + (row_base + j) * ldk + (int64_t)hk * DH;
        float part = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = lane + 64 * c;
            if (d < DH) part += qv[c] * kr[d];
        }
        const float sc = wave_sum(part) * scale;
        const float m_new = fmaxf(m, sc);
        const float factor = expf(m - m_new);
        const float p = expf(sc - m_new);
        l = l * factor + p;
        m = m_new;
        const float *vr = v + (row_base + j) * ldk + (int64_t)hk * DH;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int d = lane + 64 * c;
            acc[c] = acc[c] * factor + (d < DH ? p * vr[d] : 0.f);
        }
    }
    const float inv = 1.0f / fmaxf(l, 1e-30f);
    if (lse && lane == 0) lse[(row_base + i) * H + h] = (m + logf(fmaxf(l, 1e-30f))) * kLog2e;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        if (d < DH) o[(row_base + i) * ldo + (int64_t)h * DH + d] = acc[c] * inv;
    }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    CATNN_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) CATNN_HIP(hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cus[dev];
}

}  // namespace

// ld_qkv: row stride of q; ldk: of k and v, which hold n_heads / group
// heads; window > 0: sliding window (with causal).
static void attention_fwd(hipStream_t s, const float *q, const float *k, const float *v,
                          int64_t ld_qkv, int64_t ldk, int64_t group, int64_t window, float *ctx,
                          int64_t ldo, float *lse, int64_t batch, int64_t seq, int64_t n_heads,
                          int64_t d_head, bool causal) {
    CATNN_REQUIRE(batch >= 0 && seq >= 0 && n_heads > 0 && d_head > 0, CATNN_ERR_SHAPE_MISMATCH,
                  "attention: bad dims");
    CATNN_REQUIRE(d_head <= 256, CATNN_ERR_SHAPE_MISMATCH, "attention: d_head > 256");
    CATNN_REQUIRE(group >= 1 && n_heads % group == 0, CATNN_ERR_SHAPE_MISMATCH,
                  "attention: n_heads not a multiple of the kv groups");
    CATNN_REQUIRE(n_heads * d_head <= ld_qkv && n_heads * d_head <= ldo &&
                      (n_heads / group) * d_head <= ldk,
                  CATNN_ERR_SHAPE_MISMATCH, "attention: heads exceed the row width");
    CATNN_REQUIRE(window <= 0 || causal, CATNN_ERR_INVALID_ARGUMENT, "attention: a window needs causal");
    CATNN_REQUIRE(batch * seq < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "attention: too many rows");
    if (batch == 0 || seq == 0) return;
    const float scale = 1.0f / sqrtf((float)d_head);
    const bool mfma = (d_head == 32 || d_head == 64 || d_head == 128) && ld_qkv % 4 == 0 && ldk % 4 == 0 &&
                      ldo % 4 == 0 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(ctx);
    const int win = (int)std::min<int64_t>(std::max<int64_t>(window, 0), seq);
    if (mfma) {
        const int nqb = (int)((seq + 127) / 128);
        const int64_t blocks = batch * n_heads * nqb;
        CATNN_REQUIRE(blocks < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "attention: grid too large");
        // Two blocks per CU (d_head ≤ 64): a causal grid of exactly that many
        // blocks pairs heavy with light query blocks per CU.
        const int pair = causal && win == 0 && d_head <= 64 && nqb % 2 == 0 && blocks == 2 * (int64_t)device_cus();
        auto launch = [&](auto kern) {
            kern<<<(unsigned)blocks, 256, 0, s>>>(q, k, v, ld_qkv, ldk, (int)group, win, ctx, ldo, lse, (int)seq,
                                                  (int)n_heads, scale * kLog2e, causal ? 1 : 0, nqb, pair);
        };
        if (d_head == 32) launch(attn_mfma_kernel<32>);
        else if (d_head == 64) launch(attn_mfma_kernel<64>);
        else launch(attn_mfma_kernel<128>);
    } else {
        const int64_t waves = batch * n_heads * seq;
        const int64_t blocks = (waves + 3) / 4;
        CATNN_REQUIRE(blocks < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "attention: grid too large");
        attn_generic_kernel<<<(unsigned)blocks, 256, 0, s>>>(q, k, v, ld_qkv, ldk, (int)group, win, ctx,
                                                             ldo, lse, (int)batch, (int)seq, (int)n_heads,
                                                             (int)d_head, scale, causal ? 1 : 0);
    }
    CATNN_HIP(hipGetLastError());
}

void attention_core_f32(hipStream_t s, const float *q, const float *k, const float *v,
                        int64_t ld_qkv, float *ctx, int64_t ldo, int64_t batch, int64_t seq,
                        int64_t n_heads, int64_t d_head, bool causal) {
    attention_fwd(s, q, k, v, ld_qkv, ld_qkv, 1, 0, ctx, ldo, nullptr, batch, seq, n_heads, d_head, causal);
}

void attention_core_gqa_f32(hipStream_t s, const float *q, const float *k, const float *v, int64_t ldq,
                            int64_t ldk, int64_t group, int64_t window, float *ctx, int64_t ldo,
                            int64_t batch, int64_t seq, int64_t n_heads, int64_t d_head) {
    attention_fwd(s, q, k, v, ldq, ldk, group, window, ctx, ldo, nullptr, batch, seq, n_heads, d_head, true);
}

void attention_core_fwd_lse(hipStream_t s, const float *q, const float *k, const float *v, int64_t ld,
                            float *ctx, int64_t ldo, float *lse, int64_t batch, int64_t seq,
                            int64_t n_heads, int64_t d_head, bool causal) {
    attention_fwd(s, q, k, v, ld, ld, 1, 0, ctx, ldo, lse, batch, seq, n_heads, d_head, causal);
}

void attention_core_fwd_lse_gqa(hipStream_t s, const float *q, int64_t ldq, const float *k, const float *v,
                                int64_t ldk, int64_t group, int64_t window, float *ctx, int64_t ldo, float *lse,
                                int64_t batch, int64_t seq, int64_t n_heads, int64_t d_head) {
    attention_fwd(s, q, k, v, ldq, ldk, group, window, ctx, ldo, lse, batch, seq, n_heads, d_head, true);
}

}  // namespace k
}  // namespace catnn

using namespace catnn;

extern "C" int catnn_hip_attention_core_f32(catnn_hip_device *dev, const float *q, const float *k,
                                            const float *v, float *ctx, int64_t batch, int64_t seq,
                                            int64_t d_model, int64_t n_heads, int64_t d_head,
                                            int32_t causal) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((q && k && v && ctx) || batch * seq == 0, CATNN_ERR_INVALID_ARGUMENT,
                      "attention: null operand");
        CATNN_REQUIRE(n_heads * d_head == d_model, CATNN_ERR_SHAPE_MISMATCH,
                      "attention: n_heads*d_head != d_model");
        k::attention_core_f32(dev->stream, q, k, v, d_model, ctx, d_model, batch, seq, n_heads,
                              d_head, causal != 0);
    });
}
