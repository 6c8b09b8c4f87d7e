// Mixture-of-experts layer on gfx950.
//
// Replaces moe::moe (crates/catnn-compile/src/kernel/moe.rs:197-223), which
// loops over tokens and, per (token, selected expert), runs a [1,H] SwiGLU
// GEMV streaming the expert's three weight matrices (moe.rs:159-174).  Here
// the layer runs as five launches over all tokens at once:
//
//  1. route     logits = x·gate with the exact summation order of
//               cpu::linear_seq (cpu.rs:115-126: s = 0; s += x[p]·g[p] for
//               p ascending, separate multiply and add), then per token the
//               top-k of a stable descending order (ties → lower expert id,
//               lens/moe.rs:175-187) by a butterfly arg-max across the
//               token's lanes, and w = exp(l − max)·(1/max(Σ, 1e-30)).
//               Bit-exact logits make the indices bit-exact.
//  2. permute   stable counting sort of the flattened slots s = t·k + k'
//               by expert: per-block histograms, a wavefront prefix scan
//               for the segment starts, and a scatter that ranks slots
//               inside each wavefront with ballot + popcount.
//  3. gate/up   grouped fp32 MFMA GEMM over each expert's row segment, A rows
//               gathered from x through the permutation, W1 and W3 tiles
//               side by side, epilogue silu(a)·c → h[pos].
//  4. down      grouped fp32 MFMA GEMM h[pos]·W2 → y[pos].
//  5. combine   out[t] = (0 + w[t,0]·y[pos(t,0)]) + w[t,1]·y[pos(t,1)] …,
//               ascending k with separate multiply and add, as moe.rs:212-220.
// No floating-point atomics anywhere, so results are run-to-run identical.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"
#include "devmath.hpp"
#include "gemm_f32.hpp"
#include "kernels.hpp"
#include "train_ops.hpp"

namespace catnn {
namespace k {

namespace {

constexpr int kRouteChunk = 64;   // hidden elements staged per LDS pass
// Slots per permutation block: a block's scatter visits its slots 256 at a
// time with three barriers each, so small chunks spread that serial work
// over more CUs (config 5's 16384 slots: 4096-slot chunks, 4 blocks, took
// 17.6 us for the scatter).
constexpr int kPermChunk = 512;
constexpr int kMaxRouteExperts = 256;
constexpr int kMaxTopK = 16;

__device__ void select_topk(const float *row, int E, int K, int64_t base, int32_t *__restrict__ idx_out,
                            float *__restrict__ w_out);
__device__ __forceinline__ void finish_route(float s, bool active, int tl, int e, int E, int K, int t0,
                                             float *__restrict__ lg, int32_t *__restrict__ idx_out,
                                             float *__restrict__ w_out, float *__restrict__ logits_out);

// One thread per (token, expert); tokens_per_block = 256 / E.
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ x,
                                                    const float *__restrict__ gate, int T, int H,
                                                    int E, int K, int tpb,
                                                    int32_t *__restrict__ idx_out,
                                                    float *__restrict__ w_out,
                                                    float *__restrict__ logits_out) {
#pragma clang fp contract(off)
    extern __shared__ float smem[];
    float *xs = smem;                                  // [tpb][kRouteChunk + 1]
    float *gs = xs + tpb * (kRouteChunk + 1);          // [kRouteChunk][E]
    float *lg = gs + kRouteChunk * E;                  // [tpb][E]
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * tpb;
    const int tl = tid / E, e = tid % E;
    const bool active = tl < tpb && t0 + tl < T;
    float s = 0.0f;
    for (int p0 = 0; p0 < H; p0 += kRouteChunk) {
        const int pc = min(kRouteChunk, H - p0);
        for (int i = tid; i < tpb * kRouteChunk; i += 256) {
            const int r = i / kRouteChunk, c = i % kRouteChunk;
            xs[r * (kRouteChunk + 1) + c] =
                (t0 + r < T && c < pc) ? x[(int64_t)(t0 + r) * H + p0 + c] : 0.f;
        }
        for (int i = tid; i < kRouteChunk * E; i += 256) {
            const int r = i / E;
            gs[i] = r < pc ? gate[(int64_t)(p0 + r) * E + (i % E)] : 0.f;
        }
        __syncthreads();
        if (active) {
            const float *xr = xs + tl * (kRouteChunk + 1);
            for (int p = 0; p < pc; ++p) {
                const float prod = xr[p] * gs[p * E + e];
                s = s + prod;
            }
        }
        __syncthreads();
    }
    finish_route(s, active, tl, e, E, K, t0, lg, idx_out, w_out, logits_out);
}

// Top-k of a stable descending order (repeated first-maximum selection) and
// the softmax of the selected logits, lens/moe.rs:175-187.
__device__ void select_topk(const float *row, int E, int K, int64_t base, int32_t *__restrict__ idx_out,
                            float *__restrict__ w_out) {
#pragma clang fp contract(off)
    int sel[kMaxTopK];
    unsigned long long taken[kMaxRouteExperts / 64] = {0, 0, 0, 0};
    for (int kk = 0; kk < K; ++kk) {
        int best = -1;
        for (int c = 0; c < E; ++c) {
            if ((taken[c >> 6] >> (c & 63)) & 1ull) continue;
            if (best < 0 || row[c] > row[best]) best = c;
        }
        sel[kk] = best;
        taken[best >> 6] |= 1ull << (best & 63);
    }
    float mx = -INFINITY;
    for (int kk = 0; kk < K; ++kk) mx = fmaxf(mx, row[sel[kk]]);
    float ex[kMaxTopK];
    float sum = 0.f;
    for (int kk = 0; kk < K; ++kk) {
        ex[kk] = expf(row[sel[kk]] - mx);
        sum = sum + ex[kk];
    }
    const float inv = 1.0f / fmaxf(sum, 1e-30f);
    for (int kk = 0; kk < K; ++kk) {
        if (idx_out) idx_out[base + kk] = sel[kk];
        if (w_out) w_out[base + kk] = ex[kk] * inv;
    }
}

// The same selection with the token's E logits in E consecutive lanes of a
// wavefront (lane e holds expert e; E a power of two ≤ 64, groups aligned
// on multiples of E): K rounds of a butterfly arg-max inside the group,
// an untaken expert beating a taken one, a larger logit a smaller one, and
// equal logits going to the lower expert — the first maximum that the
// serial selection finds.  The selected logits are the same floats, so the
// softmax below is select_topk's, bit for bit.  Every lane of the group
// must call it; lane `write` stores the token's entries.
__device__ void group_topk(float v, int e, int E, int K, bool write, int64_t base, int32_t *__restrict__ idx_out,
                           float *__restrict__ w_out) {
#pragma clang fp contract(off)
    bool taken = false;
    int sel[kMaxTopK];
    float sv[kMaxTopK];
    for (int kk = 0; kk < K; ++kk) {
        float bv = v;
        int be = taken ? E : e;  // index E: taken
        for (int off = 1; off < E; off <<= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oe = __shfl_xor(be, off, 64);
            const bool better = oe < E && (be >= E || ov > bv || (ov == bv && oe < be));
            if (better) {
                bv = ov;
                be = oe;
            }
        }
        sel[kk] = be;
        sv[kk] = bv;
        if (e == be) taken = true;
    }
    if (!write) return;
    float mx = -INFINITY;
    for (int kk = 0; kk < K; ++kk) mx = fmaxf(mx, sv[kk]);
    float ex[kMaxTopK];
    float sum = 0.f;
    for (int kk = 0; kk < K; ++kk) {
        ex[kk] = expf(sv[kk] - mx);
        sum = sum + ex[kk];
    }
    const float inv = 1.0f / fmaxf(sum, 1e-30f);
    for (int kk = 0; kk < K; ++kk) {
        if (idx_out) idx_out[base + kk] = sel[kk];
        if (w_out) w_out[base + kk] = ex[kk] * inv;
    }
}

// The end of a route kernel: logits out, then the top-k by lane groups
// (E a power of two up to 64) or by one thread per token through LDS.
__device__ __forceinline__ void finish_route(float s, bool active, int tl, int e, int E, int K, int t0,
                                             float *__restrict__ lg, int32_t *__restrict__ idx_out,
                                             float *__restrict__ w_out, float *__restrict__ logits_out) {
    if (active && logits_out) logits_out[(int64_t)(t0 + tl) * E + e] = s;
    if (E <= 64 && (E & (E - 1)) == 0) {  // uniform: the group sits in one wavefront
        group_topk(s, e, E, K, active && e == 0, (int64_t)(t0 + tl) * K, idx_out, w_out);
        return;
    }
    if (active) lg[tl * E + e] = s;
    __syncthreads();
    if (!active || e != 0) return;
    select_topk(lg + tl * E, E, K, (int64_t)(t0 + tl) * K, idx_out, w_out);
}

constexpr int kRouteGateFloats = 12288;  // LDS floats for one staged gate chunk (48 KiB)

// gsT[e][p − p0] = gate[p][e] for p in [p0, p0 + pc), rows ldt floats
// apart: a block-wide transposing copy with 8 loads in flight per thread.
__device__ __forceinline__ void stage_gate_t(const float *__restrict__ gate, int p0, int pc, int E,
                                             float *__restrict__ gsT, int ldt) {
    constexpr int GB = 8;
    const int n = pc * E;
    const float *src = gate + (int64_t)p0 * E;
    for (int i0 = threadIdx.x; i0 < n; i0 += 256 * GB) {
        float v[GB];
#pragma unroll
        for (int u = 0; u < GB; ++u) {
            const int i = i0 + u * 256;
            v[u] = i < n ? src[i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < GB; ++u) {
            const int i = i0 + u * 256;
            if (i < n) {
                const int p = i / E;
                gsT[(i - p * E) * ldt + p] = v[u];
            }
        }
    }
}
constexpr int kRouteXC = 64;  // hidden elements of x per staged chunk (16 float4)

constexpr int kRouteStages = 4;  // x chunks in LDS: three in flight while one is summed

// Token rows staged in LDS by direct loads (global_load_lds_dwordx4),
// kRouteStages chunks of kRouteXC columns deep.  One wave load fills 1 KiB: the
// chunk of a group of 4 token rows, row g at 64·g floats, its float4 j at
// position (j + 2g) mod 16; groups are 260 floats apart.  With that
// rotation and the 16-byte gap, the 8 tokens a wavefront reads at one step
// sit on 8 different bank quads.  The gate is staged transposed whole
// (E·(H+4) floats).  Each thread then runs its (token, expert) sum over p
// ascending with separate multiply and add, as route_kernel, reading x and
// its expert's weights as float4 from LDS.  tpb = 16·LPW tokens per block
// (each wavefront issues LPW wave loads per chunk); needs H % kRouteXC == 0
// and 16-byte aligned rows.
template <int LPW>
__global__ __launch_bounds__(256) void route_dma_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ gate, int T, int H, int E,
                                                        int K, int tpb, int32_t *__restrict__ idx_out,
                                                        float *__restrict__ w_out,
                                                        float *__restrict__ logits_out) {
#pragma clang fp contract(off)
    extern __shared__ float smem[];
    constexpr int GROUP = 4 * kRouteXC + 4;  // floats per staged group of 4 rows
    constexpr int groups = 4 * LPW;
    float *xs = smem;                         // [kRouteStages][groups][GROUP]
    float *gsT = xs + kRouteStages * groups * GROUP;  // [E][H + 4]
    float *lg = gsT + E * (H + 4);            // [tpb][E]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * tpb;
    const int tl = tid / E, e = tid % E;
    const bool active = tl < tpb && t0 + tl < T;
    // Wave loads: group q for q = wave, wave + 4, …; lane l fills row
    // 4q + l/16 at position l mod 16 with its float4 (l − 2·(l/16)) mod 16.
    // Rows past T read row T−1 (their sums are never stored).
    const int lrow = lane >> 4, lpos = lane & 15;
    const int lcol = 4 * ((lpos - 2 * lrow) & 15);
    auto issue = [&](int c) {
        float *st = xs + (c % kRouteStages) * groups * GROUP;
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            const int q = wave + 4 * j;
            const int row = min(t0 + 4 * q + lrow, T - 1);
            load_lds16(x + (int64_t)row * H + c * kRouteXC + lcol, st + q * GROUP);
        }
    };
    const int nc = H / kRouteXC;
#pragma unroll
    for (int c = 0; c < kRouteStages - 1; ++c)
        if (c < nc) issue(c);
    stage_gate_t(gate, 0, H, E, gsT, H + 4);
    float s = 0.0f;
    const float4 *gr = reinterpret_cast<const float4 *>(gsT + e * (H + 4));
    const int rg = tl & 3;
    const int xoff = (tl >> 2) * GROUP + rg * kRouteXC;
    for (int c = 0; c < nc; ++c) {
        // Chunk c in LDS (and the gate); chunk c−1 consumed by every thread.
        // Chunks c+1 and c+2 may stay in flight.
        if (c + 2 < nc) dma_sync<2 * LPW>();
        else if (c + 1 < nc) dma_sync<LPW>();
        else dma_sync<0>();
        if (c + kRouteStages - 1 < nc) issue(c + kRouteStages - 1);
        if (active) {
            const float *xr = xs + (c % kRouteStages) * groups * GROUP + xoff;
            const float4 *gc = gr + c * (kRouteXC / 4);
            // All of the chunk's operands first (one LDS wait), then the chain.
            float4 xv[kRouteXC / 4], gv[kRouteXC / 4];
#pragma unroll
            for (int q = 0; q < kRouteXC / 4; ++q) {
                xv[q] = *reinterpret_cast<const float4 *>(xr + 4 * ((q + 2 * rg) & 15));
                gv[q] = gc[q];
            }
#pragma unroll
            for (int q = 0; q < kRouteXC / 4; ++q) {
                s = s + xv[q].x * gv[q].x;
                s = s + xv[q].y * gv[q].y;
                s = s + xv[q].z * gv[q].z;
                s = s + xv[q].w * gv[q].w;
            }
        }
    }
    finish_route(s, active, tl, e, E, K, t0, lg, idx_out, w_out, logits_out);
}

// Rows of x 16-byte aligned (H % 4 == 0): each thread streams its token's
// row straight from memory as float4 (the E threads of a token read the
// same addresses), and the gate is staged transposed in LDS, gsT[e][p] with
// row stride HC + 4, HC hidden elements per chunk (all of H for the usual
// shapes), so a thread reads its expert's weights as float4 too.  The sum
// runs over p ascending with separate multiply and add, as route_kernel.
__global__ __launch_bounds__(256) void route_vec_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ gate, int T, int H, int E,
                                                        int K, int tpb, int HC,
                                                        int32_t *__restrict__ idx_out,
                                                        float *__restrict__ w_out,
                                                        float *__restrict__ logits_out) {
#pragma clang fp contract(off)
    extern __shared__ float smem[];
    float *gsT = smem;                 // [E][HC + 4]
    float *lg = gsT + E * (HC + 4);    // [tpb][E]
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * tpb;
    const int tl = tid / E, e = tid % E;
    const bool active = tl < tpb && t0 + tl < T;
    const float4 *xr = reinterpret_cast<const float4 *>(x + (int64_t)(active ? t0 + tl : 0) * H);
    float s = 0.0f;
    for (int p0 = 0; p0 < H; p0 += HC) {
        const int pc = min(HC, H - p0);
        __syncthreads();  // the previous chunk is consumed
        stage_gate_t(gate, p0, pc, E, gsT, HC + 4);
        __syncthreads();
        if (active) {
            const float4 *gr = reinterpret_cast<const float4 *>(gsT + e * (HC + 4));
            const float4 *xc = xr + p0 / 4;
#pragma unroll 8
            for (int q = 0; q < pc / 4; ++q) {
                const float4 xv = xc[q], gv = gr[q];
                s = s + xv.x * gv.x;
                s = s + xv.y * gv.y;
                s = s + xv.z * gv.z;
                s = s + xv.w * gv.w;
            }
        }
    }
    finish_route(s, active, tl, e, E, K, t0, lg, idx_out, w_out, logits_out);
}

// Per-block expert histogram of the slots [b·chunk, (b+1)·chunk).  Slots
// with an expert id outside [0, E) are counted in bad[0] and skipped.
// Clears the permutation's bad-id counter.  A kernel rather than
// hipMemsetAsync so that the path stays a plain kernel sequence for callers
// that capture it into a graph.
__global__ void zero_i32_kernel(int32_t *__restrict__ p) { *p = 0; }

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t *__restrict__ p, int64_t n, int32_t v,
                                                       int32_t *__restrict__ zero) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
    if (zero && i == 0) *zero = 0;
}

__global__ __launch_bounds__(256) void perm_count_kernel(const int32_t *__restrict__ idx,
                                                         int64_t n, int E,
                                                         int32_t *__restrict__ block_counts,
                                                         int32_t *__restrict__ bad) {
    __shared__ int cnt[kMaxExperts];
    for (int e = threadIdx.x; e < E; e += 256) cnt[e] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kPermChunk;
    for (int i = threadIdx.x; i < kPermChunk; i += 256) {
        const int64_t s = base + i;
        if (s < n) {
            const int e = idx[s];
            if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
            else atomicAdd(bad, 1);
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 256) block_counts[(int64_t)blockIdx.x * E + e] = cnt[e];
}

// counts, offsets (exclusive prefix, length E+1) and each block's starting
// position per expert.  One wavefront; thread e owns expert e.
// With pad > 1 every expert segment starts on a multiple of pad rows.
__global__ void perm_scan_kernel(const int32_t *__restrict__ block_counts, int nb, int E, int pad,
                                 int32_t *__restrict__ block_base, int32_t *__restrict__ counts,
                                 int32_t *__restrict__ offsets) {
    __shared__ int tot[kMaxExperts + 1];
    const int e = threadIdx.x;
    // Lane e walks the blocks' counts of expert e eight at a time, the
    // eight loads issued together (integer sums: any grouping is exact).
    if (e < E) {
        int run = 0;
        for (int b0 = 0; b0 < nb; b0 += 8) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = b0 + j < nb ? block_counts[(int64_t)(b0 + j) * E + e] : 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) run += v[j];
        }
        tot[e] = run;
        counts[e] = run;
    }
    __syncthreads();
    // Segment starts: exclusive prefix of the padded totals, a wavefront
    // inclusive scan (E ≤ 64 lanes).
    const int padded = e < E ? (tot[e] + pad - 1) / pad * pad : 0;
    int incl = padded;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (e >= off) incl += o;
    }
    __syncthreads();
    if (e < E) {
        tot[e] = incl - padded;
        offsets[e] = incl - padded;
    }
    if (e == E - 1) offsets[E] = incl;
    __syncthreads();
    // block_base[b][e] = the segment start of e + the counts of e in the
    // blocks before b
    if (e < E) {
        int run = tot[e];
        for (int b0 = 0; b0 < nb; b0 += 8) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = b0 + j < nb ? block_counts[(int64_t)(b0 + j) * E + e] : 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (b0 + j < nb) block_base[(int64_t)(b0 + j) * E + e] = run;
                run += v[j];
            }
        }
    }
}

// Stable scatter: slot s goes to offsets[e] + (number of earlier slots with
// the same expert).  Slots are visited in ascending order, 256 at a time;
// inside a wavefront the rank among equal experts is the popcount of the
// ballot below the lane, across wavefronts it is the counts of the lower
// wavefronts, across iterations and blocks the running totals.
__global__ __launch_bounds__(256) void perm_scatter_kernel(const int32_t *__restrict__ idx,
                                                           int64_t n, int E,
                                                           const int32_t *__restrict__ block_base,
                                                           int32_t *__restrict__ slot_of_pos,
                                                           int32_t *__restrict__ pos_of_slot) {
    __shared__ int running[kMaxExperts];
    __shared__ int wave_cnt[4][kMaxExperts];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += 256) running[e] = block_base[(int64_t)blockIdx.x * E + e];
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kPermChunk;
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int it = 0; it < kPermChunk / 256; ++it) {
        const int64_t s = base + it * 256 + tid;
        int e = s < n ? idx[s] : -1;
        if (e >= E) e = -1;
        int rank = 0;
        for (int c = 0; c < E; ++c) {
            const unsigned long long m = __ballot(e == c);
            if (e == c) rank = __popcll(m & below);
            if (lane == 0) wave_cnt[wave][c] = __popcll(m);
        }
        __syncthreads();
        if (e >= 0) {
            int pos = running[e] + rank;
            for (int w = 0; w < wave; ++w) pos += wave_cnt[w][e];
            slot_of_pos[pos] = (int32_t)s;
            pos_of_slot[s] = pos;
        } else if (s < n) {
            pos_of_slot[s] = -1;
        }
        __syncthreads();
        for (int c = tid; c < E; c += 256)
            running[c] += wave_cnt[0][c] + wave_cnt[1][c] + wave_cnt[2][c] + wave_cnt[3][c];
        __syncthreads();
    }
}

// out[t, c] = Σ_k (ascending) w[t,k]·y[pos(t,k), c], starting from 0.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y,
                                                      const int32_t *__restrict__ pos_of_slot,
                                                      const float *__restrict__ w, int T, int K,
                                                      int H, float *__restrict__ out) {
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    if (t >= T) return;
    for (int c = threadIdx.x; c < H; c += 256) {
        float acc = 0.0f;
        for (int kk = 0; kk < K; ++kk) {
            const int64_t slot = (int64_t)t * K + kk;
            const float prod = w[slot] * y[(int64_t)pos_of_slot[slot] * H + c];
            acc = acc + prod;
        }
        out[(int64_t)t * H + c] = acc;
    }
}

// The same on float4 runs of 16-byte aligned rows.  (One wavefront per
// token with all of its slot rows loaded before the sums measured 31.6
// against 32.8 us on config 4 and was not kept.)
__global__ __launch_bounds__(256) void combine4_kernel(const float *__restrict__ y,
                                                       const int32_t *__restrict__ pos_of_slot,
                                                       const float *__restrict__ w, int T, int K,
                                                       int H, float *__restrict__ out) {
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    if (t >= T) return;
    const int h4 = H / 4;
    for (int c = threadIdx.x; c < h4; c += 256) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int kk = 0; kk < K; ++kk) {
            const int64_t slot = (int64_t)t * K + kk;
            const float ws = w[slot];
            const float4 v =
                reinterpret_cast<const float4 *>(y + (int64_t)pos_of_slot[slot] * H)[c];
            const float px = ws * v.x, py = ws * v.y, pz = ws * v.z, pw = ws * v.w;
            acc.x = acc.x + px;
            acc.y = acc.y + py;
            acc.z = acc.z + pz;
            acc.w = acc.w + pw;
        }
        reinterpret_cast<float4 *>(out + (int64_t)t * H)[c] = acc;
    }
}

uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void moe_combine(hipStream_t s, const float *y, const int32_t *pos_of_slot, const float *w,
                 int64_t tokens, int64_t top_k, int64_t hidden, float *out) {
    if (tokens <= 0) return;
    if (hidden % 4 == 0 && aligned16(out) && aligned16(y))
        combine4_kernel<<<(unsigned)tokens, 256, 0, s>>>(y, pos_of_slot, w, (int)tokens, (int)top_k,
                                                         (int)hidden, out);
    else
        combine_kernel<<<(unsigned)tokens, 256, 0, s>>>(y, pos_of_slot, w, (int)tokens, (int)top_k,
                                                        (int)hidden, out);
    CATNN_HIP(hipGetLastError());
}

// Above 64 KiB of LDS a kernel needs the opt-in; two blocks per CU still fit.
template <int LPW>
static void launch_route_dma(hipStream_t s, int64_t blocks, size_t smem, const float *x, const float *gate,
                             int64_t tokens, int64_t hidden, int E, int64_t top_k, int tpb, int32_t *idx, float *w,
                             float *logits) {
    static bool attr = false;
    if (!attr) {
        CATNN_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(route_dma_kernel<LPW>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024));
        attr = true;
    }
    route_dma_kernel<LPW><<<(unsigned)blocks, 256, smem, s>>>(x, gate, (int)tokens, (int)hidden, E, (int)top_k, tpb,
                                                              idx, w, logits);
}

void moe_route_f32(hipStream_t s, const float *x, const float *gate, int64_t tokens, int64_t hidden,
                   int64_t n_experts, int64_t top_k, int32_t *idx, float *w, float *logits) {
    CATNN_REQUIRE(tokens >= 0 && hidden > 0 && n_experts > 0, CATNN_ERR_SHAPE_MISMATCH,
                  "route: bad dims");
    CATNN_REQUIRE(n_experts <= kMaxRouteExperts, CATNN_ERR_SHAPE_MISMATCH,
                  "route: more than 256 experts");
    CATNN_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= kMaxTopK, CATNN_ERR_SHAPE_MISMATCH,
                  "route: top_k must be in [1, min(n_experts, 16)]");
    CATNN_REQUIRE(tokens < (1ll << 31) && hidden < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH,
                  "route: dims exceed 2^31");
    if (tokens == 0) return;
    const int E = (int)n_experts;
    const int tpb = std::min(64, 256 / E);  // ≤ 64 tokens keeps the LDS stage under 20 KB
    const int64_t blocks = (tokens + tpb - 1) / tpb;
    const size_t dma_smem = sizeof(float) * ((size_t)kRouteStages * (tpb / 4) * (4 * kRouteXC + 4) +
                                             (size_t)E * (hidden + 4) + (size_t)tpb * E);
    if (hidden % kRouteXC == 0 && tpb % 16 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        dma_smem <= 80 * 1024) {
        if (tpb == 16) launch_route_dma<1>(s, blocks, dma_smem, x, gate, tokens, hidden, E, top_k, tpb, idx, w, logits);
        else if (tpb == 32) launch_route_dma<2>(s, blocks, dma_smem, x, gate, tokens, hidden, E, top_k, tpb, idx, w, logits);
        else launch_route_dma<4>(s, blocks, dma_smem, x, gate, tokens, hidden, E, top_k, tpb, idx, w, logits);
    } else if (hidden % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const int HC = (int)std::min<int64_t>(hidden, (kRouteGateFloats / E - 4) & ~3);
        const size_t smem = sizeof(float) * ((size_t)E * (HC + 4) + (size_t)tpb * E);
        route_vec_kernel<<<(unsigned)blocks, 256, smem, s>>>(x, gate, (int)tokens, (int)hidden, E, (int)top_k,
                                                             tpb, HC, idx, w, logits);
    } else {
        const size_t smem = sizeof(float) * ((size_t)tpb * (kRouteChunk + 1) +
                                             (size_t)kRouteChunk * E + (size_t)tpb * E);
        route_kernel<<<(unsigned)blocks, 256, smem, s>>>(x, gate, (int)tokens, (int)hidden, E,
                                                         (int)top_k, tpb, idx, w, logits);
    }
    CATNN_HIP(hipGetLastError());
}

uint64_t moe_permute_scratch_bytes(int64_t tokens, int64_t top_k, int64_t n_experts) {
    const int64_t n = tokens * top_k;
    const int64_t nb = (n + kPermChunk - 1) / kPermChunk;
    // block_counts + block_base + bad counter
    return align256((uint64_t)nb * n_experts * 4) * 2 + 256;
}

void moe_permute(hipStream_t s, const int32_t *idx, int64_t tokens, int64_t top_k, int64_t n_experts,
                 int32_t *counts, int32_t *offsets, int32_t *slot_of_pos, int32_t *pos_of_slot,
                 void *scratch) {
    CATNN_REQUIRE(n_experts > 0 && n_experts <= kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                  "permute: n_experts must be in [1, 64]");
    CATNN_REQUIRE(tokens >= 0 && top_k >= 1 && tokens * top_k < (1ll << 31),
                  CATNN_ERR_SHAPE_MISMATCH, "permute: slot count out of range");
    const int64_t n = tokens * top_k;
    const int E = (int)n_experts;
    const int64_t nb = (n + kPermChunk - 1) / kPermChunk;
    char *sc = static_cast<char *>(scratch);
    int32_t *block_counts = reinterpret_cast<int32_t *>(sc);
    int32_t *block_base = reinterpret_cast<int32_t *>(sc + align256((uint64_t)nb * E * 4));
    int32_t *bad = reinterpret_cast<int32_t *>(sc + 2 * align256((uint64_t)nb * E * 4));
    zero_i32_kernel<<<1, 1, 0, s>>>(bad);
    CATNN_HIP(hipGetLastError());
    if (nb > 0) {
        perm_count_kernel<<<(unsigned)nb, 256, 0, s>>>(idx, n, E, block_counts, bad);
        CATNN_HIP(hipGetLastError());
    }
    perm_scan_kernel<<<1, 64, 0, s>>>(block_counts, (int)nb, E, 1, block_base, counts, offsets);
    CATNN_HIP(hipGetLastError());
    if (nb > 0) {
        perm_scatter_kernel<<<(unsigned)nb, 256, 0, s>>>(idx, n, E, block_base, slot_of_pos,
                                                         pos_of_slot);
        CATNN_HIP(hipGetLastError());
    }
}

void moe_permute_padded(hipStream_t s, const int32_t *idx, int64_t tokens, int64_t top_k,
                        int64_t n_experts, int pad, int64_t n_pos_cap, int32_t *counts,
                        int32_t *offsets, int32_t *slot_of_pos, int32_t *pos_of_slot,
                        void *scratch) {
    CATNN_REQUIRE(n_experts > 0 && n_experts <= kMaxExperts && pad >= 1, CATNN_ERR_SHAPE_MISMATCH,
                  "permute: bad expert count or pad");
    const int64_t n = tokens * top_k;
    CATNN_REQUIRE(n_pos_cap >= n + n_experts * (pad - 1) && n_pos_cap < (1ll << 31),
                  CATNN_ERR_SHAPE_MISMATCH, "permute: position capacity too small");
    const int E = (int)n_experts;
    const int64_t nb = (n + kPermChunk - 1) / kPermChunk;
    char *sc = static_cast<char *>(scratch);
    int32_t *block_counts = reinterpret_cast<int32_t *>(sc);
    int32_t *block_base = reinterpret_cast<int32_t *>(sc + align256((uint64_t)nb * E * 4));
    int32_t *bad = reinterpret_cast<int32_t *>(sc + 2 * align256((uint64_t)nb * E * 4));
    if (n_pos_cap > 0)  // padding positions, and the bad-id counter cleared by the same launch
        fill_i32_kernel<<<(unsigned)((n_pos_cap + 255) / 256), 256, 0, s>>>(slot_of_pos, n_pos_cap, -1, bad);
    else
        zero_i32_kernel<<<1, 1, 0, s>>>(bad);
    CATNN_HIP(hipGetLastError());
    if (nb > 0) {
        perm_count_kernel<<<(unsigned)nb, 256, 0, s>>>(idx, n, E, block_counts, bad);
        CATNN_HIP(hipGetLastError());
    }
    perm_scan_kernel<<<1, 64, 0, s>>>(block_counts, (int)nb, E, pad, block_base, counts, offsets);
    CATNN_HIP(hipGetLastError());
    if (nb > 0) {
        perm_scatter_kernel<<<(unsigned)nb, 256, 0, s>>>(idx, n, E, block_base, slot_of_pos,
                                                         pos_of_slot);
        CATNN_HIP(hipGetLastError());
    }
}

MoeWorkspaceLayout moe_workspace_layout(int64_t tokens, int64_t hidden, int64_t intermediate,
                                        int64_t n_experts, int64_t top_k) {
    MoeWorkspaceLayout L{};
    const uint64_t n = (uint64_t)(tokens * top_k);
    const uint64_t max_tiles = (n + gemm_tile_rows() - 1) / gemm_tile_rows() + n_experts;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t o = off;
        off += align256(bytes ? bytes : 1);
        return o;
    };
    L.idx = take(n * 4);
    L.w = take(n * 4);
    L.counts = take((uint64_t)n_experts * 4);
    L.offsets = take((uint64_t)(n_experts + 1) * 4);
    L.slot_of_pos = take(n * 4);
    L.pos_of_slot = take(n * 4);
    L.perm_scratch = take(moe_permute_scratch_bytes(tokens, top_k, n_experts));
    L.tiles = take((2 * max_tiles + 1) * 4);
    L.ptrs = 0;
    L.h = take(n * (uint64_t)intermediate * 4);
    L.y = take(n * (uint64_t)hidden * 4);
    L.total = off;
    return L;
}

void moe_f32(hipStream_t s, const float *x, const float *gate, const float *const *w1s,
             const float *const *w3s, const float *const *w2s, int64_t tokens, int64_t hidden,
             int64_t intermediate, int64_t n_experts, int64_t top_k, float *out, void *ws,
             const MoeWorkspaceLayout &L) {
    CATNN_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                  "moe: n_experts must be in [1, 64]");
    CATNN_REQUIRE(tokens >= 0 && hidden > 0 && intermediate > 0, CATNN_ERR_SHAPE_MISMATCH,
                  "moe: bad dims");
    CATNN_REQUIRE(tokens * top_k < (1ll << 31) && intermediate < (1ll << 31) &&
                      hidden < (1ll << 31),
                  CATNN_ERR_SHAPE_MISMATCH, "moe: dims exceed 2^31");
    if (tokens == 0) return;
    char *base = static_cast<char *>(ws);
    int32_t *idx = reinterpret_cast<int32_t *>(base + L.idx);
    float *w = reinterpret_cast<float *>(base + L.w);
    int32_t *counts = reinterpret_cast<int32_t *>(base + L.counts);
    int32_t *offsets = reinterpret_cast<int32_t *>(base + L.offsets);
    int32_t *slot_of_pos = reinterpret_cast<int32_t *>(base + L.slot_of_pos);
    int32_t *pos_of_slot = reinterpret_cast<int32_t *>(base + L.pos_of_slot);
    const int64_t n = tokens * top_k;
    const int max_tiles = (int)((n + gemm_tile_rows() - 1) / gemm_tile_rows() + n_experts);
    int32_t *tile_expert = reinterpret_cast<int32_t *>(base + L.tiles);
    int32_t *tile_row0 = tile_expert + max_tiles;
    int32_t *n_tiles = tile_row0 + max_tiles;
    float *h = reinterpret_cast<float *>(base + L.h);
    float *y = reinterpret_cast<float *>(base + L.y);

    moe_route_f32(s, x, gate, tokens, hidden, n_experts, top_k, idx, w, nullptr);
    moe_permute(s, idx, tokens, top_k, n_experts, counts, offsets, slot_of_pos, pos_of_slot,
                base + L.perm_scratch);
    build_tiles(s, offsets, (int)n_experts, tile_expert, tile_row0, n_tiles);

    GemmParams g{};
    g.tile_expert = tile_expert;
    g.tile_row0 = tile_row0;
    g.n_tiles = n_tiles;
    g.seg_offsets = offsets;
    g.max_tiles = max_tiles;
    g.n_experts = (int)n_experts;
    g.act = ACT_NONE;

    // gate/up: h[pos] = silu(x[token(pos)]·w1) ⊙ (x[token(pos)]·w3)
    g.A = x;
    g.lda = hidden;
    g.a_rows = slot_of_pos;
    g.a_row_div = (int)top_k;
    for (int e = 0; e < n_experts; ++e) {
        g.B_e[e] = w1s[e];
        g.B2_e[e] = w3s[e];
    }
    g.ldb = intermediate;
    g.C = h;
    g.ldc = intermediate;
    g.N = (int)intermediate;
    g.K = (int)hidden;
    gemm_grouped_launch(s, g, true);

    // down: y[pos] = h[pos]·w2
    g.A = h;
    g.lda = intermediate;
    g.a_rows = nullptr;
    g.a_row_div = 1;
    for (int e = 0; e < n_experts; ++e) {
        g.B_e[e] = w2s[e];
        g.B2_e[e] = nullptr;
    }
    g.ldb = hidden;
    g.C = y;
    g.ldc = hidden;
    g.N = (int)hidden;
    g.K = (int)intermediate;
    gemm_grouped_launch(s, g, false);

    if (hidden % 4 == 0 && aligned16(out))
        combine4_kernel<<<(unsigned)tokens, 256, 0, s>>>(y, pos_of_slot, w, (int)tokens,
                                                         (int)top_k, (int)hidden, out);
    else
        combine_kernel<<<(unsigned)tokens, 256, 0, s>>>(y, pos_of_slot, w, (int)tokens, (int)top_k,
                                                        (int)hidden, out);
    CATNN_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------
// Allocation-free MoE layer: its workspace is a fixed device array, so the
// entry point calls no hipMalloc/hipFree (for callers under HIP graph
// capture, tight serving loops, harnesses that forbid allocation).  Each GPU
// holds its own copy of the array from code-object load to process exit.
namespace noalloc {

static __device__ __align__(256) char scratch[kMoeNoAllocScratchBytes];
static_assert(kMoeNoAllocScratchBytes == CATNN_MOE_NOALLOC_SCRATCH_BYTES, "header and library agree");

std::mutex g_mu;
std::vector<void *> g_ptr;  // per device ordinal: the array's device address

}  // namespace noalloc

void *moe_noalloc_scratch(int ordinal, std::string *err) {
    // Called with `ordinal` current (catnn_hip_open).  The host-side name of
    // the array is only a stand-in: its device address comes from the
    // runtime, once per device, and only that address reaches kernels.
    std::lock_guard<std::mutex> lock(noalloc::g_mu);
    if ((int)noalloc::g_ptr.size() <= ordinal) noalloc::g_ptr.resize(ordinal + 1, nullptr);
    if (noalloc::g_ptr[ordinal]) return noalloc::g_ptr[ordinal];
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(noalloc::scratch));
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        if (err) *err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
        return nullptr;
    }
    noalloc::g_ptr[ordinal] = ptr;
    return ptr;
}

}  // namespace k
}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_hip_moe_route_f32(catnn_hip_device *dev, const float *x, const float *gate,
                            int64_t tokens, int64_t hidden, int64_t n_experts, int64_t top_k,
                            int32_t *idx, float *w, float *logits) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE((x && gate) || tokens == 0, CATNN_ERR_INVALID_ARGUMENT,
                      "route: null operand");
        k::moe_route_f32(dev->stream, x, gate, tokens, hidden, n_experts, top_k, idx, w, logits);
    });
}

int catnn_hip_moe_permute(catnn_hip_device *dev, const int32_t *idx, int64_t tokens, int64_t top_k,
                          int64_t n_experts, int32_t *counts, int32_t *offsets,
                          int32_t *slot_of_pos, int32_t *pos_of_slot) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(counts && offsets && ((idx && slot_of_pos && pos_of_slot) || tokens == 0),
                      CATNN_ERR_INVALID_ARGUMENT, "permute: null operand");
        const uint64_t bytes = k::moe_permute_scratch_bytes(tokens, top_k, n_experts);
        void *scratch = workspace(dev, dev->moe_ws, bytes);
        k::moe_permute(dev->stream, idx, tokens, top_k, n_experts, counts, offsets, slot_of_pos,
                       pos_of_slot, scratch);
        // Caller-supplied ids may be out of range: report instead of guessing.
        int32_t bad = 0;
        CATNN_HIP(hipMemcpyAsync(&bad, static_cast<char *>(scratch) + bytes - 256, 4,
                                 hipMemcpyDeviceToHost, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
        CATNN_REQUIRE(bad == 0, CATNN_ERR_SHAPE_MISMATCH,
                      "permute: " + std::to_string(bad) + " expert ids outside [0, n_experts)");
    });
}

int catnn_hip_moe_f32(catnn_hip_device *dev, const float *x, const float *gate,
                      const float *const *w1s, const float *const *w3s, const float *const *w2s,
                      int64_t tokens, int64_t hidden, int64_t intermediate, int64_t n_experts,
                      int64_t top_k, float *out, int32_t *idx, float *w, int32_t *counts) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(w1s && w3s && w2s, CATNN_ERR_INVALID_ARGUMENT, "moe: null weight table");
        CATNN_REQUIRE((x && gate && out) || tokens == 0, CATNN_ERR_INVALID_ARGUMENT,
                      "moe: null operand");
        CATNN_REQUIRE(n_experts >= 1 && n_experts <= k::kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                      "moe: n_experts must be in [1, 64]");
        for (int64_t e = 0; e < n_experts; ++e)
            CATNN_REQUIRE(w1s[e] && w3s[e] && w2s[e], CATNN_ERR_INVALID_ARGUMENT,
                          "moe: null expert weight " + std::to_string(e));
        const k::MoeWorkspaceLayout L =
            k::moe_workspace_layout(tokens, hidden, intermediate, n_experts, top_k);
        void *ws = workspace(dev, dev->moe_ws, L.total);
        k::moe_f32(dev->stream, x, gate, w1s, w3s, w2s, tokens, hidden, intermediate, n_experts,
                   top_k, out, ws, L);
        char *base = static_cast<char *>(ws);
        const uint64_t n = (uint64_t)(tokens * top_k);
        if (idx && n)
            CATNN_HIP(hipMemcpyAsync(idx, base + L.idx, n * 4, hipMemcpyDeviceToDevice, dev->stream));
        if (w && n)
            CATNN_HIP(hipMemcpyAsync(w, base + L.w, n * 4, hipMemcpyDeviceToDevice, dev->stream));
        if (counts)
            CATNN_HIP(hipMemcpyAsync(counts, base + L.counts, (uint64_t)n_experts * 4,
                                     hipMemcpyDeviceToDevice, dev->stream));
    });
}

int catnn_hip_moe_f32_noalloc(catnn_hip_device *dev, const float *x, const float *gate,
                              const float *const *w1s, const float *const *w3s,
                              const float *const *w2s, int64_t tokens, int64_t hidden,
                              int64_t intermediate, int64_t n_experts, int64_t top_k, float *out,
                              int32_t *idx, float *w, int32_t *counts) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(w1s && w3s && w2s, CATNN_ERR_INVALID_ARGUMENT, "moe: null weight table");
        CATNN_REQUIRE((x && gate && out) || tokens == 0, CATNN_ERR_INVALID_ARGUMENT,
                      "moe: null operand");
        CATNN_REQUIRE(n_experts >= 1 && n_experts <= k::kMaxExperts, CATNN_ERR_SHAPE_MISMATCH,
                      "moe: n_experts must be in [1, 64]");
        CATNN_REQUIRE(tokens >= 0 && top_k >= 1 && hidden > 0 && intermediate > 0,
                      CATNN_ERR_SHAPE_MISMATCH, "moe: bad dims");
        for (int64_t e = 0; e < n_experts; ++e)
            CATNN_REQUIRE(w1s[e] && w3s[e] && w2s[e], CATNN_ERR_INVALID_ARGUMENT,
                          "moe: null expert weight " + std::to_string(e));
        CATNN_REQUIRE(dev->noalloc_scratch, CATNN_ERR_DEVICE,
                      "moe_noalloc: no device scratch on this device (" + dev->noalloc_error + ")");
        const k::MoeWorkspaceLayout L =
            k::moe_workspace_layout(tokens, hidden, intermediate, n_experts, top_k);
        CATNN_REQUIRE(L.total <= k::kMoeNoAllocScratchBytes, CATNN_ERR_SHAPE_MISMATCH,
                      "moe_noalloc: workspace of " + std::to_string(L.total) +
                          " bytes exceeds the fixed scratch of " +
                          std::to_string(k::kMoeNoAllocScratchBytes) +
                          " bytes; use catnn_hip_moe_f32 or fewer tokens");
        void *ws = dev->noalloc_scratch;
        k::moe_f32(dev->stream, x, gate, w1s, w3s, w2s, tokens, hidden, intermediate, n_experts,
                   top_k, out, ws, L);
        char *base = static_cast<char *>(ws);
        const uint64_t n = (uint64_t)(tokens * top_k);
        if (idx && n)
            CATNN_HIP(hipMemcpyAsync(idx, base + L.idx, n * 4, hipMemcpyDeviceToDevice, dev->stream));
        if (w && n)
            CATNN_HIP(hipMemcpyAsync(w, base + L.w, n * 4, hipMemcpyDeviceToDevice, dev->stream));
        if (counts && tokens > 0)
            CATNN_HIP(hipMemcpyAsync(counts, base + L.counts, (uint64_t)n_experts * 4,
                                     hipMemcpyDeviceToDevice, dev->stream));
    });
}

}  // extern "C"
