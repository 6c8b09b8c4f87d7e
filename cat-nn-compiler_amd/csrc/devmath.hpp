// Device-side scalar helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace catnn {
namespace k {

// GELU, tanh form: 0.5·z·(1 + tanh(√(2/π)·(z + 0.044715·z³))), with the
// constant rounded to f32 and the cube evaluated left to right as
// crates/catnn-compile/src/kernel/cpu.rs:20-29 does.
__device__ __forceinline__ float gelu_tanh(float z) {
    const float c = 0.797884523868560791f;  // f32 sqrt(f32(2) / f32(pi))
    const float inner = c * (z + 0.044715f * z * z * z);
    return 0.5f * z * (1.0f + tanhf(inner));
}

// SiLU, crates/catnn-compile/src/kernel/moe.rs:12-14: x / (1 + e^{-x}).
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 2) return fmaxf(v, 0.0f);
    if (act == 3) return gelu_tanh(v);
    return v;
}

// Direct HBM → LDS loads (global_load_lds_dwordx4): the LDS destination is
// an address-space-3 pointer, uniform across the wavefront; lane l writes
// its 16 bytes at destination + 16·l.
typedef __attribute__((address_space(3))) void lds_void_t;

// Issued from inline assembly rather than __builtin_amdgcn_global_load_lds:
// for the builtin the compiler makes every later LDS access of the wavefront
// wait for all direct-to-LDS loads in flight (vmcnt(0)), whatever stage they
// fill, which turns a multi-stage pipeline into a load-then-compute loop.
// Here the compiler sees no LDS write, so the caller's dma_sync waits are the
// only ones and must cover every read of the stage a load fills.  M0 holds
// the wavefront's LDS base; one wait state separates its write from the load.
// load_lds16_at takes the destination as an LDS byte address (lds_addr),
// which saves the generic-to-LDS pointer conversion per load when the
// caller keeps the base.
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(size_t)(lds_void_t *)p; }
__device__ __forceinline__ void load_lds16_at(const void *src, uint32_t lds_wave_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_wave_base);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src)
                 : "memory", "m0");
}
__device__ __forceinline__ void load_lds16(const void *src, void *lds_wave_base) {
    load_lds16_at(src, lds_addr(lds_wave_base));
}

// s_waitcnt with vmcnt ≤ N, lgkmcnt 0 (every LDS access of this wavefront
// done), expcnt unconstrained; then the block barrier.  Direct-to-LDS loads
// count in vmcnt until their data is in LDS.  The empty asm statements keep
// the compiler from moving memory accesses across; the barrier builtin
// itself carries no fence, so the waits stay exactly these.
template <int N>
__device__ __forceinline__ void dma_sync() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Butterfly reductions across the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum over the 64 lanes without LDS round trips: DPP swaps within each
// quad (lanes ^1, ^2), then the half-row and row mirrors (lane i with
// 7 − i, then 15 − i) leave every lane of a 16-lane row holding that row's
// sum, the same value in each (each step adds a commutative pair); the four
// row sums are read from lanes 0, 16, 32, 48 and added in a fixed order.
// The result is uniform across the wavefront.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_move<0x141>(v);  // row_half_mirror
    v += dpp_move<0x140>(v);  // row_mirror
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0)), r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32)), r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Blocks of one launch are dealt round-robin to the 8 XCDs of an MI355X
// (block b runs on XCD b % 8), and each XCD has its own L2.  Renumber so
// that each XCD owns one contiguous range of logical tiles; neighbouring
// tiles share operand panels, so their reuse stays inside one L2.
__device__ __forceinline__ int xcd_remap(int pid, int nblocks) {
    if ((nblocks & 7) != 0) return pid;
    return (pid & 7) * (nblocks >> 3) + (pid >> 3);
}

// Block b of a launch over n_bh (batch, head) pairs × nb blocks each: its
// block index `blk` (0 = the heaviest under a causal mask) and pair `bh`.
// blk is the slowest-varying index, so all blocks of one weight are
// launched before the lighter ones (longest first: the last blocks to start
// are the shortest).  Blocks go to XCD b % 8 round-robin, and consecutive
// blocks take different pairs, so every XCD receives every weight equally.
__device__ __forceinline__ void split_bh_block(int b, int nb, int n_bh, int &blk, int &bh) {
    (void)nb;
    blk = b / n_bh;
    bh = b - blk * n_bh;
}

// Grouped tile order: walk `group` row-tiles down a column of tiles before
// moving right, so that blocks resident together reuse the same B panel
// and a small set of A panels.
__device__ __forceinline__ void grouped_tile(int lid, int tiles_m, int tiles_n, int group,
                                             int &tm, int &tn) {
    const int per_group = group * tiles_n;
    const int g = lid / per_group;
    const int first_m = g * group;
    const int gsz = min(tiles_m - first_m, group);
    const int in_group = lid - g * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

// Streaming (nontemporal) 16- and 8-byte accesses, for values a kernel
// reads or writes once and that no kernel right after it reads again
// through the L2.
typedef float stream_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t stream_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 load_stream(const float *q) {
    const stream_f4 v = __builtin_nontemporal_load(reinterpret_cast<const stream_f4 *>(q));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_stream(float *q, float4 v) {
    const stream_f4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<stream_f4 *>(q));
}
__device__ __forceinline__ void store_stream(uint16_t *q, uint32_t a, uint32_t b) {
    const stream_u2 w = {a, b};
    __builtin_nontemporal_store(w, reinterpret_cast<stream_u2 *>(q));
}

}  // namespace k
}  // namespace catnn
