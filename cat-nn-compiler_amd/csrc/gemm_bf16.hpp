// bf16 MFMA GEMM of the training path (gemm_bf16.hip).
//
// C[M,N] = Σ_k A[m][k]·B[n][k]: both operands bf16 and k-contiguous (the
// second one is stored "transposed", [N,K]); fp32 accumulation.  A weight
// W [K,N] therefore enters the forward as its transposed bf16 copy and the
// input-gradient GEMM as its own bf16 copy; weight gradients take both
// activations transposed.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "gemm_f32.hpp"

namespace catnn {
namespace k {

typedef uint16_t bf16_t;  // storage type of bf16 values on the host side

enum Bf16Epi : int {
    EPI_STORE = 0,       // C32 (= or +=) acc, Cb = bf16(acc)
    EPI_LINEAR = 1,      // v = acc + bias; Z = v; v = act(v); v = R + v; C32/Cb = v
    EPI_GELU_BWD = 2,    // v = acc · gelu'(Z); C32/Cb = v
    EPI_SWIGLU_FWD = 3,  // dual B: save a, c (bf16) to S1, S2; Cb = bf16(silu(a)·c)
    EPI_SWIGLU_BWD = 4,  // a = S1, c = S2: Cb = bf16(acc·c·silu'(a)), Cb2 = bf16(acc·silu(a))
};

enum Bf16Grid : int { GRID_PLAIN = 0, GRID_ROWS = 1, GRID_SEGK = 2 };

struct GemmBf16Params {
    const bf16_t *A;
    int64_t lda;
    const int32_t *a_rows;  // logical row r reads source row a_rows[r] / a_row_div
    int a_row_div;
    const bf16_t *B;
    const bf16_t *B2;       // dual mode second operand (W3ᵀ)
    int64_t ldb;
    int M, N, K;
    int epi;
    int act;
    // outputs
    float *C32;
    int64_t ldc32;
    int accumulate;
    bf16_t *Cb;
    int64_t ldcb;
    bf16_t *Cb2;
    const float *bias;
    const float *R;
    int64_t ldr;
    float *Z;               // EPI_LINEAR: pre-activation out; EPI_GELU_BWD: pre-activation in
    int64_t ldz;
    bf16_t *S1, *S2;        // SwiGLU saved a / c
    int64_t lds;
    // grouped grids
    int grid;
    const int32_t *tile_expert;
    const int32_t *tile_row0;
    const int32_t *n_tiles;
    const int32_t *seg_offsets;  // segment e starts at seg_offsets[e]
    const int32_t *seg_counts;   // ... and holds seg_counts[e] rows (null: ends at seg_offsets[e+1])
    int segk_aligned;            // GRID_SEGK: caller guarantees seg_offsets[e] % 8 == 0
    int ksplit;                  // GRID_SEGK with seg_offsets null: segment e is [e·ksplit, (e+1)·ksplit) ∩ [0, K)
    int vec_epi;                 // set by the launcher: output rows allow 16-byte epilogue accesses
    int b_kwrap;                 // > 0: B's k index wraps at b_kwrap (B has b_kwrap columns; K a multiple
                                 // of it and of 64): [x_hi | x_lo]·[w | w] without a doubled copy of w
    int max_tiles;
    const int32_t *tiles256;  // GRID_ROWS: the table of 256-row tiles (gemm_bf16_build_tiles), or null
    int max_tiles256;
    // Stream-K remainder (configuration 12): fp32 partial tiles, gemm_bf16_sk_floats() of them, or null
    // (then configuration 12 is not chosen); sk_ctas is set by the launcher.
    float *sk_part;
    int sk_ctas;
    int n_experts;
    const bf16_t *B_e[kMaxExperts];
    const bf16_t *B2_e[kMaxExperts];
    float *C_e[kMaxExperts];  // GRID_SEGK: output of expert e
};

void gemm_bf16_launch(hipStream_t s, const GemmBf16Params &p);
// The same with a fixed tile configuration (0, 2, 7, 9, 10, 11 or 12; see gemm_bf16.hip).
void gemm_bf16_launch_cfg(hipStream_t s, const GemmBf16Params &p, int cfg);
int gemm_bf16_tile_rows();
// Floats of partial-tile scratch the stream-K remainder of configuration 12
// needs on the current device (one 256 × 256 tile per CU).
int64_t gemm_bf16_sk_floats();
// Tile tables of the grouped grid for `rows` routed rows (T·k) over
// n_experts segments: 128-row and 256-row tiles of each segment, in expert
// order, built by one launch into `tiles` (gemm_bf16_tiles_ints int32s);
// gemm_bf16_use_tiles points a GRID_ROWS launch at both.
int64_t gemm_bf16_tiles_ints(int64_t rows, int n_experts);
void gemm_bf16_build_tiles(hipStream_t s, const int32_t *offsets, int n_experts, int64_t rows, int32_t *tiles);
void gemm_bf16_use_tiles(GemmBf16Params &p, const int32_t *tiles, int64_t rows, int n_experts);
// K splits for a plain store/accumulate GEMM whose tiles alone leave the
// GPU's CUs idle (1 = no split); gemm_bf16_splitk_len gives the segment.
int gemm_bf16_splitk(int64_t M, int64_t N, int64_t K);
int gemm_bf16_splitk_len(int64_t K, int splits);

}  // namespace k
}  // namespace catnn
