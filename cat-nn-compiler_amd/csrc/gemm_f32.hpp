// Parameters of the fp32 MFMA GEMM (gemm_f32.hip), shared with the MoE
// pipeline which launches its grouped form.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace catnn {
namespace k {

// Largest expert count the grouped grid accepts (per-expert weight pointers
// travel by value in the kernel arguments).
constexpr int kMaxExperts = 64;

struct GemmParams {
    // A [rows, K]; logical row r reads source row a_rows[r] / a_row_div when
    // a_rows is set (MoE: permuted slot → token), else row r.
    const float *A;
    int64_t lda;
    const int32_t *a_rows;
    int a_row_div;
    // B [K, N] (and B2 for the dual SwiGLU mode).
    const float *B;
    const float *B2;
    int64_t ldb;
    const float *bias;  // [N] or null
    const float *R;     // residual [rows, N] or null
    int64_t ldr;
    float *C;
    int64_t ldc;
    int M, N, K;
    int act;
    // Grouped grid (MoE): tiles listed by build_tiles; per-expert B pointers.
    const int32_t *tile_expert;
    const int32_t *tile_row0;
    const int32_t *n_tiles;
    const int32_t *seg_offsets;
    int max_tiles;
    int n_experts;
    const float *B_e[kMaxExperts];
    const float *B2_e[kMaxExperts];
};

int gemm_tile_rows();
void gemm_launch(hipStream_t s, const GemmParams &p, bool dual);
void gemm_grouped_launch(hipStream_t s, const GemmParams &p, bool dual);
void build_tiles(hipStream_t s, const int32_t *offsets, int n_experts, int32_t *tile_expert,
                 int32_t *tile_row0, int32_t *n_tiles);

}  // namespace k
}  // namespace catnn
