// Launch functions of the gfx950 kernels.  Each validates what its grid
// assumes on the host, launches on `s`, and returns without synchronising.
// Shape problems raise catnn::Failure (CATNN_ERR_SHAPE_MISMATCH).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace catnn {
namespace k {

enum Act : int { ACT_NONE = 0, ACT_RELU = 2, ACT_GELU = 3 };

// y = act(x·w + b) + r over row-major f32; x [m,k] (row stride lda),
// w [k,n] (ldb), y [m,n] (ldc), r [m,n] (ldr).  fp32 MFMA.
void linear_f32(hipStream_t s, const float *x, int64_t lda, const float *w, int64_t ldb,
                const float *b, const float *r, int64_t ldr, float *y, int64_t ldc,
                int64_t m, int64_t k, int64_t n, int act);

void act_f32(hipStream_t s, const float *x, float *y, int64_t n, int act);
void add_f32(hipStream_t s, const float *a, const float *b, float *y, int64_t na, int64_t nb);
void mul_f32(hipStream_t s, const float *a, const float *b, float *y, int64_t n);
void copy_f32(hipStream_t s, const float *x, float *y, int64_t n);
void layer_norm_f32(hipStream_t s, const float *x, const float *gamma, const float *beta,
                    float *y, int64_t rows, int64_t cols, float eps);
void softmax_f32(hipStream_t s, const float *x, float *y, int64_t rows, int64_t cols);

// Flash-style attention core on q/k/v with row stride ld (elements) and
// head h at column offset h·dh; ctx has row stride ldo.
void attention_core_f32(hipStream_t s, const float *q, const float *k, const float *v,
                        int64_t ld_qkv, float *ctx, int64_t ldo, int64_t batch, int64_t seq,
                        int64_t n_heads, int64_t d_head, bool causal);

// MoE pieces.
void moe_route_f32(hipStream_t s, const float *x, const float *gate, int64_t tokens,
                   int64_t hidden, int64_t n_experts, int64_t top_k, int32_t *idx, float *w,
                   float *logits);
// Permutation; `scratch` must hold moe_permute_scratch_bytes(...) bytes.
uint64_t moe_permute_scratch_bytes(int64_t tokens, int64_t top_k, int64_t n_experts);
void moe_permute(hipStream_t s, const int32_t *idx, int64_t tokens, int64_t top_k,
                 int64_t n_experts, int32_t *counts, int32_t *offsets, int32_t *slot_of_pos,
                 int32_t *pos_of_slot, void *scratch);

struct MoeWorkspaceLayout {
    uint64_t idx, w, counts, offsets, slot_of_pos, pos_of_slot, perm_scratch, tiles, ptrs, h,
        y, total;
};
MoeWorkspaceLayout moe_workspace_layout(int64_t tokens, int64_t hidden, int64_t intermediate,
                                        int64_t n_experts, int64_t top_k);
void moe_f32(hipStream_t s, const float *x, const float *gate, const float *const *w1s,
             const float *const *w3s, const float *const *w2s, int64_t tokens, int64_t hidden,
             int64_t intermediate, int64_t n_experts, int64_t top_k, float *out, void *ws,
             const MoeWorkspaceLayout &L);

}  // namespace k
}  // namespace catnn
