// Launch functions of the gfx950 kernels.  Each validates what its grid
// assumes on the host, launches on `s`, and returns without synchronising.
// Shape problems raise catnn::Failure (CATNN_ERR_SHAPE_MISMATCH).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>

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

// The same with grouped K/V heads: q rows have stride ldq and n_heads heads,
// k/v rows stride ldk and n_heads / group heads (head h reads K/V head
// h / group); causal, and window > 0 restricts query i to keys
// [i − window + 1, i].
void attention_core_gqa_f32(hipStream_t s, const float *q, const float *k, const float *v, int64_t ldq,
                            int64_t ldk, int64_t group, int64_t window, float *ctx, int64_t ldo,
                            int64_t batch, int64_t seq, int64_t n_heads, int64_t d_head);

// Decoder ops (decoder.hip).
void rms_norm_f32(hipStream_t s, const float *x, const float *w, float *y, int64_t rows, int64_t cols,
                  float eps);
// ids: n f32 token ids; *bad (device int) is set to 1 when an id ≥ vocab.
void embedding_f32(hipStream_t s, const float *ids, int64_t n, const float *table, int64_t vocab,
                   int64_t hidden, float *y, int *bad);
void mix_f32(hipStream_t s, const float *a, const float *b, const float *gate, float *y, int64_t n);
// embedding_backward (adjoint.rs:187-197): dw [vocab, hidden] from dy
// [n, hidden] and the n f32 ids, in token order per row; idi holds n ints,
// hit vocab ints (scratch).
void embedding_backward(hipStream_t s, const float *ids, int64_t n, const float *dy, int64_t vocab, int64_t hidden,
                        float *dw, int *idi, int *hit);
void transpose_f32(hipStream_t s, const float *src, int64_t rows, int64_t cols, float *dst);

// GQA scratch, in floats: packed q|k|v rows [T, qkv_ld], ctx [T, n_heads·hd]
// and the RoPE table [S, hd/2] of (cos, sin).
struct GqaLayout {
    int64_t qkv_ld, qkv, ctx, rope, floats;
};
GqaLayout gqa_layout(int64_t tokens, int64_t seq, int64_t n_heads, int64_t n_kv, int64_t head_dim);
// y = GQA(x) (+ residual).  wqkv [D, qkv_ld] = [wq | wk | wv] per row, or
// null to use the three projections separately.
void gqa_f32(hipStream_t s, const float *x, const float *wqkv, const float *wq, const float *wk,
             const float *wv, const float *wo, int64_t B, int64_t S, int64_t D, int64_t n_heads,
             int64_t n_kv, int64_t head_dim, double theta, int64_t window, const float *residual,
             float *y, float *scratch, const GqaLayout &L);
// y = (silu(x·w1) ⊙ (x·w3))·w2 (+ residual); h is [T, I] scratch.
void swiglu_f32(hipStream_t s, const float *x, const float *w1, const float *w3, const float *w2,
                int64_t T, int64_t H, int64_t I, const float *residual, float *y, float *h);

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

// The fixed device scratch of catnn_hip_moe_f32_noalloc and its size.
// moe_noalloc_scratch returns the array's device address on the current
// device `ordinal` (queried once per device), or null with `err` set.
constexpr uint64_t kMoeNoAllocScratchBytes = 128ull << 20;
void *moe_noalloc_scratch(int ordinal, std::string *err);

}  // namespace k
}  // namespace catnn
