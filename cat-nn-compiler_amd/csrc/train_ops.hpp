// Launchers of the training-step kernels (train_ops.hip, attention.hip's
// adjoint, moe.hip's padded permutation).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "gemm_bf16.hpp"

namespace catnn {
namespace k {

void fill_f32(hipStream_t s, float *y, float v, int64_t n);
void fill_bf16_zero(hipStream_t s, bf16_t *y, int64_t n);
void cast_f32_bf16(hipStream_t s, const float *x, bf16_t *y, int64_t n);
// dst[c][r] = src[map(r)][c]; map(r) = rows_map[r] / div (negative: zero row).
void transpose_bf16(hipStream_t s, const bf16_t *src, int64_t lds, const int32_t *rows_map, int div,
                    int rows, int cols, bf16_t *dst, int64_t ldd);
void transpose_f32_bf16(hipStream_t s, const float *src, int64_t lds, const int32_t *rows_map,
                        int div, int rows, int cols, bf16_t *dst, int64_t ldd);

// Split-bf16 GEMM operands: A' rows [hi | lo | hi] from fp32 rows of K
// (out row stride ldo ≥ 3K) and B' = [hi | hi | lo] rows from the columns of
// an fp32 [K, N] matrix, so the bf16 GEMM over K' = 3K yields hi·hi + hi·lo
// + lo·hi ≈ the fp32 product (relative error ~2⁻¹⁶).
void split3_rows(hipStream_t s, const float *x, int64_t ldx, int64_t rows, int K, bf16_t *out,
                 int64_t ldo);
void transpose_split3(hipStream_t s, const float *w, int64_t ldw, int K, int N, bf16_t *out,
                      int64_t ldo);

// LayerNorm forward with its mean and rstd for the adjoint; y (fp32), yb
// (bf16, row stride cols) and y3 ([hi | lo | hi] split-bf16, row stride
// 3·cols, as split3_rows) are each optional.
void ln_forward_train(hipStream_t s, const float *x, const float *g, const float *b, float *y,
                      bf16_t *yb, bf16_t *y3, float *mean, float *rstd, int64_t rows, int cols, float eps);
uint64_t ln_backward_scratch_bytes(int64_t rows, int cols);
void ln_backward(hipStream_t s, const float *x, const float *g, const float *mean, const float *rstd,
                 const float *dy, float *dx, bool accumulate, float *dg, float *db, bool acc_params,
                 int64_t rows, int cols, float *scratch);

// out (=/+=) Σ_e parts[e], e = 0 … np−1 in order, each part n floats.
void sum_parts(hipStream_t s, const float *parts, int np, int64_t n, float *out, bool accumulate);

uint64_t colsum_scratch_bytes(int64_t rows, int cols);
// y [rows, cols] (fp32, row stride cols): yt = bf16(y)ᵀ (row stride ldt),
// with out (or null) (+)= the column sums of y and yb (or null) = bf16(y)
// row-major, as transpose_f32_bf16, colsum (its scratch) and cast_f32_bf16
// would give them, in one pass.  False, with nothing launched, unless rows
// and cols are multiples of 64 with 16-byte aligned rows.
bool transpose_colsum(hipStream_t s, const float *y, int64_t rows, int cols, bf16_t *yt, int64_t ldt,
                      float *out, bool accumulate, float *scratch, bf16_t *yb = nullptr);
void colsum(hipStream_t s, const float *y, int64_t rows, int cols, float *out, bool accumulate,
            float *scratch);
void act_backward(hipStream_t s, const float *z, const float *dy, float *dx, int64_t n, int act,
                  bool accumulate);

uint64_t mse_scratch_bytes();
void mse(hipStream_t s, const float *pred, const float *tgt, float *d, int64_t n, float *loss,
         float *scratch);
void sgd(hipStream_t s, float *p, const float *g, int64_t ldg, int64_t rows, int cols, float lr,
         bf16_t *pb);
// rmsnorm_backward (adjoint.rs:147-198) of rows × cols: dx (=, or += when
// accumulate; null: not computed) and dw = Σ_rows dy·x·inv via
// prod [rows, cols] and colsum's scratch (colsum_scratch_bytes).
void rms_backward(hipStream_t s, const float *x, const float *w, const float *dy, float *dx, bool accumulate,
                  float *dw, int64_t rows, int cols, float eps, float *prod, float *colsum_scratch);
// mix_backward (deepseek.rs:241-258) over n values: da, db (= or +=, null:
// skipped) and, when dgate is given, the gate's cotangent; parts holds
// mix_scratch_bytes().
uint64_t mix_scratch_bytes();
// softmax_backward (adjoint.rs:92-104) from the forward output y [rows, cols].
void softmax_backward(hipStream_t s, const float *y, const float *dy, float *dx, bool accumulate, int64_t rows,
                      int cols);
// The dense SwiGLU: h = silu(a)·c, and the adjoint's da, dc (bf16).
void swiglu_h(hipStream_t s, const float *a, const float *c, float *h, int64_t n);
void swiglu_dadc(hipStream_t s, const float *dh, const float *a, const float *c, bf16_t *da, bf16_t *dc, int64_t n);
// One input's cotangent of Mul (adjoint.rs:787-800): dx (=/+=) dy·other.
void mul_backward(hipStream_t s, const float *dy, const float *other, float *dx, bool accumulate, int64_t n);
void mix_backward(hipStream_t s, const float *a, const float *b, const float *gate, const float *dy, float *da,
                  bool acc_a, float *db, bool acc_b, int64_t n, float *dgate, float *parts);
// cross_entropy (adjoint.rs:123-145) of logits [rows, V] against class ids
// (each < V): d [rows, V] and the mean loss; row_loss holds rows floats.
void cross_entropy(hipStream_t s, const float *logits, const uint32_t *ids, int64_t rows, int V, float *d,
                   float *loss, float *row_loss);

// The update morphism of one launch (OptimizerKind, lens/optim.rs:142-145).
// Adam's bias corrections b1t = 1 − β₁ᵗ and b2t = 1 − β₂ᵗ are computed on
// the host for the step about to run (adam_bias_corrections).
struct UpdateRule {
    int adam;  // 0: Sgd::put (optim.rs:32-42), 1: Adam::put (optim.rs:95-118)
    float lr, beta1, beta2, eps, b1t, b2t;
};
UpdateRule sgd_rule(float lr);
// Adam with the reference's defaults (β₁ 0.9, β₂ 0.999, eps 1e-8) at step t
// (t ≥ 1 is the step being taken: AdamState.t + 1).
UpdateRule adam_rule(float lr, uint64_t t);
// f32 β^t by binary exponentiation, the lowering of Rust's f32::powi for a
// run-time exponent (compiler-builtins' __powisf2).
float powi_f32(float b, int32_t t);
// p ← update(p, g) elementwise over n values; m, v are Adam's moments
// (ignored for SGD), updated in place.
void apply_update(hipStream_t s, const UpdateRule &u, float *p, const float *g, float *m, float *v,
                  int64_t n);

// One parameter of the multi-tensor update: fp32 master p [rows, cols] and
// its gradient g (same layout, or null: refresh only), and the bf16 copies
// to rewrite from the new value: b [rows, cols], bt [cols, rows] and the
// split-bf16 transposed bt3 [cols, 3·rows] = hi | hi | lo (each may be null).
struct SgdParam {
    float *p;
    const float *g;
    float *m, *v;  // Adam moments, same layout as p (null under SGD)
    bf16_t *b, *bt, *bt3;
    int ldb;      // row stride of b (≥ cols)
    int rows, cols;
    int tile0;    // first 64×64 tile of this parameter in the launch
    int tiles_c;  // tiles across cols
};
// The update rule on every parameter of `table` (device memory, n entries,
// tile0 ascending, `tiles` in total) in one launch, then the bf16 copies;
// with use_grad false only the copies are refreshed.
void sgd_multi(hipStream_t s, const SgdParam *table, int n, int tiles, const UpdateRule &u, bool use_grad);

uint64_t router_backward_scratch_bytes(int T, int H, int E);
void router_backward(hipStream_t s, const int32_t *idx, const float *w, const float *dw,
                     const float *x, int T, int H, int E, int K, float *dl, float *dgate,
                     float *scratch);
void moe_slot_grads(hipStream_t s, const int32_t *slot_of_pos, const float *w, const float *y,
                    const float *dout, int K, int H, int n_pos, bf16_t *dys, float *dw);
// fp32 slot cotangents (the fp32-precision trainer).
void moe_slot_grads_f32(hipStream_t s, const int32_t *slot_of_pos, const float *w, const float *y,
                        const float *dout, int K, int H, int n_pos, float *dys, float *dw);
// Six-part split operands (fp32-accurate GEMMs on bf16 matrix cores): each
// element of an fp32 matrix becomes six bf16 values interleaved along K,
// laid out for the A or the B role.  split6_rows: out [rows, 6K];
// split6_transpose: out[c] = the split of column c of x (rows gathered
// through rows_map[r] / div, negative → zero), [cols, 6·rows].
void split6_rows(hipStream_t s, const float *x, int64_t ldx, int64_t rows, int K, bool role_b, bf16_t *out,
                 int64_t ldo);
void split6_transpose(hipStream_t s, const float *x, int64_t ldx, const int32_t *rows_map, int div, int rows,
                      int cols, bool role_b, bf16_t *out, int64_t ldo);
void scale_i32(hipStream_t s, const int32_t *src, int n, int factor, int32_t *dst);
void swiglu_dadc_f32(hipStream_t s, const float *dh, const float *a, const float *c, float *da, float *dc,
                     int64_t n);
void moe_dx(hipStream_t s, const float *dxs, const int32_t *pos_of_slot, const float *dl,
            const float *gate, int T, int K, int H, int E, float *dx, bool accumulate);

// Permutation with every expert segment starting on a multiple of `pad`
// rows: offsets[e] = Σ_{e'<e} roundup(counts[e'], pad), offsets[E] = total;
// slot_of_pos is −1 on padding rows.  n_pos_cap must be ≥ T·k + E·(pad−1).
void moe_permute_padded(hipStream_t s, const int32_t *idx, int64_t tokens, int64_t top_k,
                        int64_t n_experts, int pad, int64_t n_pos_cap, int32_t *counts,
                        int32_t *offsets, int32_t *slot_of_pos, int32_t *pos_of_slot,
                        void *scratch);

// out[t] = Σ_k w[t,k]·y[pos(t,k)] (the MoE combine of moe.hip).
void moe_combine(hipStream_t s, const float *y, const int32_t *pos_of_slot, const float *w,
                 int64_t tokens, int64_t top_k, int64_t hidden, float *out);

// Attention forward that also stores the per-(query, head) log-sum-exp
// (log2 domain, scores pre-scaled by log2e/√dh) for the adjoint.
void attention_core_fwd_lse(hipStream_t s, const float *q, const float *k, const float *v, int64_t ld,
                            float *ctx, int64_t ldo, float *lse, int64_t batch, int64_t seq,
                            int64_t n_heads, int64_t d_head, bool causal);
// Adjoint of the attention core: dq, dk, dv (row stride ld_d, head h at
// column h·dh) from q, k, v, o (= ctx), lse and do (row stride ldo).
uint64_t attention_bwd_scratch_bytes(int64_t batch, int64_t seq, int64_t n_heads);
void attention_core_bwd(hipStream_t s, const float *q, const float *k, const float *v, int64_t ld,
                        const float *o, const float *dout, int64_t ldo, const float *lse,
                        float *dq, float *dk, float *dv, int64_t ld_d, int64_t batch, int64_t seq,
                        int64_t n_heads, int64_t d_head, bool causal, float *scratch);
// D[row·n_heads + h] = Σ_d o·dout over head h (rows of stride ld).
void attention_rowdot(hipStream_t s, const float *o, const float *dout, int64_t ld, int64_t rows, int64_t n_heads,
                      int64_t d_head, float *D);
// The attention core on bf16 MFMA (attention_bf16.hip), d_head 64, one K/V
// head per query head.  qkv: bf16 rows [q | k | v] of stride ld (n_heads·64
// each); qkvt: its transpose per batch element from transpose_bt (3·n_heads·64
// features × attention_bf16_seq_pad(seq)).  The forward writes ctx (fp32)
// and lse (log2 domain, as attention_core_fwd_lse); the adjoint takes ctx,
// dctx (fp32, stride ldo), dctx's bf16 copy dctxb (stride ldo) and its
// transpose dctxt (n_heads·64 features) and writes dq | dk | dv (fp32) into
// the columns of dqkv (stride ldd); scratch: attention_bwd_scratch_bytes.
bool attention_bf16_supported(int64_t d_head, int64_t ld);
int64_t attention_bf16_seq_pad(int64_t seq);
// y[b][f][s] = x[b·seq + s][f] for f < F, s < attention_bf16_seq_pad(seq),
// zero for s ≥ seq.
void transpose_bt(hipStream_t s, const bf16_t *x, int64_t ldx, int64_t batch, int64_t seq, int64_t F, bf16_t *y);
void attention_core_fwd_bf16(hipStream_t s, const bf16_t *qkv, int64_t ld, const bf16_t *qkvt, float *ctx,
                             int64_t ldo, float *lse, int64_t batch, int64_t seq, int64_t n_heads, bool causal);
void attention_core_bwd_bf16(hipStream_t s, const bf16_t *qkv, int64_t ld, const bf16_t *qkvt, const float *ctx,
                             const float *dctx, int64_t ldo, const bf16_t *dctxb, const bf16_t *dctxt,
                             const float *lse, float *dqkv, int64_t ldd, int64_t batch, int64_t seq,
                             int64_t n_heads, bool causal, float *scratch);
// Grouped-query forms (GqaAttention, always causal in the forward; window >
// 0: query i sees keys [i − window + 1, i]): q (and dq) rows of stride ldq
// hold n_heads heads, k, v (and dk, dv) rows of stride ldk hold
// n_heads / group heads; query head h reads K/V head h / group.  dk and dv
// of a K/V head sum its group's query heads in head order.
void attention_core_fwd_lse_gqa(hipStream_t s, const float *q, int64_t ldq, const float *k, const float *v,
                                int64_t ldk, int64_t group, int64_t window, float *ctx, int64_t ldo, float *lse,
                                int64_t batch, int64_t seq, int64_t n_heads, int64_t d_head);
void attention_core_bwd_gqa(hipStream_t s, const float *q, int64_t ldq, const float *k, const float *v,
                            int64_t ldk, int64_t group, int64_t window, const float *o, const float *dout,
                            int64_t ldo, const float *lse, float *dq, int64_t ld_dq, float *dk, float *dv,
                            int64_t ld_dkv, int64_t batch, int64_t seq, int64_t n_heads, int64_t d_head,
                            bool causal, float *scratch);
// RoPE on the first `heads` heads of width hd of each row of qk (row r is
// position r mod S), in place: table [S, hd/2] of (cos, sin) from rope_table
// (angles pos·θ^(−2i/hd) in f64, rounded to f32); sign −1 rotates by −angle,
// the adjoint of the rotation (gqa_backward's apply_rope with −θ).
void rope_table(hipStream_t s, float *tab, int64_t S, int64_t hd, double theta);
void rope_apply(hipStream_t s, float *qk, int64_t ld, int64_t rows, int64_t S, int64_t heads, int64_t hd,
                const float *tab, float sign);

}  // namespace k
}  // namespace catnn
