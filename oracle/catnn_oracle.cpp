// catnn oracle — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of the reference's CPU kernels and naïve reference
// (dkarapetyan-afk/cat-nn-compiler, Rust), used by tests/, by
// __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker
// and the timed CPU path.  Nothing in the product links or calls it.
//
// Each function follows the cited reference loop nest.  Built with
// -ffp-contract=off because Rust does not contract a·b + c into a fused
// multiply-add; f32 exp/tanh/sqrt come from the C library, as Rust's f32
// methods do on Linux.  OpenMP parallelises exactly the loops the reference
// runs under Rayon (row loops of cpu::linear, softmax_last, layer_norm);
// everything else is sequential, as in the reference.
//
// Parity status per function (how each is pinned; see tests/test_oracle.py):
//   lcg, checksum                — reference test tensor.rs:310-315 + the
//                                  published LCG/FNV-1a definitions (brute
//                                  force in Python integers).
//   relu, gelu, softmax_last,
//   layer_norm, add, mul         — known answers (cpu.rs:318-322), library
//                                  routines in float64 (torch/scipy), invariants.
//   matmul_seq / linear_seq      — bit-exact against a float32 sequential sum
//                                  done element by element in numpy; float64
//                                  matmul within 1e-6.
//   linear (f32x8 lane order)    — float64 matmul within 1e-6; the exact low
//                                  bits depend on `wide` 1.7.1's reduce_add
//                                  order and are parity unpinned at the bit
//                                  level (tolerance only, as the reference's
//                                  own test lib.rs:99-107).
//   attention (+causal)          — torch float64 scaled_dot_product_attention.
//   topk_softmax                 — known answer lens/moe.rs:208-213, stable
//                                  argsort brute force.  NaN logits: parity
//                                  unpinned (Rust's sort with a non-total
//                                  comparator is not reproduced).
//   route / swiglu / moe         — float64 dense evaluation, brute force.
//   moe_permute                  — build-defined order; bijection and
//                                  histogram invariants, brute force.
//   place_arena / arena_conflict — reference tests schedule.rs:479-498 and
//                                  invariants (no conflicts, cap respected).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

extern "C" {

// ------------------------------------------------------------- tensor.rs

// Tensor::lcg, crates/catnn-core/src/tensor.rs:259-268.
void orc_lcg(uint64_t seed, float *out, int64_t n) {
    uint64_t state = seed < 1 ? 1 : seed;
    for (int64_t i = 0; i < n; ++i) {
        state = state * 6364136223846793005ull + 1ull;
        const float unit = (float)(uint32_t)(state >> 33) / (float)UINT32_MAX;
        out[i] = unit * 2.0f - 1.0f;
    }
}

// Tensor::checksum, tensor.rs:279-288.
uint64_t orc_checksum(const float *x, int64_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (int64_t i = 0; i < n; ++i) {
        uint32_t bits;
        std::memcpy(&bits, x + i, 4);
        h ^= (uint64_t)bits;
        h *= 0x100000001b3ull;
    }
    return h;
}

// Tensor::max_abs_diff, tensor.rs:270-277.
float orc_max_abs_diff(const float *a, const float *b, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) m = std::fmax(m, std::fabs(a[i] - b[i]));
    return m;
}

// ---------------------------------------------------------------- cpu.rs

// cpu::relu, crates/catnn-compile/src/kernel/cpu.rs:14-18 (f32::max).
void orc_relu(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = std::fmax(x[i], 0.0f);
}

// cpu::gelu, cpu.rs:20-29 (reference::gelu, reference.rs:17-24, is the same).
void orc_gelu(const float *x, float *y, int64_t n) {
    const float c = std::sqrt(2.0f / (float)M_PI);
    for (int64_t i = 0; i < n; ++i) {
        const float z = x[i];
        const float inner = c * (z + 0.044715f * z * z * z);
        y[i] = 0.5f * z * (1.0f + std::tanh(inner));
    }
}

// One row of cpu::softmax_last, cpu.rs:39-50.
static void softmax_row(const float *in, float *out, int64_t last) {
    float mx = -INFINITY;
    for (int64_t j = 0; j < last; ++j) mx = std::fmax(mx, in[j]);
    float sum = 0.0f;
    for (int64_t j = 0; j < last; ++j) {
        out[j] = std::exp(in[j] - mx);
        sum += out[j];
    }
    const float inv = 1.0f / std::fmax(sum, 1e-30f);
    for (int64_t j = 0; j < last; ++j) out[j] *= inv;
}

// cpu::softmax_last, cpu.rs:31-52 (Rayon over rows).
void orc_softmax_last(const float *x, float *y, int64_t rows, int64_t last) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) softmax_row(x + r * last, y + r * last, last);
}

// reference::softmax_last, reference.rs:26-42 (sequential, same formula).
void orc_ref_softmax_last(const float *x, float *y, int64_t rows, int64_t last) {
    for (int64_t r = 0; r < rows; ++r) softmax_row(x + r * last, y + r * last, last);
}

// One row of cpu::layer_norm, cpu.rs:61-76: mean = Σx/n, var = Σ(x−mean)²/n,
// inv = 1/sqrt(var + eps), y = (x − mean)·inv·γ + β.
static void layer_norm_row(const float *in, const float *g, const float *b, float *out,
                           int64_t last, float eps) {
    const float n = (float)last;
    float s = 0.0f;
    for (int64_t i = 0; i < last; ++i) s += in[i];
    const float mean = s / n;
    float q = 0.0f;
    for (int64_t i = 0; i < last; ++i) {
        const float d = in[i] - mean;
        q += d * d;
    }
    const float var = q / n;
    const float inv = 1.0f / std::sqrt(var + eps);
    for (int64_t i = 0; i < last; ++i) out[i] = (in[i] - mean) * inv * g[i] + b[i];
}

// cpu::layer_norm, cpu.rs:54-78 (Rayon over rows).
void orc_layer_norm(const float *x, const float *g, const float *b, float *y, int64_t rows,
                    int64_t last, float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) layer_norm_row(x + r * last, g, b, y + r * last, last, eps);
}

// reference::layer_norm, reference.rs:44-57 (sequential).
void orc_ref_layer_norm(const float *x, const float *g, const float *b, float *y, int64_t rows,
                        int64_t last, float eps) {
    for (int64_t r = 0; r < rows; ++r) layer_norm_row(x + r * last, g, b, y + r * last, last, eps);
}

// cpu::add, cpu.rs:80-98.  Returns 0, or 2 (ShapeMismatch) when b is neither
// the same length nor the last dim.
int orc_add(const float *a, int64_t na, const float *b, int64_t nb, int64_t last, float *y) {
    if (na == nb) {
        for (int64_t i = 0; i < na; ++i) y[i] = a[i] + b[i];
        return 0;
    }
    if (nb == last && last > 0) {
        for (int64_t i = 0; i < na; ++i) y[i] = a[i] + b[i % last];
        return 0;
    }
    return 2;
}

// cpu::mul, cpu.rs:100-109.
int orc_mul(const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
    return 0;
}

// cpu::matmul_mk_kn_seq, cpu.rs:115-126: s = 0; s += a[i,p]·b[p,j], p ascending.
void orc_matmul_seq(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i) {
        const float *ai = a + i * k;
        for (int64_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (int64_t p = 0; p < k; ++p) s += ai[p] * b[p * n + j];
            c[i * n + j] = s;
        }
    }
}

// Bias pass of linear_inner, cpu.rs:173-182.
static void add_bias(float *y, const float *bias, int64_t m, int64_t n) {
    if (!bias) return;
    for (int64_t r = 0; r < m; ++r)
        for (int64_t j = 0; j < n; ++j) y[r * n + j] += bias[j];
}

// cpu::linear_seq, cpu.rs:128-132 → linear_inner(parallel = false).
void orc_linear_seq(const float *x, const float *w, const float *bias, float *y, int64_t m,
                    int64_t k, int64_t n) {
    orc_matmul_seq(x, w, y, m, k, n);
    add_bias(y, bias, m, n);
}

// cpu::dot_row, cpu.rs:199-232: eight lane accumulators over p in steps of
// 8 (lane l accumulates a[p+l]·b[(p+l)·n+j], multiply then add), the lanes
// reduced as wide::f32x8::reduce_add — here (l0+l4, l1+l5, l2+l6, l3+l7),
// then pairs (0+2, 1+3), then the final add — and a scalar tail.
static float dot_row(const float *a, const float *b, int64_t k, int64_t n, int64_t j) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t p = 0;
    for (; p + 8 <= k; p += 8)
        for (int l = 0; l < 8; ++l) acc[l] += a[p + l] * b[(p + l) * n + j];
    const float s4[4] = {acc[0] + acc[4], acc[1] + acc[5], acc[2] + acc[6], acc[3] + acc[7]};
    const float s2[2] = {s4[0] + s4[2], s4[1] + s4[3]};
    float s = s2[0] + s2[1];
    for (; p < k; ++p) s += a[p] * b[p * n + j];
    return s;
}

// cpu::matmul_mk_kn, cpu.rs:186-197 (Rayon over output rows; column blocks
// of 32 only change the visiting order, not any value).
void orc_matmul(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < m; ++i) {
        const float *ai = a + i * k;
        for (int64_t j = 0; j < n; ++j) c[i * n + j] = dot_row(ai, b, k, n, j);
    }
}

// cpu::linear, cpu.rs:135-184.
void orc_linear(const float *x, const float *w, const float *bias, float *y, int64_t m, int64_t k,
                int64_t n) {
    orc_matmul(x, w, y, m, k, n);
    add_bias(y, bias, m, n);
}

// reference::linear, reference.rs:63-85: naïve i, j, p with the bias added
// inside the sum.
void orc_ref_linear(const float *x, const float *w, const float *bias, float *y, int64_t m,
                    int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float s = 0.0f;
            for (int64_t p = 0; p < k; ++p) s += x[i * k + p] * w[p * n + j];
            if (bias) s += bias[j];
            y[i * n + j] = s;
        }
}

// cpu::attention, cpu.rs:235-298, on x [B,S,D] with head h at columns
// h·dh..(h+1)·dh: q, k, v and the output projection through cpu::linear
// (linear3, cpu.rs:300-304); scores, softmax and P·V sequential per (b, h).
// causal != 0 applies the masking of moe::gqa (moe.rs:104-121): query i
// attends keys j ≤ i only.  Returns 2 when n_heads·d_head > D.
int orc_attention(const float *x, const float *wq, const float *wk, const float *wv,
                  const float *wo, int64_t B, int64_t S, int64_t D, int64_t H, int64_t dh,
                  int32_t causal, float *out) {
    if (H * dh > D) return 2;
    const int64_t T = B * S;
    std::vector<float> q((size_t)(T * D)), k((size_t)(T * D)), v((size_t)(T * D)),
        ctx((size_t)(T * D), 0.0f);
    orc_linear(x, wq, nullptr, q.data(), T, D, D);
    orc_linear(x, wk, nullptr, k.data(), T, D, D);
    orc_linear(x, wv, nullptr, v.data(), T, D, D);
    const float scale = 1.0f / std::sqrt((float)dh);
    std::vector<float> scores((size_t)(S * S));
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t h = 0; h < H; ++h) {
            for (int64_t i = 0; i < S; ++i)
                for (int64_t j = 0; j < S; ++j) {
                    if (causal && j > i) {
                        scores[(size_t)(i * S + j)] = -INFINITY;
                        continue;
                    }
                    float dot = 0.0f;
                    for (int64_t t = 0; t < dh; ++t)
                        dot += q[(size_t)(bi * S * D + i * D + h * dh + t)] *
                               k[(size_t)(bi * S * D + j * D + h * dh + t)];
                    scores[(size_t)(i * S + j)] = dot * scale;
                }
            for (int64_t i = 0; i < S; ++i) {
                float *row = &scores[(size_t)(i * S)];
                const int64_t len = causal ? i + 1 : S;
                float mx = -INFINITY;
                for (int64_t j = 0; j < len; ++j) mx = std::fmax(mx, row[j]);
                float sum = 0.0f;
                for (int64_t j = 0; j < len; ++j) {
                    row[j] = std::exp(row[j] - mx);
                    sum += row[j];
                }
                const float inv = 1.0f / std::fmax(sum, 1e-30f);
                for (int64_t j = 0; j < len; ++j) row[j] *= inv;
                for (int64_t j = len; j < S; ++j) row[j] = 0.0f;
            }
            for (int64_t i = 0; i < S; ++i) {
                const int64_t len = causal ? i + 1 : S;
                for (int64_t t = 0; t < dh; ++t) {
                    float acc = 0.0f;
                    for (int64_t j = 0; j < len; ++j)
                        acc += scores[(size_t)(i * S + j)] * v[(size_t)(bi * S * D + j * D + h * dh + t)];
                    ctx[(size_t)(bi * S * D + i * D + h * dh + t)] = acc;
                }
            }
        }
    orc_linear(ctx.data(), wo, nullptr, out, T, D, D);
    return 0;
}

// ---------------------------------------------------------------- moe.rs

// lens::moe::topk_softmax, crates/catnn-core/src/lens/moe.rs:175-187: stable
// sort of expert ids by descending logit (ties keep the lower id first),
// truncate to k, w = exp(l − max_sel)·(1/max(Σ, 1e-30)).
void orc_topk_softmax(const float *logits, int64_t E, int64_t k, int32_t *idx, float *w) {
    std::vector<int32_t> order((size_t)E);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(),
                     [&](int32_t a, int32_t b) { return logits[a] > logits[b]; });
    const int64_t kk = std::min(k, E);
    float mx = -INFINITY;
    for (int64_t i = 0; i < kk; ++i) mx = std::fmax(mx, logits[order[(size_t)i]]);
    float sum = 0.0f;
    for (int64_t i = 0; i < kk; ++i) {
        idx[i] = order[(size_t)i];
        w[i] = std::exp(logits[order[(size_t)i]] - mx);
        sum += w[i];
    }
    const float inv = 1.0f / std::fmax(sum, 1e-30f);
    for (int64_t i = 0; i < kk; ++i) w[i] *= inv;
}

// moe::route, crates/catnn-compile/src/kernel/moe.rs:177-195.
void orc_route(const float *x, const float *gate, int64_t T, int64_t H, int64_t E, int64_t k,
               int32_t *idx, float *w, float *logits) {
    std::vector<float> lg((size_t)(T * E));
    orc_matmul_seq(x, gate, lg.data(), T, H, E);
    for (int64_t t = 0; t < T; ++t) orc_topk_softmax(&lg[(size_t)(t * E)], E, k, idx + t * k, w + t * k);
    if (logits) std::memcpy(logits, lg.data(), lg.size() * 4);
}

// silu, moe.rs:12-14.
static float silu(float v) { return v / (1.0f + std::exp(-v)); }

// moe::swiglu, moe.rs:159-174: three linear_seq GEMMs on x [T,H].
void orc_swiglu(const float *x, const float *w1, const float *w3, const float *w2, int64_t T,
                int64_t H, int64_t I, float *y) {
    std::vector<float> a((size_t)(T * I)), c((size_t)(T * I));
    orc_matmul_seq(x, w1, a.data(), T, H, I);
    orc_matmul_seq(x, w3, c.data(), T, H, I);
    for (size_t i = 0; i < a.size(); ++i) a[i] = silu(a[i]) * c[i];
    orc_matmul_seq(a.data(), w2, y, T, I, H);
}

// moe::reference::swiglu, moe.rs:353-381 (gate and up accumulated together).
void orc_ref_swiglu(const float *x, const float *w1, const float *w3, const float *w2, int64_t T,
                    int64_t H, int64_t I, float *y) {
    std::vector<float> h((size_t)(T * I));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t j = 0; j < I; ++j) {
            float a = 0.0f, c = 0.0f;
            for (int64_t i = 0; i < H; ++i) {
                const float xv = x[t * H + i];
                a += xv * w1[i * I + j];
                c += xv * w3[i * I + j];
            }
            h[(size_t)(t * I + j)] = silu(a) * c;
        }
    for (int64_t t = 0; t < T; ++t)
        for (int64_t i = 0; i < H; ++i) {
            float s = 0.0f;
            for (int64_t j = 0; j < I; ++j) s += h[(size_t)(t * I + j)] * w2[j * H + i];
            y[t * H + i] = s;
        }
}

// moe::moe, moe.rs:197-223: route all tokens, then per token and per
// selected expert (ascending k) out[t] += w·swiglu_e(x_t).  Expert weights
// are packed: w1s [E][H][I], w3s [E][H][I], w2s [E][I][H].  `tokens_only`
// (may be null) restricts the expert loop to a list of token rows, leaving
// the other rows of `out` untouched — per-token work is independent, so a
// subset gives the same rows as the full run.
void orc_moe(const float *x, const float *gate, const float *w1s, const float *w3s,
             const float *w2s, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
             const int64_t *tokens_only, int64_t n_only, float *out) {
    std::vector<int32_t> idx((size_t)(T * k));
    std::vector<float> w((size_t)(T * k));
    orc_route(x, gate, T, H, E, k, idx.data(), w.data(), nullptr);
    std::vector<float> y((size_t)H);
    const int64_t n_rows = tokens_only ? n_only : T;
    for (int64_t r = 0; r < n_rows; ++r) {
        const int64_t t = tokens_only ? tokens_only[r] : r;
        float *o = out + t * H;
        for (int64_t i = 0; i < H; ++i) o[i] = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) {
            const int64_t e = idx[(size_t)(t * k + kk)];
            const float wt = w[(size_t)(t * k + kk)];
            orc_swiglu(x + t * H, w1s + e * H * I, w3s + e * H * I, w2s + e * I * H, 1, H, I, y.data());
            for (int64_t i = 0; i < H; ++i) o[i] += wt * y[(size_t)i];
        }
    }
}

// moe::reference::moe, moe.rs:383-416 (per-token logits, reference swiglu).
void orc_ref_moe(const float *x, const float *gate, const float *w1s, const float *w3s,
                 const float *w2s, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                 float *out) {
    std::vector<float> logits((size_t)E), y((size_t)H);
    std::vector<int32_t> idx((size_t)k);
    std::vector<float> w((size_t)k);
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t e = 0; e < E; ++e) {
            float s = 0.0f;
            for (int64_t i = 0; i < H; ++i) s += x[t * H + i] * gate[i * E + e];
            logits[(size_t)e] = s;
        }
        orc_topk_softmax(logits.data(), E, k, idx.data(), w.data());
        float *o = out + t * H;
        for (int64_t i = 0; i < H; ++i) o[i] = 0.0f;
        for (int64_t kk = 0; kk < std::min(k, E); ++kk) {
            const int64_t e = idx[(size_t)kk];
            orc_ref_swiglu(x + t * H, w1s + e * H * I, w3s + e * H * I, w2s + e * I * H, 1, H, I, y.data());
            for (int64_t i = 0; i < H; ++i) o[i] += w[(size_t)kk] * y[(size_t)i];
        }
    }
}

// Token permutation of the backend (the reference has none: it loops over
// tokens).  Stable counting sort of the flattened slots s = t·k + k' by
// expert: counts[e], offsets[e] = Σ_{e'<e} counts[e'] (E+1 entries),
// slot_of_pos[offsets[e] + r] = the r-th slot routed to e in ascending s,
// pos_of_slot its inverse.  Returns 2 for an id outside [0, E).
int orc_moe_permute(const int32_t *idx, int64_t T, int64_t k, int64_t E, int32_t *counts,
                    int32_t *offsets, int32_t *slot_of_pos, int32_t *pos_of_slot) {
    const int64_t n = T * k;
    for (int64_t e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t s = 0; s < n; ++s) {
        if (idx[s] < 0 || idx[s] >= E) return 2;
        ++counts[idx[s]];
    }
    offsets[0] = 0;
    for (int64_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    std::vector<int32_t> next(offsets, offsets + E);
    for (int64_t s = 0; s < n; ++s) {
        const int32_t pos = next[(size_t)idx[s]]++;
        slot_of_pos[pos] = (int32_t)s;
        pos_of_slot[s] = pos;
    }
    return 0;
}

// ----------------------------------------------------------- schedule.rs

struct OrcReq {
    uint64_t bytes, live_from, live_to;
};

// schedule::place_arena, crates/catnn-compile/src/schedule.rs:79-116.
// Writes offsets[i] for request i (input order).  Returns 0, or 10
// (Fibration) with *fail_index set on overflow.
int orc_place_arena(const uint64_t *bytes, const uint64_t *live_from, const uint64_t *live_to,
                    int64_t n, uint64_t cap, uint64_t *offsets, int64_t *placement_order,
                    int64_t *fail_index) {
    std::vector<int64_t> order((size_t)n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        if (live_from[a] != live_from[b]) return live_from[a] < live_from[b];
        return bytes[a] > bytes[b];
    });
    std::vector<int64_t> placed;
    for (int64_t pi = 0; pi < n; ++pi) {
        const int64_t i = order[(size_t)pi];
        std::vector<std::pair<uint64_t, uint64_t>> forb;
        for (int64_t p : placed)
            if (live_from[p] <= live_to[i] && live_from[i] <= live_to[p])
                forb.emplace_back(offsets[p], offsets[p] + bytes[p]);
        std::stable_sort(forb.begin(), forb.end(),
                         [](const auto &a, const auto &b) { return a.first < b.first; });
        uint64_t cursor = 0;
        bool chosen = false;
        uint64_t off = 0;
        for (const auto &f : forb) {
            if (f.first >= cursor + bytes[i]) {
                off = cursor;
                chosen = true;
                break;
            }
            cursor = std::max(cursor, f.second);
        }
        if (!chosen) off = cursor;
        if (off + bytes[i] < off || off + bytes[i] > cap) {
            if (fail_index) *fail_index = i;
            return 10;
        }
        offsets[i] = off;
        if (placement_order) placement_order[pi] = i;
        placed.push_back(i);
    }
    return 0;
}

// schedule::arena_conflict, schedule.rs:123-136: 1 when two simultaneously
// live buffers overlap in the arena.
int orc_arena_conflict(const uint64_t *bytes, const uint64_t *offsets, const uint64_t *live_from,
                       const uint64_t *live_to, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        for (int64_t j = i + 1; j < n; ++j)
            if (live_from[i] <= live_to[j] && live_from[j] <= live_to[i] &&
                offsets[i] < offsets[j] + bytes[j] && offsets[j] < offsets[i] + bytes[i])
                return 1;
    return 0;
}

// ---------------------------------------------------------- Mixtral ops
// moe::rmsnorm, moe.rs:17-32: y = x · 1/sqrt(Σx²/n + eps) · w per row.
void orc_rmsnorm(const float *x, const float *w, int64_t rows, int64_t cols, float eps, float *y) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float ss = 0.0f;
        for (int64_t i = 0; i < cols; ++i) ss += row[i] * row[i];
        const float mean_sq = ss / (float)cols;
        const float inv = 1.0f / std::sqrt(mean_sq + eps);
        for (int64_t i = 0; i < cols; ++i) y[r * cols + i] = row[i] * inv * w[i];
    }
}

// The Embedding arm of eval_cpu (mod.rs:81-96) over moe::embedding
// (moe.rs:34-45): ids arrive as f32, rounded half away from zero and
// clamped to [0, u32::MAX]; an id ≥ vocab is ShapeMismatch (returns 2).
int orc_embedding(const float *ids, int64_t n, const float *table, int64_t vocab, int64_t hidden,
                  float *y) {
    for (int64_t t = 0; t < n; ++t) {
        float v = std::round(ids[t]);
        if (!(v >= 0.0f)) v = 0.0f;  // NaN and negatives clamp to 0
        if (v >= (float)vocab) return 2;
        const int64_t id = (int64_t)v;
        std::memcpy(y + t * hidden, table + id * hidden, (size_t)hidden * 4);
    }
    return 0;
}

// moe::apply_rope, moe.rs:47-60: pairs (2i, 2i+1) rotated by pos·θ^(−2i/hd),
// angles in f64, sin/cos cast to f32.
static void apply_rope(float *q, int64_t head_dim, int64_t pos, double theta) {
    for (int64_t i = 0; i < head_dim / 2; ++i) {
        const double freq = 1.0 / std::pow(theta, 2.0 * (double)i / (double)head_dim);
        const double ang = (double)pos * freq;
        const float s = (float)std::sin(ang), c = (float)std::cos(ang);
        const float a = q[2 * i], b = q[2 * i + 1];
        q[2 * i] = a * c - b * s;
        q[2 * i + 1] = a * s + b * c;
    }
}

// moe::gqa, moe.rs:62-136: q/k/v projections (linear_seq), RoPE on q and k
// at position t, per (b, h) causal softmax over keys [start, i] with
// start = i − (window − 1) when a window is given (window ≤ 0: none), kv head
// h / (n_heads / n_kv), then the output projection; n_heads·head_dim need
// not equal the model width.  Returns 2 on a shape mismatch.
int orc_gqa(const float *x, const float *wq, const float *wk, const float *wv, const float *wo, int64_t B,
            int64_t S, int64_t D, int64_t n_heads, int64_t n_kv, int64_t head_dim, double theta,
            int64_t window, float *y) {
    if (n_kv <= 0 || n_heads <= 0 || n_heads % n_kv != 0) return 2;
    const int64_t T = B * S, KV = n_kv * head_dim, QW = n_heads * head_dim;
    std::vector<float> q((size_t)(T * QW)), k((size_t)(T * KV)), v((size_t)(T * KV));
    orc_matmul_seq(x, wq, q.data(), T, D, QW);
    orc_matmul_seq(x, wk, k.data(), T, D, KV);
    orc_matmul_seq(x, wv, v.data(), T, D, KV);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t t = 0; t < S; ++t) {
            for (int64_t h = 0; h < n_heads; ++h)
                apply_rope(&q[(size_t)(((bi * S + t) * n_heads + h) * head_dim)], head_dim, t, theta);
            for (int64_t h = 0; h < n_kv; ++h)
                apply_rope(&k[(size_t)(((bi * S + t) * n_kv + h) * head_dim)], head_dim, t, theta);
        }
    const int64_t repeats = std::max<int64_t>(n_heads / std::max<int64_t>(n_kv, 1), 1);
    const float scale = 1.0f / std::sqrt((float)head_dim);
    std::vector<float> ctx((size_t)(T * QW), 0.0f), scores((size_t)S);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t h = 0; h < n_heads; ++h) {
            const int64_t kv_h = h / repeats;
            for (int64_t i = 0; i < S; ++i) {
                const int64_t start = window > 0 ? std::max<int64_t>(i - (window - 1), 0) : 0;
                const float *qi = &q[(size_t)(((bi * S + i) * n_heads + h) * head_dim)];
                float mx = -INFINITY;
                for (int64_t j = start; j <= i; ++j) {
                    const float *kj = &k[(size_t)(((bi * S + j) * n_kv + kv_h) * head_dim)];
                    float dot = 0.0f;
                    for (int64_t t = 0; t < head_dim; ++t) dot += qi[t] * kj[t];
                    scores[(size_t)j] = dot * scale;
                    mx = std::max(mx, scores[(size_t)j]);
                }
                float sum = 0.0f;
                for (int64_t j = start; j <= i; ++j) {
                    scores[(size_t)j] = std::exp(scores[(size_t)j] - mx);
                    sum += scores[(size_t)j];
                }
                const float inv = 1.0f / std::max(sum, 1e-30f);
                float *o = &ctx[(size_t)(((bi * S + i) * n_heads + h) * head_dim)];
                for (int64_t j = start; j <= i; ++j) {
                    const float wgt = scores[(size_t)j] * inv;
                    const float *vj = &v[(size_t)(((bi * S + j) * n_kv + kv_h) * head_dim)];
                    for (int64_t t = 0; t < head_dim; ++t) o[t] += wgt * vj[t];
                }
            }
        }
    orc_matmul_seq(ctx.data(), wo, y, T, QW, D);
    return 0;
}

void orc_linear_backward(const float *x, const float *w, const float *dy, int64_t m, int64_t k,
                         int64_t n, float *dx, float *dw, float *db);

// apply_rope of the adjoint module, adjoint.rs:457-470: the same rotation
// with frequencies from |θ|; a negative θ rotates by −angle (the sine cast
// to f32, then negated).
static void apply_rope_adj(float *q, int64_t head_dim, int64_t pos, double theta) {
    for (int64_t i = 0; i < head_dim / 2; ++i) {
        const double freq = 1.0 / std::pow(std::fabs(theta), 2.0 * (double)i / (double)head_dim);
        const double ang = (double)pos * freq;
        float s = (float)std::sin(ang);
        const float c = (float)std::cos(ang);
        if (theta < 0.0) s = -s;
        const float a = q[2 * i], b = q[2 * i + 1];
        q[2 * i] = a * c - b * s;
        q[2 * i + 1] = a * s + b * c;
    }
}

// gqa_backward, adjoint.rs:287-440: recompute q, k, v (linear_seq, as
// linear3 at :442-455) and RoPE on q and k, then per (b, h, i) the windowed
// causal softmax (keys [start, i], start = i − (window − 1) when a window is
// given; window ≤ 0: none) kept as `attn`; dctx and dwo by linear_backward;
// dv += a·dctx, dq += ds·scale·k, dk += ds·scale·q with ds the softmax
// adjoint over the window, in the reference's (b, h, i, j) order; dq and dk
// rotated back by −θ; dx = dxq + dxk + dxv from the three projections'
// linear_backward.  Returns 2 on a shape mismatch.
int orc_gqa_backward(const float *x, const float *wq, const float *wk, const float *wv, const float *wo,
                     int64_t B, int64_t S, int64_t D, int64_t n_heads, int64_t n_kv, int64_t head_dim,
                     double theta, int64_t window, const float *dy, float *dx, float *dwq, float *dwk,
                     float *dwv, float *dwo) {
    if (n_kv <= 0 || n_heads <= 0 || n_heads % n_kv != 0) return 2;
    const int64_t T = B * S, QW = n_heads * head_dim, KV = n_kv * head_dim;
    std::vector<float> q((size_t)(T * QW)), k((size_t)(T * KV)), v((size_t)(T * KV));
    orc_matmul_seq(x, wq, q.data(), T, D, QW);
    orc_matmul_seq(x, wk, k.data(), T, D, KV);
    orc_matmul_seq(x, wv, v.data(), T, D, KV);
    const int64_t repeats = n_heads / std::max<int64_t>(n_kv, 1);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t t = 0; t < S; ++t) {
            for (int64_t h = 0; h < n_heads; ++h)
                apply_rope_adj(&q[(size_t)(((bi * S + t) * n_heads + h) * head_dim)], head_dim, t, theta);
            for (int64_t h = 0; h < n_kv; ++h)
                apply_rope_adj(&k[(size_t)(((bi * S + t) * n_kv + h) * head_dim)], head_dim, t, theta);
        }
    const float scale = 1.0f / std::sqrt((float)head_dim);
    auto start_of = [&](int64_t i) { return window > 0 ? std::max<int64_t>(i - (window - 1), 0) : 0; };
    std::vector<float> ctx((size_t)(T * QW), 0.0f), attn((size_t)(B * n_heads * S * S), 0.0f);
    std::vector<float> scores((size_t)S);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t h = 0; h < n_heads; ++h) {
            const int64_t kv_h = h / std::max<int64_t>(repeats, 1);
            for (int64_t i = 0; i < S; ++i) {
                const int64_t start = start_of(i);
                const int64_t q_off = ((bi * S + i) * n_heads + h) * head_dim;
                std::fill(scores.begin(), scores.end(), -INFINITY);
                for (int64_t j = start; j <= i; ++j) {
                    const int64_t k_off = ((bi * S + j) * n_kv + kv_h) * head_dim;
                    float dot = 0.0f;
                    for (int64_t t = 0; t < head_dim; ++t) dot += q[(size_t)(q_off + t)] * k[(size_t)(k_off + t)];
                    scores[(size_t)j] = dot * scale;
                }
                float mx = -INFINITY;
                for (int64_t j = start; j <= i; ++j) mx = std::max(mx, scores[(size_t)j]);
                float sum = 0.0f;
                for (int64_t j = start; j <= i; ++j) {
                    scores[(size_t)j] = std::exp(scores[(size_t)j] - mx);
                    sum += scores[(size_t)j];
                }
                const float inv = 1.0f / std::max(sum, 1e-30f);
                for (int64_t j = start; j <= i; ++j) {
                    scores[(size_t)j] *= inv;
                    attn[(size_t)(((bi * n_heads + h) * S + i) * S + j)] = scores[(size_t)j];
                }
                for (int64_t j = start; j <= i; ++j) {
                    const int64_t v_off = ((bi * S + j) * n_kv + kv_h) * head_dim;
                    for (int64_t t = 0; t < head_dim; ++t)
                        ctx[(size_t)(q_off + t)] += scores[(size_t)j] * v[(size_t)(v_off + t)];
                }
            }
        }
    std::vector<float> dctx((size_t)(T * QW)), db((size_t)std::max(D, std::max(QW, KV)));
    orc_linear_backward(ctx.data(), wo, dy, T, QW, D, dctx.data(), dwo, db.data());
    std::vector<float> dq((size_t)(T * QW), 0.0f), dk((size_t)(T * KV), 0.0f), dv((size_t)(T * KV), 0.0f);
    std::vector<float> dscore((size_t)S);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t h = 0; h < n_heads; ++h) {
            const int64_t kv_h = h / std::max<int64_t>(repeats, 1);
            for (int64_t i = 0; i < S; ++i) {
                const int64_t start = start_of(i);
                const int64_t o_off = ((bi * S + i) * n_heads + h) * head_dim;
                const float *arow = &attn[(size_t)(((bi * n_heads + h) * S + i) * S)];
                std::fill(dscore.begin(), dscore.end(), 0.0f);
                for (int64_t j = start; j <= i; ++j) {
                    const int64_t v_off = ((bi * S + j) * n_kv + kv_h) * head_dim;
                    float dot = 0.0f;
                    for (int64_t t = 0; t < head_dim; ++t) dot += dctx[(size_t)(o_off + t)] * v[(size_t)(v_off + t)];
                    dscore[(size_t)j] = dot;
                }
                float dot = 0.0f;
                for (int64_t j = start; j <= i; ++j) dot += arow[j] * dscore[(size_t)j];
                for (int64_t j = start; j <= i; ++j) dscore[(size_t)j] = arow[j] * (dscore[(size_t)j] - dot);
                for (int64_t j = start; j <= i; ++j) {
                    const int64_t kv_off = ((bi * S + j) * n_kv + kv_h) * head_dim;
                    const float a = arow[j];
                    for (int64_t t = 0; t < head_dim; ++t) {
                        dv[(size_t)(kv_off + t)] += a * dctx[(size_t)(o_off + t)];
                        dq[(size_t)(o_off + t)] += dscore[(size_t)j] * scale * k[(size_t)(kv_off + t)];
                        dk[(size_t)(kv_off + t)] += dscore[(size_t)j] * scale * q[(size_t)(o_off + t)];
                    }
                }
            }
        }
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t t = 0; t < S; ++t) {
            for (int64_t h = 0; h < n_heads; ++h)
                apply_rope_adj(&dq[(size_t)(((bi * S + t) * n_heads + h) * head_dim)], head_dim, t, -theta);
            for (int64_t h = 0; h < n_kv; ++h)
                apply_rope_adj(&dk[(size_t)(((bi * S + t) * n_kv + h) * head_dim)], head_dim, t, -theta);
        }
    std::vector<float> dxk((size_t)(T * D)), dxv((size_t)(T * D));
    orc_linear_backward(x, wq, dq.data(), T, D, QW, dx, dwq, db.data());
    orc_linear_backward(x, wk, dk.data(), T, D, KV, dxk.data(), dwk, db.data());
    orc_linear_backward(x, wv, dv.data(), T, D, KV, dxv.data(), dwv, db.data());
    for (int64_t i = 0; i < T * D; ++i) dx[i] += dxk[(size_t)i];
    for (int64_t i = 0; i < T * D; ++i) dx[i] += dxv[(size_t)i];
    return 0;
}

// moe::lm_head, moe.rs:325-333: w is [V, H] (HF layout); y = x·wᵀ via the
// transposed copy and linear_seq.
void orc_lm_head(const float *x, const float *w, int64_t rows, int64_t H, int64_t V, float *y) {
    std::vector<float> wt((size_t)(H * V));
    for (int64_t i = 0; i < V; ++i)
        for (int64_t j = 0; j < H; ++j) wt[(size_t)(j * V + i)] = w[i * H + j];
    orc_matmul_seq(x, wt.data(), y, rows, H, V);
}

// deepseek::mix, deepseek.rs:229-239: y = σ(g)·a + (1 − σ(g))·b.
void orc_mix(const float *a, const float *b, float gate, int64_t n, float *y) {
    const float s = 1.0f / (1.0f + std::exp(-gate));
    for (int64_t i = 0; i < n; ++i) y[i] = s * a[i] + (1.0f - s) * b[i];
}

// embedding_backward, adjoint.rs:187-197, with the ids converted as the
// adjoint_of arm does (adjoint.rs:845: round, max 0, as u32): dw = 0, then
// per token in order dw[id] += dy[t].
void orc_embedding_backward(const float *ids, int64_t n, const float *dy, int64_t vocab, int64_t hidden, float *dw) {
    for (int64_t i = 0; i < vocab * hidden; ++i) dw[i] = 0.0f;
    for (int64_t t = 0; t < n; ++t) {
        const float r = std::max(std::round(ids[t]), 0.0f);
        const int64_t id = !(r >= 0.0f) ? 0 : r >= 4294967296.0f ? 4294967295ll : (int64_t)r;
        if (id >= vocab) continue;  // the reference indexes out of bounds; the forward refuses such ids
        for (int64_t i = 0; i < hidden; ++i) dw[id * hidden + i] += dy[t * hidden + i];
    }
}

// deepseek::mix_backward, deepseek.rs:241-258: da = dy·σ, db = dy·(1 − σ),
// dg = σ(1 − σ)·Σ (a − b)·dy summed in index order.  Returns dg.
float orc_mix_backward(const float *a, const float *b, float gate, const float *dy, int64_t n, float *da,
                       float *db) {
    const float s = 1.0f / (1.0f + std::exp(-gate));
    float dg = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        da[i] = dy[i] * s;
        db[i] = dy[i] * (1.0f - s);
        dg += (a[i] - b[i]) * dy[i];
    }
    return dg * (s * (1.0f - s));
}

}  // extern "C"

// ============================================================ adjoint.rs
// Reverse rules of crates/catnn-compile/src/kernel/adjoint.rs, restated loop
// for loop (sequential: the reference runs them single-threaded).  Pinned by
// tests/test_oracle_adjoint.py against float64 torch autograd and the
// reference's known answers (adjoint.rs:1006-1011, :1035-1042,
// optim.rs:163-176).

extern "C" {

// linear_backward, adjoint.rs:35-61: for i, j: g = dy[i,j]; db[j] += g;
// for p: dw[p,j] += x[i,p]·g; dx[i,p] += g·w[p,j].
void orc_linear_backward(const float *x, const float *w, const float *dy, int64_t m, int64_t k,
                         int64_t n, float *dx, float *dw, float *db) {
    std::fill(dx, dx + m * k, 0.0f);
    std::fill(dw, dw + k * n, 0.0f);
    std::fill(db, db + n, 0.0f);
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            const float g = dy[i * n + j];
            db[j] += g;
            for (int64_t p = 0; p < k; ++p) {
                dw[p * n + j] += x[i * k + p] * g;
                dx[i * k + p] += g * w[p * n + j];
            }
        }
}

// relu_backward, adjoint.rs:63-74.
void orc_relu_backward(const float *x, const float *dy, float *dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = x[i] <= 0.0f ? 0.0f : dy[i];
}

// gelu_backward, adjoint.rs:76-90 (derivative of the tanh form).
void orc_gelu_backward(const float *x, const float *dy, float *dx, int64_t n) {
    const float C = 0.044715f;
    const float k = std::sqrt(2.0f / (float)M_PI);
    for (int64_t i = 0; i < n; ++i) {
        const float z = x[i];
        const float u = k * (z + C * z * z * z);
        const float t = std::tanh(u);
        const float sech2 = 1.0f - t * t;
        const float du = k * (1.0f + 3.0f * C * z * z);
        const float dg = 0.5f * (1.0f + t) + 0.5f * z * sech2 * du;
        dx[i] = dy[i] * dg;
    }
}

// softmax_backward, adjoint.rs:92-104: dx = y·(dy − Σ y·dy) per row.
void orc_softmax_backward(const float *y, const float *dy, float *dx, int64_t rows, int64_t last) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *yr = y + r * last, *gr = dy + r * last;
        float dot = 0.0f;
        for (int64_t i = 0; i < last; ++i) dot += yr[i] * gr[i];
        for (int64_t i = 0; i < last; ++i) dx[r * last + i] = yr[i] * (gr[i] - dot);
    }
}

// mse_loss, adjoint.rs:106-119: loss = Σe²/n, d = 2e/n.
float orc_mse_loss(const float *pred, const float *target, int64_t n, float *d) {
    const float nf = (float)n;
    float loss = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float e = pred[i] - target[i];
        loss += e * e;
        d[i] = 2.0f * e / nf;
    }
    return loss / nf;
}

// layer_norm_backward, adjoint.rs:530-577.
// rmsnorm_backward, adjoint.rs:147-198: per row ms = Σx²/n (sequential),
// inv = 1/√(ms+eps); dw_i += dy_i·x_i·inv and dinv += dy_i·x_i·w_i in column
// order; dms = dinv·(−0.5)·(ms+eps)^(−1.5); dx_i = dy_i·inv·w_i + dms·(2·x_i/n).
void orc_rmsnorm_backward(const float *x, const float *w, const float *dy, int64_t rows, int64_t last, float eps,
                          float *dx, float *dw) {
    const float n = (float)last;
    for (int64_t i = 0; i < last; ++i) dw[i] = 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * last, *yr = dy + r * last;
        float ss = 0.0f;
        for (int64_t i = 0; i < last; ++i) ss += xr[i] * xr[i];
        const float ms = ss / n;
        const float inv = 1.0f / std::sqrt(ms + eps);
        float dinv = 0.0f;
        for (int64_t i = 0; i < last; ++i) {
            dw[i] += yr[i] * xr[i] * inv;
            dinv += yr[i] * xr[i] * w[i];
        }
        const float dms = dinv * (-0.5f) * std::pow(ms + eps, -1.5f);
        for (int64_t i = 0; i < last; ++i) dx[r * last + i] = yr[i] * inv * w[i] + dms * (2.0f * xr[i] / n);
    }
}

void orc_layer_norm_backward(const float *x, const float *gamma, const float *dy, int64_t rows,
                             int64_t last, float eps, float *dx, float *dgamma, float *dbeta) {
    std::fill(dgamma, dgamma + last, 0.0f);
    std::fill(dbeta, dbeta + last, 0.0f);
    const float n = (float)last;
    std::vector<float> xhat((size_t)last), dxhat((size_t)last);
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = x + r * last, *yrow = dy + r * last;
        float s = 0.0f;
        for (int64_t i = 0; i < last; ++i) s += row[i];
        const float mean = s / n;
        float q = 0.0f;
        for (int64_t i = 0; i < last; ++i) {
            const float d = row[i] - mean;
            q += d * d;
        }
        const float var = q / n;
        const float inv = 1.0f / std::sqrt(var + eps);
        for (int64_t i = 0; i < last; ++i) {
            xhat[(size_t)i] = (row[i] - mean) * inv;
            dbeta[i] += yrow[i];
            dgamma[i] += yrow[i] * xhat[(size_t)i];
            dxhat[(size_t)i] = yrow[i] * gamma[i];
        }
        float sd = 0.0f, sdx = 0.0f;
        for (int64_t i = 0; i < last; ++i) sd += dxhat[(size_t)i];
        for (int64_t i = 0; i < last; ++i) sdx += dxhat[(size_t)i] * xhat[(size_t)i];
        for (int64_t i = 0; i < last; ++i)
            dx[r * last + i] = (inv / n) * (n * dxhat[(size_t)i] - sd - xhat[(size_t)i] * sdx);
    }
}

// attention_backward, adjoint.rs:582-722 (recomputes the forward with
// cpu::linear projections).  causal != 0 restricts every row to keys j ≤ i
// with the window softmax and its adjoint as gqa_backward does
// (adjoint.rs:372-405).
int orc_attention_backward(const float *x, const float *wq, const float *wk, const float *wv,
                           const float *wo, int64_t B, int64_t S, int64_t D, int64_t H, int64_t dh,
                           int32_t causal, const float *dy, float *dx, float *dwq, float *dwk,
                           float *dwv, float *dwo) {
    if (D != H * dh) return 2;
    const int64_t T = B * S;
    std::vector<float> q((size_t)(T * D)), k((size_t)(T * D)), v((size_t)(T * D));
    orc_linear(x, wq, nullptr, q.data(), T, D, D);
    orc_linear(x, wk, nullptr, k.data(), T, D, D);
    orc_linear(x, wv, nullptr, v.data(), T, D, D);
    const float scale = 1.0f / std::sqrt((float)dh);
    std::vector<float> attn((size_t)(B * H * S * S), 0.0f), ctx((size_t)(T * D), 0.0f);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t h = 0; h < H; ++h) {
            float *sc = &attn[(size_t)((bi * H + h) * S * S)];
            for (int64_t i = 0; i < S; ++i) {
                const int64_t len = causal ? i + 1 : S;
                for (int64_t j = 0; j < len; ++j) {
                    float dot = 0.0f;
                    for (int64_t t = 0; t < dh; ++t)
                        dot += q[(size_t)(bi * S * D + i * D + h * dh + t)] *
                               k[(size_t)(bi * S * D + j * D + h * dh + t)];
                    sc[i * S + j] = dot * scale;
                }
                float mx = -INFINITY;
                for (int64_t j = 0; j < len; ++j) mx = std::fmax(mx, sc[i * S + j]);
                float sum = 0.0f;
                for (int64_t j = 0; j < len; ++j) {
                    sc[i * S + j] = std::exp(sc[i * S + j] - mx);
                    sum += sc[i * S + j];
                }
                const float inv = 1.0f / std::fmax(sum, 1e-30f);
                for (int64_t j = 0; j < len; ++j) sc[i * S + j] *= inv;
            }
            for (int64_t i = 0; i < S; ++i) {
                const int64_t len = causal ? i + 1 : S;
                for (int64_t t = 0; t < dh; ++t) {
                    float acc = 0.0f;
                    for (int64_t j = 0; j < len; ++j)
                        acc += sc[i * S + j] * v[(size_t)(bi * S * D + j * D + h * dh + t)];
                    ctx[(size_t)(bi * S * D + i * D + h * dh + t)] = acc;
                }
            }
        }
    std::vector<float> dctx((size_t)(T * D)), dbias((size_t)D);
    orc_linear_backward(ctx.data(), wo, dy, T, D, D, dctx.data(), dwo, dbias.data());
    std::vector<float> dq((size_t)(T * D), 0.0f), dk((size_t)(T * D), 0.0f), dv((size_t)(T * D), 0.0f);
    std::vector<float> dattn((size_t)S);
    for (int64_t bi = 0; bi < B; ++bi)
        for (int64_t h = 0; h < H; ++h) {
            const float *a = &attn[(size_t)((bi * H + h) * S * S)];
            for (int64_t i = 0; i < S; ++i) {
                const int64_t len = causal ? i + 1 : S;
                for (int64_t j = 0; j < len; ++j) {
                    float g = 0.0f;
                    for (int64_t t = 0; t < dh; ++t) {
                        const float dc = dctx[(size_t)(bi * S * D + i * D + h * dh + t)];
                        g += dc * v[(size_t)(bi * S * D + j * D + h * dh + t)];
                        dv[(size_t)(bi * S * D + j * D + h * dh + t)] += a[i * S + j] * dc;
                    }
                    dattn[(size_t)j] = g;
                }
                float dot = 0.0f;
                for (int64_t j = 0; j < len; ++j) dot += a[i * S + j] * dattn[(size_t)j];
                for (int64_t j = 0; j < len; ++j) {
                    const float g = a[i * S + j] * (dattn[(size_t)j] - dot) * scale;
                    for (int64_t t = 0; t < dh; ++t) {
                        dq[(size_t)(bi * S * D + i * D + h * dh + t)] +=
                            g * k[(size_t)(bi * S * D + j * D + h * dh + t)];
                        dk[(size_t)(bi * S * D + j * D + h * dh + t)] +=
                            g * q[(size_t)(bi * S * D + i * D + h * dh + t)];
                    }
                }
            }
        }
    std::vector<float> dxq((size_t)(T * D)), dxk((size_t)(T * D)), dxv((size_t)(T * D));
    orc_linear_backward(x, wq, dq.data(), T, D, D, dxq.data(), dwq, dbias.data());
    orc_linear_backward(x, wk, dk.data(), T, D, D, dxk.data(), dwk, dbias.data());
    orc_linear_backward(x, wv, dv.data(), T, D, D, dxv.data(), dwv, dbias.data());
    for (int64_t i = 0; i < T * D; ++i) dx[i] = dxq[(size_t)i] + dxk[(size_t)i] + dxv[(size_t)i];
    return 0;
}

static float silu_grad(float v) {
    const float s = 1.0f / (1.0f + std::exp(-v));
    return s + v * s * (1.0f - s);
}

// swiglu_backward, adjoint.rs:217-251 (gradients accumulate into dw*).
static void swiglu_backward_acc(const float *x, const float *w1, const float *w3, const float *w2,
                                int64_t T, int64_t H, int64_t I, const float *dy, float *dx,
                                float *dw1, float *dw3, float *dw2) {
    std::vector<float> a((size_t)(T * I)), c((size_t)(T * I)), h((size_t)(T * I));
    orc_matmul_seq(x, w1, a.data(), T, H, I);
    orc_matmul_seq(x, w3, c.data(), T, H, I);
    for (size_t i = 0; i < h.size(); ++i) h[i] = silu(a[i]) * c[i];
    std::vector<float> dh((size_t)(T * I)), tw2((size_t)(I * H)), tb((size_t)std::max(H, I));
    orc_linear_backward(h.data(), w2, dy, T, I, H, dh.data(), tw2.data(), tb.data());
    std::vector<float> da((size_t)(T * I)), dc((size_t)(T * I));
    for (size_t i = 0; i < h.size(); ++i) {
        da[i] = dh[i] * c[i] * silu_grad(a[i]);
        dc[i] = dh[i] * silu(a[i]);
    }
    std::vector<float> dx1((size_t)(T * H)), dx3((size_t)(T * H)), tw1((size_t)(H * I)), tw3((size_t)(H * I));
    orc_linear_backward(x, w1, da.data(), T, H, I, dx1.data(), tw1.data(), tb.data());
    orc_linear_backward(x, w3, dc.data(), T, H, I, dx3.data(), tw3.data(), tb.data());
    for (int64_t i = 0; i < T * H; ++i) dx[i] = dx1[(size_t)i] + dx3[(size_t)i];
    for (int64_t i = 0; i < H * I; ++i) {
        dw1[i] += tw1[(size_t)i];
        dw3[i] += tw3[(size_t)i];
    }
    for (int64_t i = 0; i < I * H; ++i) dw2[i] += tw2[(size_t)i];
}

void orc_swiglu_backward(const float *x, const float *w1, const float *w3, const float *w2, int64_t T,
                         int64_t H, int64_t I, const float *dy, float *dx, float *dw1, float *dw3,
                         float *dw2) {
    std::fill(dw1, dw1 + H * I, 0.0f);
    std::fill(dw3, dw3 + H * I, 0.0f);
    std::fill(dw2, dw2 + I * H, 0.0f);
    swiglu_backward_acc(x, w1, w3, w2, T, H, I, dy, dx, dw1, dw3, dw2);
}

// router_backward_ste, adjoint.rs:255-284: per token, the softmax Jacobian
// on the selected subset; then linear_backward through the gate.
void orc_router_backward_ste(const float *x, const float *gate, int64_t T, int64_t H, int64_t E,
                             int64_t k, const float *d_weights, float *dx, float *dgate) {
    std::vector<float> logits((size_t)(T * E)), dl((size_t)(T * E), 0.0f), db((size_t)E);
    orc_matmul_seq(x, gate, logits.data(), T, H, E);
    std::vector<int32_t> idx((size_t)k);
    std::vector<float> w((size_t)k);
    for (int64_t t = 0; t < T; ++t) {
        orc_topk_softmax(&logits[(size_t)(t * E)], E, k, idx.data(), w.data());
        float dot = 0.0f;
        for (int64_t j = 0; j < k; ++j) dot += w[(size_t)j] * d_weights[t * k + j];
        for (int64_t j = 0; j < k; ++j)
            dl[(size_t)(t * E + idx[(size_t)j])] += w[(size_t)j] * (d_weights[t * k + j] - dot);
    }
    orc_linear_backward(x, gate, dl.data(), T, H, E, dx, dgate, db.data());
}

// moe_backward, adjoint.rs:471-526.  Expert weights packed as in orc_moe.
void orc_moe_backward(const float *x, const float *gate, const float *w1s, const float *w3s,
                      const float *w2s, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k,
                      const float *dy, float *dx, float *dgate, float *dw1s, float *dw3s,
                      float *dw2s) {
    std::vector<int32_t> idx((size_t)(T * k));
    std::vector<float> wts((size_t)(T * k)), d_wts((size_t)(T * k), 0.0f);
    orc_route(x, gate, T, H, E, k, idx.data(), wts.data(), nullptr);
    std::fill(dx, dx + T * H, 0.0f);
    std::fill(dw1s, dw1s + E * H * I, 0.0f);
    std::fill(dw3s, dw3s + E * H * I, 0.0f);
    std::fill(dw2s, dw2s + E * I * H, 0.0f);
    std::vector<float> y((size_t)H), dye((size_t)H), dxe((size_t)H);
    for (int64_t t = 0; t < T; ++t) {
        const float *xt = x + t * H, *dyt = dy + t * H;
        for (int64_t j = 0; j < k; ++j) {
            const int64_t e = idx[(size_t)(t * k + j)];
            const float wt = wts[(size_t)(t * k + j)];
            const float *w1 = w1s + e * H * I, *w3 = w3s + e * H * I, *w2 = w2s + e * I * H;
            orc_swiglu(xt, w1, w3, w2, 1, H, I, y.data());
            float s = 0.0f;
            for (int64_t i = 0; i < H; ++i) s += y[(size_t)i] * dyt[i];
            d_wts[(size_t)(t * k + j)] = s;
            for (int64_t i = 0; i < H; ++i) dye[(size_t)i] = dyt[i] * wt;
            swiglu_backward_acc(xt, w1, w3, w2, 1, H, I, dye.data(), dxe.data(), dw1s + e * H * I,
                                dw3s + e * H * I, dw2s + e * I * H);
            for (int64_t i = 0; i < H; ++i) dx[t * H + i] += dxe[(size_t)i];
        }
    }
    std::vector<float> dxg((size_t)(T * H));
    orc_router_backward_ste(x, gate, T, H, E, k, d_wts.data(), dxg.data(), dgate);
    for (int64_t i = 0; i < T * H; ++i) dx[i] += dxg[(size_t)i];
}

// cross_entropy, crates/catnn-compile/src/kernel/adjoint.rs:123-145: probs
// = softmax_last(logits); d = probs with every element of row r divided by
// rows and 1/rows subtracted at the target; loss = Σ_r −ln(max(p_t, 1e-30))
// summed in row order, divided by rows.  Returns 0 and writes d and *loss,
// or −1 (ShapeMismatch) for a target ≥ last.
int orc_cross_entropy(const float *logits, const uint32_t *targets, int64_t rows, int64_t last, float *d,
                      float *loss) {
    orc_softmax_last(logits, d, rows, last);
    const float rf = (float)rows;
    float l = 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t t = targets[r];
        if (t >= last) return -1;
        const float p = std::max(d[r * last + t], 1e-30f);
        l -= std::log(p);
        for (int64_t j = 0; j < last; ++j) d[r * last + j] /= rf;
        d[r * last + t] -= 1.0f / rf;
    }
    *loss = l / rf;
    return 0;
}

// Sgd::put, crates/catnn-core/src/lens/optim.rs:32-42: p −= lr·g.
void orc_sgd(float *p, const float *g, int64_t n, float lr) {
    for (int64_t i = 0; i < n; ++i) p[i] -= lr * g[i];
}

// f32::powi for a run-time exponent.  The reference calls b1.powi(t as i32)
// (optim.rs:102-103); rustc lowers that to llvm.powi.f32, which for a
// non-constant exponent becomes a call of __powisf2 from Rust's
// compiler-builtins crate (the version pinned by the toolchain, absent
// here): binary exponentiation — multiply the result by the base when the
// low bit is set, halve the exponent, square the base — in f32, reciprocal
// for a negative exponent.
float orc_powi(float b, int32_t t) {
    const bool recip = t < 0;
    uint32_t e = recip ? 0u - (uint32_t)t : (uint32_t)t;
    float r = 1.f;
    for (;;) {
        if (e & 1u) r *= b;
        e >>= 1;
        if (e == 0) break;
        b *= b;
    }
    return recip ? 1.f / r : r;
}

// Adam::put, crates/catnn-core/src/lens/optim.rs:95-118, on n values in
// place: `t` is AdamState.t before the step (t' = t saturating_add 1),
// b1t = 1 − β₁^t', b2t = 1 − β₂^t', then per element m' = β₁m + (1−β₁)g,
// v' = β₂v + (1−β₂)·g·g (left to right), p' = p − lr·m̂/(√v̂ + eps) with
// m̂ = m'/max(b1t, 1e-30), v̂ = v'/max(b2t, 1e-30).  Built with
// -ffp-contract=off, so every operation rounds as Rust's does.
void orc_adam(float *p, const float *g, float *m, float *v, int64_t n, uint64_t t, float lr, float beta1,
              float beta2, float eps) {
    const uint64_t t1 = t == UINT64_MAX ? t : t + 1;
    const float b1t = 1.0f - orc_powi(beta1, (int32_t)t1);
    const float b2t = 1.0f - orc_powi(beta2, (int32_t)t1);
    for (int64_t i = 0; i < n; ++i) {
        const float gi = g[i];
        const float mi = beta1 * m[i] + (1.0f - beta1) * gi;
        const float vi = beta2 * v[i] + (1.0f - beta2) * gi * gi;
        m[i] = mi;
        v[i] = vi;
        const float mhat = mi / std::max(b1t, 1e-30f);
        const float vhat = vi / std::max(b2t, 1e-30f);
        p[i] = p[i] - lr * mhat / (std::sqrt(vhat) + eps);
    }
}

}  // extern "C"
