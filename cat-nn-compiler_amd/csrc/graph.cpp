// IR graph, per-op dispatch and the three execution seams of the backend:
//
//  * catnn_hip_run_kernel — DeviceHandler::run_kernel (crates/catnn-rt/src/handler.rs:34-57)
//    with host tensors in and out, params riding in the node;
//  * catnn_hip_run_node   — the same node on arena buffer ids (device-resident);
//  * catnn_hip_install / catnn_hip_forward — a whole IrGraph on one device,
//    evaluated in IrGraph::topo order as eval_graph_cpu does
//    (crates/catnn-compile/src/lib.rs:48-68), with activations in one HBM
//    region planned by place_arena over forward lifetimes.
//
// Fusion.  Realization.fusions (place::propose_fusions, crates/catnn-compile/src/place.rs:184-208)
// pairs a Linear with a following Relu/Gelu on the same device; the reference
// records but never executes them (cpu.rs:306-310 has no callers).  The
// program honours them: the Linear's GEMM applies the activation in its
// epilogue and writes the activation node's buffer.  It also folds a
// ResidualAdd into the GEMM that produces one of its operands (a Linear, a
// fused Linear+activation, or an Attention output projection) when that
// operand has no other consumer and the other operand is computed earlier.
// Fusion only removes intermediate buffers; the arithmetic per element is
// the same sequence of operations.
#include <algorithm>
#include <cstring>
#include <numeric>
#include <set>

#include "arena.hpp"
#include "graph.hpp"
#include "kernels.hpp"
#include "train_ops.hpp"

namespace catnn {

std::string op_name(int32_t kind) {
    // OpenOp::name, crates/catnn-core/src/category/morphism.rs:119-145.
    static const char *names[] = {"id",     "linear",  "relu",      "gelu",        "softmax",
                                  "layernorm", "add",  "mul",       "matmul",      "transpose",
                                  "reshape", "attention", "residual_add", "embedding", "rmsnorm",
                                  "gqa",    "swiglu",  "router",    "moe",         "lm_head",
                                  "mla",    "deepseek_moe", "mix"};
    if (kind < 0 || kind >= (int32_t)(sizeof(names) / sizeof(names[0]))) return "unknown";
    return names[kind];
}

std::string dims_str(const std::vector<int64_t> &d) {
    std::string s = "f32[";
    for (size_t i = 0; i < d.size(); ++i) s += (i ? "," : "") + std::to_string(d[i]);
    return s + "]";
}

static int64_t numel_of(const std::vector<int64_t> &d) {
    int64_t n = 1;
    for (int64_t v : d) n *= v;
    return n;
}

static HostTensor from_c(const catnn_tensor &t, bool need_data) {
    CATNN_REQUIRE(t.rank >= 0 && t.rank <= CATNN_MAX_RANK, CATNN_ERR_SHAPE_MISMATCH,
                  "tensor rank out of range");
    HostTensor h;
    h.dtype = t.dtype;
    for (int i = 0; i < t.rank; ++i) {
        CATNN_REQUIRE(t.dims[i] >= 0, CATNN_ERR_SHAPE_MISMATCH, "negative dimension");
        h.dims.push_back(t.dims[i]);
    }
    if (need_data) {
        const int64_t n = h.numel();
        CATNN_REQUIRE(t.data || n == 0, CATNN_ERR_INVALID_ARGUMENT, "tensor without data");
        h.data.assign(t.data, t.data + n);
    }
    return h;
}

static Node node_from_c(const catnn_node *c, bool need_param_data = true) {
    CATNN_REQUIRE(c, CATNN_ERR_INVALID_ARGUMENT, "null node");
    Node n;
    n.id = c->id;
    n.name = c->name ? c->name : "";
    n.op = c->op;
    n.output_ty = from_c(c->output_ty, false);
    CATNN_REQUIRE(c->n_params >= 0 && (c->n_params == 0 || c->params), CATNN_ERR_INVALID_ARGUMENT,
                  "node params");
    for (int i = 0; i < c->n_params; ++i) {
        CATNN_REQUIRE(c->params[i].port, CATNN_ERR_INVALID_ARGUMENT, "param without port name");
        n.params.emplace_back(c->params[i].port, from_c(c->params[i].value, need_param_data));
    }
    return n;
}

Node node_shape_from_c(const catnn_node *c) { return node_from_c(c, false); }

std::vector<int64_t> dims_from_c(const catnn_tensor &t) { return from_c(t, false).dims; }

static const std::vector<int64_t> &pdims(const Node &n, const std::string &port) {
    const HostTensor *t = n.param(port);
    if (!t) fail(CATNN_ERR_UNKNOWN_PORT, "unknown port " + port + " on interface " + n.name);
    return t->dims;
}

static std::string expert_port(int64_t e, const char *w) {
    return "e" + std::to_string(e) + "." + w;
}

// Weight of a Linear/MatMul: "w", else the first param (kernel/mod.rs:46-50).
static const std::pair<std::string, HostTensor> *linear_weight(const Node &n) {
    for (auto &p : n.params)
        if (p.first == "w") return &p;
    return n.params.empty() ? nullptr : &n.params.front();
}

std::vector<int64_t> infer_dims(const Node &node, const std::vector<std::vector<int64_t>> &ins) {
    const int32_t kind = node.op.kind;
    if (ins.empty()) {
        if (kind == CATNN_OP_IDENTITY) return node.output_ty.dims;  // zeros (mod.rs:22-24)
        fail(CATNN_ERR_WIRING, "node " + node.name + " (" + op_name(kind) + ") has no inputs");
    }
    const std::vector<int64_t> &x = ins[0];
    switch (kind) {
        case CATNN_OP_IDENTITY:
        case CATNN_OP_RESHAPE:
        case CATNN_OP_TRANSPOSE:  // data pass-through, as eval_cpu (mod.rs:27)
        case CATNN_OP_RELU:
        case CATNN_OP_GELU:
        case CATNN_OP_SOFTMAX:
            return x;
        case CATNN_OP_ADD:
        case CATNN_OP_RESIDUAL_ADD: {
            if (ins.size() < 2) return x;
            const int64_t na = numel_of(x), nb = numel_of(ins[1]);
            if (na == nb) return x;
            const int64_t last = x.empty() ? na : x.back();
            if (nb == last) return x;
            fail(CATNN_ERR_SHAPE_MISMATCH, "add " + dims_str(x) + " vs " + dims_str(ins[1]));
        }
        case CATNN_OP_MUL:
            if (ins.size() >= 2 && numel_of(x) != numel_of(ins[1]))
                fail(CATNN_ERR_SHAPE_MISMATCH, "mul length");
            return x;
        case CATNN_OP_LINEAR:
        case CATNN_OP_MATMUL: {
            const auto *w = linear_weight(node);
            if (!w) fail(CATNN_ERR_UNKNOWN_COMPONENT, "unknown component " + node.name);
            const auto &wd = w->second.dims;
            if (x.size() < 2 || wd.size() != 2)
                fail(CATNN_ERR_SHAPE_MISMATCH, "linear " + dims_str(x) + " @ " + dims_str(wd));
            const int64_t k = x.back();
            if (wd[0] != k)
                fail(CATNN_ERR_SHAPE_MISMATCH,
                     "linear K " + std::to_string(k) + " vs " + std::to_string(wd[0]));
            if (const HostTensor *b = node.param("b"))
                if (b->numel() != wd[1]) fail(CATNN_ERR_SHAPE_MISMATCH, "bias length");
            std::vector<int64_t> out = x;
            out.back() = wd[1];
            return out;
        }
        case CATNN_OP_LAYER_NORM: {
            const auto &g = pdims(node, "gamma");
            const auto &b = pdims(node, "beta");
            if (x.empty()) fail(CATNN_ERR_SHAPE_MISMATCH, "ln scalar");
            if (numel_of(g) != x.back() || numel_of(b) != x.back())
                fail(CATNN_ERR_SHAPE_MISMATCH, "ln gamma/beta length");
            return x;
        }
        case CATNN_OP_ATTENTION: {
            if (x.size() != 3) fail(CATNN_ERR_SHAPE_MISMATCH, "attention expects [B,S,D]");
            const int64_t d = x[2], heads = node.op.a[0], dh = node.op.a[2];
            for (const char *p : {"wq", "wk", "wv", "wo"}) {
                const auto &wd = pdims(node, p);
                if (wd.size() != 2 || wd[0] != d || wd[1] != d)
                    fail(CATNN_ERR_SHAPE_MISMATCH,
                         std::string("attention ") + p + " " + dims_str(wd) + " for d_model " +
                             std::to_string(d));
            }
            if (heads <= 0 || dh <= 0 || heads * dh != d)
                fail(CATNN_ERR_SHAPE_MISMATCH, "attention n_heads*d_head != d_model");
            return x;
        }
        case CATNN_OP_MOE: {
            const int64_t E = node.op.a[0], K = node.op.a[1];
            if (x.empty()) fail(CATNN_ERR_SHAPE_MISMATCH, "moe on scalar");
            const int64_t hid = x.back();
            const auto &gd = pdims(node, "gate");
            if (gd.size() != 2 || gd[0] != hid || gd[1] != E)
                fail(CATNN_ERR_SHAPE_MISMATCH, "moe gate " + dims_str(gd));
            if (K < 1 || K > E) fail(CATNN_ERR_SHAPE_MISMATCH, "moe top_k out of range");
            int64_t inter = -1;
            for (int64_t e = 0; e < E; ++e) {
                const auto &w1 = pdims(node, expert_port(e, "w1"));
                const auto &w3 = pdims(node, expert_port(e, "w3"));
                const auto &w2 = pdims(node, expert_port(e, "w2"));
                if (w1.size() != 2 || w1[0] != hid) fail(CATNN_ERR_SHAPE_MISMATCH, "moe w1");
                if (inter < 0) inter = w1[1];
                if (w1[1] != inter || w3 != w1 || w2.size() != 2 || w2[0] != inter || w2[1] != hid)
                    fail(CATNN_ERR_SHAPE_MISMATCH, "moe expert " + std::to_string(e) + " shapes");
            }
            return x;
        }
        case CATNN_OP_ROUTER:  // identity in eval_cpu (mod.rs:128)
            return x;
        case CATNN_OP_RMS_NORM: {  // moe.rs:17-22
            if (x.empty()) fail(CATNN_ERR_SHAPE_MISMATCH, "rms scalar");
            if (numel_of(pdims(node, "w")) != x.back()) fail(CATNN_ERR_SHAPE_MISMATCH, "rmsnorm weight");
            return x;
        }
        case CATNN_OP_EMBEDDING: {  // mod.rs:81-96: [B,S] ids → [B,S,hidden], else [n, hidden]
            const int64_t hidden = node.op.a[1];
            const auto &t = pdims(node, "w");
            if (t.size() != 2 || t[1] != hidden)
                fail(CATNN_ERR_SHAPE_MISMATCH,
                     "embedding table " + dims_str(t) + " for hidden " + std::to_string(hidden));
            if (x.size() == 2) return {x[0], x[1], hidden};
            return {numel_of(x), hidden};
        }
        case CATNN_OP_GQA_ATTENTION: {  // moe.rs:64-82
            if (x.size() != 3) fail(CATNN_ERR_SHAPE_MISMATCH, "gqa expects [B,S,H]");
            const int64_t nh = node.op.a[0], nkv = node.op.a[1], hd = node.op.a[2], d = x[2];
            if (nh <= 0 || nkv <= 0 || hd <= 0 || nh % nkv != 0)
                fail(CATNN_ERR_SHAPE_MISMATCH, "gqa: n_heads must be a positive multiple of n_kv_heads");
            const int64_t qw = nh * hd, kw = nkv * hd;
            const std::pair<const char *, std::vector<int64_t>> want[] = {
                {"wq", {d, qw}}, {"wk", {d, kw}}, {"wv", {d, kw}}, {"wo", {qw, d}}};
            for (const auto &w : want)
                if (pdims(node, w.first) != w.second)
                    fail(CATNN_ERR_SHAPE_MISMATCH, std::string("gqa ") + w.first + " " +
                                                       dims_str(pdims(node, w.first)) + ", expected " +
                                                       dims_str(w.second));
            return x;
        }
        case CATNN_OP_SWIGLU: {  // moe.rs:159-174
            if (x.empty()) fail(CATNN_ERR_SHAPE_MISMATCH, "swiglu on scalar");
            const int64_t hid = x.back();
            const auto &w1 = pdims(node, "w1");
            if (w1.size() != 2 || w1[0] != hid || pdims(node, "w3") != w1 ||
                pdims(node, "w2") != std::vector<int64_t>{w1[1], hid})
                fail(CATNN_ERR_SHAPE_MISMATCH, "swiglu weights " + dims_str(w1) + " for hidden " +
                                                   std::to_string(hid));
            return x;
        }
        case CATNN_OP_LM_HEAD: {  // moe.rs:325-333: w [V, H], [B,S,H] → [B,S,V]
            if (x.size() != 3) fail(CATNN_ERR_SHAPE_MISMATCH, "lm_head expects [B,S,H]");
            const int64_t vocab = node.op.a[1];
            if (pdims(node, "w") != std::vector<int64_t>{vocab, x[2]})
                fail(CATNN_ERR_SHAPE_MISMATCH, "lm_head w " + dims_str(pdims(node, "w")));
            return {x[0], x[1], vocab};
        }
        case CATNN_OP_MIX:  // mod.rs:186-193, deepseek.rs:229-232
            if (ins.size() < 2) fail(CATNN_ERR_WIRING, "mix needs two inputs");
            if (numel_of(x) != numel_of(ins[1])) fail(CATNN_ERR_SHAPE_MISMATCH, "mix operands differ");
            return x;
        default:
            fail(CATNN_ERR_UNSUPPORTED,
                 "op " + op_name(kind) + " (node " + node.name + ") is not executable on the HIP backend");
    }
}

static int64_t moe_intermediate(const Node &node) { return pdims(node, "e0.w1")[1]; }

static k::GqaLayout gqa_layout_of(const Node &node, const std::vector<int64_t> &x) {
    return k::gqa_layout(x[0] * x[1], x[1], node.op.a[0], node.op.a[1], node.op.a[2]);
}

uint64_t scratch_bytes(const Node &node, const std::vector<std::vector<int64_t>> &ins) {
    if (ins.empty()) return 0;
    if (node.op.kind == CATNN_OP_ATTENTION) {
        const auto &x = ins[0];
        const uint64_t t = (uint64_t)(x[0] * x[1]), d = (uint64_t)x[2];
        return (t * 3 * d + t * d) * 4;
    }
    if (node.op.kind == CATNN_OP_MOE) {
        const auto &x = ins[0];
        const int64_t hid = x.back();
        return k::moe_workspace_layout(numel_of(x) / hid, hid, moe_intermediate(node),
                                       node.op.a[0], node.op.a[1])
            .total;
    }
    if (node.op.kind == CATNN_OP_EMBEDDING) return 256;  // the bad-id flag
    if (node.op.kind == CATNN_OP_GQA_ATTENTION) return (uint64_t)gqa_layout_of(node, ins[0]).floats * 4;
    if (node.op.kind == CATNN_OP_SWIGLU) {
        const int64_t hid = ins[0].back();
        return (uint64_t)(numel_of(ins[0]) / hid) * (uint64_t)pdims(node, "w1")[1] * 4;
    }
    if (node.op.kind == CATNN_OP_LM_HEAD) return (uint64_t)numel_of(pdims(node, "w")) * 4;  // wᵀ
    return 0;
}

void exec_node(catnn_hip_device *dev, const Node &node, const ExecArgs &a) {
    hipStream_t s = dev->stream;
    const int32_t kind = node.op.kind;
    const std::vector<int64_t> out_dims = infer_dims(node, a.in_dims);
    const int64_t n_out = numel_of(out_dims);
    bool residual_done = false;
    auto need = [&](const std::string &port) {
        const float *p = a.param(port);
        if (!p) fail(CATNN_ERR_UNKNOWN_PORT, "unknown port " + port + " on interface " + node.name);
        return p;
    };
    if (a.inputs.empty()) {  // Identity without inputs → zeros of output_ty
        CATNN_HIP(hipMemsetAsync(a.out, 0, (size_t)n_out * 4, s));
        return;
    }
    const float *x = a.inputs[0];
    const int64_t nx = numel_of(a.in_dims[0]);
    switch (kind) {
        case CATNN_OP_IDENTITY:
        case CATNN_OP_RESHAPE:
        case CATNN_OP_TRANSPOSE:
            k::copy_f32(s, x, a.out, nx);
            break;
        case CATNN_OP_RELU:
        case CATNN_OP_GELU:
            k::act_f32(s, x, a.out, nx, kind);
            break;
        case CATNN_OP_SOFTMAX: {
            const int64_t last = a.in_dims[0].empty() ? 0 : a.in_dims[0].back();
            if (last == 0) k::copy_f32(s, x, a.out, nx);  // scalar / empty: unchanged
            else k::softmax_f32(s, x, a.out, nx / last, last);
            break;
        }
        case CATNN_OP_ADD:
        case CATNN_OP_RESIDUAL_ADD:
            if (a.inputs.size() > 1) k::add_f32(s, x, a.inputs[1], a.out, nx, numel_of(a.in_dims[1]));
            else k::copy_f32(s, x, a.out, nx);
            break;
        case CATNN_OP_MUL:
            if (a.inputs.size() > 1) k::mul_f32(s, x, a.inputs[1], a.out, nx);
            else k::copy_f32(s, x, a.out, nx);
            break;
        case CATNN_OP_LINEAR:
        case CATNN_OP_MATMUL: {
            const auto *w = linear_weight(node);
            const int64_t kdim = w->second.dims[0], n = w->second.dims[1];
            const float *wp = need(w->first);
            const float *bp = node.param("b") ? need("b") : nullptr;
            k::linear_f32(s, x, kdim, wp, n, bp, a.residual, n, a.out, n, nx / std::max<int64_t>(kdim, 1),
                          kdim, n, a.fused_act);
            residual_done = true;
            break;
        }
        case CATNN_OP_LAYER_NORM: {
            const int64_t last = a.in_dims[0].back();
            const float eps = (float)node.op.a[0] * 1e-6f;  // eps_e6 as f32 · 1e-6 (mod.rs:65)
            k::layer_norm_f32(s, x, need("gamma"), need("beta"), a.out, nx / last, last, eps);
            break;
        }
        case CATNN_OP_ATTENTION: {
            const auto &xd = a.in_dims[0];
            const int64_t B = xd[0], S = xd[1], D = xd[2], T = B * S;
            const int64_t heads = node.op.a[0], dh = node.op.a[2];
            const bool causal = (node.op.flags & CATNN_FLAG_CAUSAL) != 0;
            CATNN_REQUIRE(a.scratch && a.scratch_bytes >= (uint64_t)(T * 4 * D) * 4,
                          CATNN_ERR_INVALID_ARGUMENT, "attention: scratch too small");
            float *qkv = a.scratch;          // [T, 3D]
            float *ctx = a.scratch + T * 3 * D;  // [T, D]
            if (a.derived) {
                k::linear_f32(s, x, D, a.derived, 3 * D, nullptr, nullptr, 0, qkv, 3 * D, T, D,
                              3 * D, 0);
            } else {
                k::linear_f32(s, x, D, need("wq"), D, nullptr, nullptr, 0, qkv, 3 * D, T, D, D, 0);
                k::linear_f32(s, x, D, need("wk"), D, nullptr, nullptr, 0, qkv + D, 3 * D, T, D, D, 0);
                k::linear_f32(s, x, D, need("wv"), D, nullptr, nullptr, 0, qkv + 2 * D, 3 * D, T, D, D,
                              0);
            }
            k::attention_core_f32(s, qkv, qkv + D, qkv + 2 * D, 3 * D, ctx, D, B, S, heads, dh, causal);
            k::linear_f32(s, ctx, D, need("wo"), D, nullptr, a.residual, D, a.out, D, T, D, D, 0);
            residual_done = true;
            break;
        }
        case CATNN_OP_MOE: {
            const int64_t hid = a.in_dims[0].back();
            const int64_t E = node.op.a[0], K = node.op.a[1];
            const int64_t inter = moe_intermediate(node);
            const int64_t T = nx / hid;
            std::vector<const float *> w1(E), w3(E), w2(E);
            for (int64_t e = 0; e < E; ++e) {
                w1[e] = need(expert_port(e, "w1"));
                w3[e] = need(expert_port(e, "w3"));
                w2[e] = need(expert_port(e, "w2"));
            }
            const k::MoeWorkspaceLayout L = k::moe_workspace_layout(T, hid, inter, E, K);
            CATNN_REQUIRE(a.scratch && a.scratch_bytes >= L.total, CATNN_ERR_INVALID_ARGUMENT,
                          "moe: scratch too small");
            k::moe_f32(s, x, need("gate"), w1.data(), w3.data(), w2.data(), T, hid, inter, E, K,
                       a.out, a.scratch, L);
            break;
        }
        case CATNN_OP_ROUTER:
            k::copy_f32(s, x, a.out, nx);
            break;
        case CATNN_OP_RMS_NORM: {
            const int64_t last = a.in_dims[0].back();
            const float eps = (float)node.op.a[0] * 1e-6f;  // eps_e6 as f32 · 1e-6 (mod.rs:79)
            k::rms_norm_f32(s, x, need("w"), a.out, nx / last, last, eps);
            break;
        }
        case CATNN_OP_EMBEDDING: {
            const int64_t vocab = pdims(node, "w")[0], hidden = node.op.a[1];
            CATNN_REQUIRE(a.scratch && a.scratch_bytes >= 4, CATNN_ERR_INVALID_ARGUMENT,
                          "embedding: scratch too small");
            if (a.embed_flag) {  // a program reads the flag once, after its last step
                k::embedding_f32(s, x, nx, need("w"), vocab, hidden, a.out, a.embed_flag);
                break;
            }
            int *bad = reinterpret_cast<int *>(a.scratch);
            CATNN_HIP(hipMemsetAsync(bad, 0, sizeof(int), s));
            k::embedding_f32(s, x, nx, need("w"), vocab, hidden, a.out, bad);
            // The reference fails the op on an out-of-range id (moe.rs:38-40):
            // read the flag back before anything consumes the rows.
            int host_bad = 0;
            CATNN_HIP(hipMemcpyAsync(&host_bad, bad, sizeof(int), hipMemcpyDeviceToHost, s));
            CATNN_HIP(hipStreamSynchronize(s));
            if (host_bad)
                fail(CATNN_ERR_SHAPE_MISMATCH, "embedding " + node.name + ": token id >= vocab " +
                                                   std::to_string(vocab));
            break;
        }
        case CATNN_OP_GQA_ATTENTION: {
            const auto &xd = a.in_dims[0];
            const k::GqaLayout L = gqa_layout_of(node, xd);
            CATNN_REQUIRE(a.scratch && a.scratch_bytes >= (uint64_t)L.floats * 4, CATNN_ERR_INVALID_ARGUMENT,
                          "gqa: scratch too small");
            const bool packed = a.derived != nullptr;
            // sliding_window None is −1 here; Some(0) behaves as no window, as the
            // reference's saturating start does in a release build (moe.rs:102).
            k::gqa_f32(s, x, a.derived, packed ? nullptr : need("wq"), packed ? nullptr : need("wk"),
                       packed ? nullptr : need("wv"), need("wo"), xd[0], xd[1], xd[2], node.op.a[0],
                       node.op.a[1], node.op.a[2], (double)node.op.a[5], node.op.a[4], a.residual, a.out,
                       a.scratch, L);
            residual_done = true;
            break;
        }
        case CATNN_OP_SWIGLU: {
            const int64_t hid = a.in_dims[0].back(), inter = pdims(node, "w1")[1];
            const int64_t T = nx / hid;
            CATNN_REQUIRE(a.scratch && a.scratch_bytes >= (uint64_t)(T * inter) * 4, CATNN_ERR_INVALID_ARGUMENT,
                          "swiglu: scratch too small");
            k::swiglu_f32(s, x, need("w1"), need("w3"), need("w2"), T, hid, inter, a.residual, a.out,
                          a.scratch);
            residual_done = true;
            break;
        }
        case CATNN_OP_LM_HEAD: {
            const auto &xd = a.in_dims[0];
            const int64_t vocab = node.op.a[1], hid = xd[2], T = xd[0] * xd[1];
            const float *wt = a.derived;
            if (!wt) {
                CATNN_REQUIRE(a.scratch && a.scratch_bytes >= (uint64_t)(vocab * hid) * 4,
                              CATNN_ERR_INVALID_ARGUMENT, "lm_head: scratch too small");
                k::transpose_f32(s, need("w"), vocab, hid, a.scratch);
                wt = a.scratch;
            }
            k::linear_f32(s, x, hid, wt, vocab, nullptr, a.residual, vocab, a.out, vocab, T, hid, vocab, 0);
            residual_done = true;
            break;
        }
        case CATNN_OP_MIX:
            k::mix_f32(s, x, a.inputs[1], a.param("gate"), a.out, nx);
            break;
        default:
            fail(CATNN_ERR_UNSUPPORTED, "op " + op_name(kind) + " (node " + node.name +
                                            ") is not executable on the HIP backend");
    }
    if (a.fused_act && kind != CATNN_OP_LINEAR && kind != CATNN_OP_MATMUL)
        k::act_f32(s, a.out, a.out, n_out, a.fused_act);
    if (a.residual && !residual_done) k::add_f32(s, a.residual, a.out, a.out, n_out, n_out);
}

}  // namespace catnn

// ------------------------------------------------------------ IrGraph

const catnn::Node &catnn_graph::node(uint32_t id) const {
    auto it = nodes.find(id);
    if (it == nodes.end()) catnn::fail(CATNN_ERR_WIRING, "edge names unknown node " + std::to_string(id));
    return it->second;
}

std::vector<uint32_t> catnn_graph::preds(uint32_t id) const {
    std::vector<uint32_t> out;
    for (const auto &e : edges)
        if (e.dst == id) out.push_back(e.src);
    return out;
}

std::vector<uint32_t> catnn_graph::succs(uint32_t id) const {
    std::vector<uint32_t> out;
    for (const auto &e : edges)
        if (e.src == id) out.push_back(e.dst);
    return out;
}

// Kahn's algorithm exactly as IrGraph::topo (ir.rs:67-92): zero-indegree ids
// sorted ascending and popped from the back; each popped node's successors
// (one entry per edge) sorted ascending and pushed when they reach zero.
std::vector<uint32_t> catnn_graph::topo() const {
    std::map<uint32_t, size_t> indeg;
    for (uint32_t id : node_order) indeg[id] = 0;
    for (const auto &e : edges) {
        auto it = indeg.find(e.dst);
        if (it == indeg.end() || !indeg.count(e.src))
            catnn::fail(CATNN_ERR_WIRING, "edge " + std::to_string(e.src) + "->" +
                                              std::to_string(e.dst) + " names an unknown node");
        ++it->second;
    }
    std::vector<uint32_t> q;
    for (uint32_t id : node_order)
        if (indeg[id] == 0) q.push_back(id);
    std::sort(q.begin(), q.end());
    std::vector<uint32_t> out;
    while (!q.empty()) {
        const uint32_t n = q.back();
        q.pop_back();
        out.push_back(n);
        std::vector<uint32_t> nexts;
        for (const auto &e : edges)
            if (e.src == n) nexts.push_back(e.dst);
        std::sort(nexts.begin(), nexts.end());
        for (uint32_t s : nexts)
            if (--indeg[s] == 0) q.push_back(s);
    }
    if (out.size() != nodes.size()) catnn::fail(CATNN_ERR_WIRING, "IR graph has a cycle");
    return out;
}

// ------------------------------------------------------------ program

namespace catnn {

struct Step {
    uint32_t node;
    size_t tick;                   // topo index of the executing node
    std::vector<uint32_t> ins;     // value ids read as inputs (preds, edge order)
    uint32_t out;                  // value id written
    int fused_act = 0;
    int64_t residual = -1;         // value id added in the epilogue
    std::vector<std::vector<int64_t>> in_dims;
    uint64_t scratch = 0;
    bool is_input = false;
};

}  // namespace catnn

struct catnn_hip_program {
    catnn_hip_device *dev = nullptr;
    catnn_graph graph;
    std::vector<catnn::Step> steps;
    std::map<uint32_t, std::vector<int64_t>> dims;  // per materialised value
    std::vector<catnn::ArenaAlloc> plan;
    uint64_t reserved = 0;
    void *base = nullptr;
    std::map<std::string, float *> ptr;  // buffer id → device pointer
    std::vector<uint32_t> input_vals;
    uint32_t output_val = 0;
    // Per-step timing (catnn_hip_program_profile).
    bool profiling = false;
    std::vector<size_t> exec_steps;                  // indices of non-input steps
    std::vector<std::vector<hipEvent_t>> pending;    // one event set per timed forward
    std::vector<std::vector<hipEvent_t>> event_pool;
    std::vector<double> total_ms;
    std::vector<int32_t> calls;
    // A device's stage of a placed graph (catnn_hip_install_placed): values
    // that arrive from elsewhere ("in") or leave ("out"), by name, and the
    // wave state of the current forward pass (coord.rs:592-686).
    bool placed = false;
    std::map<std::string, uint32_t> port_in, port_out;
    std::set<uint32_t> have;       // values present on the device this pass
    std::vector<char> step_done;   // per step, this pass
    // Embeddings raise one device flag on an id ≥ vocab (moe.rs:38-40); it
    // is copied to pinned host memory after the last step and checked when
    // the program next synchronises, so no forward stalls mid-graph.
    bool has_embedding = false;
    int *embed_flag = nullptr;       // device (arena)
    int *embed_flag_host = nullptr;  // pinned
};

namespace catnn {

static std::string act_id(uint32_t v) { return "act:" + std::to_string(v); }
static std::string param_id(const Node &n, const std::string &port) {
    return "param:" + n.name + ":" + port;
}
static std::string scratch_id(const Node &n) { return "scratch:" + n.name; }
static std::string derived_id(const Node &n) { return "derived:" + n.name; }

static bool fusion_listed(const catnn_graph &g, const std::string &a, const std::string &b) {
    for (const auto &f : g.fusions)
        for (size_t i = 0; i + 1 < f.size(); ++i)
            if (f[i] == a && f[i + 1] == b) return true;
    return false;
}

static void build_program(catnn_hip_program &p) {
    const catnn_graph &g = p.graph;
    CATNN_REQUIRE(!g.outputs.empty(), CATNN_ERR_WIRING, "graph has no outputs");
    const std::vector<uint32_t> order = g.topo();
    std::map<uint32_t, size_t> tick;
    for (size_t i = 0; i < order.size(); ++i) tick[order[i]] = i;
    std::set<uint32_t> inputs(g.inputs.begin(), g.inputs.end());
    std::set<uint32_t> done;
    const uint32_t final_out = g.outputs.back();

    for (size_t i = 0; i < order.size(); ++i) {
        const uint32_t id = order[i];
        if (done.count(id)) continue;
        const Node &n = g.node(id);
        Step st;
        st.node = id;
        st.tick = i;
        st.out = id;
        if (inputs.count(id)) {
            st.is_input = true;
            p.dims[id] = n.output_ty.dims;
            p.input_vals.push_back(id);
            p.steps.push_back(st);
            continue;
        }
        st.ins = g.preds(id);
        for (uint32_t v : st.ins) {
            CATNN_REQUIRE(p.dims.count(v), CATNN_ERR_WIRING,
                          "node " + n.name + " reads a value that is not materialised");
            st.in_dims.push_back(p.dims[v]);
        }
        std::vector<int64_t> out_dims = infer_dims(n, st.in_dims);
        const bool gemm_like = n.op.kind == CATNN_OP_LINEAR || n.op.kind == CATNN_OP_MATMUL;
        // Linear → Relu/Gelu listed in Realization.fusions, sole consumer.
        if (gemm_like && !g.outputs.empty()) {
            const auto sc = g.succs(id);
            if (sc.size() == 1 && std::find(g.outputs.begin(), g.outputs.end(), id) == g.outputs.end()) {
                const Node &nx = g.node(sc[0]);
                if ((nx.op.kind == CATNN_OP_RELU || nx.op.kind == CATNN_OP_GELU) &&
                    g.preds(sc[0]).size() == 1 && fusion_listed(g, n.name, nx.name)) {
                    st.fused_act = nx.op.kind;
                    st.out = sc[0];
                    done.insert(sc[0]);
                }
            }
        }
        // ResidualAdd folded into the producing GEMM's epilogue.
        if (gemm_like || n.op.kind == CATNN_OP_ATTENTION || n.op.kind == CATNN_OP_GQA_ATTENTION ||
            n.op.kind == CATNN_OP_SWIGLU) {
            const auto sc = g.succs(st.out);
            const bool is_out =
                std::find(g.outputs.begin(), g.outputs.end(), st.out) != g.outputs.end();
            if (sc.size() == 1 && !is_out) {
                const Node &r = g.node(sc[0]);
                const auto rp = g.preds(sc[0]);
                if (r.op.kind == CATNN_OP_RESIDUAL_ADD && rp.size() == 2 && rp[0] != rp[1] &&
                    (rp[0] == st.out || rp[1] == st.out)) {
                    const uint32_t other = rp[0] == st.out ? rp[1] : rp[0];
                    if (p.dims.count(other) && tick[other] < i &&
                        numel_of(p.dims[other]) == numel_of(out_dims)) {
                        st.residual = other;
                        st.out = sc[0];
                        done.insert(sc[0]);
                    }
                }
            }
        }
        // LmHead reads the wᵀ copy made at install instead of scratch.
        st.scratch = n.op.kind == CATNN_OP_LM_HEAD && n.param("w") ? 0 : scratch_bytes(n, st.in_dims);
        p.dims[st.out] = out_dims;
        p.steps.push_back(st);
    }
    CATNN_REQUIRE(p.dims.count(final_out), CATNN_ERR_WIRING, "graph output is not materialised");
    p.output_val = final_out;
    for (size_t i = 0; i < p.steps.size(); ++i)
        if (!p.steps[i].is_input) p.exec_steps.push_back(i);
    p.total_ms.assign(p.exec_steps.size(), 0.0);
    p.calls.assign(p.exec_steps.size(), 0);
}

// Weight copies made once at install (host side, from the params): the
// projections of Attention / GqaAttention packed per row as [wq | wk | wv],
// so q, k and v come from one GEMM, and LmHead's wᵀ [H, V], so the head is a
// plain GEMM (moe.rs:328 transposes per call).
static int64_t derived_floats(const Node &n) {
    if ((n.op.kind == CATNN_OP_ATTENTION || n.op.kind == CATNN_OP_GQA_ATTENTION) && n.param("wq") &&
        n.param("wk") && n.param("wv"))
        return n.param("wq")->numel() + n.param("wk")->numel() + n.param("wv")->numel();
    if (n.op.kind == CATNN_OP_LM_HEAD && n.param("w")) return n.param("w")->numel();
    return 0;
}

static std::vector<float> derived_weight(const Node &n) {
    std::vector<float> out((size_t)derived_floats(n));
    if (n.op.kind == CATNN_OP_LM_HEAD) {
        const HostTensor &w = *n.param("w");
        const int64_t V = w.dims[0], H = w.dims[1];
        for (int64_t v = 0; v < V; ++v)
            for (int64_t h = 0; h < H; ++h) out[(size_t)(h * V + v)] = w.data[(size_t)(v * H + h)];
        return out;
    }
    const HostTensor *parts[3] = {n.param("wq"), n.param("wk"), n.param("wv")};
    const int64_t rows = parts[0]->dims[0];
    int64_t ld = 0;
    for (const HostTensor *t : parts) ld += t->dims[1];
    int64_t col = 0;
    for (const HostTensor *t : parts) {
        const int64_t c = t->dims[1];
        for (int64_t r = 0; r < rows; ++r)
            std::memcpy(&out[(size_t)(r * ld + col)], &t->data[(size_t)(r * c)], (size_t)c * 4);
        col += c;
    }
    return out;
}

static void plan_and_upload(catnn_hip_program &p) {
    catnn_hip_device *dev = p.dev;
    const catnn_graph &g = p.graph;
    const uint64_t n_ticks = g.nodes.size();
    std::vector<BufferReq> reqs;
    // Activations: live from the producing step to the last reading step.
    std::map<uint32_t, uint64_t> first, last;
    for (const Step &st : p.steps) {
        first[st.out] = st.tick;
        last[st.out] = std::max<uint64_t>(last[st.out], st.tick);
        for (uint32_t v : st.ins) last[v] = std::max<uint64_t>(last[v], st.tick);
        if (st.residual >= 0) last[(uint32_t)st.residual] = std::max<uint64_t>(last[(uint32_t)st.residual], st.tick);
    }
    for (uint32_t o : g.outputs)
        if (p.dims.count(o)) last[o] = n_ticks;
    if (p.placed)  // steps run in waves as remote values arrive, not in tick order: no aliasing
        for (auto &kv : first) {
            kv.second = 0;
            last[kv.first] = n_ticks;
        }
    for (const auto &kv : first) {
        const uint64_t bytes = (uint64_t)numel_of(p.dims[kv.first]) * 4;
        reqs.push_back(BufferReq{act_id(kv.first), bytes, kv.second, last[kv.first], false});
    }
    // Step scratch: live for its own tick only.
    for (const Step &st : p.steps)
        if (st.scratch) reqs.push_back(BufferReq{scratch_id(g.node(st.node)), st.scratch, st.tick, st.tick, false});
    // Params (and the derived weight copies) live throughout.
    for (uint32_t id : g.node_order) {
        const Node &n = g.node(id);
        for (const auto &pr : n.params)
            reqs.push_back(BufferReq{param_id(n, pr.first), (uint64_t)pr.second.numel() * 4, 0, n_ticks, false});
        if (derived_floats(n))
            reqs.push_back(BufferReq{derived_id(n), (uint64_t)derived_floats(n) * 4, 0, n_ticks, false});
    }
    for (const Step &st : p.steps)
        if (!st.is_input && g.node(st.node).op.kind == CATNN_OP_EMBEDDING) p.has_embedding = true;
    if (p.has_embedding) reqs.push_back(BufferReq{"flags:embedding", 256, 0, n_ticks, false});
    // Every buffer starts on a 256-byte boundary: round sizes up.
    for (auto &r : reqs) r.bytes = (r.bytes + 255) & ~uint64_t(255);
    hipDeviceProp_t prop;
    CATNN_HIP(hipGetDeviceProperties(&prop, dev->ordinal));
    p.plan = place_arena(reqs, prop.totalGlobalMem);
    p.reserved = 0;
    for (const auto &a : p.plan) p.reserved = std::max(p.reserved, a.offset + a.bytes);
    if (p.reserved) {
        hipError_t e = hipMalloc(&p.base, p.reserved);
        if (e != hipSuccess)
            fail(CATNN_ERR_FIBRATION, "buffer arena: hipMalloc of " + std::to_string(p.reserved) +
                                          " B failed (" + hipGetErrorString(e) + ")");
    }
    for (const auto &a : p.plan)
        p.ptr[a.id] = reinterpret_cast<float *>(static_cast<char *>(p.base) + a.offset);
    if (p.has_embedding) {
        p.embed_flag = reinterpret_cast<int *>(p.ptr.at("flags:embedding"));
        CATNN_HIP(hipHostMalloc(reinterpret_cast<void **>(&p.embed_flag_host), sizeof(int), hipHostMallocDefault));
        *p.embed_flag_host = 0;
        k::fill_f32(dev->stream, reinterpret_cast<float *>(p.embed_flag), 0.f, 1);
    }
    // Params are uploaded once, here.
    for (uint32_t id : g.node_order) {
        const Node &n = g.node(id);
        for (const auto &pr : n.params)
            if (pr.second.numel())
                CATNN_HIP(hipMemcpyAsync(p.ptr[param_id(n, pr.first)], pr.second.data.data(),
                                         (size_t)pr.second.numel() * 4, hipMemcpyHostToDevice,
                                         dev->stream));
        if (derived_floats(n)) {
            const std::vector<float> d = derived_weight(n);
            CATNN_HIP(hipMemcpyAsync(p.ptr[derived_id(n)], d.data(), d.size() * 4,
                                     hipMemcpyHostToDevice, dev->stream));
            CATNN_HIP(hipStreamSynchronize(dev->stream));
        }
    }
    CATNN_HIP(hipStreamSynchronize(dev->stream));
}

static void exec_step(catnn_hip_program &p, const Step &st) {
    const catnn_graph &g = p.graph;
    const Node &n = g.node(st.node);
    ExecArgs a;
    for (uint32_t v : st.ins) a.inputs.push_back(p.ptr.at(act_id(v)));
    a.in_dims = st.in_dims;
    a.param = [&](const std::string &port) -> const float * {
        auto it = p.ptr.find(param_id(n, port));
        return it == p.ptr.end() ? nullptr : it->second;
    };
    a.out = p.ptr.at(act_id(st.out));
    a.fused_act = st.fused_act;
    a.residual = st.residual >= 0 ? p.ptr.at(act_id((uint32_t)st.residual)) : nullptr;
    if (st.scratch) {
        a.scratch = p.ptr.at(scratch_id(n));
        a.scratch_bytes = st.scratch;
    }
    if (derived_floats(n)) a.derived = p.ptr.at(derived_id(n));
    a.embed_flag = p.embed_flag;
    exec_node(p.dev, n, a);
}

// The forward's embedding flag, copied behind its last step.
static void post_embed_flag(catnn_hip_program &p) {
    if (p.has_embedding)
        CATNN_HIP(hipMemcpyAsync(p.embed_flag_host, p.embed_flag, sizeof(int), hipMemcpyDeviceToHost, p.dev->stream));
}

// After a synchronisation: an out-of-range token id seen by the forward
// fails it as moe::embedding does (ShapeMismatch, moe.rs:38-40).
static void check_embed_flag(catnn_hip_program &p) {
    if (!p.has_embedding || !*p.embed_flag_host) return;
    *p.embed_flag_host = 0;
    k::fill_f32(p.dev->stream, reinterpret_cast<float *>(p.embed_flag), 0.f, 1);
    fail(CATNN_ERR_SHAPE_MISMATCH, "embedding: token id >= vocab in the last forward of " + p.graph.name);
}

static void run_program(catnn_hip_program &p) {
    std::vector<hipEvent_t> *evs = nullptr;
    if (p.profiling) {
        std::vector<hipEvent_t> set;
        if (!p.event_pool.empty()) {
            set = std::move(p.event_pool.back());
            p.event_pool.pop_back();
        } else {
            set.resize(p.exec_steps.size() + 1);
            for (auto &e : set) CATNN_HIP(hipEventCreate(&e));
        }
        p.pending.push_back(std::move(set));
        evs = &p.pending.back();
        CATNN_HIP(hipEventRecord((*evs)[0], p.dev->stream));
    }
    size_t executed = 0;
    for (const Step &st : p.steps) {
        if (st.is_input) continue;
        exec_step(p, st);
        ++executed;
        if (evs) CATNN_HIP(hipEventRecord((*evs)[executed], p.dev->stream));
    }
    post_embed_flag(p);
}

// One forward wave of a placed stage (forward_device, coord.rs:622-676):
// every step not yet run this pass whose inputs are all present runs, in
// topo order; its output becomes present.  Returns the steps fired.
static int forward_wave(catnn_hip_program &p) {
    int fired = 0;
    for (size_t i = 0; i < p.steps.size(); ++i) {
        const Step &st = p.steps[i];
        if (st.is_input || p.step_done[i]) continue;
        bool ready = true;
        for (uint32_t v : st.ins) ready = ready && p.have.count(v);
        if (st.residual >= 0) ready = ready && p.have.count((uint32_t)st.residual);
        if (!ready) continue;
        exec_step(p, st);
        p.step_done[i] = 1;
        p.have.insert(st.out);
        ++fired;
    }
    if (fired) post_embed_flag(p);
    return fired;
}

static void collect_timings(catnn_hip_program &p) {
    for (auto &set : p.pending) {
        CATNN_HIP(hipEventSynchronize(set.back()));
        for (size_t i = 0; i + 1 < set.size(); ++i) {
            float ms = 0.f;
            CATNN_HIP(hipEventElapsedTime(&ms, set[i], set[i + 1]));
            p.total_ms[i] += ms;
            p.calls[i] += 1;
        }
        p.event_pool.push_back(std::move(set));
    }
    p.pending.clear();
}

static void destroy_events(catnn_hip_program &p) {
    for (auto *sets : {&p.pending, &p.event_pool})
        for (auto &set : *sets)
            for (hipEvent_t e : set) (void)hipEventDestroy(e);
    p.pending.clear();
    p.event_pool.clear();
}

// The stage of `g` that Placement puts on `device` (placement.get(name)
// .unwrap_or(default_device), as forward_device reads it, coord.rs:629):
// its nodes keep their ids; a value produced elsewhere and read here enters
// as an input node "{producer}#recv" (the buffer schedule_device names
// act:{producer}#recv, pipeline.rs:319-327); a local value read elsewhere,
// or a graph output placed here, is an output of the stage.
static catnn_graph stage_of(const catnn_graph &g, const std::map<std::string, std::string> &assign,
                            const std::string &device, const std::string &default_device,
                            std::map<std::string, uint32_t> &port_in, std::map<std::string, uint32_t> &port_out) {
    auto home = [&](const Node &n) {
        auto it = assign.find(n.name);
        return it == assign.end() ? default_device : it->second;
    };
    catnn_graph st;
    st.name = g.name + "@" + device;
    st.fusions = g.fusions;
    uint32_t next_id = 0;
    for (const auto &kv : g.nodes) next_id = std::max(next_id, kv.first + 1);
    std::map<uint32_t, uint32_t> recv_of;  // remote producer id → recv node id
    const std::set<uint32_t> inputs(g.inputs.begin(), g.inputs.end());
    for (uint32_t id : g.node_order) {
        const Node &n = g.node(id);
        if (home(n) != device) continue;
        st.node_order.push_back(id);
        st.nodes[id] = n;
        if (inputs.count(id)) {
            st.inputs.push_back(id);
            port_in[n.name] = id;
        }
    }
    CATNN_REQUIRE(!st.nodes.empty(), CATNN_ERR_UNKNOWN_REALIZATION,
                  "no node of graph " + g.name + " is placed on device " + device);
    for (const Edge &e : g.edges) {
        if (!st.nodes.count(e.dst)) continue;
        if (st.nodes.count(e.src)) {
            st.edges.push_back(e);
            continue;
        }
        auto it = recv_of.find(e.src);
        if (it == recv_of.end()) {
            const Node &src = g.node(e.src);
            Node r;
            r.id = next_id++;
            r.name = src.name + "#recv";
            std::memset(&r.op, 0, sizeof(r.op));
            r.op.kind = CATNN_OP_IDENTITY;
            r.output_ty = src.output_ty;
            CATNN_REQUIRE(!r.output_ty.dims.empty(), CATNN_ERR_SHAPE_MISMATCH,
                          "node " + src.name + " has no declared output type to receive");
            st.nodes[r.id] = r;
            st.node_order.push_back(r.id);
            st.inputs.push_back(r.id);
            port_in[r.name] = r.id;
            it = recv_of.emplace(e.src, r.id).first;
        }
        Edge re = e;
        re.src = it->second;
        st.edges.push_back(re);
    }
    std::set<uint32_t> outs;
    for (const Edge &e : g.edges)
        if (st.nodes.count(e.src) && !st.nodes.count(e.dst) && !recv_of.count(e.src)) outs.insert(e.src);
    for (uint32_t o : g.outputs)
        if (st.nodes.count(o)) outs.insert(o);
    for (uint32_t id : st.node_order)
        if (outs.count(id)) {
            st.outputs.push_back(id);
            port_out[st.nodes.at(id).name] = id;
        }
    if (st.outputs.empty()) {  // a stage whose values all stay local: its last node
        st.outputs.push_back(st.topo().back());
        port_out[st.nodes.at(st.outputs.back()).name] = st.outputs.back();
    }
    return st;
}

}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_graph_new(const char *name, catnn_graph **out) {
    return guard([&] {
        CATNN_REQUIRE(out, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        auto *g = new catnn_graph();
        g->name = name ? name : "";
        *out = g;
    });
}

int catnn_graph_free(catnn_graph *g) {
    return guard([&] { delete g; });
}

int catnn_graph_add_node(catnn_graph *g, const catnn_node *node) {
    return guard([&] {
        CATNN_REQUIRE(g, CATNN_ERR_INVALID_ARGUMENT, "null graph");
        Node n = node_from_c(node);
        if (!g->nodes.count(n.id)) g->node_order.push_back(n.id);
        g->nodes[n.id] = std::move(n);  // IndexMap::insert keeps the first position
    });
}

int catnn_graph_add_edge(catnn_graph *g, uint32_t src, uint32_t dst, const char *src_port,
                         const char *dst_port) {
    return guard([&] {
        CATNN_REQUIRE(g, CATNN_ERR_INVALID_ARGUMENT, "null graph");
        g->edges.push_back(Edge{src, dst, src_port ? src_port : "data", dst_port ? dst_port : "data"});
    });
}

int catnn_graph_add_input(catnn_graph *g, uint32_t id) {
    return guard([&] {
        CATNN_REQUIRE(g, CATNN_ERR_INVALID_ARGUMENT, "null graph");
        g->inputs.push_back(id);
    });
}

int catnn_graph_add_output(catnn_graph *g, uint32_t id) {
    return guard([&] {
        CATNN_REQUIRE(g, CATNN_ERR_INVALID_ARGUMENT, "null graph");
        g->outputs.push_back(id);
    });
}

int catnn_graph_add_fusion(catnn_graph *g, const char *const *op_names, int32_t n) {
    return guard([&] {
        CATNN_REQUIRE(g && n >= 0 && (n == 0 || op_names), CATNN_ERR_INVALID_ARGUMENT,
                      "null argument");
        std::vector<std::string> f;
        for (int32_t i = 0; i < n; ++i) f.emplace_back(op_names[i] ? op_names[i] : "");
        g->fusions.push_back(std::move(f));
    });
}

int catnn_graph_topo(const catnn_graph *g, uint32_t *order, int32_t cap, int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(g && n, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        const std::vector<uint32_t> o = g->topo();
        *n = (int32_t)o.size();
        for (int32_t i = 0; order && i < cap && i < (int32_t)o.size(); ++i) order[i] = o[(size_t)i];
    });
}

int catnn_hip_run_kernel(catnn_hip_device *dev, const catnn_node *node, const catnn_tensor *inputs,
                         int32_t n_inputs, catnn_tensor *out) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(out && n_inputs >= 0 && (n_inputs == 0 || inputs), CATNN_ERR_INVALID_ARGUMENT,
                      "null argument");
        const Node n = node_from_c(node);
        std::vector<HostTensor> ins;
        std::vector<std::vector<int64_t>> in_dims;
        for (int32_t i = 0; i < n_inputs; ++i) {
            ins.push_back(from_c(inputs[i], true));
            in_dims.push_back(ins.back().dims);
        }
        const std::vector<int64_t> od = infer_dims(n, in_dims);
        const int64_t n_out = numel_of(od);
        CATNN_REQUIRE(od.size() <= CATNN_MAX_RANK, CATNN_ERR_SHAPE_MISMATCH, "output rank > 8");
        int64_t cap = 1;
        for (int i = 0; i < out->rank; ++i) cap *= out->dims[i];
        CATNN_REQUIRE(out->rank >= 0 && cap >= n_out && (out->data || n_out == 0),
                      CATNN_ERR_SHAPE_MISMATCH,
                      "output buffer holds " + std::to_string(cap) + " values, node " + n.name +
                          " produces " + dims_str(od));
        // Lay out inputs, params, output and scratch in one device workspace.
        const uint64_t scr = scratch_bytes(n, in_dims);
        auto rnd = [](uint64_t b) { return (b + 255) & ~uint64_t(255); };
        uint64_t total = 0;
        std::vector<uint64_t> in_off, p_off;
        for (const auto &t : ins) { in_off.push_back(total); total += rnd((uint64_t)t.numel() * 4); }
        for (const auto &pr : n.params) { p_off.push_back(total); total += rnd((uint64_t)pr.second.numel() * 4); }
        const uint64_t out_off = total;
        total += rnd((uint64_t)n_out * 4);
        const uint64_t scr_off = total;
        total += rnd(scr);
        char *base = static_cast<char *>(workspace(dev, dev->moe_ws, std::max<uint64_t>(total, 256)));
        for (size_t i = 0; i < ins.size(); ++i)
            if (ins[i].numel())
                CATNN_HIP(hipMemcpyAsync(base + in_off[i], ins[i].data.data(), (size_t)ins[i].numel() * 4,
                                         hipMemcpyHostToDevice, dev->stream));
        for (size_t i = 0; i < n.params.size(); ++i)
            if (n.params[i].second.numel())
                CATNN_HIP(hipMemcpyAsync(base + p_off[i], n.params[i].second.data.data(),
                                         (size_t)n.params[i].second.numel() * 4,
                                         hipMemcpyHostToDevice, dev->stream));
        ExecArgs a;
        for (size_t i = 0; i < ins.size(); ++i) a.inputs.push_back(reinterpret_cast<float *>(base + in_off[i]));
        a.in_dims = in_dims;
        a.param = [&](const std::string &port) -> const float * {
            for (size_t i = 0; i < n.params.size(); ++i)
                if (n.params[i].first == port) return reinterpret_cast<float *>(base + p_off[i]);
            return nullptr;
        };
        a.out = reinterpret_cast<float *>(base + out_off);
        if (scr) {
            a.scratch = reinterpret_cast<float *>(base + scr_off);
            a.scratch_bytes = scr;
        }
        push_device_event(dev, n.name, CATNN_EV_KERNEL_START, 0);
        exec_node(dev, n, a);
        const size_t end_ev = push_device_event(dev, n.name, CATNN_EV_KERNEL_END, 0);
        if (n_out)
            CATNN_HIP(hipMemcpyAsync(out->data, base + out_off, (size_t)n_out * 4,
                                     hipMemcpyDeviceToHost, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
        out->rank = (int32_t)od.size();
        for (size_t i = 0; i < od.size(); ++i) out->dims[i] = od[i];
        out->dtype = ins.empty() ? n.output_ty.dtype : ins[0].dtype;
        dev->events[end_ev].checksum = fnv1a_f32(out->data, (uint64_t)n_out);
    });
}

int catnn_hip_run_node(catnn_hip_device *dev, const catnn_node *node, const char *const *in_ids,
                       const catnn_tensor *in_types, int32_t n_in, const char *out_id,
                       int32_t fused_act, const char *residual_id) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(out_id && n_in >= 0 && (n_in == 0 || (in_ids && in_types)),
                      CATNN_ERR_INVALID_ARGUMENT, "null argument");
        CATNN_REQUIRE(fused_act == 0 || fused_act == CATNN_OP_RELU || fused_act == CATNN_OP_GELU,
                      CATNN_ERR_INVALID_ARGUMENT, "fused_act must be 0, 2 (relu) or 3 (gelu)");
        const Node n = node_from_c(node, false);
        ExecArgs a;
        for (int32_t i = 0; i < n_in; ++i) {
            CATNN_REQUIRE(in_ids[i], CATNN_ERR_INVALID_ARGUMENT, "null input id");
            uint64_t cap = 0;
            a.inputs.push_back(static_cast<float *>(buffer(dev, in_ids[i], &cap)));
            a.in_dims.push_back(from_c(in_types[i], false).dims);
            CATNN_REQUIRE((uint64_t)numel_of(a.in_dims.back()) * 4 <= cap, CATNN_ERR_SHAPE_MISMATCH,
                          std::string("input buffer ") + in_ids[i] + " smaller than its type " +
                              dims_str(a.in_dims.back()));
        }
        uint64_t out_cap = 0;
        a.out = static_cast<float *>(buffer(dev, out_id, &out_cap));
        const std::vector<int64_t> od = infer_dims(n, a.in_dims);
        CATNN_REQUIRE((uint64_t)numel_of(od) * 4 <= out_cap, CATNN_ERR_SHAPE_MISMATCH,
                      std::string("output buffer ") + out_id + " too small for " + dims_str(od));
        a.param = [&](const std::string &port) -> const float * {
            auto it = dev->bindings.find("param:" + n.name + ":" + port);
            if (it == dev->bindings.end()) return nullptr;
            return reinterpret_cast<float *>(static_cast<char *>(dev->arena) + it->second.offset);
        };
        a.fused_act = fused_act;
        a.residual = residual_id ? static_cast<float *>(buffer(dev, residual_id)) : nullptr;
        const uint64_t scr = scratch_bytes(n, a.in_dims);
        if (scr) {
            a.scratch = static_cast<float *>(workspace(dev, dev->moe_ws, scr));
            a.scratch_bytes = scr;
        }
        push_device_event(dev, n.name, CATNN_EV_KERNEL_START, 0);
        exec_node(dev, n, a);
        const size_t end_ev = push_device_event(dev, n.name, CATNN_EV_KERNEL_END, 0);
        if (dev->trace_checksums) {
            const int64_t n_out = numel_of(od);
            std::vector<float> host((size_t)n_out);
            if (n_out)
                CATNN_HIP(hipMemcpyAsync(host.data(), a.out, (size_t)n_out * 4, hipMemcpyDeviceToHost,
                                         dev->stream));
            CATNN_HIP(hipStreamSynchronize(dev->stream));
            dev->events[end_ev].checksum = fnv1a_f32(host.data(), (uint64_t)n_out);
        }
    });
}

int catnn_hip_install(catnn_hip_device *dev, const catnn_graph *g, catnn_hip_program **out) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(g && out, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        auto *p = new catnn_hip_program();
        try {
            p->dev = dev;
            p->graph = *g;
            build_program(*p);
            plan_and_upload(*p);
        } catch (...) {
            if (p->base) (void)hipFree(p->base);
            delete p;
            throw;
        }
        *out = p;
    });
}

int catnn_hip_install_placed(catnn_hip_device *dev, const catnn_graph *g, const catnn_placement_entry *assign,
                             int32_t n_assign, const char *device_id, const char *default_device,
                             catnn_hip_program **out) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(g && out && device_id && default_device && (assign || n_assign == 0),
                      CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        std::map<std::string, std::string> a;
        for (int32_t i = 0; i < n_assign; ++i) {
            CATNN_REQUIRE(assign[i].op && assign[i].device, CATNN_ERR_INVALID_ARGUMENT, "null placement entry");
            a[assign[i].op] = assign[i].device;  // IndexMap::insert: a later entry replaces an earlier one
        }
        auto *p = new catnn_hip_program();
        try {
            p->dev = dev;
            p->placed = true;
            p->graph = stage_of(*g, a, device_id, default_device, p->port_in, p->port_out);
            build_program(*p);
            plan_and_upload(*p);
            p->step_done.assign(p->steps.size(), 0);
        } catch (...) {
            if (p->base) (void)hipFree(p->base);
            delete p;
            throw;
        }
        *out = p;
    });
}

int catnn_hip_program_ports(catnn_hip_program *p, char (*in_names)[CATNN_ID_CAP], int32_t in_cap, int32_t *n_in,
                            char (*out_names)[CATNN_ID_CAP], int32_t out_cap, int32_t *n_out) {
    return guard([&] {
        CATNN_REQUIRE(p && n_in && n_out, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        auto fill = [](const std::map<std::string, uint32_t> &m, const std::vector<uint32_t> &order,
                       const catnn_graph &g, char (*names)[CATNN_ID_CAP], int32_t cap, int32_t *n) {
            int32_t k = 0;
            for (uint32_t id : order) {
                const std::string &nm = g.node(id).name;
                if (!m.count(nm)) continue;
                if (names && k < cap) {
                    std::memset(names[k], 0, CATNN_ID_CAP);
                    std::strncpy(names[k], nm.c_str(), CATNN_ID_CAP - 1);
                }
                ++k;
            }
            *n = k;
        };
        std::map<std::string, uint32_t> in = p->port_in, outp = p->port_out;
        if (!p->placed) {  // an installed whole graph: its inputs and final output
            for (uint32_t v : p->input_vals) in[p->graph.node(v).name] = v;
            outp[p->graph.node(p->output_val).name] = p->output_val;
        }
        fill(in, p->graph.inputs, p->graph, in_names, in_cap, n_in);
        fill(outp, p->graph.outputs, p->graph, out_names, out_cap, n_out);
    });
}

int catnn_hip_program_new_pass(catnn_hip_program *p) {
    return guard([&] {
        CATNN_REQUIRE(p, CATNN_ERR_INVALID_ARGUMENT, "null program");
        p->have.clear();
        p->step_done.assign(p->steps.size(), 0);
    });
}

int catnn_hip_program_set_value(catnn_hip_program *p, const char *name, const catnn_tensor *value) {
    return guard([&] {
        CATNN_REQUIRE(p && name && value, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(p->dev);
        uint32_t id = UINT32_MAX;
        auto it = p->port_in.find(name);
        if (it != p->port_in.end()) id = it->second;
        for (uint32_t v : p->input_vals)
            if (!p->placed && p->graph.node(v).name == name) id = v;
        CATNN_REQUIRE(id != UINT32_MAX, CATNN_ERR_UNKNOWN_PORT,
                      std::string("unknown port ") + name + " on interface " + p->graph.name);
        const HostTensor in = from_c(*value, true);
        CATNN_REQUIRE(in.numel() == numel_of(p->dims[id]), CATNN_ERR_SHAPE_MISMATCH,
                      std::string(name) + ": " + dims_str(in.dims) + " vs " + dims_str(p->dims[id]));
        if (in.numel())
            CATNN_HIP(hipMemcpyAsync(p->ptr.at(act_id(id)), in.data.data(), (size_t)in.numel() * 4,
                                     hipMemcpyHostToDevice, p->dev->stream));
        CATNN_HIP(hipStreamSynchronize(p->dev->stream));  // the host tensor is borrowed for the call only
        p->have.insert(id);
    });
}

int catnn_hip_forward_wave(catnn_hip_program *p, int32_t *fired) {
    return guard([&] {
        CATNN_REQUIRE(p, CATNN_ERR_INVALID_ARGUMENT, "null program");
        require_device(p->dev);
        if (p->step_done.size() != p->steps.size()) p->step_done.assign(p->steps.size(), 0);
        const int n = forward_wave(*p);
        if (fired) *fired = n;
    });
}

int catnn_hip_program_get_value(catnn_hip_program *p, const char *name, catnn_tensor *out) {
    return guard([&] {
        CATNN_REQUIRE(p && name && out, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(p->dev);
        uint32_t id = UINT32_MAX;
        auto it = p->port_out.find(name);
        if (it != p->port_out.end()) id = it->second;
        if (!p->placed && p->graph.node(p->output_val).name == name) id = p->output_val;
        CATNN_REQUIRE(id != UINT32_MAX, CATNN_ERR_UNKNOWN_PORT,
                      std::string("unknown port ") + name + " on interface " + p->graph.name);
        CATNN_REQUIRE(!p->placed || p->have.count(id), CATNN_ERR_WIRING,
                      std::string(name) + " has not been computed in this pass");
        const auto &od = p->dims[id];
        const int64_t n = numel_of(od);
        int64_t cap = 1;
        for (int i = 0; i < out->rank; ++i) cap *= out->dims[i];
        CATNN_REQUIRE(cap >= n && (out->data || n == 0), CATNN_ERR_SHAPE_MISMATCH,
                      "output buffer holds " + std::to_string(cap) + " values, " + name + " has " + dims_str(od));
        if (n)
            CATNN_HIP(hipMemcpyAsync(out->data, p->ptr.at(act_id(id)), (size_t)n * 4, hipMemcpyDeviceToHost,
                                     p->dev->stream));
        CATNN_HIP(hipStreamSynchronize(p->dev->stream));
        check_embed_flag(*p);
        out->rank = (int32_t)od.size();
        for (size_t i = 0; i < od.size(); ++i) out->dims[i] = od[i];
        out->dtype = CATNN_F32;
    });
}

int catnn_hip_program_free(catnn_hip_program *p) {
    return guard([&] {
        if (!p) return;
        (void)hipSetDevice(p->dev->ordinal);
        (void)hipStreamSynchronize(p->dev->stream);
        destroy_events(*p);
        if (p->base) (void)hipFree(p->base);
        if (p->embed_flag_host) (void)hipHostFree(p->embed_flag_host);
        delete p;
    });
}

int catnn_hip_program_profile(catnn_hip_program *p, int32_t enable) {
    return guard([&] {
        CATNN_REQUIRE(p, CATNN_ERR_INVALID_ARGUMENT, "null program");
        require_device(p->dev);
        collect_timings(*p);
        p->profiling = enable != 0;
        std::fill(p->total_ms.begin(), p->total_ms.end(), 0.0);
        std::fill(p->calls.begin(), p->calls.end(), 0);
    });
}

int catnn_hip_program_timings(catnn_hip_program *p, catnn_step_timing *out, int32_t cap,
                              int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(p && n, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(p->dev);
        collect_timings(*p);
        *n = (int32_t)p->exec_steps.size();
        for (int32_t i = 0; out && i < cap && i < *n; ++i) {
            const Node &node = p->graph.node(p->steps[p->exec_steps[(size_t)i]].node);
            std::memset(out[i].name, 0, CATNN_ID_CAP);
            std::strncpy(out[i].name, node.name.c_str(), CATNN_ID_CAP - 1);
            out[i].kind = node.op.kind;
            out[i].calls = p->calls[(size_t)i];
            out[i].total_ms = p->total_ms[(size_t)i];
        }
    });
}

int catnn_hip_forward_resident(catnn_hip_program *p) {
    return guard([&] {
        CATNN_REQUIRE(p, CATNN_ERR_INVALID_ARGUMENT, "null program");
        require_device(p->dev);
        run_program(*p);
    });
}

int catnn_hip_program_check(catnn_hip_program *p) {
    return guard([&] {
        CATNN_REQUIRE(p, CATNN_ERR_INVALID_ARGUMENT, "null program");
        require_device(p->dev);
        CATNN_HIP(hipStreamSynchronize(p->dev->stream));
        check_embed_flag(*p);
    });
}

int catnn_hip_forward(catnn_hip_program *p, const catnn_tensor *input, catnn_tensor *output) {
    return guard([&] {
        CATNN_REQUIRE(p && output, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(p->dev);
        catnn_hip_device *dev = p->dev;
        if (!p->input_vals.empty()) {
            CATNN_REQUIRE(input, CATNN_ERR_INVALID_ARGUMENT, "graph has inputs but none given");
            const HostTensor in = from_c(*input, true);
            for (uint32_t v : p->input_vals) {
                CATNN_REQUIRE(in.numel() == numel_of(p->dims[v]), CATNN_ERR_SHAPE_MISMATCH,
                              "input " + dims_str(in.dims) + " vs graph input " + dims_str(p->dims[v]));
                if (in.numel())
                    CATNN_HIP(hipMemcpyAsync(p->ptr.at(act_id(v)), in.data.data(), (size_t)in.numel() * 4,
                                             hipMemcpyHostToDevice, dev->stream));
            }
        }
        run_program(*p);
        const auto &od = p->dims[p->output_val];
        const int64_t n_out = numel_of(od);
        int64_t cap = 1;
        for (int i = 0; i < output->rank; ++i) cap *= output->dims[i];
        CATNN_REQUIRE(cap >= n_out && (output->data || n_out == 0), CATNN_ERR_SHAPE_MISMATCH,
                      "output buffer holds " + std::to_string(cap) + " values, graph produces " +
                          dims_str(od));
        if (n_out)
            CATNN_HIP(hipMemcpyAsync(output->data, p->ptr.at(act_id(p->output_val)), (size_t)n_out * 4,
                                     hipMemcpyDeviceToHost, dev->stream));
        CATNN_HIP(hipStreamSynchronize(dev->stream));
        check_embed_flag(*p);
        output->rank = (int32_t)od.size();
        for (size_t i = 0; i < od.size(); ++i) output->dims[i] = od[i];
        output->dtype = CATNN_F32;
    });
}

int catnn_hip_program_io(catnn_hip_program *p, void **in_dptr, uint64_t *in_bytes, void **out_dptr,
                         uint64_t *out_bytes) {
    return guard([&] {
        CATNN_REQUIRE(p, CATNN_ERR_INVALID_ARGUMENT, "null program");
        if (in_dptr) *in_dptr = p->input_vals.empty() ? nullptr : p->ptr.at(act_id(p->input_vals[0]));
        if (in_bytes)
            *in_bytes = p->input_vals.empty() ? 0 : (uint64_t)numel_of(p->dims[p->input_vals[0]]) * 4;
        if (out_dptr) *out_dptr = p->ptr.at(act_id(p->output_val));
        if (out_bytes) *out_bytes = (uint64_t)numel_of(p->dims[p->output_val]) * 4;
    });
}

int catnn_hip_program_arena(catnn_hip_program *p, catnn_arena_alloc *out, int32_t cap, int32_t *n,
                            uint64_t *reserved_bytes) {
    return guard([&] {
        CATNN_REQUIRE(p && n, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *n = (int32_t)p->plan.size();
        if (reserved_bytes) *reserved_bytes = p->reserved;
        for (int32_t i = 0; out && i < cap && i < (int32_t)p->plan.size(); ++i) {
            const auto &a = p->plan[(size_t)i];
            std::memset(out[i].id, 0, CATNN_ID_CAP);
            std::strncpy(out[i].id, a.id.c_str(), CATNN_ID_CAP - 1);
            out[i].bytes = a.bytes;
            out[i].offset = a.offset;
            out[i].live_from = a.live_from;
            out[i].live_to = a.live_to;
        }
    });
}

}  // extern "C"
