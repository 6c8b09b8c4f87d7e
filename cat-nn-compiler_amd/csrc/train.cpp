// Training step of an IrGraph on one device: the device counterpart of
// pipeline::reference_train (crates/catnn-compile/src/pipeline.rs:476-547)
// for one step with MSE and SGD, i.e. of the three seams that bypass the
// handler in the reference's training wave — adjoint_of (coord.rs:413),
// rematerialisation (coord.rs:470, not needed: every tape is kept) and
// apply_update (coord.rs:481).
//
//   forward   topo order; every op stores the tape its adjoint needs;
//   loss      as loss_and_grad picks it (pipeline.rs:430-451): cross-entropy
//             against class ids when the output node is an LmHead
//             (adjoint.rs:123-145), else MSE against the target
//             (adjoint.rs:106-119);
//   backward  reverse topo order, adjoint_of per node (adjoint.rs:762-951);
//             a value's cotangent is written by the first of its consumers
//             to run and accumulated by the others (add_tensors,
//             adjoint.rs:22-24);
//   update    the optimizer on the fp32 master weights — Sgd::put
//             (lens/optim.rs:32-42) or Adam::put (:95-118) with its moments
//             resident beside them, as apply_update (pipeline.rs:455-472)
//             chooses — then the bf16 copies are refreshed.
//
// Precision: every GEMM runs on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation.  Linear, MatMul, LmHead and the dense SwiGLU take bf16
// operands.  The attention projections take split-bf16 operands (hi|lo|hi
// against hi|hi|lo over 3K: the fp32 product to ~2⁻¹⁶): with plain bf16
// there the gradients of wq and wk move about 1.3× further from the fp32
// path.  The MoE gate/up GEMM takes its input split (hi|lo against the
// weights' hi|hi, 2K: x at split precision, the expert weights rounded
// once), because the rounding of its input reaches the router's gradient;
// the rest of the MoE expert forward and every backward GEMM take plain
// bf16 operands.  The attention core (d_head 64) runs on bf16 MFMA with
// q, k, v, the normalised P, dO and dS rounded (attention_bf16.hip); other
// head sizes on fp32 MFMA.  Master weights, the residual stream, LayerNorm,
// softmax statistics, the router and all cotangent accumulation stay fp32.
//
// Memory: every buffer (params, their bf16 copies and gradients, values,
// cotangents, tapes, scratch) is a BufferReq on the reference's logical
// ticks (pipeline.rs:280-284: forward = topo index t, loss = n, backward of
// t = 2n − t, update = 2n + 1), placed by place_arena and backed by one
// hipMalloc — the arena of schedule_device (pipeline.rs:272-401) made real.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <set>

#include "arena.hpp"
#include "gemm_bf16.hpp"
#include "graph.hpp"
#include "kernels.hpp"
#include "train_ops.hpp"

namespace catnn {

using k::bf16_t;

namespace {

int64_t numel(const std::vector<int64_t> &d) {
    int64_t n = 1;
    for (int64_t v : d) n *= v;
    return n;
}

constexpr int kPad = 128;  // MoE expert segments start on multiples of the GEMM tile

// The MoE gate/up B operand wraps its k index at H (whole 64-deep chunks).
bool moe_kwrap(int64_t H) { return H % 64 == 0; }

// The bf16 step runs an Attention node's core on bf16 MFMA (attention_bf16.hip)
// where that kernel covers its head size; q, k, v then live as bf16.
bool attn_core_bf16(const Node &nd, int64_t D) {
    return nd.op.kind == CATNN_OP_ATTENTION && k::attention_bf16_supported(nd.op.a[2], 3 * D);
}

struct TParam {
    std::string name;       // "param:{node}:{port}"
    int64_t rows = 0, cols = 0;
    std::vector<float> init;  // host values uploaded at install
    bool want_b = false, want_bt = false, want_bt3 = false;
    // Row stride of the bf16 copy b (0: cols).  b_with: b lives inside that
    // parameter's copy, b_col columns in (MoE w1 | w3 rows side by side, the
    // B operand of one input-gradient GEMM over both).
    int64_t b_ld = 0, b_col = 0;
    TParam *b_with = nullptr;
    float *master = nullptr, *grad = nullptr;
    float *m = nullptr, *v = nullptr;  // Adam moments "adam:{node}:{port}:m|v"
    bf16_t *b = nullptr, *bt = nullptr;
    bf16_t *bt3 = nullptr;  // [cols, 3·rows] split-bf16 transposed copy (hi | hi | lo)
    // fp32 precision: six-part split copies in the B role, of the rows
    // ([rows, 6·cols], the input-gradient GEMM) and of the columns
    // ([cols, 6·rows], the forward).
    bool want_b6 = false, want_bt6 = false;
    bf16_t *b6 = nullptr, *bt6 = nullptr;
    // Held as the transpose of the graph's tensor (LmHead's w [V, H] is kept
    // as wᵀ [H, V], a Linear weight, as adjoint.rs:903-913 transposes it);
    // reads transpose back.
    bool transposed = false;
};

struct TNode {
    uint32_t id;
    const Node *node;
    size_t tick;
    int kind;
    std::vector<uint32_t> ins;
    std::vector<std::vector<int64_t>> in_dims;
    std::vector<bool> first_writer;  // per input: this adjoint overwrites the cotangent
    // Linear(A) → GELU → Linear(B) with single consumers: B's input-gradient
    // GEMM applies gelu'(A's output) in its epilogue and writes A's cotangent
    // (fp32 and its bf16 copy); the GELU node's adjoint is then skipped.
    bool skip_bwd = false;         // this GELU node's adjoint runs inside B's GEMM
    uint32_t gelu_pre = UINT32_MAX;  // on B: the Linear A before the GELU
    bool dyb_ready = false;        // on A: its bf16 cotangent is written by B
    // The forward of the same pattern: A's GEMM epilogue applies the GELU
    // and writes B's bf16 input operand (its "xb" tape) directly; the GELU
    // node's forward and B's cast are skipped.
    bool skip_fwd = false;            // on the GELU node
    uint32_t gelu_next = UINT32_MAX;  // on A: B
    bool xb_ready = false;            // on B
    size_t xb_from = 0;               // on B: the tick its xb tape is written (A's)
    // LayerNorm → its only consumer: the LN forward writes the consumer's
    // GEMM operand (a Linear's bf16 "xb", an attention's split-bf16 "x3")
    // instead of its fp32 output, which nothing else reads.
    uint32_t ln_next = UINT32_MAX;    // on the LayerNorm
    bool x3_ready = false;            // on the attention node
    size_t x3_from = 0;
    // GEMM → Add (its only consumer): the GEMM's epilogue adds the other
    // addend and writes the Add's value; the Add's forward is skipped and
    // its value is live from the GEMM's tick.
    uint32_t res_into = UINT32_MAX, res_other = UINT32_MAX;  // on the GEMM node
    size_t val_from = SIZE_MAX;       // on the Add: the tick its value is written
    std::vector<int64_t> dims;
    std::map<std::string, TParam *> params;
    // tapes and scratch (named pointers, assigned after planning)
    std::map<std::string, void *> buf;
    void *&B(const std::string &n) { return buf[n]; }
};

}  // namespace
}  // namespace catnn

struct catnn_hip_trainer {
    catnn_hip_device *dev = nullptr;
    float *sk_part = nullptr;  // the device's stream-K scratch for the bf16 GEMMs
    catnn_graph graph;
    float lr = 0.05f;
    int opt = CATNN_OPT_SGD;
    int prec = CATNN_PREC_BF16;
    uint64_t arena_cap = 0;  // 0: the device's memory
    // Residual adds and LayerNorm outputs fused into the neighbouring GEMMs
    // (their values are then not recomputable); off when a capped arena
    // needs more checkpoints than the fused plan offers.
    bool fuse_values = true;
    uint64_t adam_t = 0;  // AdamState.t shared by every trained parameter
    // Activation checkpoints (schedule.rs:155-212): value id → where its
    // forward buffer ends and where the recomputed copy lives.
    struct Ckpt {
        size_t req = 0;            // index of act:{id} in reqs
        uint64_t fwd_last = 0;     // last forward tick that reads the value
        uint64_t bwd_first = 0;    // first backward tick that reads it
        size_t first_reader = 0;   // nodes[] index of the node whose backward runs at bwd_first
    };
    std::map<uint32_t, Ckpt> ckpt_candidates, ckpt;
    std::map<uint32_t, float *> val_fwd, val_recomp;  // per checkpointed value
    bool input_grads = false;  // keep the graph inputs' cotangents (run_adjoint)
    std::vector<catnn::TNode> nodes;
    std::map<uint32_t, size_t> index;                 // node id → nodes[]
    std::vector<std::unique_ptr<catnn::TParam>> params;
    std::map<uint32_t, float *> val, grad;            // value / cotangent per node id
    std::map<uint32_t, std::vector<int64_t>> dims;
    std::set<uint32_t> input_ids;
    std::set<uint32_t> has_grad;  // ids whose cotangent some adjoint (or the loss) writes
    uint32_t out_id = 0;
    bool classes = false;  // the output is an LmHead: TrainTarget::Classes, cross-entropy
    int64_t class_rows = 0, vocab = 0;
    uint32_t *class_ids = nullptr;
    float *target = nullptr, *loss = nullptr, *mse_scratch = nullptr, *ce_rows = nullptr;
    catnn::k::SgdParam *sgd_table = nullptr;  // device copy of every parameter's update entry
    int sgd_n = 0, sgd_tiles = 0;
    std::vector<catnn::BufferReq> reqs;
    std::vector<void **> req_slot;
    std::vector<catnn::ArenaAlloc> plan;
    void *base = nullptr;
    uint64_t reserved = 0;
};

namespace catnn {

namespace {

using Tr = catnn_hip_trainer;

void request(Tr &t, const std::string &id, uint64_t bytes, uint64_t from, uint64_t to, void **slot) {
    t.reqs.push_back(BufferReq{id, (bytes + 255) & ~uint64_t(255), from, to, false});
    t.req_slot.push_back(slot);
}

// The stream-K scratch of the trainer whose step (or adjoint pass) this
// thread is running, for every GEMM it launches (SkScope sets it).
thread_local float *tl_sk_part = nullptr;

struct SkScope {
    float *prev;
    explicit SkScope(float *p) : prev(tl_sk_part) { tl_sk_part = p; }
    ~SkScope() { tl_sk_part = prev; }
};

k::GemmBf16Params gp() {
    k::GemmBf16Params p{};
    p.a_row_div = 1;
    p.sk_part = tl_sk_part;
    return p;
}

// The device's stream-K scratch (allocated on first use, freed with the device).
float *device_sk_scratch(catnn_hip_device *dev) {
    if (!dev->sk_ws.ptr) {
        const uint64_t bytes = (uint64_t)k::gemm_bf16_sk_floats() * 4;
        CATNN_HIP(hipMalloc(&dev->sk_ws.ptr, bytes));
        dev->sk_ws.bytes = bytes;
    }
    return (float *)dev->sk_ws.ptr;
}

// Bytes of split-K partial sums gemm_nt needs for an M×N×K product (at
// least one 256-byte block, so that the request is never empty).
uint64_t wparts_bytes(int64_t M, int64_t N, int64_t K) {
    const int sp = k::gemm_bf16_splitk(M, N, K);
    return sp > 1 ? (uint64_t)sp * M * N * 4 : 256;
}

// C32 (=/+=) A[M,K]·B[N,K]ᵀ on bf16 operands.  With `wparts` (wparts_bytes
// of scratch) a grid too small for the GPU is split along K: each segment
// stores its partial product there and sum_parts adds them into C in order.
void gemm_nt(hipStream_t s, const bf16_t *A, int64_t lda, const bf16_t *B, int64_t ldb, int M, int N,
             int K, float *C, int64_t ldc, bool accumulate, float *wparts = nullptr) {
    const int sp = wparts ? k::gemm_bf16_splitk(M, N, K) : 1;
    if (sp > 1 && ldc == N) {
        k::GemmBf16Params p = gp();
        p.A = A;
        p.lda = lda;
        p.B = B;
        p.ldb = ldb;
        p.M = M;
        p.N = N;
        p.K = K;
        p.epi = k::EPI_STORE;
        p.ldc32 = N;
        p.grid = k::GRID_SEGK;
        p.ksplit = k::gemm_bf16_splitk_len(K, sp);
        p.segk_aligned = p.ksplit % 8 == 0;
        p.n_experts = sp;
        for (int e = 0; e < sp; ++e) p.C_e[e] = wparts + (int64_t)e * M * N;
        k::gemm_bf16_launch(s, p);
        k::sum_parts(s, wparts, sp, (int64_t)M * N, C, accumulate);
        return;
    }
    k::GemmBf16Params p = gp();
    p.A = A;
    p.lda = lda;
    p.B = B;
    p.ldb = ldb;
    p.M = M;
    p.N = N;
    p.K = K;
    p.epi = k::EPI_STORE;
    p.C32 = C;
    p.ldc32 = ldc;
    p.accumulate = accumulate ? 1 : 0;
    k::gemm_bf16_launch(s, p);
}

void add_into(hipStream_t s, float *dst, const float *src, int64_t n, bool overwrite) {
    if (overwrite) k::copy_f32(s, src, dst, n);
    else k::add_f32(s, dst, src, dst, n, n);
}

// The host values of trainer parameter `port` of node `nd`, in the layout
// the trainer keeps it: Attention's "wqkv" packs [wq | wk | wv] per row
// ([D, 3D]); LmHead's "w" [V, H] is held as wᵀ [H, V]; every other port is
// the node's tensor as it is.
std::vector<float> param_values(const Node &nd, const std::string &port) {
    auto host = [&](const std::string &p) {
        const HostTensor *h = nd.param(p);
        if (!h) fail(CATNN_ERR_UNKNOWN_PORT, "unknown port " + p + " on interface " + nd.name);
        return h;
    };
    if ((nd.op.kind == CATNN_OP_ATTENTION || nd.op.kind == CATNN_OP_GQA_ATTENTION) && port == "wqkv") {
        // [wq | wk | wv] per row: widths QW, KW, KW (Attention: all D).
        const HostTensor *wq = host("wq"), *wk = host("wk"), *wv = host("wv");
        CATNN_REQUIRE(wq->dims.size() == 2 && wk->dims.size() == 2 && wv->dims == wk->dims &&
                          wk->dims[0] == wq->dims[0],
                      CATNN_ERR_SHAPE_MISMATCH, "attention projections");
        const int64_t D = wq->dims[0], QW = wq->dims[1], KW = wk->dims[1], LD = QW + 2 * KW;
        std::vector<float> packed((size_t)(D * LD));
        for (int64_t r = 0; r < D; ++r) {
            std::memcpy(&packed[(size_t)(r * LD)], &wq->data[(size_t)(r * QW)], (size_t)QW * 4);
            std::memcpy(&packed[(size_t)(r * LD + QW)], &wk->data[(size_t)(r * KW)], (size_t)KW * 4);
            std::memcpy(&packed[(size_t)(r * LD + QW + KW)], &wv->data[(size_t)(r * KW)], (size_t)KW * 4);
        }
        return packed;
    }
    if (nd.op.kind == CATNN_OP_LM_HEAD && port == "w") {
        const HostTensor *w = host("w");
        const int64_t V = nd.op.a[1], K = nd.op.a[0];
        CATNN_REQUIRE(w->numel() == V * K, CATNN_ERR_SHAPE_MISMATCH, "lm_head w");
        std::vector<float> wt((size_t)(V * K));
        for (int64_t v = 0; v < V; ++v)
            for (int64_t h = 0; h < K; ++h) wt[(size_t)(h * V + v)] = w->data[(size_t)(v * K + h)];
        return wt;
    }
    return host(port)->data;
}

}  // namespace

static void refresh_split_copies(Tr &t);

static void plan_trainer(Tr &t) {
    const catnn_graph &g = t.graph;
    const std::vector<uint32_t> order = g.topo();
    const uint64_t n = order.size();
    auto bwd = [&](uint64_t tick) { return 2 * n - tick; };
    const uint64_t upd = 2 * n + 1;
    CATNN_REQUIRE(!g.outputs.empty(), CATNN_ERR_WIRING, "graph has no outputs");
    t.out_id = g.outputs.back();
    t.input_ids.insert(g.inputs.begin(), g.inputs.end());
    for (size_t i = 0; i < order.size(); ++i) t.index[order[i]] = i;

    // Shapes and nodes.
    t.nodes.reserve(order.size());
    for (size_t i = 0; i < order.size(); ++i) {
        const uint32_t id = order[i];
        const Node &nd = g.node(id);
        TNode tn;
        tn.id = id;
        tn.node = &nd;
        tn.tick = i;
        tn.kind = nd.op.kind;
        if (t.input_ids.count(id)) {
            tn.dims = nd.output_ty.dims;
        } else {
            tn.ins = g.preds(id);
            for (uint32_t v : tn.ins) tn.in_dims.push_back(t.dims.at(v));
            tn.dims = infer_dims(nd, tn.in_dims);
            switch (tn.kind) {
                case CATNN_OP_IDENTITY: case CATNN_OP_RESHAPE: case CATNN_OP_TRANSPOSE:
                case CATNN_OP_RELU: case CATNN_OP_GELU: case CATNN_OP_LINEAR: case CATNN_OP_MATMUL:
                case CATNN_OP_LAYER_NORM: case CATNN_OP_ATTENTION: case CATNN_OP_MOE:
                case CATNN_OP_LM_HEAD: case CATNN_OP_RMS_NORM: case CATNN_OP_EMBEDDING:
                case CATNN_OP_SWIGLU: case CATNN_OP_GQA_ATTENTION:
                    break;
                case CATNN_OP_MIX:
                    CATNN_REQUIRE(tn.ins.size() == 2, CATNN_ERR_WIRING, "mix adjoint needs two inputs");
                    CATNN_REQUIRE(numel(tn.in_dims[0]) == numel(tn.in_dims[1]), CATNN_ERR_SHAPE_MISMATCH,
                                  "mix operands differ");
                    break;
                case CATNN_OP_SOFTMAX:
                    break;
                case CATNN_OP_ROUTER:  // adjoint.rs:915-920
                    fail(CATNN_ERR_UNLAWFUL,
                         "router adjoint is the straight-through estimator inside MoE, not a standalone op");
                case CATNN_OP_MUL:
                    CATNN_REQUIRE(tn.ins.size() != 2 || numel(tn.in_dims[0]) == numel(tn.in_dims[1]),
                                  CATNN_ERR_SHAPE_MISMATCH, "mul operands differ");
                    break;
                case CATNN_OP_ADD: case CATNN_OP_RESIDUAL_ADD:
                    CATNN_REQUIRE(tn.ins.size() != 2 || numel(tn.in_dims[0]) == numel(tn.in_dims[1]),
                                  CATNN_ERR_UNSUPPORTED,
                                  "training: broadcast add (" + nd.name + ") has no device adjoint");
                    break;
                default:
                    fail(CATNN_ERR_UNSUPPORTED, "training: op " + op_name(tn.kind) + " (node " + nd.name +
                                                    ") has no device adjoint");
            }
        }
        t.dims[id] = tn.dims;
        t.nodes.push_back(std::move(tn));
    }
    // Which cotangents exist: the output's, and (backwards) every input of a
    // node that itself has one.
    t.has_grad.insert(t.out_id);
    for (auto it = t.nodes.rbegin(); it != t.nodes.rend(); ++it)
        if (t.has_grad.count(it->id))
            for (uint32_t v : it->ins) t.has_grad.insert(v);
    // Who writes each cotangent first: consumers run their adjoints in reverse
    // topo order, so the consumer with the largest tick writes first.
    std::map<uint32_t, size_t> first_consumer_tick;
    for (auto &tn : t.nodes)
        for (uint32_t v : tn.ins) {
            if (!t.has_grad.count(tn.id)) continue;  // skipped in the backward pass
            auto it = first_consumer_tick.find(v);
            if (it == first_consumer_tick.end() || tn.tick > it->second) first_consumer_tick[v] = tn.tick;
        }
    for (auto &tn : t.nodes) {
        std::set<uint32_t> seen;
        for (uint32_t v : tn.ins) {
            // Only the first occurrence of v in this node's inputs may overwrite.
            const bool first = first_consumer_tick[v] == tn.tick && !seen.count(v);
            tn.first_writer.push_back(first);
            seen.insert(v);
        }
    }

    // GELU adjoints fused into the next Linear's input-gradient GEMM.
    std::map<uint32_t, std::vector<uint32_t>> consumers;
    for (auto &tn : t.nodes)
        for (uint32_t v : tn.ins) consumers[v].push_back(tn.id);
    auto is_linear = [&](const TNode &x) { return x.kind == CATNN_OP_LINEAR || x.kind == CATNN_OP_MATMUL; };
    std::map<uint32_t, uint64_t> grad_from;  // cotangents first written earlier than their first consumer
    for (auto &gn : t.nodes) {
        if (t.prec != CATNN_PREC_BF16) break;  // the fused epilogue writes the bf16 operand of the bf16 path
        if (gn.kind != CATNN_OP_GELU || gn.ins.size() != 1 || gn.id == t.out_id || !t.has_grad.count(gn.id)) continue;
        const uint32_t a = gn.ins[0];
        const auto &ca = consumers[a], &cg = consumers[gn.id];
        if (ca.size() != 1 || cg.size() != 1 || t.input_ids.count(a) || a == t.out_id) continue;
        TNode &an = t.nodes[t.index.at(a)], &bn = t.nodes[t.index.at(cg[0])];
        if (!is_linear(an) || !is_linear(bn) || bn.ins.size() != 1 || !t.has_grad.count(bn.id)) continue;
        gn.skip_bwd = true;
        bn.gelu_pre = a;
        an.dyb_ready = true;
        grad_from[a] = bwd(bn.tick);
        if (an.kind == CATNN_OP_LINEAR || an.kind == CATNN_OP_MATMUL) {
            gn.skip_fwd = true;
            an.gelu_next = bn.id;
            bn.xb_ready = true;
            bn.xb_from = an.tick;
        }
    }

    for (auto &an : t.nodes) {
        if (t.prec != CATNN_PREC_BF16 || !t.fuse_values) break;
        if ((an.kind != CATNN_OP_ADD && an.kind != CATNN_OP_RESIDUAL_ADD) || an.ins.size() != 2 ||
            an.ins[0] == an.ins[1] || an.dims != t.dims[an.ins[0]] || an.dims != t.dims[an.ins[1]])
            continue;
        for (int j = 0; j < 2; ++j) {
            const uint32_t g = an.ins[j], o = an.ins[1 - j];
            if (t.input_ids.count(g) || g == t.out_id || consumers[g].size() != 1) continue;
            TNode &gn = t.nodes[t.index.at(g)];
            const bool gemm = (is_linear(gn) && gn.gelu_next == UINT32_MAX) ||
                              (gn.kind == CATNN_OP_ATTENTION && attn_core_bf16(*gn.node, gn.in_dims[0].back()));
            // the other addend must exist when the GEMM runs
            const bool ready = t.input_ids.count(o) || t.nodes[t.index.at(o)].tick < gn.tick;
            if (!gemm || !ready) continue;
            gn.res_into = an.id;
            gn.res_other = o;
            an.skip_fwd = true;
            an.val_from = gn.tick;
            break;
        }
    }

    for (auto &ln : t.nodes) {
        if (t.prec != CATNN_PREC_BF16 || !t.fuse_values) break;
        if (ln.kind != CATNN_OP_LAYER_NORM || ln.id == t.out_id || t.input_ids.count(ln.id)) continue;
        const auto &cs = consumers[ln.id];
        if (cs.size() != 1) continue;
        TNode &cn = t.nodes[t.index.at(cs[0])];
        if (cn.ins.size() != 1) continue;
        if (is_linear(cn) && !cn.xb_ready) {
            ln.ln_next = cn.id;
            cn.xb_ready = true;
            cn.xb_from = ln.tick;
        } else if (cn.kind == CATNN_OP_ATTENTION || cn.kind == CATNN_OP_GQA_ATTENTION) {
            ln.ln_next = cn.id;
            cn.x3_ready = true;
            cn.x3_from = ln.tick;
        }
    }

    // Values and cotangents.
    std::map<uint32_t, uint64_t> last_read;  // last tick a value is read
    for (auto &tn : t.nodes) {
        last_read[tn.id] = std::max<uint64_t>(last_read[tn.id], tn.tick);
        // softmax_backward reads the forward output (adjoint.rs:92-104).
        if (tn.kind == CATNN_OP_SOFTMAX) last_read[tn.id] = std::max<uint64_t>(last_read[tn.id], bwd(tn.tick));
        for (uint32_t v : tn.ins) last_read[v] = std::max<uint64_t>(last_read[v], bwd(tn.tick));
    }
    // The output value stays readable after the step (catnn_hip_train_read_value).
    last_read[t.out_id] = upd;
    // Values that may be checkpointed: produced by a node (not a graph
    // input, not the output the loss reads), read again in the backward
    // pass, by a producer whose forward uses no forward-only scratch (it is
    // re-run at the first backward tick that reads the value).
    std::map<uint32_t, uint64_t> fwd_last, bwd_first;
    std::map<uint32_t, size_t> first_reader;
    auto bwd_read = [&](uint32_t v, size_t i) {
        const uint64_t b = bwd(t.nodes[i].tick);
        if (!bwd_first.count(v) || b < bwd_first[v]) {
            bwd_first[v] = b;
            first_reader[v] = i;
        }
    };
    for (size_t i = 0; i < t.nodes.size(); ++i) {
        const TNode &tn = t.nodes[i];
        for (uint32_t v : tn.ins) {
            fwd_last[v] = std::max<uint64_t>(fwd_last[v], tn.tick);
            bwd_read(v, i);
        }
        if (tn.kind == CATNN_OP_SOFTMAX) bwd_read(tn.id, i);  // softmax_backward reads its own output
        if (tn.gelu_pre != UINT32_MAX) bwd_read(tn.gelu_pre, i);  // the fused GELU adjoint reads A's output
    }
    for (auto &tn : t.nodes) {
        const uint64_t bytes = (uint64_t)numel(tn.dims) * 4;
        // The batch (inputs and target) stays resident across steps: set_batch
        // once, step many times.
        const bool is_input = t.input_ids.count(tn.id) != 0;
        const bool fscratch_fwd = t.prec == CATNN_PREC_FP32 &&
            (tn.kind == CATNN_OP_LINEAR || tn.kind == CATNN_OP_MATMUL || tn.kind == CATNN_OP_LM_HEAD ||
             tn.kind == CATNN_OP_SWIGLU || tn.kind == CATNN_OP_ATTENTION || tn.kind == CATNN_OP_GQA_ATTENTION ||
             tn.kind == CATNN_OP_MOE);
        // Values a fused forward writes elsewhere (or in another node's
        // epilogue) are not recomputed.
        const bool fused = tn.skip_fwd || tn.res_into != UINT32_MAX || tn.ln_next != UINT32_MAX;
        if (!is_input && tn.id != t.out_id && !fscratch_fwd && !fused && fwd_last.count(tn.id) &&
            last_read[tn.id] > fwd_last[tn.id] && bwd_first.count(tn.id)) {
            catnn_hip_trainer::Ckpt c;
            c.req = t.reqs.size();
            c.fwd_last = fwd_last[tn.id];
            c.bwd_first = bwd_first[tn.id];
            c.first_reader = first_reader[tn.id];
            t.ckpt_candidates[tn.id] = c;
        }
        request(t, "act:" + std::to_string(tn.id), bytes, is_input ? 0 : std::min<size_t>(tn.tick, tn.val_from),
                is_input ? upd : last_read[tn.id], reinterpret_cast<void **>(&t.val[tn.id]));
        if (is_input) {
            // An input's cotangent, when kept, stays readable after the pass.
            if (t.input_grads && first_consumer_tick.count(tn.id))
                request(t, "grad:" + std::to_string(tn.id), bytes, bwd(first_consumer_tick[tn.id]), upd,
                        reinterpret_cast<void **>(&t.grad[tn.id]));
            continue;
        }
        uint64_t from = tn.id == t.out_id ? n : bwd(first_consumer_tick.count(tn.id) ? first_consumer_tick[tn.id] : tn.tick);
        if (grad_from.count(tn.id)) from = std::min(from, grad_from[tn.id]);
        request(t, "grad:" + std::to_string(tn.id), bytes, std::min<uint64_t>(from, bwd(tn.tick)),
                bwd(tn.tick), reinterpret_cast<void **>(&t.grad[tn.id]));
    }
    t.classes = g.node(t.out_id).op.kind == CATNN_OP_LM_HEAD;
    if (t.classes) {  // pipeline.rs:430-441: an LmHead output trains on class ids
        t.vocab = t.dims[t.out_id].back();
        t.class_rows = numel(t.dims[t.out_id]) / std::max<int64_t>(t.vocab, 1);
        request(t, "classes", (uint64_t)t.class_rows * 4, 0, upd, reinterpret_cast<void **>(&t.class_ids));
        request(t, "ce_rows", (uint64_t)t.class_rows * 4, n, n, reinterpret_cast<void **>(&t.ce_rows));
    } else {
        request(t, "target", (uint64_t)numel(t.dims[t.out_id]) * 4, 0, upd, reinterpret_cast<void **>(&t.target));
        request(t, "mse_scratch", k::mse_scratch_bytes(), n, n, reinterpret_cast<void **>(&t.mse_scratch));
    }
    request(t, "loss", 256, n, upd, reinterpret_cast<void **>(&t.loss));

    auto add_param = [&](TNode &tn, const std::string &port, int64_t rows, int64_t cols, bool b, bool bt,
                         std::vector<float> init, bool bt3 = false, int64_t b_ld = 0, TParam *b_with = nullptr,
                         int64_t b_col = 0) {
        auto p = std::make_unique<TParam>();
        p->name = "param:" + tn.node->name + ":" + port;
        p->rows = rows;
        p->cols = cols;
        p->init = std::move(init);
        p->want_b = b || bt;
        p->want_bt = bt;
        p->want_bt3 = bt3;
        if (t.prec == CATNN_PREC_FP32) {  // every GEMM weight: the two six-part copies instead
            p->want_b6 = p->want_bt6 = b || bt || bt3;
            p->want_b = p->want_bt = p->want_bt3 = false;
        }
        const uint64_t e = (uint64_t)(rows * cols);
        p->b_ld = b_ld;
        p->b_with = b_with;
        p->b_col = b_col;
        request(t, p->name, e * 4, 0, upd, reinterpret_cast<void **>(&p->master));
        request(t, "grad:" + p->name, e * 4, bwd(tn.tick), upd, reinterpret_cast<void **>(&p->grad));
        if (t.opt == CATNN_OPT_ADAM)  // pipeline.rs:366-376
            for (const char *mom : {"m", "v"})
                request(t, "adam:" + tn.node->name + ":" + port + ":" + mom, e * 4, 0, upd,
                        reinterpret_cast<void **>(mom[0] == 'm' ? &p->m : &p->v));
        if (p->want_b && !p->b_with)
            request(t, "bf16:" + p->name, (uint64_t)(rows * (b_ld ? b_ld : cols)) * 2, 0, upd,
                    reinterpret_cast<void **>(&p->b));
        if (p->want_bt) request(t, "bf16t:" + p->name, e * 2, 0, upd, reinterpret_cast<void **>(&p->bt));
        if (p->want_bt3) request(t, "bf16t3:" + p->name, e * 6, 0, upd, reinterpret_cast<void **>(&p->bt3));
        if (p->want_b6) request(t, "bf16x6:" + p->name, e * 12, 0, upd, reinterpret_cast<void **>(&p->b6));
        if (p->want_bt6) request(t, "bf16x6t:" + p->name, e * 12, 0, upd, reinterpret_cast<void **>(&p->bt6));
        tn.params[port] = p.get();
        t.params.push_back(std::move(p));
    };
    auto host = [](const Node &nd, const std::string &port) {
        const HostTensor *h = nd.param(port);
        if (!h) fail(CATNN_ERR_UNKNOWN_PORT, "unknown port " + port + " on interface " + nd.name);
        return h;
    };
    auto tape = [&](TNode &tn, const std::string &nm, uint64_t bytes, bool keep = false) {
        request(t, "tape:" + tn.node->name + ":" + nm, bytes, tn.tick, keep ? upd : bwd(tn.tick), &tn.B(nm));
    };
    auto scratch = [&](TNode &tn, const std::string &nm, uint64_t bytes) {
        request(t, "scratch:" + tn.node->name + ":" + nm, bytes, bwd(tn.tick), bwd(tn.tick), &tn.B(nm));
    };
    auto fscratch = [&](TNode &tn, const std::string &nm, uint64_t bytes) {  // forward tick only
        request(t, "fscratch:" + tn.node->name + ":" + nm, bytes, tn.tick, tn.tick, &tn.B(nm));
    };
    constexpr uint64_t X6 = 12;  // bytes per element of a six-part split operand

    for (auto &tn : t.nodes) {
        if (t.input_ids.count(tn.id)) continue;
        if (t.prec != CATNN_PREC_FP32) continue;
        // fp32 precision: every GEMM on six-part split operands (an fp32
        // product on the bf16 matrix cores), every tape and cotangent fp32.
        const Node &nd = *tn.node;
        const auto &x = tn.in_dims.empty() ? tn.dims : tn.in_dims[0];
        switch (tn.kind) {
            case CATNN_OP_LINEAR: case CATNN_OP_MATMUL: case CATNN_OP_LM_HEAD: {
                int64_t K, N;
                if (tn.kind == CATNN_OP_LM_HEAD) {
                    const HostTensor *w = host(nd, "w");
                    K = nd.op.a[0];
                    N = nd.op.a[1];
                    CATNN_REQUIRE(w->numel() == N * K, CATNN_ERR_SHAPE_MISMATCH, "lm_head w");
                    add_param(tn, "w", K, N, true, false, param_values(nd, "w"), true);
                    tn.params["w"]->transposed = true;
                } else {
                    const HostTensor *w = nd.param("w") ? nd.param("w") : (nd.params.empty() ? nullptr : &nd.params.front().second);
                    CATNN_REQUIRE(w, CATNN_ERR_UNKNOWN_COMPONENT, "unknown component " + nd.name);
                    K = w->dims[0];
                    N = w->dims[1];
                    add_param(tn, nd.param("w") ? "w" : nd.params.front().first, K, N, true, false, w->data, true);
                    if (const HostTensor *b = nd.param("b")) add_param(tn, "b", 1, N, false, false, b->data);
                }
                const int64_t M = numel(x) / K;
                fscratch(tn, "x6", (uint64_t)(M * K) * X6);
                scratch(tn, "dy6", (uint64_t)(M * N) * X6);
                scratch(tn, "xt6", (uint64_t)(M * K) * X6);
                scratch(tn, "dyt6", (uint64_t)(M * N) * X6);
                scratch(tn, "colsum", k::colsum_scratch_bytes(M, (int)N));
                scratch(tn, "wparts", wparts_bytes(K, N, 6 * M));
                break;
            }
            case CATNN_OP_SWIGLU: {
                const int64_t H = nd.op.a[0], I = nd.op.a[1], M = numel(x) / std::max<int64_t>(H, 1);
                CATNN_REQUIRE(x.back() == H, CATNN_ERR_SHAPE_MISMATCH, "swiglu input");
                const HostTensor *w1 = host(nd, "w1"), *w3 = host(nd, "w3"), *w2 = host(nd, "w2");
                CATNN_REQUIRE(w1->numel() == H * I && w3->numel() == H * I && w2->numel() == I * H,
                              CATNN_ERR_SHAPE_MISMATCH, "swiglu weights");
                add_param(tn, "w1", H, I, true, false, w1->data, true);
                add_param(tn, "w3", H, I, true, false, w3->data, true);
                add_param(tn, "w2", I, H, true, false, w2->data, true);
                for (const char *nm : {"a", "c", "h"}) tape(tn, nm, (uint64_t)(M * I) * 4);
                fscratch(tn, "x6", (uint64_t)(M * H) * X6);
                fscratch(tn, "h6", (uint64_t)(M * I) * X6);
                scratch(tn, "dy6", (uint64_t)(M * H) * X6);
                for (const char *nm : {"dh", "da", "dc"}) scratch(tn, nm, (uint64_t)(M * I) * 4);
                for (const char *nm : {"da6", "dc6", "dat6", "dct6", "ht6"}) scratch(tn, nm, (uint64_t)(M * I) * X6);
                scratch(tn, "xt6", (uint64_t)(M * H) * X6);
                scratch(tn, "dyt6", (uint64_t)(M * H) * X6);
                scratch(tn, "wparts", std::max(wparts_bytes(H, I, 6 * M), wparts_bytes(I, H, 6 * M)));
                break;
            }
            case CATNN_OP_ATTENTION: case CATNN_OP_GQA_ATTENTION: {
                const bool gqa = tn.kind == CATNN_OP_GQA_ATTENTION;
                const int64_t Bt = x[0], S = x[1], D = x[2], T = Bt * S, H = nd.op.a[0];
                const int64_t hd = gqa ? nd.op.a[2] : nd.op.a[2], HKV = gqa ? nd.op.a[1] : H;
                const int64_t QW = H * hd, KW = HKV * hd, LD = QW + 2 * KW;
                add_param(tn, "wqkv", D, LD, true, false, param_values(nd, "wqkv"), true);
                add_param(tn, "wo", QW, D, true, false, host(nd, "wo")->data, true);
                tape(tn, "qkv", (uint64_t)(T * LD) * 4);
                tape(tn, "ctx", (uint64_t)(T * QW) * 4);
                tape(tn, "lse", (uint64_t)(T * H) * 4);
                if (gqa) tape(tn, "rope", (uint64_t)(S * std::max<int64_t>(hd / 2, 1)) * 8);
                fscratch(tn, "x6", (uint64_t)(T * D) * X6);
                fscratch(tn, "ctx6", (uint64_t)(T * QW) * X6);
                scratch(tn, "dy6", (uint64_t)(T * D) * X6);
                scratch(tn, "dctx", (uint64_t)(T * QW) * 4);
                scratch(tn, "ctxt6", (uint64_t)(T * QW) * X6);
                scratch(tn, "dyt6", (uint64_t)(T * D) * X6);
                scratch(tn, "dqkv", (uint64_t)(T * LD) * 4);
                scratch(tn, "dqkv6", (uint64_t)(T * LD) * X6);
                scratch(tn, "xt6", (uint64_t)(T * D) * X6);
                scratch(tn, "dqkvt6", (uint64_t)(T * LD) * X6);
                scratch(tn, "dscr", k::attention_bwd_scratch_bytes(Bt, S, H));
                scratch(tn, "wparts", std::max(wparts_bytes(QW, D, 6 * T), wparts_bytes(D, LD, 6 * T)));
                break;
            }
            case CATNN_OP_MOE: {
                const int64_t E = nd.op.a[0], K = nd.op.a[1], H = x.back(), T = numel(x) / H;
                const int64_t I = host(nd, "e0.w1")->dims[1];
                const int64_t P = T * K + E * (kPad - 1);
                const int64_t Pr = (P + kPad - 1) / kPad * kPad;
                add_param(tn, "gate", H, E, false, false, host(nd, "gate")->data);
                for (int64_t e = 0; e < E; ++e) {
                    const std::string p = "e" + std::to_string(e);
                    add_param(tn, p + ".w1", H, I, true, false, host(nd, p + ".w1")->data);
                    add_param(tn, p + ".w3", H, I, true, false, host(nd, p + ".w3")->data);
                    add_param(tn, p + ".w2", I, H, true, false, host(nd, p + ".w2")->data);
                }
                tape(tn, "idx", (uint64_t)(T * K) * 4, true);  // readable after the step
                tape(tn, "w", (uint64_t)(T * K) * 4);
                tape(tn, "counts", (uint64_t)E * 4);
                tape(tn, "offsets", (uint64_t)(E + 1) * 4);
                tape(tn, "sop", (uint64_t)Pr * 4);
                tape(tn, "pos", (uint64_t)(T * K) * 4);
                tape(tn, "tiles", (uint64_t)k::gemm_bf16_tiles_ints(T * K, (int)E) * 4);
                tape(tn, "perm_scratch", k::moe_permute_scratch_bytes(T, K, E));
                for (const char *nm : {"a", "c", "h"}) tape(tn, nm, (uint64_t)(Pr * I) * 4);
                tape(tn, "ys", (uint64_t)(Pr * H) * 4);
                fscratch(tn, "x6", (uint64_t)(T * H) * X6);
                fscratch(tn, "h6", (uint64_t)(Pr * I) * X6);
                scratch(tn, "dys", (uint64_t)(Pr * H) * 4);
                scratch(tn, "dw", (uint64_t)(T * K) * 4);
                scratch(tn, "dys6", (uint64_t)(Pr * H) * X6);
                for (const char *nm : {"dh", "da", "dc"}) scratch(tn, nm, (uint64_t)(Pr * I) * 4);
                for (const char *nm : {"da6", "dc6", "ht6", "dat6", "dct6"}) scratch(tn, nm, (uint64_t)(Pr * I) * X6);
                scratch(tn, "dxs", (uint64_t)(Pr * H) * 4);
                scratch(tn, "xpt6", (uint64_t)(Pr * H) * X6);
                scratch(tn, "dyst6", (uint64_t)(Pr * H) * X6);
                scratch(tn, "seg6", (uint64_t)(2 * E + 1) * 4);
                scratch(tn, "dl", (uint64_t)(T * E) * 4);
                scratch(tn, "router", k::router_backward_scratch_bytes((int)T, (int)H, (int)E));
                break;
            }
            default:
                break;
        }
    }

    for (auto &tn : t.nodes) {
        if (t.input_ids.count(tn.id)) continue;
        if (t.prec == CATNN_PREC_FP32 &&
            (tn.kind == CATNN_OP_LINEAR || tn.kind == CATNN_OP_MATMUL || tn.kind == CATNN_OP_LM_HEAD ||
             tn.kind == CATNN_OP_SWIGLU || tn.kind == CATNN_OP_ATTENTION || tn.kind == CATNN_OP_GQA_ATTENTION ||
             tn.kind == CATNN_OP_MOE))
            continue;  // planned above
        const Node &nd = *tn.node;
        const auto &x = tn.in_dims.empty() ? tn.dims : tn.in_dims[0];
        switch (tn.kind) {
            case CATNN_OP_LINEAR:
            case CATNN_OP_MATMUL: {
                const HostTensor *w = nd.param("w") ? nd.param("w") : (nd.params.empty() ? nullptr : &nd.params.front().second);
                CATNN_REQUIRE(w, CATNN_ERR_UNKNOWN_COMPONENT, "unknown component " + nd.name);
                const int64_t K = w->dims[0], N = w->dims[1], M = numel(x) / K;
                add_param(tn, nd.param("w") ? "w" : nd.params.front().first, K, N, true, true, w->data);
                if (const HostTensor *b = nd.param("b")) add_param(tn, "b", 1, N, false, false, b->data);
                if (tn.xb_ready)  // written by the previous Linear's epilogue (the fused GELU)
                    request(t, "tape:" + tn.node->name + ":xb", (uint64_t)(M * K) * 2, tn.xb_from, bwd(tn.tick),
                            &tn.B("xb"));
                else
                    tape(tn, "xb", (uint64_t)(M * K) * 2);
                scratch(tn, "xbt", (uint64_t)(M * K) * 2);
                if (tn.dyb_ready)  // written by the next Linear's backward (the fused GELU adjoint)
                    request(t, "scratch:" + tn.node->name + ":dyb", (uint64_t)(M * N) * 2, grad_from.at(tn.id),
                            bwd(tn.tick), &tn.B("dyb"));
                else
                    scratch(tn, "dyb", (uint64_t)(M * N) * 2);
                scratch(tn, "dybt", (uint64_t)(M * N) * 2);
                scratch(tn, "colsum", k::colsum_scratch_bytes(M, (int)N));
                scratch(tn, "wparts", wparts_bytes(K, N, M));
                break;
            }
            case CATNN_OP_SWIGLU: {  // moe.rs:159-174; adjoint.rs:217-251
                const int64_t H = nd.op.a[0], I = nd.op.a[1], M = numel(x) / std::max<int64_t>(H, 1);
                CATNN_REQUIRE(x.back() == H, CATNN_ERR_SHAPE_MISMATCH, "swiglu input");
                const HostTensor *w1 = host(nd, "w1"), *w3 = host(nd, "w3"), *w2 = host(nd, "w2");
                CATNN_REQUIRE(w1->numel() == H * I && w3->numel() == H * I && w2->numel() == I * H,
                              CATNN_ERR_SHAPE_MISMATCH, "swiglu weights");
                add_param(tn, "w1", H, I, true, true, w1->data);
                add_param(tn, "w3", H, I, true, true, w3->data);
                add_param(tn, "w2", I, H, true, true, w2->data);
                tape(tn, "xb", (uint64_t)(M * H) * 2);
                tape(tn, "a", (uint64_t)(M * I) * 4);
                tape(tn, "c", (uint64_t)(M * I) * 4);
                tape(tn, "h", (uint64_t)(M * I) * 4);
                tape(tn, "hb", (uint64_t)(M * I) * 2);
                scratch(tn, "dyb", (uint64_t)(M * H) * 2);
                scratch(tn, "dybt", (uint64_t)(M * H) * 2);
                scratch(tn, "dh", (uint64_t)(M * I) * 4);
                for (const char *nm : {"dab", "dcb", "dabt", "dcbt", "hbt"}) scratch(tn, nm, (uint64_t)(M * I) * 2);
                scratch(tn, "xbt", (uint64_t)(M * H) * 2);
                scratch(tn, "wparts", std::max(wparts_bytes(H, I, M), wparts_bytes(I, H, M)));
                break;
            }
            case CATNN_OP_EMBEDDING: {
                const int64_t V = nd.op.a[0], H = nd.op.a[1], n_ids = numel(x);
                // Its ids are checked on the host when the batch is set: they
                // must come from a graph input (an id ≥ vocab fails the step as
                // moe::embedding fails, moe.rs:38-40, instead of training on
                // zero rows).
                CATNN_REQUIRE(!tn.ins.empty() && t.input_ids.count(tn.ins[0]), CATNN_ERR_UNSUPPORTED,
                              "training: Embedding " + nd.name + " reads a computed value; its ids must come "
                              "from a graph input, where they are checked against the vocabulary");
                const HostTensor *w = host(nd, "w");
                CATNN_REQUIRE(w->numel() == V * H, CATNN_ERR_SHAPE_MISMATCH, "embedding table");
                add_param(tn, "w", V, H, false, false, w->data);
                tape(tn, "bad", 256);
                scratch(tn, "idi", (uint64_t)n_ids * 4);
                scratch(tn, "hit", (uint64_t)V * 4);
                break;
            }
            case CATNN_OP_MIX: {
                if (const HostTensor *g = nd.param("gate")) {
                    CATNN_REQUIRE(g->numel() == 1, CATNN_ERR_SHAPE_MISMATCH, "mix gate");
                    add_param(tn, "gate", 1, 1, false, false, g->data);
                }
                scratch(tn, "parts", k::mix_scratch_bytes());
                break;
            }
            case CATNN_OP_RMS_NORM: {
                const int64_t C = x.back(), R = numel(x) / C;
                const HostTensor *w = host(nd, "w");
                CATNN_REQUIRE(w->numel() == C, CATNN_ERR_SHAPE_MISMATCH, "rmsnorm w");  // adjoint.rs:155-157
                add_param(tn, "w", 1, C, false, false, w->data);
                scratch(tn, "prod", (uint64_t)(R * C) * 4);
                scratch(tn, "colsum", k::colsum_scratch_bytes(R, (int)C));
                break;
            }
            case CATNN_OP_LM_HEAD: {
                // logits = x·wᵀ: a bias-free Linear with weight wᵀ [H, V].
                const HostTensor *w = host(nd, "w");
                const int64_t V = nd.op.a[1], K = nd.op.a[0], M = numel(x) / K;
                CATNN_REQUIRE(w->numel() == V * K, CATNN_ERR_SHAPE_MISMATCH, "lm_head w");
                add_param(tn, "w", K, V, true, true, param_values(nd, "w"));
                tn.params["w"]->transposed = true;
                tape(tn, "xb", (uint64_t)(M * K) * 2);
                scratch(tn, "xbt", (uint64_t)(M * K) * 2);
                scratch(tn, "dyb", (uint64_t)(M * V) * 2);
                scratch(tn, "dybt", (uint64_t)(M * V) * 2);
                scratch(tn, "wparts", wparts_bytes(K, V, M));
                break;
            }
            case CATNN_OP_LAYER_NORM: {
                const int64_t C = x.back(), R = numel(x) / C;
                add_param(tn, "gamma", 1, C, false, false, host(nd, "gamma")->data);
                add_param(tn, "beta", 1, C, false, false, host(nd, "beta")->data);
                tape(tn, "mean", (uint64_t)R * 4);
                tape(tn, "rstd", (uint64_t)R * 4);
                scratch(tn, "parts", k::ln_backward_scratch_bytes(R, (int)C));
                break;
            }
            case CATNN_OP_ATTENTION: {
                const int64_t Bt = x[0], S = x[1], D = x[2], T = Bt * S, H = nd.op.a[0];
                add_param(tn, "wqkv", D, 3 * D, true, false, param_values(nd, "wqkv"), true);
                add_param(tn, "wo", D, D, true, false, host(nd, "wo")->data, true);
                if (tn.x3_ready)  // written by the LayerNorm before it
                    request(t, "tape:" + tn.node->name + ":x3", (uint64_t)(T * 3 * D) * 2, tn.x3_from, bwd(tn.tick),
                            &tn.B("x3"));
                else
                    tape(tn, "x3", (uint64_t)(T * 3 * D) * 2);
                if (attn_core_bf16(nd, D)) {
                    const uint64_t Sp = (uint64_t)k::attention_bf16_seq_pad(S);
                    tape(tn, "qkvb", (uint64_t)(T * 3 * D) * 2);
                    tape(tn, "qkvt", (uint64_t)(Bt * 3 * D) * Sp * 2);
                    scratch(tn, "dctxb", (uint64_t)(T * D) * 2);
                    scratch(tn, "dctxt", (uint64_t)(Bt * D) * Sp * 2);
                } else {
                    tape(tn, "qkv", (uint64_t)(T * 3 * D) * 4);
                }
                tape(tn, "ctx", (uint64_t)(T * D) * 4);
                tape(tn, "ctx3", (uint64_t)(T * 3 * D) * 2);
                tape(tn, "lse", (uint64_t)(T * H) * 4);
                scratch(tn, "dyb", (uint64_t)(T * D) * 2);
                scratch(tn, "dybt", (uint64_t)(T * D) * 2);
                scratch(tn, "ctxt", (uint64_t)(T * D) * 2);
                scratch(tn, "dctx", (uint64_t)(T * D) * 4);
                scratch(tn, "dqkv", (uint64_t)(T * 3 * D) * 4);
                scratch(tn, "dqkvb", (uint64_t)(T * 3 * D) * 2);
                scratch(tn, "dqkvt", (uint64_t)(T * 3 * D) * 2);
                scratch(tn, "xbt", (uint64_t)(T * D) * 2);
                scratch(tn, "dscr", k::attention_bwd_scratch_bytes(Bt, S, H));
                scratch(tn, "wparts", std::max(wparts_bytes(D, D, T), wparts_bytes(D, 3 * D, T)));
                break;
            }
            case CATNN_OP_GQA_ATTENTION: {  // moe.rs:62-136; gqa_backward, adjoint.rs:287-440
                const int64_t Bt = x[0], S = x[1], D = x[2], T = Bt * S;
                const int64_t H = nd.op.a[0], HKV = nd.op.a[1], hd = nd.op.a[2];
                const int64_t QW = H * hd, KW = HKV * hd, LD = QW + 2 * KW;
                add_param(tn, "wqkv", D, LD, true, false, param_values(nd, "wqkv"), true);
                add_param(tn, "wo", QW, D, true, false, host(nd, "wo")->data, true);
                if (tn.x3_ready)  // written by the LayerNorm before it
                    request(t, "tape:" + tn.node->name + ":x3", (uint64_t)(T * 3 * D) * 2, tn.x3_from, bwd(tn.tick),
                            &tn.B("x3"));
                else
                    tape(tn, "x3", (uint64_t)(T * 3 * D) * 2);
                tape(tn, "qkv", (uint64_t)(T * LD) * 4);  // q and k after RoPE
                tape(tn, "ctx", (uint64_t)(T * QW) * 4);
                tape(tn, "ctx3", (uint64_t)(T * 3 * QW) * 2);
                tape(tn, "lse", (uint64_t)(T * H) * 4);
                tape(tn, "rope", (uint64_t)(S * std::max<int64_t>(hd / 2, 1)) * 8);
                scratch(tn, "dyb", (uint64_t)(T * D) * 2);
                scratch(tn, "dybt", (uint64_t)(T * D) * 2);
                scratch(tn, "ctxt", (uint64_t)(T * QW) * 2);
                scratch(tn, "dctx", (uint64_t)(T * QW) * 4);
                scratch(tn, "dqkv", (uint64_t)(T * LD) * 4);
                scratch(tn, "dqkvb", (uint64_t)(T * LD) * 2);
                scratch(tn, "dqkvt", (uint64_t)(T * LD) * 2);
                scratch(tn, "xbt", (uint64_t)(T * D) * 2);
                scratch(tn, "dscr", k::attention_bwd_scratch_bytes(Bt, S, H));
                scratch(tn, "wparts", std::max(wparts_bytes(QW, D, T), wparts_bytes(D, LD, T)));
                break;
            }
            case CATNN_OP_MOE: {
                const int64_t E = nd.op.a[0], K = nd.op.a[1], H = x.back(), T = numel(x) / H;
                const int64_t I = host(nd, "e0.w1")->dims[1];
                const int64_t P = T * K + E * (kPad - 1);
                const int64_t Pr = (P + kPad - 1) / kPad * kPad;  // transposed operands' row stride
                add_param(tn, "gate", H, E, false, false, host(nd, "gate")->data);
                for (int64_t e = 0; e < E; ++e) {
                    const std::string p = "e" + std::to_string(e);
                    // w1's bf16 copy holds [w1 | w3] per row: the B operand of dx = [da | dc]·[w1 | w3]ᵀ.
                    // The gate/up GEMM reads wᵀ twice over K = 2H ([x_hi | x_lo]·[wᵀ | wᵀ]): as a
                    // k-wrapping B on the plain transposed copy, or as the first 2H of the split copy.
                    const bool wrap = moe_kwrap(H);
                    add_param(tn, p + ".w1", H, I, true, wrap, host(nd, p + ".w1")->data, !wrap, 2 * I);
                    add_param(tn, p + ".w3", H, I, true, wrap, host(nd, p + ".w3")->data, !wrap, 2 * I,
                              tn.params[p + ".w1"], I);
                    add_param(tn, p + ".w2", I, H, true, true, host(nd, p + ".w2")->data);
                }
                tape(tn, "x3", (uint64_t)(T * 3 * H) * 2);
                tape(tn, "idx", (uint64_t)(T * K) * 4, true);  // readable after the step
                tape(tn, "w", (uint64_t)(T * K) * 4);
                tape(tn, "counts", (uint64_t)E * 4);
                tape(tn, "offsets", (uint64_t)(E + 1) * 4);
                tape(tn, "sop", (uint64_t)Pr * 4);
                tape(tn, "pos", (uint64_t)(T * K) * 4);
                tape(tn, "tiles", (uint64_t)k::gemm_bf16_tiles_ints(T * K, (int)E) * 4);
                tape(tn, "perm_scratch", k::moe_permute_scratch_bytes(T, K, E));
                tape(tn, "a", (uint64_t)(Pr * I) * 2);
                tape(tn, "c", (uint64_t)(Pr * I) * 2);
                tape(tn, "h", (uint64_t)(Pr * I) * 2);
                tape(tn, "ys", (uint64_t)(Pr * H) * 4);
                scratch(tn, "dys", (uint64_t)(Pr * H) * 2);
                scratch(tn, "dw", (uint64_t)(T * K) * 4);
                scratch(tn, "dadc", (uint64_t)(Pr * 2 * I) * 2);  // [da | dc] per slot row
                scratch(tn, "dxs", (uint64_t)(Pr * H) * 4);
                scratch(tn, "xpt", (uint64_t)(H * Pr) * 2);
                scratch(tn, "ht", (uint64_t)(I * Pr) * 2);
                scratch(tn, "dyst", (uint64_t)(H * Pr) * 2);
                scratch(tn, "dadct", (uint64_t)(2 * I * Pr) * 2);
                scratch(tn, "dl", (uint64_t)(T * E) * 4);
                scratch(tn, "router", k::router_backward_scratch_bytes((int)T, (int)H, (int)E));
                break;
            }
            default:
                break;
        }
    }
    // One multi-tensor update entry per parameter.
    request(t, "sgd_table", (uint64_t)t.params.size() * sizeof(k::SgdParam), 0, upd,
            reinterpret_cast<void **>(&t.sgd_table));
}

// The multi-tensor update table: every parameter, trained ones (nodes that
// receive a cotangent) with their gradient, in 64×64 tiles.
static void build_sgd_table(Tr &t, std::vector<k::SgdParam> &tab) {
    int tiles = 0;
    for (auto &tn : t.nodes) {
        if (t.input_ids.count(tn.id)) continue;
        const bool trained = t.has_grad.count(tn.id) != 0;
        for (auto &kv : tn.params) {
            TParam *p = kv.second;
            k::SgdParam e{};
            e.p = p->master;
            e.g = trained ? p->grad : nullptr;
            e.m = p->m;
            e.v = p->v;
            e.b = p->want_b ? p->b : nullptr;
            e.ldb = (int)(p->b_ld ? p->b_ld : p->cols);
            e.bt = p->want_bt ? p->bt : nullptr;
            e.bt3 = p->want_bt3 ? p->bt3 : nullptr;
            e.rows = (int)p->rows;
            e.cols = (int)p->cols;
            e.tiles_c = (int)((p->cols + 63) / 64);
            e.tile0 = tiles;
            const int64_t nt = (int64_t)((p->rows + 63) / 64) * e.tiles_c;
            CATNN_REQUIRE(tiles + nt < (1ll << 31), CATNN_ERR_SHAPE_MISMATCH, "training: too many parameter tiles");
            tiles += (int)nt;
            tab.push_back(e);
        }
    }
    t.sgd_tiles = tiles;
    t.sgd_n = (int)tab.size();
}

// Masters from the host copies, then the bf16 operand copies from the
// masters; Adam's moments start at zero (AdamState::zeros_like, optim.rs:71-75).
static void upload_params(Tr &t) {
    hipStream_t s = t.dev->stream;
    for (auto &p : t.params) {
        CATNN_HIP(hipMemcpyAsync(p->master, p->init.data(), p->init.size() * 4, hipMemcpyHostToDevice, s));
        if (p->m) k::fill_f32(s, p->m, 0.f, p->rows * p->cols);
        if (p->v) k::fill_f32(s, p->v, 0.f, p->rows * p->cols);
    }
    t.adam_t = 0;
    k::sgd_multi(s, t.sgd_table, t.sgd_n, t.sgd_tiles, k::sgd_rule(0.f), false);
    if (t.prec == CATNN_PREC_FP32) refresh_split_copies(t);
}

// place_arena under the cap; when the arena misses, checkpoint the value
// with the largest bytes × lifetime — its buffer then ends at its last
// forward read and a copy "act:{id}#recomp" lives from its first backward
// read, recomputed there by re-running its producer — as schedule() does
// for one buffer (schedule.rs:155-212), repeated until the plan fits or
// nothing is left to checkpoint.
static void plan_arena(Tr &t, uint64_t cap) {
    for (;;) {
        try {
            t.plan = place_arena(t.reqs, cap);
            return;
        } catch (const Failure &f) {
            if (f.code != CATNN_ERR_FIBRATION) throw;
            uint32_t best = UINT32_MAX;
            uint64_t best_cost = 0;
            for (const auto &kv : t.ckpt_candidates) {
                if (t.ckpt.count(kv.first)) continue;
                const BufferReq &r = t.reqs[kv.second.req];
                const uint64_t cost = r.bytes * (r.live_to - r.live_from + 1);
                if (best == UINT32_MAX || cost > best_cost) {
                    best = kv.first;
                    best_cost = cost;
                }
            }
            if (best == UINT32_MAX)
                fail(CATNN_ERR_FIBRATION, f.msg + " (no activation left to checkpoint)");
            const catnn_hip_trainer::Ckpt c = t.ckpt_candidates.at(best);
            BufferReq &r = t.reqs[c.req];
            const uint64_t t1 = r.live_to;
            r.live_to = c.fwd_last;
            r.checkpoint = true;
            const uint64_t bytes = r.bytes;
            const std::string id = r.id + "#recomp";
            t.reqs.push_back(BufferReq{id, bytes, c.bwd_first, t1, true});
            t.req_slot.push_back(reinterpret_cast<void **>(&t.val_recomp[best]));
            t.ckpt[best] = c;
        }
    }
}

static void reserve_and_upload(Tr &t) {
    hipDeviceProp_t prop;
    CATNN_HIP(hipGetDeviceProperties(&prop, t.dev->ordinal));
    plan_arena(t, t.arena_cap ? std::min<uint64_t>(t.arena_cap, prop.totalGlobalMem) : prop.totalGlobalMem);
    t.reserved = 0;
    for (const auto &a : t.plan) t.reserved = std::max(t.reserved, a.offset + a.bytes);
    hipError_t e = hipMalloc(&t.base, t.reserved);
    if (e != hipSuccess)
        fail(CATNN_ERR_FIBRATION, "training arena: hipMalloc of " + std::to_string(t.reserved) +
                                      " B failed (" + hipGetErrorString(e) + ")");
    std::map<std::string, uint64_t> off;
    for (const auto &a : t.plan) off[a.id] = a.offset;
    for (size_t i = 0; i < t.reqs.size(); ++i)
        *t.req_slot[i] = static_cast<char *>(t.base) + off.at(t.reqs[i].id);
    for (auto &p : t.params)
        if (p->b_with) p->b = p->b_with->b + p->b_col;
    for (const auto &kv : t.ckpt) t.val_fwd[kv.first] = t.val.at(kv.first);
    for (auto &p : t.params)
        CATNN_REQUIRE((int64_t)p->init.size() == p->rows * p->cols, CATNN_ERR_SHAPE_MISMATCH,
                      p->name + ": parameter size");
    std::vector<k::SgdParam> tab;
    build_sgd_table(t, tab);
    CATNN_REQUIRE(tab.size() == t.params.size(), CATNN_ERR_WIRING, "training: update table size");
    CATNN_HIP(hipMemcpyAsync(t.sgd_table, tab.data(), tab.size() * sizeof(k::SgdParam), hipMemcpyHostToDevice,
                             t.dev->stream));
    upload_params(t);
    CATNN_HIP(hipStreamSynchronize(t.dev->stream));  // before `tab` goes out of scope
}

// ------------------------------------------------- fp32 precision GEMMs
// Every GEMM of these ops on six-part split operands (k::split6_*): A rows
// from fp32 values, B from the weights' six-part copies (b6, bt6) or from
// fp32 values transposed; K' = 6K.  Tapes and cotangents stay fp32.

static bool is_gemm_op(int kind) {
    return kind == CATNN_OP_LINEAR || kind == CATNN_OP_MATMUL || kind == CATNN_OP_LM_HEAD ||
           kind == CATNN_OP_SWIGLU || kind == CATNN_OP_ATTENTION || kind == CATNN_OP_GQA_ATTENTION ||
           kind == CATNN_OP_MOE;
}

// C = A6·B6ᵀ over the six-part K' = 6K (EPI_LINEAR: + bias).
static void gemm6(hipStream_t s, const bf16_t *A6, int64_t lda, const bf16_t *B6, int64_t ldb, int64_t M, int64_t N,
                  int64_t K, float *C, int64_t ldc, const float *bias = nullptr) {
    k::GemmBf16Params p = gp();
    p.A = A6; p.lda = lda; p.B = B6; p.ldb = ldb;
    p.M = (int)M; p.N = (int)N; p.K = (int)(6 * K);
    p.epi = k::EPI_LINEAR; p.bias = bias;
    p.C32 = C; p.ldc32 = ldc;
    k::gemm_bf16_launch(s, p);
}

static void forward_gemm_f32(Tr &t, TNode &tn) {
    hipStream_t s = t.dev->stream;
    const Node &nd = *tn.node;
    float *y = t.val.at(tn.id);
    const float *x = t.val.at(tn.ins[0]);
    const auto &xd = tn.in_dims[0];
    const int64_t nx = numel(xd);
    switch (tn.kind) {
        case CATNN_OP_LINEAR: case CATNN_OP_MATMUL: case CATNN_OP_LM_HEAD: {
            TParam *w = tn.params.begin()->second;
            for (auto &kv : tn.params) if (kv.first != "b") w = kv.second;
            TParam *b = tn.params.count("b") ? tn.params["b"] : nullptr;
            const int64_t K = w->rows, N = w->cols, M = nx / K;
            bf16_t *x6 = (bf16_t *)tn.B("x6");
            k::split6_rows(s, x, K, M, (int)K, false, x6, 6 * K);
            gemm6(s, x6, 6 * K, w->bt6, 6 * K, M, N, K, y, N, b ? b->master : nullptr);
            break;
        }
        case CATNN_OP_SWIGLU: {
            TParam *w1 = tn.params["w1"], *w3 = tn.params["w3"], *w2 = tn.params["w2"];
            const int64_t H = w1->rows, I = w1->cols, M = nx / H;
            bf16_t *x6 = (bf16_t *)tn.B("x6"), *h6 = (bf16_t *)tn.B("h6");
            float *a = (float *)tn.B("a"), *c = (float *)tn.B("c"), *h = (float *)tn.B("h");
            k::split6_rows(s, x, H, M, (int)H, false, x6, 6 * H);
            gemm6(s, x6, 6 * H, w1->bt6, 6 * H, M, I, H, a, I);
            gemm6(s, x6, 6 * H, w3->bt6, 6 * H, M, I, H, c, I);
            k::swiglu_h(s, a, c, h, M * I);
            k::split6_rows(s, h, I, M, (int)I, false, h6, 6 * I);
            gemm6(s, h6, 6 * I, w2->bt6, 6 * I, M, H, I, y, H);
            break;
        }
        case CATNN_OP_ATTENTION: case CATNN_OP_GQA_ATTENTION: {
            const bool gqa = tn.kind == CATNN_OP_GQA_ATTENTION;
            const int64_t Bt = xd[0], S = xd[1], D = xd[2], T = Bt * S;
            const int64_t H = nd.op.a[0], hd = nd.op.a[2], HKV = gqa ? nd.op.a[1] : H;
            const int64_t QW = H * hd, KW = HKV * hd, LD = QW + 2 * KW;
            bf16_t *x6 = (bf16_t *)tn.B("x6"), *ctx6 = (bf16_t *)tn.B("ctx6");
            float *qkv = (float *)tn.B("qkv"), *ctx = (float *)tn.B("ctx"), *lse = (float *)tn.B("lse");
            k::split6_rows(s, x, D, T, (int)D, false, x6, 6 * D);
            gemm6(s, x6, 6 * D, tn.params["wqkv"]->bt6, 6 * D, T, LD, D, qkv, LD);
            if (gqa) {
                float *rope = (float *)tn.B("rope");
                k::rope_table(s, rope, S, hd, (double)nd.op.a[5]);
                k::rope_apply(s, qkv, LD, T, S, H + HKV, hd, rope, 1.0f);
                k::attention_core_fwd_lse_gqa(s, qkv, LD, qkv + QW, qkv + QW + KW, LD, H / HKV,
                                              nd.op.a[4] > 0 ? nd.op.a[4] : 0, ctx, QW, lse, Bt, S, H, hd);
            } else {
                k::attention_core_fwd_lse(s, qkv, qkv + D, qkv + 2 * D, 3 * D, ctx, D, lse, Bt, S, H, hd,
                                          (nd.op.flags & CATNN_FLAG_CAUSAL) != 0);
            }
            k::split6_rows(s, ctx, QW, T, (int)QW, false, ctx6, 6 * QW);
            gemm6(s, ctx6, 6 * QW, tn.params["wo"]->bt6, 6 * QW, T, D, QW, y, D);
            break;
        }
        case CATNN_OP_MOE: {
            const int64_t E = nd.op.a[0], K = nd.op.a[1], H = xd.back(), T = nx / H;
            const int64_t I = tn.params["e0.w1"]->cols;
            const int64_t P = T * K + E * (kPad - 1);
            const int64_t Pr = (P + kPad - 1) / kPad * kPad;
            int32_t *idx = (int32_t *)tn.B("idx"), *counts = (int32_t *)tn.B("counts");
            int32_t *offs = (int32_t *)tn.B("offsets"), *sop = (int32_t *)tn.B("sop");
            int32_t *pos = (int32_t *)tn.B("pos"), *tiles = (int32_t *)tn.B("tiles");
            float *w = (float *)tn.B("w");
            float *a = (float *)tn.B("a"), *c = (float *)tn.B("c"), *h = (float *)tn.B("h");
            k::moe_route_f32(s, x, tn.params["gate"]->master, T, H, E, K, idx, w, nullptr);
            k::moe_permute_padded(s, idx, T, K, E, kPad, Pr, counts, offs, sop, pos, tn.B("perm_scratch"));
            k::gemm_bf16_build_tiles(s, offs, (int)E, T * K, tiles);
            bf16_t *x6 = (bf16_t *)tn.B("x6"), *h6 = (bf16_t *)tn.B("h6");
            k::split6_rows(s, x, H, T, (int)H, false, x6, 6 * H);
            k::GemmBf16Params p = gp();
            p.grid = k::GRID_ROWS;
            k::gemm_bf16_use_tiles(p, tiles, T * K, (int)E);
            p.seg_offsets = offs; p.seg_counts = counts; p.n_experts = (int)E;
            p.epi = k::EPI_STORE;
            // a = x·w1, c = x·w3 per expert segment, rows gathered through the permutation
            p.A = x6; p.lda = 6 * H; p.a_rows = sop; p.a_row_div = (int)K;
            p.ldb = 6 * H; p.M = 0; p.N = (int)I; p.K = (int)(6 * H);
            p.ldc32 = I;
            for (const char *port : {".w1", ".w3"}) {
                for (int64_t e = 0; e < E; ++e) p.B_e[e] = tn.params["e" + std::to_string(e) + port]->bt6;
                p.C32 = port[2] == '1' ? a : c;
                k::gemm_bf16_launch(s, p);
            }
            k::swiglu_h(s, a, c, h, Pr * I);
            k::split6_rows(s, h, I, Pr, (int)I, false, h6, 6 * I);
            // ys = h·w2
            p.A = h6; p.lda = 6 * I; p.a_rows = nullptr; p.a_row_div = 1;
            for (int64_t e = 0; e < E; ++e) p.B_e[e] = tn.params["e" + std::to_string(e) + ".w2"]->bt6;
            p.ldb = 6 * I; p.N = (int)H; p.K = (int)(6 * I);
            p.C32 = (float *)tn.B("ys"); p.ldc32 = H;
            k::gemm_bf16_launch(s, p);
            k::moe_combine(s, (float *)tn.B("ys"), pos, w, T, K, H, y);
            break;
        }
        default:
            fail(CATNN_ERR_UNSUPPORTED, "training: op " + op_name(tn.kind));
    }
}

static void backward_gemm_f32(Tr &t, TNode &tn) {
    hipStream_t s = t.dev->stream;
    const Node &nd = *tn.node;
    const float *dy = t.grad.at(tn.id);
    float *dx = t.input_ids.count(tn.ins[0]) && !t.input_grads ? nullptr : t.grad.at(tn.ins[0]);
    const bool acc = !tn.first_writer[0];
    const float *x = t.val.at(tn.ins[0]);
    const auto &xd = tn.in_dims[0];
    const int64_t nx = numel(xd);
    switch (tn.kind) {
        case CATNN_OP_LINEAR: case CATNN_OP_MATMUL: case CATNN_OP_LM_HEAD: {
            TParam *w = tn.params.begin()->second;
            for (auto &kv : tn.params) if (kv.first != "b") w = kv.second;
            TParam *b = tn.params.count("b") ? tn.params["b"] : nullptr;
            const int64_t K = w->rows, N = w->cols, M = nx / K;
            bf16_t *dy6 = (bf16_t *)tn.B("dy6"), *xt6 = (bf16_t *)tn.B("xt6"), *dyt6 = (bf16_t *)tn.B("dyt6");
            k::split6_rows(s, dy, N, M, (int)N, false, dy6, 6 * N);
            if (dx) gemm_nt(s, dy6, 6 * N, w->b6, 6 * N, (int)M, (int)K, (int)(6 * N), dx, K, acc);
            k::split6_transpose(s, x, K, nullptr, 1, (int)M, (int)K, false, xt6, 6 * M);
            k::split6_transpose(s, dy, N, nullptr, 1, (int)M, (int)N, true, dyt6, 6 * M);
            gemm_nt(s, xt6, 6 * M, dyt6, 6 * M, (int)K, (int)N, (int)(6 * M), w->grad, N, false,
                    (float *)tn.B("wparts"));
            if (b) k::colsum(s, dy, M, (int)N, b->grad, false, (float *)tn.B("colsum"));
            break;
        }
        case CATNN_OP_SWIGLU: {  // swiglu_backward, adjoint.rs:217-251
            TParam *w1 = tn.params["w1"], *w3 = tn.params["w3"], *w2 = tn.params["w2"];
            const int64_t H = w1->rows, I = w1->cols, M = nx / H;
            auto B = [&](const char *nm) { return (bf16_t *)tn.B(nm); };
            auto F = [&](const char *nm) { return (float *)tn.B(nm); };
            float *wparts = F("wparts");
            k::split6_rows(s, dy, H, M, (int)H, false, B("dy6"), 6 * H);
            gemm_nt(s, B("dy6"), 6 * H, w2->b6, 6 * H, (int)M, (int)I, (int)(6 * H), F("dh"), I, false);
            k::swiglu_dadc_f32(s, F("dh"), F("a"), F("c"), F("da"), F("dc"), M * I);
            k::split6_rows(s, F("da"), I, M, (int)I, false, B("da6"), 6 * I);
            k::split6_rows(s, F("dc"), I, M, (int)I, false, B("dc6"), 6 * I);
            if (dx) {
                gemm_nt(s, B("da6"), 6 * I, w1->b6, 6 * I, (int)M, (int)H, (int)(6 * I), dx, H, acc);
                gemm_nt(s, B("dc6"), 6 * I, w3->b6, 6 * I, (int)M, (int)H, (int)(6 * I), dx, H, true);
            }
            k::split6_transpose(s, x, H, nullptr, 1, (int)M, (int)H, false, B("xt6"), 6 * M);
            k::split6_transpose(s, F("da"), I, nullptr, 1, (int)M, (int)I, true, B("dat6"), 6 * M);
            k::split6_transpose(s, F("dc"), I, nullptr, 1, (int)M, (int)I, true, B("dct6"), 6 * M);
            gemm_nt(s, B("xt6"), 6 * M, B("dat6"), 6 * M, (int)H, (int)I, (int)(6 * M), w1->grad, I, false, wparts);
            gemm_nt(s, B("xt6"), 6 * M, B("dct6"), 6 * M, (int)H, (int)I, (int)(6 * M), w3->grad, I, false, wparts);
            k::split6_transpose(s, F("h"), I, nullptr, 1, (int)M, (int)I, false, B("ht6"), 6 * M);
            k::split6_transpose(s, dy, H, nullptr, 1, (int)M, (int)H, true, B("dyt6"), 6 * M);
            gemm_nt(s, B("ht6"), 6 * M, B("dyt6"), 6 * M, (int)I, (int)H, (int)(6 * M), w2->grad, H, false, wparts);
            break;
        }
        case CATNN_OP_ATTENTION: case CATNN_OP_GQA_ATTENTION: {
            const bool gqa = tn.kind == CATNN_OP_GQA_ATTENTION;
            const int64_t Bt = xd[0], S = xd[1], D = xd[2], T = Bt * S;
            const int64_t H = nd.op.a[0], hd = nd.op.a[2], HKV = gqa ? nd.op.a[1] : H;
            const int64_t QW = H * hd, KW = HKV * hd, LD = QW + 2 * KW;
            TParam *wqkv = tn.params["wqkv"], *wo = tn.params["wo"];
            auto B = [&](const char *nm) { return (bf16_t *)tn.B(nm); };
            auto F = [&](const char *nm) { return (float *)tn.B(nm); };
            float *qkv = F("qkv"), *ctx = F("ctx"), *dqkv = F("dqkv"), *wparts = F("wparts");
            k::split6_rows(s, dy, D, T, (int)D, false, B("dy6"), 6 * D);
            gemm_nt(s, B("dy6"), 6 * D, wo->b6, 6 * D, (int)T, (int)QW, (int)(6 * D), F("dctx"), QW, false);
            k::split6_transpose(s, ctx, QW, nullptr, 1, (int)T, (int)QW, false, B("ctxt6"), 6 * T);
            k::split6_transpose(s, dy, D, nullptr, 1, (int)T, (int)D, true, B("dyt6"), 6 * T);
            gemm_nt(s, B("ctxt6"), 6 * T, B("dyt6"), 6 * T, (int)QW, (int)D, (int)(6 * T), wo->grad, D, false, wparts);
            if (gqa) {
                k::attention_core_bwd_gqa(s, qkv, LD, qkv + QW, qkv + QW + KW, LD, H / HKV,
                                          nd.op.a[4] > 0 ? nd.op.a[4] : 0, ctx, F("dctx"), QW, F("lse"), dqkv, LD,
                                          dqkv + QW, dqkv + QW + KW, LD, Bt, S, H, hd, true, F("dscr"));
                k::rope_apply(s, dqkv, LD, T, S, H + HKV, hd, F("rope"), -1.0f);
            } else {
                k::attention_core_bwd(s, qkv, qkv + D, qkv + 2 * D, 3 * D, ctx, F("dctx"), D, F("lse"), dqkv,
                                      dqkv + D, dqkv + 2 * D, 3 * D, Bt, S, H, hd,
                                      (nd.op.flags & CATNN_FLAG_CAUSAL) != 0, F("dscr"));
            }
            k::split6_rows(s, dqkv, LD, T, (int)LD, false, B("dqkv6"), 6 * LD);
            if (dx) gemm_nt(s, B("dqkv6"), 6 * LD, wqkv->b6, 6 * LD, (int)T, (int)D, (int)(6 * LD), dx, D, acc);
            k::split6_transpose(s, x, D, nullptr, 1, (int)T, (int)D, false, B("xt6"), 6 * T);
            k::split6_transpose(s, dqkv, LD, nullptr, 1, (int)T, (int)LD, true, B("dqkvt6"), 6 * T);
            gemm_nt(s, B("xt6"), 6 * T, B("dqkvt6"), 6 * T, (int)D, (int)LD, (int)(6 * T), wqkv->grad, LD, false,
                    wparts);
            break;
        }
        case CATNN_OP_MOE: {
            const int64_t E = nd.op.a[0], K = nd.op.a[1], H = xd.back(), T = nx / H;
            const int64_t I = tn.params["e0.w1"]->cols;
            const int64_t P = T * K + E * (kPad - 1);
            const int64_t Pr = (P + kPad - 1) / kPad * kPad;
            auto B = [&](const char *nm) { return (bf16_t *)tn.B(nm); };
            auto F = [&](const char *nm) { return (float *)tn.B(nm); };
            int32_t *idx = (int32_t *)tn.B("idx"), *counts = (int32_t *)tn.B("counts");
            int32_t *offs = (int32_t *)tn.B("offsets"), *sop = (int32_t *)tn.B("sop");
            int32_t *pos = (int32_t *)tn.B("pos"), *tiles = (int32_t *)tn.B("tiles");
            int32_t *seg6 = (int32_t *)tn.B("seg6");
            float *w = F("w"), *dw = F("dw"), *dys = F("dys");
            k::moe_slot_grads_f32(s, sop, w, F("ys"), dy, (int)K, (int)H, (int)Pr, dys, dw);
            k::split6_rows(s, dys, H, Pr, (int)H, false, B("dys6"), 6 * H);
            k::GemmBf16Params p = gp();
            p.grid = k::GRID_ROWS;
            k::gemm_bf16_use_tiles(p, tiles, T * K, (int)E);
            p.seg_offsets = offs; p.seg_counts = counts; p.n_experts = (int)E;
            p.epi = k::EPI_STORE;
            // dh = dys·w2ᵀ
            p.A = B("dys6"); p.lda = 6 * H; p.ldb = 6 * H; p.N = (int)I; p.K = (int)(6 * H);
            for (int64_t e = 0; e < E; ++e) p.B_e[e] = tn.params["e" + std::to_string(e) + ".w2"]->b6;
            p.C32 = F("dh"); p.ldc32 = I;
            k::gemm_bf16_launch(s, p);
            k::swiglu_dadc_f32(s, F("dh"), F("a"), F("c"), F("da"), F("dc"), Pr * I);
            k::split6_rows(s, F("da"), I, Pr, (int)I, false, B("da6"), 6 * I);
            k::split6_rows(s, F("dc"), I, Pr, (int)I, false, B("dc6"), 6 * I);
            // dxs = da·w1ᵀ + dc·w3ᵀ
            p.lda = 6 * I; p.ldb = 6 * I; p.N = (int)H; p.K = (int)(6 * I);
            p.C32 = F("dxs"); p.ldc32 = H;
            p.A = B("da6"); p.accumulate = 0;
            for (int64_t e = 0; e < E; ++e) p.B_e[e] = tn.params["e" + std::to_string(e) + ".w1"]->b6;
            k::gemm_bf16_launch(s, p);
            p.A = B("dc6"); p.accumulate = 1;
            for (int64_t e = 0; e < E; ++e) p.B_e[e] = tn.params["e" + std::to_string(e) + ".w3"]->b6;
            k::gemm_bf16_launch(s, p);
            // Expert weight gradients: segments of the six-part K are six times the rows'.
            k::scale_i32(s, offs, (int)(E + 1), 6, seg6);
            k::scale_i32(s, counts, (int)E, 6, seg6 + E + 1);
            k::split6_transpose(s, x, H, sop, (int)K, (int)Pr, (int)H, false, B("xpt6"), 6 * Pr);
            k::split6_transpose(s, F("h"), I, nullptr, 1, (int)Pr, (int)I, false, B("ht6"), 6 * Pr);
            k::split6_transpose(s, dys, H, nullptr, 1, (int)Pr, (int)H, true, B("dyst6"), 6 * Pr);
            k::split6_transpose(s, F("da"), I, nullptr, 1, (int)Pr, (int)I, true, B("dat6"), 6 * Pr);
            k::split6_transpose(s, F("dc"), I, nullptr, 1, (int)Pr, (int)I, true, B("dct6"), 6 * Pr);
            k::GemmBf16Params r = gp();
            r.grid = k::GRID_SEGK; r.seg_offsets = seg6; r.seg_counts = seg6 + E + 1; r.segk_aligned = 1;
            r.n_experts = (int)E; r.epi = k::EPI_STORE;
            auto segk = [&](const bf16_t *A, const bf16_t *Bm, int M, int N, const char *port) {
                r.A = A; r.lda = 6 * Pr; r.B = Bm; r.ldb = 6 * Pr; r.M = M; r.N = N; r.K = (int)(6 * Pr); r.ldc32 = N;
                for (int64_t e = 0; e < E; ++e) r.C_e[e] = tn.params["e" + std::to_string(e) + port]->grad;
                k::gemm_bf16_launch(s, r);
            };
            segk(B("ht6"), B("dyst6"), (int)I, (int)H, ".w2");
            segk(B("xpt6"), B("dat6"), (int)H, (int)I, ".w1");
            segk(B("xpt6"), B("dct6"), (int)H, (int)I, ".w3");
            // Router (straight-through on the indices) and the input cotangent.
            float *dl = F("dl");
            k::router_backward(s, idx, w, dw, x, (int)T, (int)H, (int)E, (int)K, dl, tn.params["gate"]->grad,
                               F("router"));
            if (dx) k::moe_dx(s, F("dxs"), pos, dl, tn.params["gate"]->master, (int)T, (int)K, (int)H, (int)E, dx, acc);
            break;
        }
        default:
            fail(CATNN_ERR_UNSUPPORTED, "training: op " + op_name(tn.kind));
    }
}

// The six-part copies of every GEMM weight from its fp32 master.
static void refresh_split_copies(Tr &t) {
    hipStream_t s = t.dev->stream;
    for (auto &p : t.params) {
        if (p->want_b6) k::split6_rows(s, p->master, p->cols, p->rows, (int)p->cols, true, p->b6, 6 * p->cols);
        if (p->want_bt6)
            k::split6_transpose(s, p->master, p->cols, nullptr, 1, (int)p->rows, (int)p->cols, true, p->bt6,
                                6 * p->rows);
    }
}

// ------------------------------------------------------------ forward

static void forward_node(Tr &t, TNode &tn) {
    if (tn.skip_fwd) return;  // a GELU applied by the producing Linear's epilogue
    if (t.prec == CATNN_PREC_FP32 && is_gemm_op(tn.kind)) return forward_gemm_f32(t, tn);
    hipStream_t s = t.dev->stream;
    const Node &nd = *tn.node;
    float *y = t.val.at(tn.id);
    const float *x = tn.ins.empty() ? nullptr : t.val.at(tn.ins[0]);
    const auto &xd = tn.ins.empty() ? tn.dims : tn.in_dims[0];
    const int64_t nx = numel(xd);
    switch (tn.kind) {
        case CATNN_OP_IDENTITY: case CATNN_OP_RESHAPE: case CATNN_OP_TRANSPOSE:
            if (x) k::copy_f32(s, x, y, nx);
            else k::fill_f32(s, y, 0.f, numel(tn.dims));
            break;
        case CATNN_OP_RELU: case CATNN_OP_GELU:
            k::act_f32(s, x, y, nx, tn.kind);
            break;
        case CATNN_OP_ADD: case CATNN_OP_RESIDUAL_ADD:
            if (tn.ins.size() > 1) k::add_f32(s, x, t.val.at(tn.ins[1]), y, nx, nx);
            else k::copy_f32(s, x, y, nx);
            break;
        case CATNN_OP_MUL:
            if (tn.ins.size() > 1) k::mul_f32(s, x, t.val.at(tn.ins[1]), y, nx);
            else k::copy_f32(s, x, y, nx);
            break;
        case CATNN_OP_SOFTMAX: {
            const int64_t C = xd.back();
            k::softmax_f32(s, x, y, nx / C, C);
            break;
        }
        case CATNN_OP_LINEAR: case CATNN_OP_MATMUL: case CATNN_OP_LM_HEAD: {
            TParam *w = tn.params.begin()->second;
            for (auto &kv : tn.params) if (kv.first != "b") w = kv.second;
            TParam *b = tn.params.count("b") ? tn.params["b"] : nullptr;
            const int64_t K = w->rows, N = w->cols, M = nx / K;
            bf16_t *xb = (bf16_t *)tn.B("xb");
            if (!tn.xb_ready) k::cast_f32_bf16(s, x, xb, M * K);
            k::GemmBf16Params p = gp();
            p.A = xb; p.lda = K; p.B = w->bt; p.ldb = K;
            p.M = (int)M; p.N = (int)N; p.K = (int)K;
            p.epi = k::EPI_LINEAR; p.bias = b ? b->master : nullptr;
            if (tn.gelu_next != UINT32_MAX) {
                // y = x·w + b (the GELU adjoint's Z), then GELU into the next
                // Linear's bf16 operand.
                p.Z = y; p.ldz = N; p.act = 3;
                p.Cb = (bf16_t *)t.nodes[t.index.at(tn.gelu_next)].B("xb"); p.ldcb = N;
            } else if (tn.res_into != UINT32_MAX) {
                // the Add after it: other + (x·w + b)
                p.R = t.val.at(tn.res_other); p.ldr = N;
                p.C32 = t.val.at(tn.res_into); p.ldc32 = N;
            } else {
                p.C32 = y; p.ldc32 = N;
            }
            k::gemm_bf16_launch(s, p);
            break;
        }
        case CATNN_OP_SWIGLU: {
            // a = x·w1, c = x·w3 and y = h·w2 with h = silu(a)·c, each GEMM on
            // bf16 operands as Linear's forward.
            TParam *w1 = tn.params["w1"], *w3 = tn.params["w3"], *w2 = tn.params["w2"];
            const int64_t H = w1->rows, I = w1->cols, M = nx / H;
            bf16_t *xb = (bf16_t *)tn.B("xb"), *hb = (bf16_t *)tn.B("hb");
            float *a = (float *)tn.B("a"), *c = (float *)tn.B("c"), *h = (float *)tn.B("h");
            auto bf16_gemm = [&](const bf16_t *A, int64_t K, const TParam *w, float *C) {
                k::GemmBf16Params p = gp();
                p.A = A; p.lda = K; p.B = w->bt; p.ldb = K;
                p.M = (int)M; p.N = (int)w->cols; p.K = (int)K;
                p.epi = k::EPI_LINEAR; p.C32 = C; p.ldc32 = w->cols;
                k::gemm_bf16_launch(s, p);
            };
            k::cast_f32_bf16(s, x, xb, M * H);
            bf16_gemm(xb, H, w1, a);
            bf16_gemm(xb, H, w3, c);
            k::swiglu_h(s, a, c, h, M * I);
            k::cast_f32_bf16(s, h, hb, M * I);
            bf16_gemm(hb, I, w2, y);
            break;
        }
        case CATNN_OP_EMBEDDING:  // ids are checked against the vocabulary by set_batch
            k::embedding_f32(s, x, nx, tn.params["w"]->master, nd.op.a[0], nd.op.a[1], y, (int *)tn.B("bad"));
            break;
        case CATNN_OP_MIX: {
            const float *gate = tn.params.count("gate") ? tn.params["gate"]->master : nullptr;
            k::mix_f32(s, x, t.val.at(tn.ins[1]), gate, y, nx);
            break;
        }
        case CATNN_OP_RMS_NORM: {
            const int64_t C = xd.back();
            k::rms_norm_f32(s, x, tn.params["w"]->master, y, nx / C, C, (float)nd.op.a[0] * 1e-6f);
            break;
        }
        case CATNN_OP_LAYER_NORM: {
            const int64_t C = xd.back();
            const float eps = (float)nd.op.a[0] * 1e-6f;
            bf16_t *yb = nullptr, *y3 = nullptr;
            if (tn.ln_next != UINT32_MAX) {
                TNode &cn = t.nodes[t.index.at(tn.ln_next)];
                if (cn.x3_ready) y3 = (bf16_t *)cn.B("x3");
                else yb = (bf16_t *)cn.B("xb");
            }
            k::ln_forward_train(s, x, tn.params["gamma"]->master, tn.params["beta"]->master,
                                tn.ln_next != UINT32_MAX ? nullptr : y, yb, y3, (float *)tn.B("mean"),
                                (float *)tn.B("rstd"), nx / C, (int)C, eps);
            break;
        }
        case CATNN_OP_ATTENTION: {
            const int64_t Bt = xd[0], S = xd[1], D = xd[2], T = Bt * S;
            const int64_t H = nd.op.a[0], dh = nd.op.a[2];
            const bool causal = (nd.op.flags & CATNN_FLAG_CAUSAL) != 0;
            bf16_t *x3 = (bf16_t *)tn.B("x3"), *ctx3 = (bf16_t *)tn.B("ctx3");
            float *ctx = (float *)tn.B("ctx");
            // Both projections split-bf16 (K' = 3D).
            if (!tn.x3_ready) k::split3_rows(s, x, D, T, (int)D, x3, 3 * D);
            if (attn_core_bf16(nd, D)) {
                // q, k, v in bf16 (and transposed per batch element) for the
                // core on bf16 MFMA.
                bf16_t *qkvb = (bf16_t *)tn.B("qkvb"), *qkvt = (bf16_t *)tn.B("qkvt");
                k::GemmBf16Params p = gp();
                p.A = x3; p.lda = 3 * D; p.B = tn.params["wqkv"]->bt3; p.ldb = 3 * D;
                p.M = (int)T; p.N = (int)(3 * D); p.K = (int)(3 * D);
                p.epi = k::EPI_STORE; p.Cb = qkvb; p.ldcb = 3 * D;
                k::gemm_bf16_launch(s, p);
                k::transpose_bt(s, qkvb, 3 * D, Bt, S, 3 * D, qkvt);
                k::attention_core_fwd_bf16(s, qkvb, 3 * D, qkvt, ctx, D, (float *)tn.B("lse"), Bt, S, H, causal);
            } else {
                float *qkv = (float *)tn.B("qkv");
                gemm_nt(s, x3, 3 * D, tn.params["wqkv"]->bt3, 3 * D, (int)T, (int)(3 * D), (int)(3 * D), qkv,
                        3 * D, false);
                k::attention_core_fwd_lse(s, qkv, qkv + D, qkv + 2 * D, 3 * D, ctx, D, (float *)tn.B("lse"), Bt,
                                          S, H, dh, causal);
            }
            k::split3_rows(s, ctx, D, T, (int)D, ctx3, 3 * D);
            if (tn.res_into != UINT32_MAX) {  // the Add after it: other + ctx·wo
                k::GemmBf16Params p = gp();
                p.A = ctx3; p.lda = 3 * D; p.B = tn.params["wo"]->bt3; p.ldb = 3 * D;
                p.M = (int)T; p.N = (int)D; p.K = (int)(3 * D);
                p.epi = k::EPI_LINEAR; p.R = t.val.at(tn.res_other); p.ldr = D;
                p.C32 = t.val.at(tn.res_into); p.ldc32 = D;
                k::gemm_bf16_launch(s, p);
            } else {
                gemm_nt(s, ctx3, 3 * D, tn.params["wo"]->bt3, 3 * D, (int)T, (int)D, (int)(3 * D), y, D, false);
            }
            break;
        }
        case CATNN_OP_GQA_ATTENTION: {
            const int64_t Bt = xd[0], S = xd[1], D = xd[2], T = Bt * S;
            const int64_t H = nd.op.a[0], HKV = nd.op.a[1], hd = nd.op.a[2];
            const int64_t QW = H * hd, KW = HKV * hd, LD = QW + 2 * KW;
            // sliding_window None is −1; Some(0) means no window, as the inference path.
            const int64_t window = nd.op.a[4] > 0 ? nd.op.a[4] : 0;
            bf16_t *x3 = (bf16_t *)tn.B("x3"), *ctx3 = (bf16_t *)tn.B("ctx3");
            float *qkv = (float *)tn.B("qkv"), *ctx = (float *)tn.B("ctx"), *rope = (float *)tn.B("rope");
            // Projections split-bf16 as Attention's; RoPE on q and k in place;
            // the grouped, windowed causal core on fp32 MFMA with its lse kept.
            if (!tn.x3_ready) k::split3_rows(s, x, D, T, (int)D, x3, 3 * D);
            gemm_nt(s, x3, 3 * D, tn.params["wqkv"]->bt3, 3 * D, (int)T, (int)LD, (int)(3 * D), qkv, LD, false);
            k::rope_table(s, rope, S, hd, (double)nd.op.a[5]);
            k::rope_apply(s, qkv, LD, T, S, H + HKV, hd, rope, 1.0f);
            k::attention_core_fwd_lse_gqa(s, qkv, LD, qkv + QW, qkv + QW + KW, LD, H / HKV, window, ctx, QW,
                                          (float *)tn.B("lse"), Bt, S, H, hd);
            k::split3_rows(s, ctx, QW, T, (int)QW, ctx3, 3 * QW);
            gemm_nt(s, ctx3, 3 * QW, tn.params["wo"]->bt3, 3 * QW, (int)T, (int)D, (int)(3 * QW), y, D, false);
            break;
        }
        case CATNN_OP_MOE: {
            const int64_t E = nd.op.a[0], K = nd.op.a[1], H = xd.back(), T = nx / H;
            const int64_t I = tn.params["e0.w1"]->cols;
            const int64_t P = T * K + E * (kPad - 1);
            const int64_t Pr = (P + kPad - 1) / kPad * kPad;
            int32_t *idx = (int32_t *)tn.B("idx"), *counts = (int32_t *)tn.B("counts");
            int32_t *offs = (int32_t *)tn.B("offsets"), *sop = (int32_t *)tn.B("sop");
            int32_t *pos = (int32_t *)tn.B("pos"), *tiles = (int32_t *)tn.B("tiles");
            float *w = (float *)tn.B("w");
            k::moe_route_f32(s, x, tn.params["gate"]->master, T, H, E, K, idx, w, nullptr);
            k::moe_permute_padded(s, idx, T, K, E, kPad, Pr, counts, offs, sop, pos, tn.B("perm_scratch"));
            k::gemm_bf16_build_tiles(s, offs, (int)E, T * K, tiles);
            bf16_t *x3 = (bf16_t *)tn.B("x3");
            k::split3_rows(s, x, H, T, (int)H, x3, 3 * H);
            k::GemmBf16Params p = gp();
            p.grid = k::GRID_ROWS;
            k::gemm_bf16_use_tiles(p, tiles, T * K, (int)E);
            p.seg_offsets = offs; p.seg_counts = counts; p.n_experts = (int)E;
            // gate/up: h = silu(x·w1)·(x·w3), a and c kept for the adjoint;
            // [hi|lo] of x against [hi|hi] of the weights over 2H.
            const bool wrap = moe_kwrap(H);
            p.A = x3; p.lda = 3 * H; p.a_rows = sop; p.a_row_div = (int)K;
            for (int64_t e = 0; e < E; ++e) {
                const TParam *w1 = tn.params["e" + std::to_string(e) + ".w1"];
                const TParam *w3 = tn.params["e" + std::to_string(e) + ".w3"];
                p.B_e[e] = wrap ? w1->bt : w1->bt3;
                p.B2_e[e] = wrap ? w3->bt : w3->bt3;
            }
            p.ldb = wrap ? H : 3 * H; p.b_kwrap = wrap ? (int)H : 0;
            p.M = 0; p.N = (int)I; p.K = (int)(2 * H);
            p.epi = k::EPI_SWIGLU_FWD;
            p.Cb = (bf16_t *)tn.B("h"); p.ldcb = I;
            p.S1 = (bf16_t *)tn.B("a"); p.S2 = (bf16_t *)tn.B("c"); p.lds = I;
            k::gemm_bf16_launch(s, p);
            // down: ys = h·w2
            k::GemmBf16Params q = p;
            q.A = (bf16_t *)tn.B("h"); q.lda = I; q.a_rows = nullptr; q.a_row_div = 1;
            for (int64_t e = 0; e < E; ++e) {
                q.B_e[e] = tn.params["e" + std::to_string(e) + ".w2"]->bt;
                q.B2_e[e] = nullptr;
            }
            q.ldb = I; q.N = (int)H; q.K = (int)I; q.b_kwrap = 0;
            q.epi = k::EPI_STORE; q.Cb = nullptr; q.S1 = q.S2 = nullptr;
            q.C32 = (float *)tn.B("ys"); q.ldc32 = H;
            k::gemm_bf16_launch(s, q);
            k::moe_combine(s, (float *)tn.B("ys"), pos, w, T, K, H, y);
            break;
        }
        default:
            fail(CATNN_ERR_UNSUPPORTED, "training: op " + op_name(tn.kind));
    }
}

// ----------------------------------------------------------- backward

static void backward_node(Tr &t, TNode &tn) {
    if (t.prec == CATNN_PREC_FP32 && is_gemm_op(tn.kind)) return backward_gemm_f32(t, tn);
    hipStream_t s = t.dev->stream;
    const Node &nd = *tn.node;
    const float *dy = t.grad.at(tn.id);
    auto dst = [&](size_t i) -> float * {
        return t.input_ids.count(tn.ins[i]) && !t.input_grads ? nullptr : t.grad.at(tn.ins[i]);
    };
    const float *x = tn.ins.empty() ? nullptr : t.val.at(tn.ins[0]);
    const auto &xd = tn.ins.empty() ? tn.dims : tn.in_dims[0];
    const int64_t nx = numel(xd);
    switch (tn.kind) {
        case CATNN_OP_IDENTITY: case CATNN_OP_RESHAPE: case CATNN_OP_TRANSPOSE:
            if (!tn.ins.empty() && dst(0)) add_into(s, dst(0), dy, nx, tn.first_writer[0]);
            break;
        case CATNN_OP_ADD: case CATNN_OP_RESIDUAL_ADD:
            for (size_t i = 0; i < tn.ins.size(); ++i)
                if (dst(i)) add_into(s, dst(i), dy, nx, tn.first_writer[i]);
            break;
        case CATNN_OP_MUL:  // adjoint.rs:787-800
            if (tn.ins.size() == 1) {
                if (dst(0)) add_into(s, dst(0), dy, nx, tn.first_writer[0]);
            } else {
                if (dst(0)) k::mul_backward(s, dy, t.val.at(tn.ins[1]), dst(0), !tn.first_writer[0], nx);
                if (dst(1)) k::mul_backward(s, dy, x, dst(1), !tn.first_writer[1], nx);
            }
            break;
        case CATNN_OP_SOFTMAX: {
            const int64_t C = xd.back();
            if (dst(0)) k::softmax_backward(s, t.val.at(tn.id), dy, dst(0), !tn.first_writer[0], nx / C, (int)C);
            break;
        }
        case CATNN_OP_RELU: case CATNN_OP_GELU:
            if (dst(0)) k::act_backward(s, x, dy, dst(0), nx, tn.kind, !tn.first_writer[0]);
            break;
        case CATNN_OP_LINEAR: case CATNN_OP_MATMUL: case CATNN_OP_LM_HEAD: {
            TParam *w = tn.params.begin()->second;
            for (auto &kv : tn.params) if (kv.first != "b") w = kv.second;
            TParam *b = tn.params.count("b") ? tn.params["b"] : nullptr;
            const int64_t K = w->rows, N = w->cols, M = nx / K;
            bf16_t *dyb = (bf16_t *)tn.B("dyb"), *dybt = (bf16_t *)tn.B("dybt");
            bf16_t *xb = (bf16_t *)tn.B("xb"), *xbt = (bf16_t *)tn.B("xbt");
            // dyb = bf16(dy) (unless the GELU-adjoint epilogue wrote it), its
            // transpose and the bias gradient in one pass over dy where the
            // shape allows; else the cast, the transpose of dyb and the
            // column sums.
            float *cs = b ? (float *)tn.B("colsum") : nullptr;
            bool t_done = false, b_done = false;
            if (!tn.dyb_ready) {
                t_done = k::transpose_colsum(s, dy, M, (int)N, dybt, M, b ? b->grad : nullptr, false, cs, dyb);
                b_done = t_done && b;
                if (!t_done) k::cast_f32_bf16(s, dy, dyb, M * N);
            }
            if (tn.gelu_pre != UINT32_MAX) {
                // dA = (dy·Wᵀ) ∘ gelu'(A's output): A's cotangent and its bf16 copy.
                TNode &an = t.nodes[t.index.at(tn.gelu_pre)];
                k::GemmBf16Params p = gp();
                p.A = dyb; p.lda = N; p.B = w->b; p.ldb = N;
                p.M = (int)M; p.N = (int)K; p.K = (int)N;
                p.epi = k::EPI_GELU_BWD; p.Z = t.val.at(an.id); p.ldz = K;
                p.C32 = t.grad.at(an.id); p.ldc32 = K; p.accumulate = 0;
                p.Cb = (bf16_t *)an.B("dyb"); p.ldcb = K;
                k::gemm_bf16_launch(s, p);
            } else if (dst(0)) {
                gemm_nt(s, dyb, N, w->b, N, (int)M, (int)K, (int)N, dst(0), K, !tn.first_writer[0]);
            }
            if (!t_done && b) t_done = b_done = k::transpose_colsum(s, dy, M, (int)N, dybt, M, b->grad, false, cs);
            if (!t_done) k::transpose_bf16(s, dyb, N, nullptr, 1, (int)M, (int)N, dybt, M);
            k::transpose_bf16(s, xb, K, nullptr, 1, (int)M, (int)K, xbt, M);
            gemm_nt(s, xbt, M, dybt, M, (int)K, (int)N, (int)M, w->grad, N, false, (float *)tn.B("wparts"));
            if (b && !b_done) k::colsum(s, dy, M, (int)N, b->grad, false, cs);
            break;
        }
        case CATNN_OP_SWIGLU: {  // swiglu_backward, adjoint.rs:217-251
            TParam *w1 = tn.params["w1"], *w3 = tn.params["w3"], *w2 = tn.params["w2"];
            const int64_t H = w1->rows, I = w1->cols, M = nx / H;
            bf16_t *dyb = (bf16_t *)tn.B("dyb"), *dybt = (bf16_t *)tn.B("dybt"), *dab = (bf16_t *)tn.B("dab"),
                   *dcb = (bf16_t *)tn.B("dcb"), *dabt = (bf16_t *)tn.B("dabt"), *dcbt = (bf16_t *)tn.B("dcbt"),
                   *xbt = (bf16_t *)tn.B("xbt"), *hbt = (bf16_t *)tn.B("hbt"), *xb = (bf16_t *)tn.B("xb"),
                   *hb = (bf16_t *)tn.B("hb");
            float *dh = (float *)tn.B("dh"), *wparts = (float *)tn.B("wparts");
            k::cast_f32_bf16(s, dy, dyb, M * H);
            gemm_nt(s, dyb, H, w2->b, H, (int)M, (int)I, (int)H, dh, I, false);  // dh = dy·w2ᵀ
            k::swiglu_dadc(s, dh, (const float *)tn.B("a"), (const float *)tn.B("c"), dab, dcb, M * I);
            if (dst(0)) {  // dx = da·w1ᵀ + dc·w3ᵀ
                gemm_nt(s, dab, I, w1->b, I, (int)M, (int)H, (int)I, dst(0), H, !tn.first_writer[0]);
                gemm_nt(s, dcb, I, w3->b, I, (int)M, (int)H, (int)I, dst(0), H, true);
            }
            k::transpose_bf16(s, xb, H, nullptr, 1, (int)M, (int)H, xbt, M);
            k::transpose_bf16(s, dab, I, nullptr, 1, (int)M, (int)I, dabt, M);
            k::transpose_bf16(s, dcb, I, nullptr, 1, (int)M, (int)I, dcbt, M);
            gemm_nt(s, xbt, M, dabt, M, (int)H, (int)I, (int)M, w1->grad, I, false, wparts);  // dw1 = xᵀ·da
            gemm_nt(s, xbt, M, dcbt, M, (int)H, (int)I, (int)M, w3->grad, I, false, wparts);  // dw3 = xᵀ·dc
            k::transpose_bf16(s, hb, I, nullptr, 1, (int)M, (int)I, hbt, M);
            k::transpose_bf16(s, dyb, H, nullptr, 1, (int)M, (int)H, dybt, M);
            gemm_nt(s, hbt, M, dybt, M, (int)I, (int)H, (int)M, w2->grad, H, false, wparts);  // dw2 = hᵀ·dy
            break;
        }
        case CATNN_OP_EMBEDDING:
            // adjoint.rs:843-848: the ids receive the zero cotangent.
            if (dst(0) && tn.first_writer[0]) k::fill_f32(s, dst(0), 0.f, nx);
            k::embedding_backward(s, x, nx, dy, nd.op.a[0], nd.op.a[1], tn.params["w"]->grad, (int *)tn.B("idi"),
                                  (int *)tn.B("hit"));
            break;
        case CATNN_OP_MIX: {
            TParam *g = tn.params.count("gate") ? tn.params["gate"] : nullptr;
            k::mix_backward(s, x, t.val.at(tn.ins[1]), g ? g->master : nullptr, dy, dst(0),
                            dst(0) && !tn.first_writer[0], dst(1), dst(1) && !tn.first_writer[1], nx,
                            g ? g->grad : nullptr, (float *)tn.B("parts"));
            break;
        }
        case CATNN_OP_RMS_NORM: {
            const int64_t C = xd.back();
            float *dx = dst(0);
            k::rms_backward(s, x, tn.params["w"]->master, dy, dx, dx && !tn.first_writer[0], tn.params["w"]->grad,
                            nx / C, (int)C, (float)nd.op.a[0] * 1e-6f, (float *)tn.B("prod"),
                            (float *)tn.B("colsum"));
            break;
        }
        case CATNN_OP_LAYER_NORM: {
            const int64_t C = xd.back();
            float *dx = dst(0);  // null when the input is the graph input
            k::ln_backward(s, x, tn.params["gamma"]->master, (float *)tn.B("mean"), (float *)tn.B("rstd"), dy,
                           dx, dx && !tn.first_writer[0], tn.params["gamma"]->grad,
                           tn.params["beta"]->grad, false, nx / C, (int)C, (float *)tn.B("parts"));
            break;
        }
        case CATNN_OP_ATTENTION: {
            const int64_t Bt = xd[0], S = xd[1], D = xd[2], T = Bt * S;
            const int64_t H = nd.op.a[0], dh = nd.op.a[2];
            const bool causal = (nd.op.flags & CATNN_FLAG_CAUSAL) != 0;
            TParam *wqkv = tn.params["wqkv"], *wo = tn.params["wo"];
            bf16_t *dyb = (bf16_t *)tn.B("dyb"), *dybt = (bf16_t *)tn.B("dybt"), *ctxt = (bf16_t *)tn.B("ctxt");
            float *dctx = (float *)tn.B("dctx"), *dqkv = (float *)tn.B("dqkv");
            bf16_t *dqkvb = (bf16_t *)tn.B("dqkvb"), *dqkvt = (bf16_t *)tn.B("dqkvt");
            bf16_t *x3 = (bf16_t *)tn.B("x3"), *xbt = (bf16_t *)tn.B("xbt");
            const bool core_bf16 = attn_core_bf16(nd, D);
            // bf16(dy) and its transpose in one pass where the shape allows
            const bool dy_t = k::transpose_colsum(s, dy, T, (int)D, dybt, T, nullptr, false, nullptr, dyb);
            if (!dy_t) k::cast_f32_bf16(s, dy, dyb, T * D);
            {  // dctx = dy·woᵀ (and its bf16 copy for the bf16 core)
                k::GemmBf16Params p = gp();
                p.A = dyb; p.lda = D; p.B = wo->b; p.ldb = D;
                p.M = (int)T; p.N = (int)D; p.K = (int)D;
                p.epi = k::EPI_STORE; p.C32 = dctx; p.ldc32 = D;
                if (core_bf16) { p.Cb = (bf16_t *)tn.B("dctxb"); p.ldcb = D; }
                k::gemm_bf16_launch(s, p);
            }
            if (!dy_t) k::transpose_bf16(s, dyb, D, nullptr, 1, (int)T, (int)D, dybt, T);
            k::transpose_bf16(s, (bf16_t *)tn.B("ctx3"), 3 * D, nullptr, 1, (int)T, (int)D, ctxt, T);
            gemm_nt(s, ctxt, T, dybt, T, (int)D, (int)D, (int)T, wo->grad, D, false, (float *)tn.B("wparts"));
            if (core_bf16) {
                bf16_t *dctxb = (bf16_t *)tn.B("dctxb"), *dctxt = (bf16_t *)tn.B("dctxt");
                k::transpose_bt(s, dctxb, D, Bt, S, D, dctxt);
                k::attention_core_bwd_bf16(s, (bf16_t *)tn.B("qkvb"), 3 * D, (bf16_t *)tn.B("qkvt"),
                                           (float *)tn.B("ctx"), dctx, D, dctxb, dctxt, (float *)tn.B("lse"), dqkv,
                                           3 * D, Bt, S, H, causal, (float *)tn.B("dscr"));
            } else {
                float *qkv = (float *)tn.B("qkv");
                k::attention_core_bwd(s, qkv, qkv + D, qkv + 2 * D, 3 * D, (float *)tn.B("ctx"), dctx, D,
                                      (float *)tn.B("lse"), dqkv, dqkv + D, dqkv + 2 * D, 3 * D, Bt, S, H, dh,
                                      causal, (float *)tn.B("dscr"));
            }
            const bool dqkv_t = k::transpose_colsum(s, dqkv, T, (int)(3 * D), dqkvt, T, nullptr, false, nullptr, dqkvb);
            if (!dqkv_t) k::cast_f32_bf16(s, dqkv, dqkvb, T * 3 * D);
            if (dst(0))
                gemm_nt(s, dqkvb, 3 * D, wqkv->b, 3 * D, (int)T, (int)D, (int)(3 * D), dst(0), D,
                        !tn.first_writer[0]);
            if (!dqkv_t) k::transpose_bf16(s, dqkvb, 3 * D, nullptr, 1, (int)T, (int)(3 * D), dqkvt, T);
            k::transpose_bf16(s, x3, 3 * D, nullptr, 1, (int)T, (int)D, xbt, T);
            gemm_nt(s, xbt, T, dqkvt, T, (int)D, (int)(3 * D), (int)T, wqkv->grad, 3 * D, false,
                    (float *)tn.B("wparts"));
            break;
        }
        case CATNN_OP_GQA_ATTENTION: {  // gqa_backward, adjoint.rs:287-440
            const int64_t Bt = xd[0], S = xd[1], D = xd[2], T = Bt * S;
            const int64_t H = nd.op.a[0], HKV = nd.op.a[1], hd = nd.op.a[2];
            const int64_t QW = H * hd, KW = HKV * hd, LD = QW + 2 * KW;
            const int64_t window = nd.op.a[4] > 0 ? nd.op.a[4] : 0;
            TParam *wqkv = tn.params["wqkv"], *wo = tn.params["wo"];
            bf16_t *dyb = (bf16_t *)tn.B("dyb"), *dybt = (bf16_t *)tn.B("dybt"), *ctxt = (bf16_t *)tn.B("ctxt");
            bf16_t *dqkvb = (bf16_t *)tn.B("dqkvb"), *dqkvt = (bf16_t *)tn.B("dqkvt");
            bf16_t *x3 = (bf16_t *)tn.B("x3"), *xbt = (bf16_t *)tn.B("xbt");
            float *dctx = (float *)tn.B("dctx"), *dqkv = (float *)tn.B("dqkv"), *qkv = (float *)tn.B("qkv");
            float *wparts = (float *)tn.B("wparts");
            // dctx = dy·woᵀ, dwo = ctxᵀ·dy
            k::cast_f32_bf16(s, dy, dyb, T * D);
            gemm_nt(s, dyb, D, wo->b, D, (int)T, (int)QW, (int)D, dctx, QW, false);
            k::transpose_bf16(s, dyb, D, nullptr, 1, (int)T, (int)D, dybt, T);
            k::transpose_bf16(s, (bf16_t *)tn.B("ctx3"), 3 * QW, nullptr, 1, (int)T, (int)QW, ctxt, T);
            gemm_nt(s, ctxt, T, dybt, T, (int)QW, (int)D, (int)T, wo->grad, D, false, wparts);
            // The core's adjoint on the rotated q, k: dk, dv of a K/V head sum
            // its query heads in head order; then dq, dk rotated back by −θ.
            k::attention_core_bwd_gqa(s, qkv, LD, qkv + QW, qkv + QW + KW, LD, H / HKV, window,
                                      (float *)tn.B("ctx"), dctx, QW, (float *)tn.B("lse"), dqkv, LD, dqkv + QW,
                                      dqkv + QW + KW, LD, Bt, S, H, hd, true, (float *)tn.B("dscr"));
            k::rope_apply(s, dqkv, LD, T, S, H + HKV, hd, (float *)tn.B("rope"), -1.0f);
            // dx = dqkv·wqkvᵀ (dxq + dxk + dxv), dwqkv = xᵀ·dqkv
            k::cast_f32_bf16(s, dqkv, dqkvb, T * LD);
            if (dst(0))
                gemm_nt(s, dqkvb, LD, wqkv->b, LD, (int)T, (int)D, (int)LD, dst(0), D, !tn.first_writer[0]);
            k::transpose_bf16(s, dqkvb, LD, nullptr, 1, (int)T, (int)LD, dqkvt, T);
            k::transpose_bf16(s, x3, 3 * D, nullptr, 1, (int)T, (int)D, xbt, T);  // hi part of x
            gemm_nt(s, xbt, T, dqkvt, T, (int)D, (int)LD, (int)T, wqkv->grad, LD, false, wparts);
            break;
        }
        case CATNN_OP_MOE: {
            const int64_t E = nd.op.a[0], K = nd.op.a[1], H = xd.back(), T = nx / H;
            const int64_t I = tn.params["e0.w1"]->cols;
            const int64_t P = T * K + E * (kPad - 1);
            const int64_t Pr = (P + kPad - 1) / kPad * kPad;
            int32_t *idx = (int32_t *)tn.B("idx"), *counts = (int32_t *)tn.B("counts");
            int32_t *offs = (int32_t *)tn.B("offsets"), *sop = (int32_t *)tn.B("sop");
            int32_t *pos = (int32_t *)tn.B("pos"), *tiles = (int32_t *)tn.B("tiles");
            float *w = (float *)tn.B("w"), *dw = (float *)tn.B("dw");
            bf16_t *dys = (bf16_t *)tn.B("dys"), *dadc = (bf16_t *)tn.B("dadc");
            float *dxs = (float *)tn.B("dxs");
            // Per slot: dys = w·dout[token], dw = <ys, dout[token]> (moe_backward's d_wts).
            k::moe_slot_grads(s, sop, w, (float *)tn.B("ys"), dy, (int)K, (int)H, (int)Pr, dys, dw);
            k::GemmBf16Params p = gp();
            p.grid = k::GRID_ROWS;
            k::gemm_bf16_use_tiles(p, tiles, T * K, (int)E);
            p.seg_offsets = offs; p.seg_counts = counts; p.n_experts = (int)E;
            // dh = dys·w2ᵀ, then da = dh·c·silu'(a), dc = dh·silu(a), side by
            // side in one row: [da | dc]
            p.A = dys; p.lda = H;
            for (int64_t e = 0; e < E; ++e) p.B_e[e] = tn.params["e" + std::to_string(e) + ".w2"]->b;
            p.ldb = H; p.N = (int)I; p.K = (int)H;
            p.epi = k::EPI_SWIGLU_BWD; p.Cb = dadc; p.Cb2 = dadc + I; p.ldcb = 2 * I;
            p.S1 = (bf16_t *)tn.B("a"); p.S2 = (bf16_t *)tn.B("c"); p.lds = I;
            k::gemm_bf16_launch(s, p);
            // dxs = da·w1ᵀ + dc·w3ᵀ = [da | dc]·[w1 | w3]ᵀ, one GEMM over K = 2I
            k::GemmBf16Params q = p;
            q.epi = k::EPI_STORE; q.Cb = q.Cb2 = nullptr; q.S1 = q.S2 = nullptr;
            q.A = dadc; q.lda = 2 * I; q.ldb = 2 * I; q.N = (int)H; q.K = (int)(2 * I);
            q.C32 = dxs; q.ldc32 = H; q.accumulate = 0;
            for (int64_t e = 0; e < E; ++e) q.B_e[e] = tn.params["e" + std::to_string(e) + ".w1"]->b;
            k::gemm_bf16_launch(s, q);
            // Expert weight gradients: each expert reduces over its own segment.
            bf16_t *xpt = (bf16_t *)tn.B("xpt"), *ht = (bf16_t *)tn.B("ht"), *dyst = (bf16_t *)tn.B("dyst");
            bf16_t *dat = (bf16_t *)tn.B("dadct"), *dct = dat + I * Pr;
            k::transpose_bf16(s, (bf16_t *)tn.B("x3"), 3 * H, sop, (int)K, (int)Pr, (int)H, xpt, Pr);  // hi part of x
            k::transpose_bf16(s, (bf16_t *)tn.B("h"), I, nullptr, 1, (int)Pr, (int)I, ht, Pr);
            k::transpose_bf16(s, dys, H, nullptr, 1, (int)Pr, (int)H, dyst, Pr);
            // [daᵀ; dcᵀ].  (Written by the SwiGLU-adjoint GEMM's staged epilogue
            // as 16-byte column runs instead, the transposed stores made that
            // GEMM 92 us slower on config 5, as much as this transpose takes.)
            k::transpose_bf16(s, dadc, 2 * I, nullptr, 1, (int)Pr, (int)(2 * I), dat, Pr);
            k::GemmBf16Params r = gp();
            r.grid = k::GRID_SEGK; r.seg_offsets = offs; r.seg_counts = counts; r.segk_aligned = 1;
            r.n_experts = (int)E; r.epi = k::EPI_STORE;
            auto segk = [&](const bf16_t *A, const bf16_t *B, int M, int N, const char *port) {
                r.A = A; r.lda = Pr; r.B = B; r.ldb = Pr; r.M = M; r.N = N; r.K = (int)Pr; r.ldc32 = N;
                for (int64_t e = 0; e < E; ++e) r.C_e[e] = tn.params["e" + std::to_string(e) + port]->grad;
                k::gemm_bf16_launch(s, r);
            };
            segk(ht, dyst, (int)I, (int)H, ".w2");
            segk(xpt, dat, (int)H, (int)I, ".w1");
            segk(xpt, dct, (int)H, (int)I, ".w3");
            // Router (straight-through on the indices) and the input cotangent.
            float *dl = (float *)tn.B("dl");
            k::router_backward(s, idx, w, dw, x, (int)T, (int)H, (int)E, (int)K, dl, tn.params["gate"]->grad,
                               (float *)tn.B("router"));
            if (dst(0))
                k::moe_dx(s, dxs, pos, dl, tn.params["gate"]->master, (int)T, (int)K, (int)H, (int)E, dst(0),
                          !tn.first_writer[0]);
            break;
        }
        default:
            fail(CATNN_ERR_UNSUPPORTED, "training: op " + op_name(tn.kind));
    }
}

// Checkpointed values: the forward writes their own buffer; before the
// backward step of their first backward reader, their producer runs again
// into the "#recomp" copy, which the rest of the backward pass reads
// (ensure_act's rematerialisation, coord.rs:441-470, on the device).
static void forward_values_home(Tr &t) {
    for (const auto &kv : t.val_fwd) t.val[kv.first] = kv.second;
}

static void recompute_before(Tr &t, size_t reader) {
    for (const auto &kv : t.ckpt) {
        if (kv.second.first_reader != reader) continue;
        t.val[kv.first] = t.val_recomp.at(kv.first);
        forward_node(t, t.nodes[t.index.at(kv.first)]);
    }
}

static void reverse_steps(Tr &t) {
    for (size_t i = t.nodes.size(); i-- > 0;) {
        TNode &tn = t.nodes[i];
        if (!t.ckpt.empty()) recompute_before(t, i);
        if (!t.input_ids.count(tn.id) && t.has_grad.count(tn.id) && !tn.skip_bwd) backward_node(t, tn);
    }
}

static void train_step(Tr &t) {
    hipStream_t s = t.dev->stream;
    SkScope sk(t.sk_part);
    forward_values_home(t);
    for (auto &tn : t.nodes)
        if (!t.input_ids.count(tn.id)) forward_node(t, tn);
    const int64_t n_out = numel(t.dims[t.out_id]);
    if (t.classes)
        k::cross_entropy(s, t.val.at(t.out_id), t.class_ids, t.class_rows, (int)t.vocab, t.grad.at(t.out_id), t.loss,
                         t.ce_rows);
    else
        k::mse(s, t.val.at(t.out_id), t.target, t.grad.at(t.out_id), n_out, t.loss, t.mse_scratch);
    // A node whose output nobody reads receives no cotangent and is skipped,
    // as reference_train skips ids without an entry in `grads`.
    reverse_steps(t);
    // apply_update on the parameters of every node that received a
    // cotangent, and the refresh of their bf16 copies, in one launch.
    const k::UpdateRule rule = t.opt == CATNN_OPT_ADAM ? k::adam_rule(t.lr, ++t.adam_t) : k::sgd_rule(t.lr);
    k::sgd_multi(s, t.sgd_table, t.sgd_n, t.sgd_tiles, rule, true);
    if (t.prec == CATNN_PREC_FP32) refresh_split_copies(t);
}

// adjoint_of over the graph (no loss, no update): the forward for the
// tapes, then — once the caller has put the output's cotangent in place, at
// the loss tick of the plan — the reverse pass.
static void forward_pass(Tr &t) {
    SkScope sk(t.sk_part);
    forward_values_home(t);
    for (auto &tn : t.nodes)
        if (!t.input_ids.count(tn.id)) forward_node(t, tn);
}

static void reverse_pass(Tr &t) {
    SkScope sk(t.sk_part);
    reverse_steps(t);
}

static TParam *find_param(Tr &t, uint32_t node_id, const std::string &port, int64_t *col0,
                          int64_t *ncols) {
    auto it = t.index.find(node_id);
    CATNN_REQUIRE(it != t.index.end(), CATNN_ERR_UNKNOWN_COMPONENT, "unknown node " + std::to_string(node_id));
    TNode &tn = t.nodes[it->second];
    *col0 = 0;
    if (tn.kind == CATNN_OP_ATTENTION && (port == "wq" || port == "wk" || port == "wv")) {
        TParam *p = tn.params.at("wqkv");
        *col0 = port == "wq" ? 0 : port == "wk" ? p->rows : 2 * p->rows;
        *ncols = p->rows;
        return p;
    }
    if (tn.kind == CATNN_OP_GQA_ATTENTION && (port == "wq" || port == "wk" || port == "wv")) {
        TParam *p = tn.params.at("wqkv");
        const int64_t QW = tn.node->op.a[0] * tn.node->op.a[2], KW = tn.node->op.a[1] * tn.node->op.a[2];
        *col0 = port == "wq" ? 0 : port == "wk" ? QW : QW + KW;
        *ncols = port == "wq" ? QW : KW;
        return p;
    }
    auto pit = tn.params.find(port);
    CATNN_REQUIRE(pit != tn.params.end(), CATNN_ERR_UNKNOWN_PORT,
                  "unknown port " + port + " on interface " + tn.node->name);
    *ncols = pit->second->cols;
    return pit->second;
}

static void read_cols(Tr &t, const float *src, int64_t rows, int64_t cols, int64_t col0, int64_t ncols,
                      float *host, int64_t n);

// An Embedding that reads a graph input gets its ids checked here, on the
// host, before the step: the forward's conversion (round half away from
// zero, negative and NaN → 0), then id < vocab, as the handler refuses it.
static void check_embedding_ids(const Tr &t, const float *data, int64_t n) {
    for (const auto &tn : t.nodes) {
        if (tn.kind != CATNN_OP_EMBEDDING || tn.ins.empty() || !t.input_ids.count(tn.ins[0])) continue;
        const int64_t vocab = tn.node->op.a[0];
        for (int64_t i = 0; i < n; ++i) {
            const float r = std::round(data[i]);
            const int64_t id = !(r >= 0.f) ? 0 : r >= 4294967296.0f ? 4294967295ll : (int64_t)r;
            CATNN_REQUIRE(id < vocab, CATNN_ERR_SHAPE_MISMATCH,
                          "embedding " + tn.node->name + ": id " + std::to_string(id) + " >= vocab " +
                              std::to_string(vocab));
        }
    }
}

// A parameter-shaped buffer of p (master, gradient or moment) in the
// graph's layout: columns col0 … col0+ncols, or the whole transpose back
// when p is held transposed.
static void read_param_buf(Tr &t, const TParam *p, const float *src, int64_t col0, int64_t ncols, float *host,
                           int64_t n) {
    if (!p->transposed) {
        read_cols(t, src, p->rows, p->cols, col0, ncols, host, n);
        return;
    }
    std::vector<float> tmp((size_t)(p->rows * p->cols));
    read_cols(t, src, p->rows, p->cols, 0, p->cols, tmp.data(), p->rows * p->cols);
    CATNN_REQUIRE(n == p->rows * p->cols, CATNN_ERR_SHAPE_MISMATCH,
                  "host buffer holds " + std::to_string(n) + " values, tensor has " + std::to_string(p->rows * p->cols));
    for (int64_t r = 0; r < p->rows; ++r)
        for (int64_t c = 0; c < p->cols; ++c) host[c * p->rows + r] = tmp[(size_t)(r * p->cols + c)];
}

// Copies rows × ncols starting at column col0 of a [rows, cols] fp32 buffer.
static void read_cols(Tr &t, const float *src, int64_t rows, int64_t cols, int64_t col0, int64_t ncols,
                      float *host, int64_t n) {
    CATNN_REQUIRE(n == rows * ncols, CATNN_ERR_SHAPE_MISMATCH,
                  "host buffer holds " + std::to_string(n) + " values, tensor has " + std::to_string(rows * ncols));
    CATNN_HIP(hipMemcpy2DAsync(host, (size_t)ncols * 4, src + col0, (size_t)cols * 4, (size_t)ncols * 4,
                               (size_t)rows, hipMemcpyDeviceToHost, t.dev->stream));
    CATNN_HIP(hipStreamSynchronize(t.dev->stream));
}

// ------------------------------------------------ adjoint_of plan cache
// catnn_hip_run_adjoint keeps the one-node trainers it builds, keyed by the
// node's shape (op, flags, fields, input dims, parameter ports and dims), so
// a training wave that calls adjoint_of on the same nodes every step plans
// and hipMallocs each of them once.  At most kAdjointCacheEntries trainers
// and kAdjointCacheBytes of arena are kept; the least recently used goes
// first.
constexpr size_t kAdjointCacheEntries = 16;
constexpr uint64_t kAdjointCacheBytes = 16ull << 30;

struct TrainerFree {
    void operator()(catnn_hip_trainer *t) const {
        if (!t) return;
        (void)hipSetDevice(t->dev->ordinal);
        (void)hipStreamSynchronize(t->dev->stream);
        if (t->base) (void)hipFree(t->base);
        delete t;
    }
};

}  // namespace catnn

struct catnn_adjoint_cache {
    struct Entry {
        std::string key;
        std::unique_ptr<catnn_hip_trainer, catnn::TrainerFree> t;
        uint64_t used;
    };
    std::vector<Entry> entries;
    uint64_t clock = 0;
};

namespace catnn {

static std::string adjoint_key(const catnn_node *node, const catnn_tensor *inputs, int32_t n_inputs) {
    std::string k = std::to_string(node->op.kind) + "|" + std::to_string(node->op.flags);
    for (int i = 0; i < 8; ++i) k += "," + std::to_string(node->op.a[i]);
    for (int32_t i = 0; i < n_inputs; ++i) {
        k += "|in";
        for (int64_t d : dims_from_c(inputs[i])) k += "," + std::to_string(d);
    }
    for (int32_t j = 0; j < node->n_params; ++j) {
        k += "|" + std::string(node->params[j].port ? node->params[j].port : "");
        for (int64_t d : dims_from_c(node->params[j].value)) k += "," + std::to_string(d);
    }
    return k;
}

static catnn_hip_trainer *adjoint_cache_find(catnn_hip_device *dev, const std::string &key) {
    if (!dev->adj_cache) return nullptr;
    for (auto &e : dev->adj_cache->entries)
        if (e.key == key) {
            e.used = ++dev->adj_cache->clock;
            return e.t.get();
        }
    return nullptr;
}

static catnn_hip_trainer *adjoint_cache_insert(catnn_hip_device *dev, const std::string &key,
                                               std::unique_ptr<catnn_hip_trainer, TrainerFree> t) {
    if (!dev->adj_cache) dev->adj_cache = new catnn_adjoint_cache();
    auto &es = dev->adj_cache->entries;
    auto bytes = [&] {
        uint64_t b = t->reserved;
        for (auto &e : es) b += e.t->reserved;
        return b;
    };
    while (!es.empty() && (es.size() >= kAdjointCacheEntries || bytes() > kAdjointCacheBytes)) {
        auto lru = std::min_element(es.begin(), es.end(), [](const auto &a, const auto &b) { return a.used < b.used; });
        es.erase(lru);
    }
    es.push_back({key, std::move(t), ++dev->adj_cache->clock});
    return es.back().t.get();
}

void free_adjoint_cache(catnn_hip_device *dev) {
    delete dev->adj_cache;
    dev->adj_cache = nullptr;
}

}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_hip_gemm_bf16_nt(catnn_hip_device *dev, const uint16_t *a, int64_t lda, const uint16_t *b,
                           int64_t ldb, float *c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                           int32_t accumulate, int32_t tile_cfg) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m < (1ll << 31) && n < (1ll << 31) && k < (1ll << 31),
                      CATNN_ERR_SHAPE_MISMATCH, "gemm_bf16: dims");
        CATNN_REQUIRE(lda >= k && ldb >= k && ldc >= n, CATNN_ERR_SHAPE_MISMATCH, "gemm_bf16: leading dims");
        CATNN_REQUIRE((a && b && c) || m * n == 0, CATNN_ERR_INVALID_ARGUMENT, "gemm_bf16: null operand");
        CATNN_REQUIRE(tile_cfg == -1 || tile_cfg == 0 || tile_cfg == 2 || tile_cfg == 7 || tile_cfg == 9 ||
                          tile_cfg == 10 || tile_cfg == 11 || tile_cfg == 12,
                      CATNN_ERR_INVALID_ARGUMENT, "gemm_bf16: tile_cfg");
        k::GemmBf16Params p = gp();
        if (m * n > 0) p.sk_part = device_sk_scratch(dev);
        p.A = a; p.lda = lda; p.B = b; p.ldb = ldb;
        p.M = (int)m; p.N = (int)n; p.K = (int)k;
        p.epi = k::EPI_STORE; p.C32 = c; p.ldc32 = ldc; p.accumulate = accumulate ? 1 : 0;
        if (tile_cfg < 0) k::gemm_bf16_launch(dev->stream, p);
        else k::gemm_bf16_launch_cfg(dev->stream, p, tile_cfg);
    });
}

int catnn_hip_train_install(catnn_hip_device *dev, const catnn_graph *g, float lr,
                            catnn_hip_trainer **out) {
    return catnn_hip_train_install_opt(dev, g, CATNN_OPT_SGD, lr, out);
}

int catnn_hip_train_install_opt(catnn_hip_device *dev, const catnn_graph *g, int32_t optimizer, float lr,
                                catnn_hip_trainer **out) {
    const catnn_train_options o{optimizer, lr, CATNN_PREC_BF16, 0};
    return catnn_hip_train_install_ex(dev, g, &o, out);
}

int catnn_hip_train_install_ex(catnn_hip_device *dev, const catnn_graph *g, const catnn_train_options *opts,
                               catnn_hip_trainer **out) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(g && out && opts, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        const int32_t optimizer = opts->optimizer, precision = opts->precision;
        const float lr = opts->lr;
        CATNN_REQUIRE(optimizer == CATNN_OPT_SGD || optimizer == CATNN_OPT_ADAM, CATNN_ERR_INVALID_ARGUMENT,
                      "unknown optimizer " + std::to_string(optimizer) + " (expected sgd or adam)");
        CATNN_REQUIRE(precision == CATNN_PREC_BF16 || precision == CATNN_PREC_FP32, CATNN_ERR_INVALID_ARGUMENT,
                      "unknown precision " + std::to_string(precision) + " (expected bf16 or fp32)");
        *out = nullptr;
        auto make = [&](bool fuse) {
            auto *t = new catnn_hip_trainer();
            try {
                t->dev = dev;
                t->graph = *g;
                t->lr = lr;
                t->opt = optimizer;
                t->prec = precision;
                t->arena_cap = opts->arena_cap;
                t->fuse_values = fuse;
                plan_trainer(*t);
                reserve_and_upload(*t);
                if (t->prec == CATNN_PREC_BF16) t->sk_part = device_sk_scratch(dev);
            } catch (...) {
                if (t->base) (void)hipFree(t->base);
                delete t;
                throw;
            }
            return t;
        };
        try {
            *out = make(true);
        } catch (const Failure &f) {
            // Under a cap, the unfused plan has more recomputable activations.
            if (f.code != CATNN_ERR_FIBRATION || !opts->arena_cap || precision != CATNN_PREC_BF16) throw;
            *out = make(false);
        }
    });
}

int catnn_hip_train_free(catnn_hip_trainer *t) {
    return guard([&] {
        if (!t) return;
        (void)hipSetDevice(t->dev->ordinal);
        (void)hipStreamSynchronize(t->dev->stream);
        if (t->base) (void)hipFree(t->base);
        delete t;
    });
}

int catnn_hip_train_set_batch(catnn_hip_trainer *t, const catnn_tensor *input, const catnn_tensor *target) {
    return guard([&] {
        CATNN_REQUIRE(t && input && target, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(t->dev);
        hipStream_t s = t->dev->stream;
        CATNN_REQUIRE(!t->classes, CATNN_ERR_INVALID_ARGUMENT,
                      "the output is an LmHead: its targets are class ids (catnn_hip_train_set_batch_classes)");
        int64_t ni = 1, nt = 1;
        for (int i = 0; i < input->rank; ++i) ni *= input->dims[i];
        for (int i = 0; i < target->rank; ++i) nt *= target->dims[i];
        CATNN_REQUIRE(nt == numel(t->dims[t->out_id]) && (target->data || nt == 0), CATNN_ERR_SHAPE_MISMATCH,
                      "target size");
        for (uint32_t id : t->input_ids) {
            CATNN_REQUIRE(ni == numel(t->dims[id]) && (input->data || ni == 0), CATNN_ERR_SHAPE_MISMATCH,
                          "input size");
            if (ni) check_embedding_ids(*t, input->data, ni);
            CATNN_HIP(hipMemcpyAsync(t->val.at(id), input->data, (size_t)ni * 4, hipMemcpyHostToDevice, s));
        }
        CATNN_HIP(hipMemcpyAsync(t->target, target->data, (size_t)nt * 4, hipMemcpyHostToDevice, s));
        CATNN_HIP(hipStreamSynchronize(s));
    });
}

int catnn_hip_train_set_batch_classes(catnn_hip_trainer *t, const catnn_tensor *input, const uint32_t *ids,
                                      int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(t && input && (ids || n == 0), CATNN_ERR_INVALID_ARGUMENT, "null argument");
        CATNN_REQUIRE(t->classes, CATNN_ERR_INVALID_ARGUMENT,
                      "the output is not an LmHead: its target is a tensor (catnn_hip_train_set_batch)");
        require_device(t->dev);
        CATNN_REQUIRE(n == t->class_rows, CATNN_ERR_SHAPE_MISMATCH, "ce targets");  // adjoint.rs:126-128
        for (int64_t r = 0; r < n; ++r)  // adjoint.rs:134-136
            CATNN_REQUIRE((int64_t)ids[r] < t->vocab, CATNN_ERR_SHAPE_MISMATCH,
                          "target " + std::to_string(ids[r]) + " >= " + std::to_string(t->vocab));
        hipStream_t s = t->dev->stream;
        int64_t ni = 1;
        for (int i = 0; i < input->rank; ++i) ni *= input->dims[i];
        for (uint32_t id : t->input_ids) {
            CATNN_REQUIRE(ni == numel(t->dims[id]) && (input->data || ni == 0), CATNN_ERR_SHAPE_MISMATCH,
                          "input size");
            if (ni) check_embedding_ids(*t, input->data, ni);
            CATNN_HIP(hipMemcpyAsync(t->val.at(id), input->data, (size_t)ni * 4, hipMemcpyHostToDevice, s));
        }
        if (n) CATNN_HIP(hipMemcpyAsync(t->class_ids, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
        CATNN_HIP(hipStreamSynchronize(s));
    });
}

int catnn_hip_train_step(catnn_hip_trainer *t, float *loss) {
    return guard([&] {
        CATNN_REQUIRE(t, CATNN_ERR_INVALID_ARGUMENT, "null trainer");
        require_device(t->dev);
        train_step(*t);
        if (loss) {
            CATNN_HIP(hipMemcpyAsync(loss, t->loss, 4, hipMemcpyDeviceToHost, t->dev->stream));
            CATNN_HIP(hipStreamSynchronize(t->dev->stream));
        }
    });
}

int catnn_hip_train_reset(catnn_hip_trainer *t) {
    return guard([&] {
        CATNN_REQUIRE(t, CATNN_ERR_INVALID_ARGUMENT, "null trainer");
        require_device(t->dev);
        upload_params(*t);
    });
}

int catnn_hip_train_read_param(catnn_hip_trainer *t, uint32_t node_id, const char *port, float *host,
                               int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(t && port && host, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(t->dev);
        int64_t col0, ncols;
        TParam *p = find_param(*t, node_id, port, &col0, &ncols);
        read_param_buf(*t, p, p->master, col0, ncols, host, n);
    });
}

int catnn_hip_train_read_grad(catnn_hip_trainer *t, uint32_t node_id, const char *port, float *host,
                              int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(t && port && host, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(t->dev);
        int64_t col0, ncols;
        TParam *p = find_param(*t, node_id, port, &col0, &ncols);
        read_param_buf(*t, p, p->grad, col0, ncols, host, n);
    });
}

int catnn_hip_train_read_moment(catnn_hip_trainer *t, uint32_t node_id, const char *port, int32_t which,
                                float *host, int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(t && port && host, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        CATNN_REQUIRE(which == 0 || which == 1, CATNN_ERR_INVALID_ARGUMENT, "moment: 0 (m) or 1 (v)");
        CATNN_REQUIRE(t->opt == CATNN_OPT_ADAM, CATNN_ERR_UNSUPPORTED, "trainer was installed with SGD: no moments");
        require_device(t->dev);
        int64_t col0, ncols;
        TParam *p = find_param(*t, node_id, port, &col0, &ncols);
        read_param_buf(*t, p, which == 0 ? p->m : p->v, col0, ncols, host, n);
    });
}

int catnn_hip_train_adam_step(catnn_hip_trainer *t, uint64_t *step) {
    return guard([&] {
        CATNN_REQUIRE(t && step, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *step = t->adam_t;
    });
}

int catnn_hip_sgd_f32(catnn_hip_device *dev, float *p, const float *g, int64_t n, float lr) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(n >= 0, CATNN_ERR_SHAPE_MISMATCH, "sgd: negative length");
        CATNN_REQUIRE((p && g) || n == 0, CATNN_ERR_INVALID_ARGUMENT, "sgd: null buffer");
        k::apply_update(dev->stream, k::sgd_rule(lr), p, g, nullptr, nullptr, n);
    });
}

int catnn_hip_adam_f32(catnn_hip_device *dev, float *p, const float *g, float *m, float *v, int64_t n,
                       uint64_t t, float lr) {
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(n >= 0, CATNN_ERR_SHAPE_MISMATCH, "adam: negative length");
        CATNN_REQUIRE((p && g && m && v) || n == 0, CATNN_ERR_INVALID_ARGUMENT, "adam: null buffer");
        const uint64_t next = t == UINT64_MAX ? t : t + 1;  // saturating_add (optim.rs:98)
        k::apply_update(dev->stream, k::adam_rule(lr, next), p, g, m, v, n);
    });
}

int catnn_hip_run_adjoint(catnn_hip_device *dev, const catnn_node *node, const catnn_tensor *inputs,
                          int32_t n_inputs, const catnn_tensor *output, const catnn_tensor *dy,
                          catnn_tensor *dx, catnn_tensor *dparams, int32_t n_dparams) {
    (void)output;  // recomputed from the inputs on the device
    return guard([&] {
        require_device(dev);
        CATNN_REQUIRE(node && dy && (n_inputs == 0 || (inputs && dx)) && (n_dparams == 0 || dparams),
                      CATNN_ERR_INVALID_ARGUMENT, "null argument");
        // adjoint.rs:768-770
        CATNN_REQUIRE(n_inputs > 0, CATNN_ERR_WIRING,
                      std::string(node->name ? node->name : "?") + " adjoint has no inputs");
        CATNN_REQUIRE(n_inputs <= 16, CATNN_ERR_INVALID_ARGUMENT, "run_adjoint: more than 16 inputs");
        CATNN_REQUIRE(n_dparams == node->n_params, CATNN_ERR_SHAPE_MISMATCH,
                      "run_adjoint: " + std::to_string(n_dparams) + " parameter cotangents for " +
                          std::to_string(node->n_params) + " params");
        auto ok = [](int rc) {
            if (rc != CATNN_OK) fail(rc, catnn_hip_last_error());
        };
        const uint32_t nid = (uint32_t)n_inputs;
        const std::string key = adjoint_key(node, inputs, n_inputs);
        catnn_hip_trainer *t = adjoint_cache_find(dev, key);
        if (t) {
            // The same node shape ran before: its plan and arena are reused and
            // only the parameter values are replaced.
            catnn_graph tmp;
            catnn_node self = *node;
            self.id = nid;
            ok(catnn_graph_add_node(&tmp, &self));
            Node &cached = t->graph.nodes.at(nid);
            cached.params = tmp.nodes.at(nid).params;
            cached.name = tmp.nodes.at(nid).name;
            TNode &tn = t->nodes[t->index.at(nid)];
            for (auto &kv : tn.params) kv.second->init = param_values(cached, kv.first);
            upload_params(*t);
        } else {
            // The one-node graph in0 … in{n-1} → node, its preds in edge order.
            catnn_graph g;
            g.name = "adjoint";
            std::vector<std::string> names;
            for (int32_t i = 0; i < n_inputs; ++i) names.push_back("in" + std::to_string(i));
            for (int32_t i = 0; i < n_inputs; ++i) {
                catnn_node in{};
                in.id = (uint32_t)i;
                in.name = names[(size_t)i].c_str();
                in.op.kind = CATNN_OP_IDENTITY;
                in.output_ty = inputs[i];
                in.output_ty.data = nullptr;
                ok(catnn_graph_add_node(&g, &in));
                ok(catnn_graph_add_input(&g, in.id));
            }
            catnn_node self = *node;
            self.id = nid;
            ok(catnn_graph_add_node(&g, &self));
            for (int32_t i = 0; i < n_inputs; ++i) ok(catnn_graph_add_edge(&g, (uint32_t)i, nid, "out", "in"));
            ok(catnn_graph_add_output(&g, nid));
            std::unique_ptr<catnn_hip_trainer, TrainerFree> fresh(new catnn_hip_trainer());
            fresh->dev = dev;
            fresh->graph = g;
            fresh->lr = 0.f;
            fresh->prec = CATNN_PREC_FP32;  // adjoint_of is fp32 throughout (adjoint.rs:35-61)
            fresh->input_grads = true;
            plan_trainer(*fresh);
            reserve_and_upload(*fresh);
            t = adjoint_cache_insert(dev, key, std::move(fresh));
        }
        hipStream_t s = dev->stream;
        for (int32_t i = 0; i < n_inputs; ++i) {
            const int64_t ni = numel(dims_from_c(inputs[i]));
            CATNN_REQUIRE(inputs[i].data || ni == 0, CATNN_ERR_INVALID_ARGUMENT, "input " + std::to_string(i) + ": no data");
            if (ni) check_embedding_ids(*t, inputs[i].data, ni);
            if (ni) CATNN_HIP(hipMemcpyAsync(t->val.at((uint32_t)i), inputs[i].data, (size_t)ni * 4,
                                             hipMemcpyHostToDevice, s));
        }
        const std::vector<int64_t> &od = t->dims.at(nid);
        const int64_t nd = numel(dims_from_c(*dy));
        const std::string span = std::string(node->name ? node->name : "?") + ".bwd";
        CATNN_REQUIRE(nd == numel(od) && (dy->data || nd == 0), CATNN_ERR_SHAPE_MISMATCH,
                      "dy has " + std::to_string(nd) + " values, " + t->graph.node(nid).name + " produces " +
                          dims_str(od));
        // note_kernel("{name}.bwd", dy.checksum()) of the training wave (coord.rs:412), stamped on the device.
        push_device_event(dev, span, CATNN_EV_KERNEL_START, 0);
        forward_pass(*t);
        // dy's buffer is planned from the loss tick on: forward-only scratch may share it.
        if (nd) CATNN_HIP(hipMemcpyAsync(t->grad.at(nid), dy->data, (size_t)nd * 4, hipMemcpyHostToDevice, s));
        reverse_pass(*t);
        push_device_event(dev, span, CATNN_EV_KERNEL_END, fnv1a_f32(dy->data, (uint64_t)nd));
        for (int32_t i = 0; i < n_inputs; ++i) {
            const std::vector<int64_t> &xd = t->dims.at((uint32_t)i);
            const int64_t nx = numel(xd);
            int64_t cap = 1;
            for (int r = 0; r < dx[i].rank; ++r) cap *= dx[i].dims[r];
            CATNN_REQUIRE(dx[i].rank >= 0 && cap >= nx && (dx[i].data || nx == 0), CATNN_ERR_SHAPE_MISMATCH,
                          "dx[" + std::to_string(i) + "] holds " + std::to_string(cap) + " values, input has " +
                              dims_str(xd));
            if (nx) read_cols(*t, t->grad.at((uint32_t)i), 1, nx, 0, nx, dx[i].data, nx);
            dx[i].rank = (int32_t)xd.size();
            for (size_t r = 0; r < xd.size(); ++r) dx[i].dims[r] = xd[r];
            dx[i].dtype = inputs[i].dtype;
        }
        const Node &self_node = t->graph.node(nid);
        for (int32_t j = 0; j < n_dparams; ++j) {
            const auto &pr = self_node.params[(size_t)j];
            int64_t col0, ncols;
            TParam *p = find_param(*t, nid, pr.first, &col0, &ncols);
            const int64_t np = pr.second.numel();
            int64_t cap = 1;
            for (int r = 0; r < dparams[j].rank; ++r) cap *= dparams[j].dims[r];
            CATNN_REQUIRE(dparams[j].rank >= 0 && cap >= np && (dparams[j].data || np == 0),
                          CATNN_ERR_SHAPE_MISMATCH,
                          "dparams[" + std::to_string(j) + "] (" + pr.first + ") holds " + std::to_string(cap) +
                              " values, the param has " + std::to_string(np));
            if (np) read_param_buf(*t, p, p->grad, col0, ncols, dparams[j].data, np);
            dparams[j].rank = (int32_t)pr.second.dims.size();
            for (size_t r = 0; r < pr.second.dims.size(); ++r) dparams[j].dims[r] = pr.second.dims[r];
            dparams[j].dtype = CATNN_F32;
        }
        CATNN_HIP(hipStreamSynchronize(s));
    });
}

int catnn_hip_train_read_value(catnn_hip_trainer *t, uint32_t node_id, float *host, int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(t && host, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(t->dev);
        auto it = t->val.find(node_id);
        CATNN_REQUIRE(it != t->val.end(), CATNN_ERR_UNKNOWN_COMPONENT, "unknown node " + std::to_string(node_id));
        // Other values share arena space with later buffers once their last reader ran.
        CATNN_REQUIRE(node_id == t->out_id || t->input_ids.count(node_id), CATNN_ERR_UNSUPPORTED,
                      "value of node " + std::to_string(node_id) +
                          " is not kept past its last use; only graph inputs and the output are");
        read_cols(*t, it->second, 1, numel(t->dims[node_id]), 0, numel(t->dims[node_id]), host, n);
    });
}

int catnn_hip_train_read_routing(catnn_hip_trainer *t, uint32_t node_id, int32_t *idx, int64_t n) {
    return guard([&] {
        CATNN_REQUIRE(t && idx, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        require_device(t->dev);
        auto it = t->index.find(node_id);
        CATNN_REQUIRE(it != t->index.end() && t->nodes[it->second].kind == CATNN_OP_MOE,
                      CATNN_ERR_UNKNOWN_COMPONENT, "node " + std::to_string(node_id) + " is not a MoE node");
        TNode &tn = t->nodes[it->second];
        const int64_t T = numel(tn.in_dims[0]) / tn.in_dims[0].back();
        CATNN_REQUIRE(n == T * tn.node->op.a[1], CATNN_ERR_SHAPE_MISMATCH, "routing buffer size");
        CATNN_HIP(hipMemcpyAsync(idx, tn.B("idx"), (size_t)n * 4, hipMemcpyDeviceToHost, t->dev->stream));
        CATNN_HIP(hipStreamSynchronize(t->dev->stream));
    });
}

int catnn_hip_train_checkpointed(catnn_hip_trainer *t, char (*ids)[CATNN_ID_CAP], int32_t cap, int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(t && n, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        int32_t k = 0;
        for (const auto &kv : t->ckpt) {
            if (ids && k < cap) {
                std::memset(ids[k], 0, CATNN_ID_CAP);
                std::strncpy(ids[k], ("act:" + std::to_string(kv.first)).c_str(), CATNN_ID_CAP - 1);
            }
            ++k;
        }
        *n = k;
    });
}

int catnn_hip_train_arena(catnn_hip_trainer *t, catnn_arena_alloc *out, int32_t cap, int32_t *n,
                          uint64_t *reserved_bytes) {
    return guard([&] {
        CATNN_REQUIRE(t && n, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *n = (int32_t)t->plan.size();
        if (reserved_bytes) *reserved_bytes = t->reserved;
        for (int32_t i = 0; out && i < cap && i < *n; ++i) {
            const auto &a = t->plan[(size_t)i];
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
