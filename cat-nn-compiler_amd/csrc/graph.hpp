// Host-side IR graph (crates/catnn-compile/src/ir.rs:13-97) and the per-op
// dispatch shared by the three execution seams.
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "common.hpp"

namespace catnn {

struct HostTensor {
    std::vector<int64_t> dims;
    int32_t dtype = CATNN_F32;
    std::vector<float> data;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : dims) n *= d;
        return n;
    }
};

struct Node {
    uint32_t id;
    std::string name;
    catnn_op op;
    HostTensor output_ty;  // type only
    std::vector<std::pair<std::string, HostTensor>> params;  // IndexMap order
    const HostTensor *param(const std::string &port) const {
        for (auto &p : params)
            if (p.first == port) return &p.second;
        return nullptr;
    }
};

struct Edge {
    uint32_t src, dst;
    std::string src_port, dst_port;
};

std::string op_name(int32_t kind);
std::string dims_str(const std::vector<int64_t> &d);

// Output dims the backend produces for `node` given its input dims, checked
// the way the reference kernels check them (ShapeMismatch / UnknownPort /
// Wiring failures).  `param_dims` looks up a parameter's dims by port.
std::vector<int64_t> infer_dims(const Node &node, const std::vector<std::vector<int64_t>> &ins);

// Device pointers for one node execution.
struct ExecArgs {
    std::vector<const float *> inputs;
    std::vector<std::vector<int64_t>> in_dims;
    std::function<const float *(const std::string &port)> param;  // null if absent
    float *out = nullptr;
    int fused_act = 0;
    const float *residual = nullptr;
    // Attention scratch: qkv [T, 3D] and ctx [T, D]; MoE workspace.
    float *scratch = nullptr;
    uint64_t scratch_bytes = 0;
    // Weight copy made at install: Attention/GqaAttention [wq | wk | wv] per
    // row, LmHead wᵀ [H, V].  Null: built from the params (or scratch) per call.
    const float *derived = nullptr;
    // Programs: the device flag an Embedding raises on an id ≥ vocab, read
    // once at the end of the forward (null: checked right after the node).
    int *embed_flag = nullptr;
};

// A node from its C form with parameter types only (no data), and the dims
// of a C tensor; both check ranks and dimensions.
Node node_shape_from_c(const catnn_node *c);
std::vector<int64_t> dims_from_c(const catnn_tensor &t);

// Scratch bytes `node` needs beyond its output (0 for most ops).
uint64_t scratch_bytes(const Node &node, const std::vector<std::vector<int64_t>> &ins);

// Launch the kernels of one node on dev's stream.
void exec_node(catnn_hip_device *dev, const Node &node, const ExecArgs &a);

}  // namespace catnn

struct catnn_graph {
    std::string name;
    std::vector<uint32_t> node_order;  // insertion order (IndexMap)
    std::map<uint32_t, catnn::Node> nodes;
    std::vector<catnn::Edge> edges;
    std::vector<uint32_t> inputs, outputs;
    std::vector<std::vector<std::string>> fusions;

    std::vector<uint32_t> topo() const;
    std::vector<uint32_t> preds(uint32_t id) const;
    std::vector<uint32_t> succs(uint32_t id) const;
    const catnn::Node &node(uint32_t id) const;
};
