// IrGraph ingest and export in the reference's serde JSON form
// (crates/catnn-compile/src/ir.rs:13-41 with serde defaults), so a graph
// the Rust compiler serialises — e.g. the graph a coordinator ships to a
// member — loads straight into the backend.  The serde encoding:
//   IrGraph   {"name", "nodes": {"<id>": IrNode, ...} (IndexMap order),
//              "edges": [IrEdge], "inputs": [id], "outputs": [id]}
//   IrNode    {"id", "name", "op", "output_ty", "params": {"<port>": Tensor}}
//   OpenOp    unit variants as "snake_case", struct variants as
//             {"snake_case": {fields}} (morphism.rs:17-116, rename_all)
//   TensorType {"shape": {"dims": [..]}, "dtype": "f32"} (tensor.rs:17-27, 81-83, 181-184)
//   Tensor    {"ty": TensorType, "data": [f32...]} (tensor.rs:226-229);
//             serde_json writes non-finite floats as null.
// Large parameter sets ride in a side blob instead (the control plane caps
// a frame at 64 MiB): a parameter whose "data" is [] takes its numel floats
// from the blob, in node order, then port order.  Two extensions the
// reference ignores: "causal": true inside "attention", and a top-level
// "fusions": [["linear", "relu"], ...] (Realization.fusions).
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "graph.hpp"

namespace catnn {
namespace {

// ------------------------------------------------------------------ parser

struct JValue {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    std::string s;  // STR text, or NUM literal as written
    std::vector<JValue> arr;
    std::vector<std::pair<std::string, JValue>> obj;  // in document order

    const JValue *get(const std::string &k) const {
        for (auto &kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

class Parser {
public:
    Parser(const char *p, size_t n) : p_(p), n_(n) {}

    JValue parse() {
        JValue v = value(0);
        ws();
        if (i_ != n_) err("trailing characters");
        return v;
    }

private:
    const char *p_;
    size_t n_, i_ = 0;

    [[noreturn]] void err(const std::string &what) {
        fail(CATNN_ERR_PARSE, "IrGraph JSON: " + what + " at byte " + std::to_string(i_));
    }
    void ws() {
        while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\n' || p_[i_] == '\r' || p_[i_] == '\t')) ++i_;
    }
    bool lit(const char *w) {
        const size_t k = std::strlen(w);
        if (i_ + k <= n_ && std::memcmp(p_ + i_, w, k) == 0) {
            i_ += k;
            return true;
        }
        return false;
    }
    JValue value(int depth) {
        if (depth > 64) err("nesting too deep");
        ws();
        if (i_ >= n_) err("unexpected end");
        JValue v;
        const char c = p_[i_];
        if (c == '{') {
            v.kind = JValue::OBJ;
            ++i_;
            ws();
            if (i_ < n_ && p_[i_] == '}') {
                ++i_;
                return v;
            }
            for (;;) {
                ws();
                if (i_ >= n_ || p_[i_] != '"') err("expected a key");
                std::string k = str();
                ws();
                if (i_ >= n_ || p_[i_] != ':') err("expected ':'");
                ++i_;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (i_ < n_ && p_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < n_ && p_[i_] == '}') {
                    ++i_;
                    return v;
                }
                err("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = JValue::ARR;
            ++i_;
            ws();
            if (i_ < n_ && p_[i_] == ']') {
                ++i_;
                return v;
            }
            for (;;) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (i_ < n_ && p_[i_] == ',') {
                    ++i_;
                    continue;
                }
                if (i_ < n_ && p_[i_] == ']') {
                    ++i_;
                    return v;
                }
                err("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = JValue::STR;
            v.s = str();
            return v;
        }
        if (lit("true")) {
            v.kind = JValue::BOOL;
            v.b = true;
            return v;
        }
        if (lit("false")) {
            v.kind = JValue::BOOL;
            return v;
        }
        if (lit("null")) return v;
        const size_t s0 = i_;
        if (i_ < n_ && (p_[i_] == '-' || p_[i_] == '+')) ++i_;
        while (i_ < n_ && (std::isdigit((unsigned char)p_[i_]) || p_[i_] == '.' || p_[i_] == 'e' ||
                           p_[i_] == 'E' || p_[i_] == '-' || p_[i_] == '+'))
            ++i_;
        if (i_ == s0) err("unexpected character");
        v.kind = JValue::NUM;
        v.s.assign(p_ + s0, i_ - s0);
        return v;
    }
    std::string str() {
        ++i_;  // opening quote
        std::string out;
        while (i_ < n_ && p_[i_] != '"') {
            char c = p_[i_++];
            if (c == '\\') {
                if (i_ >= n_) err("bad escape");
                const char e = p_[i_++];
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (i_ + 4 > n_) err("bad \\u escape");
                        const unsigned cp = (unsigned)std::strtoul(std::string(p_ + i_, 4).c_str(), nullptr, 16);
                        i_ += 4;
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            out += (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: err("bad escape");
                }
            } else {
                out += c;
            }
        }
        if (i_ >= n_) err("unterminated string");
        ++i_;
        return out;
    }
};

[[noreturn]] void bad(const std::string &what) { fail(CATNN_ERR_PARSE, "IrGraph JSON: " + what); }

const JValue &need(const JValue &o, const char *k, const std::string &where) {
    if (o.kind != JValue::OBJ) bad(where + " is not an object");
    const JValue *v = o.get(k);
    if (!v) bad(where + " has no \"" + k + "\"");
    return *v;
}

int64_t as_int(const JValue &v, const std::string &where) {
    if (v.kind != JValue::NUM) bad(where + " is not a number");
    char *end = nullptr;
    const long long x = std::strtoll(v.s.c_str(), &end, 10);
    if (!end || *end) bad(where + " is not an integer");
    return x;
}

float as_f32(const JValue &v) {
    if (v.kind == JValue::NUL) return NAN;  // serde_json writes non-finite floats as null
    if (v.kind != JValue::NUM) bad("tensor data holds a non-number");
    return std::strtof(v.s.c_str(), nullptr);
}

// OpenOp variants: serde name, discriminant, field names in declaration order
// (morphism.rs:19-116; rename_all = "snake_case" puts '_' before every
// capital after the first).
struct OpSpec {
    const char *serde;
    int32_t kind;
    std::vector<const char *> fields;
};

const std::vector<OpSpec> &op_specs() {
    static const std::vector<OpSpec> specs = {
        {"identity", CATNN_OP_IDENTITY, {}},
        {"linear", CATNN_OP_LINEAR, {"in_features", "out_features", "bias"}},
        {"relu", CATNN_OP_RELU, {}},
        {"gelu", CATNN_OP_GELU, {}},
        {"softmax", CATNN_OP_SOFTMAX, {"axis"}},
        {"layer_norm", CATNN_OP_LAYER_NORM, {"eps_e6"}},
        {"add", CATNN_OP_ADD, {}},
        {"mul", CATNN_OP_MUL, {}},
        {"mat_mul", CATNN_OP_MATMUL, {}},
        {"transpose", CATNN_OP_TRANSPOSE, {"dim0", "dim1"}},
        {"reshape", CATNN_OP_RESHAPE, {"out"}},
        {"attention", CATNN_OP_ATTENTION, {"n_heads", "d_model", "d_head"}},
        {"residual_add", CATNN_OP_RESIDUAL_ADD, {}},
        {"embedding", CATNN_OP_EMBEDDING, {"vocab", "hidden"}},
        {"rms_norm", CATNN_OP_RMS_NORM, {"eps_e6"}},
        {"gqa_attention", CATNN_OP_GQA_ATTENTION,
         {"n_heads", "n_kv_heads", "head_dim", "d_model", "sliding_window", "rope_theta"}},
        {"swi_glu", CATNN_OP_SWIGLU, {"hidden", "intermediate"}},
        {"router", CATNN_OP_ROUTER, {"n_experts", "top_k"}},
        {"mo_e", CATNN_OP_MOE, {"n_experts", "top_k", "hidden", "intermediate"}},
        {"lm_head", CATNN_OP_LM_HEAD, {"hidden", "vocab"}},
        {"mla", CATNN_OP_MLA, {"n_heads", "q_lora", "kv_lora", "qk_nope", "qk_rope", "v_dim", "rope_theta"}},
        {"deep_seek_moe", CATNN_OP_DEEPSEEK_MOE,
         {"n_routed", "n_shared", "top_k", "n_group", "topk_group", "hidden", "moe_intermediate",
          "routed_scale_milli"}},
        {"mix", CATNN_OP_MIX, {}},
    };
    return specs;
}

catnn_op parse_op(const JValue &v, const std::string &where) {
    catnn_op op{};
    std::string name;
    const JValue *body = nullptr;
    if (v.kind == JValue::STR) {
        name = v.s;
    } else if (v.kind == JValue::OBJ && v.obj.size() == 1) {
        name = v.obj[0].first;
        body = &v.obj[0].second;
    } else {
        bad(where + ".op is neither a variant name nor a one-key object");
    }
    for (const OpSpec &sp : op_specs()) {
        if (name != sp.serde) continue;
        op.kind = sp.kind;
        if (sp.fields.empty()) {
            if (body) bad(where + ".op: " + name + " takes no fields");
            return op;
        }
        if (!body || body->kind != JValue::OBJ) bad(where + ".op: " + name + " needs its fields");
        if (sp.kind == CATNN_OP_RESHAPE) {
            const JValue &out = need(*body, "out", where + ".op.reshape");
            if (out.kind != JValue::ARR || out.arr.size() > 8) bad(where + ".op.reshape.out: up to 8 dims");
            for (size_t i = 0; i < out.arr.size(); ++i) op.a[i] = as_int(out.arr[i], where + ".op.reshape.out");
            return op;
        }
        for (size_t i = 0; i < sp.fields.size(); ++i) {
            const JValue &f = need(*body, sp.fields[i], where + ".op." + name);
            if (f.kind == JValue::BOOL) op.a[i] = f.b ? 1 : 0;
            else if (f.kind == JValue::NUL) op.a[i] = -1;  // Option::None (gqa sliding_window)
            else op.a[i] = as_int(f, where + ".op." + name + "." + sp.fields[i]);
        }
        if (sp.kind == CATNN_OP_ATTENTION) {
            const JValue *c = body->get("causal");
            if (c && c->kind == JValue::BOOL && c->b) op.flags |= CATNN_FLAG_CAUSAL;
        }
        return op;
    }
    bad(where + ".op: unknown variant \"" + name + "\"");
}

int32_t parse_dtype(const std::string &s, const std::string &where) {
    static const char *names[] = {"f32", "f16", "bf16", "fp8", "fp4", "i32", "bool"};
    for (int i = 0; i < 7; ++i)
        if (s == names[i]) return i;
    bad(where + ": unknown dtype \"" + s + "\"");
}

HostTensor parse_type(const JValue &v, const std::string &where) {
    HostTensor t;
    const JValue &dims = need(need(v, "shape", where), "dims", where + ".shape");
    if (dims.kind != JValue::ARR || dims.arr.size() > CATNN_MAX_RANK) bad(where + ".shape.dims: up to 8 dims");
    for (auto &d : dims.arr) {
        const int64_t x = as_int(d, where + ".shape.dims");
        if (x < 0) bad(where + ".shape.dims: negative dim");
        t.dims.push_back(x);
    }
    const JValue &dt = need(v, "dtype", where);
    if (dt.kind != JValue::STR) bad(where + ".dtype is not a string");
    t.dtype = parse_dtype(dt.s, where + ".dtype");
    return t;
}

// ---------------------------------------------------------------- writer

void put_str(std::string &o, const std::string &s) {
    o += '"';
    for (char c : s) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if ((unsigned char)c < 0x20) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\u%04x", (unsigned)c);
                    o += b;
                } else {
                    o += c;
                }
        }
    }
    o += '"';
}

void put_type(std::string &o, const HostTensor &t) {
    static const char *names[] = {"f32", "f16", "bf16", "fp8", "fp4", "i32", "bool"};
    o += "{\"shape\":{\"dims\":[";
    for (size_t i = 0; i < t.dims.size(); ++i) {
        if (i) o += ',';
        o += std::to_string(t.dims[i]);
    }
    o += "]},\"dtype\":\"";
    o += (t.dtype >= 0 && t.dtype < 7) ? names[t.dtype] : "f32";
    o += "\"}";
}

void put_op(std::string &o, const catnn_op &op) {
    const OpSpec *sp = nullptr;
    for (const OpSpec &s : op_specs())
        if (s.kind == op.kind) sp = &s;
    if (!sp) fail(CATNN_ERR_UNKNOWN_REALIZATION, "IrGraph JSON: op kind " + std::to_string(op.kind));
    if (sp->fields.empty()) {
        put_str(o, sp->serde);
        return;
    }
    o += "{\"";
    o += sp->serde;
    o += "\":{";
    if (op.kind == CATNN_OP_RESHAPE) {
        int n = 8;
        while (n > 0 && op.a[n - 1] == 0) --n;
        o += "\"out\":[";
        for (int i = 0; i < n; ++i) {
            if (i) o += ',';
            o += std::to_string(op.a[i]);
        }
        o += "]";
    } else {
        for (size_t i = 0; i < sp->fields.size(); ++i) {
            if (i) o += ',';
            put_str(o, sp->fields[i]);
            o += ':';
            if (op.kind == CATNN_OP_LINEAR && i == 2) o += op.a[i] ? "true" : "false";
            else if (op.kind == CATNN_OP_GQA_ATTENTION && i == 4 && op.a[i] < 0) o += "null";
            else o += std::to_string(op.a[i]);
        }
        if (op.kind == CATNN_OP_ATTENTION && (op.flags & CATNN_FLAG_CAUSAL)) o += ",\"causal\":true";
    }
    o += "}}";
}

void put_f32(std::string &o, float v) {
    if (!std::isfinite(v)) {
        o += "null";
        return;
    }
    char b[32];
    std::snprintf(b, sizeof b, "%.9g", (double)v);  // 9 significant digits round-trip any f32
    o += b;
}

}  // namespace
}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_graph_from_json(const char *json, uint64_t len, const float *blob, uint64_t blob_floats,
                          catnn_graph **out) {
    return guard([&] {
        CATNN_REQUIRE(json && out, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        const JValue root = Parser(json, (size_t)len).parse();
        auto g = std::make_unique<catnn_graph>();
        const JValue &name = need(root, "name", "graph");
        if (name.kind != JValue::STR) bad("graph.name is not a string");
        g->name = name.s;
        const JValue &nodes = need(root, "nodes", "graph");
        if (nodes.kind != JValue::OBJ) bad("graph.nodes is not an object");
        uint64_t used = 0;
        for (auto &kv : nodes.obj) {
            const std::string where = "nodes[" + kv.first + "]";
            const JValue &nv = kv.second;
            Node n;
            n.id = (uint32_t)as_int(need(nv, "id", where), where + ".id");
            if (std::to_string(n.id) != kv.first) bad(where + ": key and id differ");
            const JValue &nm = need(nv, "name", where);
            if (nm.kind != JValue::STR) bad(where + ".name is not a string");
            n.name = nm.s;
            n.op = parse_op(need(nv, "op", where), where);
            n.output_ty = parse_type(need(nv, "output_ty", where), where + ".output_ty");
            const JValue &params = need(nv, "params", where);
            if (params.kind != JValue::OBJ) bad(where + ".params is not an object");
            for (auto &pv : params.obj) {
                const std::string pw = where + ".params." + pv.first;
                HostTensor t = parse_type(need(pv.second, "ty", pw), pw + ".ty");
                const JValue &data = need(pv.second, "data", pw);
                if (data.kind != JValue::ARR) bad(pw + ".data is not an array");
                const int64_t numel = t.numel();
                if (data.arr.empty() && numel > 0) {
                    CATNN_REQUIRE(blob && used + (uint64_t)numel <= blob_floats, CATNN_ERR_SHAPE_MISMATCH,
                                  pw + ": parameter data is neither inline nor in the blob");
                    t.data.assign(blob + used, blob + used + numel);
                    used += (uint64_t)numel;
                } else {
                    CATNN_REQUIRE((int64_t)data.arr.size() == numel, CATNN_ERR_SHAPE_MISMATCH,
                                  pw + ": data len " + std::to_string(data.arr.size()) + " != numel " +
                                      std::to_string(numel));
                    t.data.resize((size_t)numel);
                    for (int64_t i = 0; i < numel; ++i) t.data[(size_t)i] = as_f32(data.arr[(size_t)i]);
                }
                n.params.emplace_back(pv.first, std::move(t));
            }
            if (g->nodes.count(n.id)) bad(where + ": duplicate node id");
            g->node_order.push_back(n.id);
            g->nodes[n.id] = std::move(n);
        }
        CATNN_REQUIRE(used == blob_floats || !blob, CATNN_ERR_SHAPE_MISMATCH,
                      "blob holds " + std::to_string(blob_floats) + " floats, the graph's parameters " +
                          std::to_string(used));
        const JValue &edges = need(root, "edges", "graph");
        if (edges.kind != JValue::ARR) bad("graph.edges is not an array");
        for (size_t i = 0; i < edges.arr.size(); ++i) {
            const std::string where = "edges[" + std::to_string(i) + "]";
            const JValue &e = edges.arr[i];
            const JValue &sp = need(e, "src_port", where), &dp = need(e, "dst_port", where);
            if (sp.kind != JValue::STR || dp.kind != JValue::STR) bad(where + ": ports are not strings");
            g->edges.push_back(Edge{(uint32_t)as_int(need(e, "src", where), where + ".src"),
                                    (uint32_t)as_int(need(e, "dst", where), where + ".dst"), sp.s, dp.s});
        }
        for (const char *key : {"inputs", "outputs"}) {
            const JValue &ids = need(root, key, "graph");
            if (ids.kind != JValue::ARR) bad(std::string("graph.") + key + " is not an array");
            for (auto &id : ids.arr)
                (key[0] == 'i' ? g->inputs : g->outputs).push_back((uint32_t)as_int(id, std::string("graph.") + key));
        }
        if (const JValue *fus = root.get("fusions")) {
            if (fus->kind != JValue::ARR) bad("graph.fusions is not an array");
            for (auto &grp : fus->arr) {
                if (grp.kind != JValue::ARR) bad("graph.fusions holds a non-array");
                std::vector<std::string> names;
                for (auto &s : grp.arr) {
                    if (s.kind != JValue::STR) bad("graph.fusions holds a non-string");
                    names.push_back(s.s);
                }
                g->fusions.push_back(std::move(names));
            }
        }
        *out = g.release();
    });
}

int catnn_graph_to_json(const catnn_graph *g, int32_t inline_params, char *buf, uint64_t cap, uint64_t *len,
                        float *blob, uint64_t blob_cap, uint64_t *blob_floats) {
    return guard([&] {
        CATNN_REQUIRE(g && len, CATNN_ERR_INVALID_ARGUMENT, "null argument");
        std::string o;
        uint64_t nb = 0;
        o += "{\"name\":";
        put_str(o, g->name);
        o += ",\"nodes\":{";
        for (size_t i = 0; i < g->node_order.size(); ++i) {
            const Node &n = g->nodes.at(g->node_order[i]);
            if (i) o += ',';
            o += '"' + std::to_string(n.id) + "\":{\"id\":" + std::to_string(n.id) + ",\"name\":";
            put_str(o, n.name);
            o += ",\"op\":";
            put_op(o, n.op);
            o += ",\"output_ty\":";
            put_type(o, n.output_ty);
            o += ",\"params\":{";
            for (size_t j = 0; j < n.params.size(); ++j) {
                const HostTensor &t = n.params[j].second;
                if (j) o += ',';
                put_str(o, n.params[j].first);
                o += ":{\"ty\":";
                put_type(o, t);
                o += ",\"data\":[";
                if (inline_params) {
                    for (size_t k = 0; k < t.data.size(); ++k) {
                        if (k) o += ',';
                        put_f32(o, t.data[k]);
                    }
                } else {
                    if (blob && nb + t.data.size() <= blob_cap)
                        std::memcpy(blob + nb, t.data.data(), t.data.size() * 4);
                    nb += t.data.size();
                }
                o += "]}";
            }
            o += "}}";
        }
        o += "},\"edges\":[";
        for (size_t i = 0; i < g->edges.size(); ++i) {
            const Edge &e = g->edges[i];
            if (i) o += ',';
            o += "{\"src\":" + std::to_string(e.src) + ",\"dst\":" + std::to_string(e.dst) + ",\"src_port\":";
            put_str(o, e.src_port);
            o += ",\"dst_port\":";
            put_str(o, e.dst_port);
            o += '}';
        }
        for (int k = 0; k < 2; ++k) {
            const auto &ids = k == 0 ? g->inputs : g->outputs;
            o += k == 0 ? "],\"inputs\":[" : "],\"outputs\":[";
            for (size_t i = 0; i < ids.size(); ++i) {
                if (i) o += ',';
                o += std::to_string(ids[i]);
            }
        }
        o += ']';
        if (!g->fusions.empty()) {
            o += ",\"fusions\":[";
            for (size_t i = 0; i < g->fusions.size(); ++i) {
                if (i) o += ',';
                o += '[';
                for (size_t j = 0; j < g->fusions[i].size(); ++j) {
                    if (j) o += ',';
                    put_str(o, g->fusions[i][j]);
                }
                o += ']';
            }
            o += ']';
        }
        o += '}';
        *len = o.size();
        if (blob_floats) *blob_floats = nb;
        if (buf && cap > o.size()) {
            std::memcpy(buf, o.data(), o.size());
            buf[o.size()] = 0;
        }
        CATNN_REQUIRE(!blob || nb <= blob_cap, CATNN_ERR_SHAPE_MISMATCH, "blob buffer too small");
    });
}

}  // extern "C"
