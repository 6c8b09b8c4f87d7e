// describe(): the kernels a node launches on gfx950, with the launch
// geometry its launcher would choose for the given input types and each
// kernel's resources as built (kernel_table.hpp) — the HIP counterpart of
// kernel::resource::describe (crates/catnn-compile/src/kernel/resource.rs:
// 155-186), whose CUDA and CPU sizes are estimates; here every figure is
// read from this build's code objects.
//
// The geometry below restates each launcher's choice (gemm_f32.hip
// gemm_launch / gemm_grouped_launch, rowops.hip, attention.hip
// attention_fwd, moe.hip, decoder.hip) for buffers aligned as the program
// arena aligns them (256 bytes); tests check every kernel named here exists
// in the table exactly once.
#include <algorithm>
#include <cstring>

#include "graph.hpp"
#include "kernel_table.hpp"

namespace catnn {

namespace {

struct Launch {
    std::string pattern;  // a substring that names exactly one kernel
    uint32_t grid;
    uint32_t block;
    uint64_t dyn_lds;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

uint32_t clamp_grid(int64_t g) { return (uint32_t)std::max<int64_t>(1, std::min<int64_t>(g, (1ll << 31) - 1)); }

// rowops.hip grid_for / decoder.hip: 256 threads, per_thread elements each,
// at least one block and at most 2^20 (grid-stride beyond).
uint32_t grid_for(int64_t n, int64_t per_thread) {
    return (uint32_t)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256 * per_thread), 1 << 20));
}

// gemm_f32.hip: 128 × 128 tiles (64 output columns in the dual SwiGLU mode);
// when K, N and both row strides are multiples of 4 (16-byte rows) the
// direct-to-LDS kernel with 4 stages of 16 KiB dynamic LDS, otherwise the
// register-staged kernel of the plain or the grouped grid.
void gemm_f32(std::vector<Launch> &L, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, bool dual,
              int64_t grouped_tiles) {
    const bool vec = K % 4 == 0 && N % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0;
    const bool grouped = grouped_tiles > 0;
    const int64_t bn = dual ? 64 : 128;
    const int64_t tiles = grouped ? grouped_tiles * cdiv(N, bn) : cdiv(M, 128) * cdiv(N, bn);
    if (tiles == 0) return;
    const std::string d = dual ? "1" : "0";
    if (vec) {
        L.push_back({"15gemm_dma_kernelILi4ELb" + d + "ELb" + (grouped ? "1" : "0") + "E", clamp_grid(tiles), 256,
                     4 * 16384});
        return;
    }
    std::string p = grouped ? "19gemm_grouped_kernelILi128ELi128ELi16ELb0ELb" : "17gemm_plain_kernelILi128ELi128ELi16ELb0ELb";
    L.push_back({p + d + "E", clamp_grid(tiles), 256, 0});
}

// rowops.hip / decoder.hip row kernels: one wavefront per row, 4 rows per
// block, NV float4 per lane.
std::string nv_suffix(int64_t c4, const int *nvs, int n_nv) {
    for (int i = 0; i < n_nv; ++i)
        if (c4 <= 64 * nvs[i]) return "ILi" + std::to_string(nvs[i]) + "EE";
    return "";
}

// full: the kernel also takes <bool FULL>, true when the row fills its NV
// float4 per lane exactly (decoder.hip rms_norm_f32).
void row_kernel(std::vector<Launch> &L, const std::string &reg, const std::string &any, int64_t rows, int64_t cols,
                bool full = false) {
    static const int nvs[] = {1, 2, 4, 8, 16};
    std::string sfx = cols % 4 == 0 ? nv_suffix(cols / 4, nvs, 5) : "";
    if (full && !sfx.empty()) {
        int nv = 0;
        for (int v : nvs)
            if (cols / 4 <= 64 * v) {
                nv = v;
                break;
            }
        sfx = "ILi" + std::to_string(nv) + "ELb" + (cols == 256 * nv ? "1" : "0") + "EE";
    }
    L.push_back({sfx.empty() ? any : reg + sfx, clamp_grid(cdiv(rows, 4)), 256, 0});
}

// attention.hip attention_fwd.
void attention(std::vector<Launch> &L, int64_t B, int64_t S, int64_t H, int64_t dh, int64_t ldq, int64_t ldk,
               int64_t ldo) {
    if (dh == 64 && ldq % 4 == 0 && ldk % 4 == 0 && ldo % 4 == 0)
        L.push_back({"16attn_mfma_kernelILi64EE", clamp_grid(B * H * cdiv(S, 128)), 256, 0});
    else
        L.push_back({"19attn_generic_kernel", clamp_grid(cdiv(B * H * S, 4)), 256, 0});
}

int64_t numel(const std::vector<int64_t> &d) {
    int64_t n = 1;
    for (int64_t v : d) n *= v;
    return n;
}

const std::vector<int64_t> &pd(const Node &n, const char *port) {
    const HostTensor *t = n.param(port);
    if (!t) fail(CATNN_ERR_UNKNOWN_PORT, std::string("unknown port ") + port + " on interface " + n.name);
    return t->dims;
}

std::vector<Launch> launches_of(const Node &node, const std::vector<std::vector<int64_t>> &ins) {
    std::vector<Launch> L;
    if (ins.empty()) return L;  // Identity without inputs: a fill
    const std::vector<int64_t> &x = ins[0];
    const int64_t nx = numel(x);
    const int64_t last = x.empty() ? 1 : x.back();
    switch (node.op.kind) {
        case CATNN_OP_IDENTITY:
        case CATNN_OP_RESHAPE:
        case CATNN_OP_TRANSPOSE:
        case CATNN_OP_ROUTER:
            break;  // device-to-device copies, no kernel
        case CATNN_OP_RELU:
        case CATNN_OP_GELU:
            if (nx > 0) L.push_back({"10act_kernelE", grid_for(nx, 4), 256, 0});
            break;
        case CATNN_OP_SOFTMAX:
            if (nx > 0 && last > 0) row_kernel(L, "18softmax_reg_kernel", "18softmax_any_kernel", nx / last, last);
            break;
        case CATNN_OP_ADD:
        case CATNN_OP_RESIDUAL_ADD: {
            if (ins.size() < 2 || nx == 0) break;
            const int64_t nb = numel(ins[1]);
            if (nb == nx && nx % 4 == 0) L.push_back({"11add4_kernel", grid_for(nx, 4), 256, 0});
            else L.push_back({"10add_kernel", grid_for(nx, 1), 256, 0});
            break;
        }
        case CATNN_OP_MUL:
            if (ins.size() >= 2 && nx > 0) L.push_back({"10mul_kernel", grid_for(nx, 1), 256, 0});
            break;
        case CATNN_OP_LINEAR:
        case CATNN_OP_MATMUL: {
            const HostTensor *w = node.param("w") ? node.param("w") : (node.params.empty() ? nullptr : &node.params.front().second);
            if (!w) fail(CATNN_ERR_UNKNOWN_COMPONENT, "unknown component " + node.name);
            const int64_t k = w->dims[0], n = w->dims[1];
            gemm_f32(L, nx / std::max<int64_t>(k, 1), n, k, k, n, false, 0);
            break;
        }
        case CATNN_OP_LAYER_NORM:
            row_kernel(L, "21layer_norm_reg_kernel", "21layer_norm_any_kernel", nx / last, last);
            break;
        case CATNN_OP_ATTENTION: {
            const int64_t B = x[0], S = x[1], D = x[2], T = B * S;
            gemm_f32(L, T, 3 * D, D, D, 3 * D, false, 0);  // packed q|k|v projection
            attention(L, B, S, node.op.a[0], node.op.a[2], 3 * D, 3 * D, D);
            gemm_f32(L, T, D, D, D, D, false, 0);
            break;
        }
        case CATNN_OP_MOE: {
            const int64_t H = last, T = nx / H, E = node.op.a[0], K = node.op.a[1];
            const int64_t I = pd(node, "e0.w1")[1];
            const int64_t tpb = std::min<int64_t>(64, 256 / E);
            // moe.hip moe_route_f32: the LDS-staged kernel (four 64-column chunks of 4-row
            // groups, whole transposed gate) when it fits 80 KiB, else the streaming one
            const uint64_t dma = 4 * (uint64_t)(4 * (tpb / 4) * (4 * 64 + 4) + E * (H + 4) + tpb * E);
            if (H % 64 == 0 && tpb % 16 == 0 && dma <= 80 * 1024) {
                L.push_back({"16route_dma_kernelILi" + std::to_string(tpb / 16) + "EE", clamp_grid(cdiv(T, tpb)), 256,
                             dma});
            } else if (H % 4 == 0) {
                const int64_t HC = std::min<int64_t>(H, (12288 / E - 4) & ~int64_t(3));
                L.push_back({"16route_vec_kernel", clamp_grid(cdiv(T, tpb)), 256,
                             (uint64_t)(4 * (E * (HC + 4) + tpb * E))});
            } else {
                L.push_back({"12route_kernel", clamp_grid(cdiv(T, tpb)), 256,
                             (uint64_t)(4 * (tpb * 65 + 64 * E + tpb * E))});
            }
            const int64_t n = T * K, nb = cdiv(n, 4096);
            if (nb > 0) L.push_back({"17perm_count_kernel", clamp_grid(nb), 256, 0});
            L.push_back({"16perm_scan_kernel", 1, 64, 0});
            if (nb > 0) L.push_back({"19perm_scatter_kernel", clamp_grid(nb), 256, 0});
            L.push_back({"18build_tiles_kernel", 1, 64, 0});
            const int64_t max_tiles = cdiv(n, 128) + E;
            gemm_f32(L, n, I, H, H, I, true, max_tiles);
            gemm_f32(L, n, H, I, I, H, false, max_tiles);
            L.push_back({H % 4 == 0 ? "15combine4_kernel" : "14combine_kernel", clamp_grid(T), 256, 0});
            break;
        }
        case CATNN_OP_RMS_NORM:
            row_kernel(L, "19rms_norm_reg_kernel", "19rms_norm_any_kernel", nx / last, last, true);
            break;
        case CATNN_OP_EMBEDDING: {
            const int64_t hidden = node.op.a[1];
            if (hidden == 1024)  // two tokens a wavefront
                L.push_back({"21embedding_pair_kernel", clamp_grid(cdiv(cdiv(nx, 2), 4)), 256, 0});
            else
                L.push_back({hidden % 4 == 0 ? "16embedding_kernelILb1E" : "16embedding_kernelILb0E",
                             clamp_grid(cdiv(nx, 4)), 256, 0});
            break;
        }
        case CATNN_OP_GQA_ATTENTION: {
            const int64_t B = x[0], S = x[1], D = x[2], T = B * S;
            const int64_t nh = node.op.a[0], nkv = node.op.a[1], hd = node.op.a[2];
            const int64_t QW = nh * hd, LD = (nh + 2 * nkv) * hd, half = hd / 2;
            gemm_f32(L, T, LD, D, D, LD, false, 0);
            if (half > 0) {
                L.push_back({"17rope_table_kernel", clamp_grid(cdiv(S * half, 256)), 256, 0});
                if (half % 2 == 0 && LD % 4 == 0)  // two pairs a thread
                    L.push_back({"18rope_apply2_kernel", clamp_grid(cdiv(T * (nh + nkv) * half / 2, 256)), 256, 0});
                else
                    L.push_back({"17rope_apply_kernel", clamp_grid(cdiv(T * (nh + nkv) * half, 256)), 256, 0});
            }
            attention(L, B, S, nh, hd, LD, LD, QW);
            gemm_f32(L, T, D, QW, QW, D, false, 0);
            break;
        }
        case CATNN_OP_SWIGLU: {
            const int64_t H = last, T = nx / H, I = pd(node, "w1")[1];
            gemm_f32(L, T, I, H, H, I, true, 0);
            gemm_f32(L, T, H, I, I, H, false, 0);
            break;
        }
        case CATNN_OP_LM_HEAD: {  // installed graphs: the GEMM on the Wᵀ copy
            const int64_t H = last, V = node.op.a[1];
            gemm_f32(L, nx / H, V, H, H, V, false, 0);
            break;
        }
        case CATNN_OP_MIX:
            if (nx > 0) L.push_back({"10mix_kernel", std::min<uint32_t>(grid_for(nx, 4), 1u << 20), 256, 0});
            break;
        default:
            fail(CATNN_ERR_UNSUPPORTED,
                 "op " + op_name(node.op.kind) + " (node " + node.name + ") is not executable on the HIP backend");
    }
    return L;
}

const KernelInfo &lookup(const std::string &pattern) {
    const KernelInfo *hit = nullptr;
    for (int i = 0; i < kKernelTableSize; ++i)
        if (std::strstr(kKernelTable[i].symbol, pattern.c_str())) {
            CATNN_REQUIRE(!hit, CATNN_ERR_INVALID_ARGUMENT, "describe: kernel pattern " + pattern + " is ambiguous");
            hit = &kKernelTable[i];
        }
    CATNN_REQUIRE(hit, CATNN_ERR_INVALID_ARGUMENT, "describe: no kernel matches " + pattern);
    return *hit;
}

void fill_static(catnn_kernel_launch &o, const KernelInfo &k) {
    std::memset(o.kernel, 0, sizeof(o.kernel));
    std::strncpy(o.kernel, k.symbol, sizeof(o.kernel) - 1);
    o.code_bytes = k.code_bytes;
    o.vgprs = k.vgprs;
    o.agprs = k.agprs;
    o.sgprs = k.sgprs;
    o.static_lds_bytes = k.lds_static;
    o.kernarg_bytes = k.kernarg_bytes;
    o.scratch_bytes_per_lane = k.scratch_per_lane;
}

}  // namespace

}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_hip_describe(const catnn_node *node, const catnn_tensor *in_types, int32_t n_in,
                       catnn_kernel_resource *out, catnn_kernel_launch *launches, int32_t cap) {
    return guard([&] {
        CATNN_REQUIRE(node && out && n_in >= 0 && (n_in == 0 || in_types) && cap >= 0 && (cap == 0 || launches),
                      CATNN_ERR_INVALID_ARGUMENT, "describe: null argument");
        const Node n = node_shape_from_c(node);
        std::vector<std::vector<int64_t>> ins;
        for (int32_t i = 0; i < n_in; ++i) ins.push_back(dims_from_c(in_types[i]));
        infer_dims(n, ins);  // the node's shape checks, with their error kinds
        const std::vector<Launch> L = launches_of(n, ins);
        std::memset(out, 0, sizeof(*out));
        out->code_estimated = 0;
        out->temp_bytes = scratch_bytes(n, ins);
        out->n_launches = (int32_t)L.size();
        std::vector<const KernelInfo *> seen;
        uint64_t most = 0;
        for (size_t i = 0; i < L.size(); ++i) {
            const KernelInfo &k = lookup(L[i].pattern);
            if (std::find(seen.begin(), seen.end(), &k) == seen.end()) {
                seen.push_back(&k);
                out->code_bytes += k.code_bytes;
            }
            // .vgpr_count of gfx950 code objects is the unified VGPR + AGPR allocation
            out->registers_per_thread = std::max(out->registers_per_thread, k.vgprs);
            out->static_smem_bytes = std::max(out->static_smem_bytes, k.lds_static);
            out->dynamic_smem_bytes = std::max(out->dynamic_smem_bytes, L[i].dyn_lds);
            out->launch_arg_bytes = std::max(out->launch_arg_bytes, k.kernarg_bytes);
            const uint64_t items = (uint64_t)L[i].grid * L[i].block;
            if (items > most) {
                most = items;
                out->grid[0] = L[i].grid;
                out->grid[1] = out->grid[2] = 1;
                out->block[0] = L[i].block;
                out->block[1] = out->block[2] = 1;
            }
            if ((int32_t)i < cap) {
                catnn_kernel_launch &o = launches[i];
                fill_static(o, k);
                o.grid[0] = L[i].grid;
                o.grid[1] = o.grid[2] = 1;
                o.block[0] = L[i].block;
                o.block[1] = o.block[2] = 1;
                o.dynamic_lds_bytes = L[i].dyn_lds;
            }
        }
    });
}

int catnn_hip_kernel_table_size(int32_t *n) {
    return guard([&] {
        CATNN_REQUIRE(n, CATNN_ERR_INVALID_ARGUMENT, "null out pointer");
        *n = kKernelTableSize;
    });
}

int catnn_hip_kernel_table_entry(int32_t i, catnn_kernel_launch *out) {
    return guard([&] {
        CATNN_REQUIRE(out && i >= 0 && i < kKernelTableSize, CATNN_ERR_INVALID_ARGUMENT,
                      "kernel table index out of range");
        std::memset(out, 0, sizeof(*out));
        fill_static(*out, kKernelTable[i]);
        out->block[0] = kKernelTable[i].max_workgroup;
    });
}

}  // extern "C"
