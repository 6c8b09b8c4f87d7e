/*
 * catnn_hip.h — C ABI of the MI355X (gfx950) execution backend for catnn's
 * lowered IR.
 *
 * The reference (dkarapetyan-afk/cat-nn-compiler, Rust) executes every IR node
 * through `DeviceHandler::run_kernel(&mut self, node: &IrNode,
 * inputs: &[Tensor]) -> CatResult<Tensor>` (crates/catnn-rt/src/handler.rs:34),
 * which calls `kernel::eval_cpu` (crates/catnn-compile/src/kernel/mod.rs:21)
 * even for GPU-placed nodes (handler.rs:43-46).  This header is what a Rust
 * `-sys` crate (or any FFI) binds to replace that call for a new
 * `KernelBackend::Hip` target.  Every function is `extern "C"`, takes plain
 * pointers and sizes, returns an `int` status (0 = ok, otherwise one of the
 * CATNN_ERR_* codes that map 1:1 onto `CatError` variants,
 * crates/catnn-core/src/error.rs:9-54), and leaves a message in the calling
 * thread's `catnn_hip_last_error()`.
 *
 * Threading contract (mirrors the reference's wave model, dist.rs:441-517):
 * a device handle is used by one host thread at a time; each device owns one
 * in-order HIP stream, so arena buffers whose lifetimes do not overlap may
 * alias safely.
 *
 * Ownership: host pointers passed in are borrowed for the duration of the
 * call only.  Device pointers returned by catnn_hip_buffer_ptr /
 * catnn_hip_alloc stay owned by the library.
 */
#ifndef CATNN_HIP_H
#define CATNN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
/* CatError variants, crates/catnn-core/src/error.rs:9-54 (same order). */
enum catnn_status {
    CATNN_OK = 0,
    CATNN_ERR_INTERFACE_MISMATCH = 1,   /* error.rs:11 */
    CATNN_ERR_SHAPE_MISMATCH = 2,       /* error.rs:14 */
    CATNN_ERR_DTYPE_MISMATCH = 3,       /* error.rs:17 */
    CATNN_ERR_UNKNOWN_PORT = 4,         /* error.rs:20 */
    CATNN_ERR_UNKNOWN_COMPONENT = 5,    /* error.rs:23 */
    CATNN_ERR_UNKNOWN_ARCHITECTURE = 6, /* error.rs:26 */
    CATNN_ERR_UNKNOWN_REALIZATION = 7,  /* error.rs:29 */
    CATNN_ERR_WIRING = 8,               /* error.rs:32 (cycles, missing preds) */
    CATNN_ERR_PARSE = 9,                /* error.rs:35 */
    CATNN_ERR_FIBRATION = 10,           /* error.rs:38 (arena overflow, schedule.rs:101-105) */
    CATNN_ERR_WITNESS = 11,             /* error.rs:41 */
    CATNN_ERR_DESCENT = 12,             /* error.rs:44 */
    CATNN_ERR_INTERVAL = 13,            /* error.rs:47 */
    CATNN_ERR_UNLAWFUL = 14,            /* error.rs:50 */
    CATNN_ERR_IO = 15,                  /* error.rs:53 */
    /* Backend-only conditions with no CatError counterpart: */
    CATNN_ERR_DEVICE = 100,             /* a HIP runtime call failed, or no GPU */
    CATNN_ERR_UNSUPPORTED = 101,        /* op kind not executable on this backend */
    CATNN_ERR_INVALID_ARGUMENT = 102    /* null handle / pointer, bad enum value */
};

/* Message for the last failing call on this thread ("" after success). */
const char *catnn_hip_last_error(void);

/* ------------------------------------------------------------ data types */
/* DType tag, crates/catnn-core/src/tensor.rs:17-27.  Storage is always f32
 * on the host, as in the reference (tensor.rs:223-229). */
enum catnn_dtype {
    CATNN_F32 = 0, CATNN_F16 = 1, CATNN_BF16 = 2, CATNN_FP8 = 3,
    CATNN_FP4 = 4, CATNN_I32 = 5, CATNN_BOOL = 6
};

#define CATNN_MAX_RANK 8

/* Host tensor: `Tensor { ty: TensorType { shape, dtype }, data: Vec<f32> }`
 * (tensor.rs:181-229).  `data` may be NULL when only the type matters
 * (IrNode.output_ty). */
typedef struct catnn_tensor {
    float *data;
    int64_t dims[CATNN_MAX_RANK];
    int32_t rank;
    int32_t dtype;
} catnn_tensor;

/* OpenOp discriminant, crates/catnn-core/src/category/morphism.rs:19-116
 * (declaration order). */
enum catnn_op_kind {
    CATNN_OP_IDENTITY = 0,
    CATNN_OP_LINEAR = 1,        /* a = {in_features, out_features, bias} */
    CATNN_OP_RELU = 2,
    CATNN_OP_GELU = 3,
    CATNN_OP_SOFTMAX = 4,       /* a = {axis} (last axis only, as cpu.rs:31) */
    CATNN_OP_LAYER_NORM = 5,    /* a = {eps_e6} */
    CATNN_OP_ADD = 6,
    CATNN_OP_MUL = 7,
    CATNN_OP_MATMUL = 8,        /* executed as Linear with param "w" */
    CATNN_OP_TRANSPOSE = 9,     /* a = {dim0, dim1}; data copy as eval_cpu */
    CATNN_OP_RESHAPE = 10,      /* a = {out dims...}; data copy as eval_cpu */
    CATNN_OP_ATTENTION = 11,    /* a = {n_heads, d_model, d_head} */
    CATNN_OP_RESIDUAL_ADD = 12,
    CATNN_OP_EMBEDDING = 13,    /* a = {vocab, hidden}; param "w" [vocab, hidden]; ids as f32 */
    CATNN_OP_RMS_NORM = 14,     /* a = {eps_e6}; param "w" */
    CATNN_OP_GQA_ATTENTION = 15, /* a = {n_heads, n_kv_heads, head_dim, d_model,
                                    sliding_window (-1: None), rope_theta} */
    CATNN_OP_SWIGLU = 16,       /* a = {hidden, intermediate}; params w1, w3, w2 */
    CATNN_OP_ROUTER = 17,       /* a = {n_experts, top_k}; identity, as eval_cpu */
    CATNN_OP_MOE = 18,          /* a = {n_experts, top_k, hidden, intermediate} */
    CATNN_OP_LM_HEAD = 19,      /* a = {hidden, vocab}; param "w" [vocab, hidden] */
    CATNN_OP_MLA = 20,          /* not executable here: CATNN_ERR_UNSUPPORTED */
    CATNN_OP_DEEPSEEK_MOE = 21, /* not executable here: CATNN_ERR_UNSUPPORTED */
    CATNN_OP_MIX = 22           /* two inputs; optional param "gate" [1] */
};

/* Attention extension: causal mask with the masking convention of
 * moe::gqa (crates/catnn-compile/src/kernel/moe.rs:105-121).  The reference
 * Attention op has no mask (cpu.rs:235-298); with the flag clear the backend
 * computes exactly that. */
#define CATNN_FLAG_CAUSAL 0x1

typedef struct catnn_op {
    int32_t kind;      /* enum catnn_op_kind */
    int32_t flags;     /* CATNN_FLAG_* */
    int64_t a[8];      /* the variant's fields in declaration order */
} catnn_op;

/* `Tensor::lcg(ty, seed)` (crates/catnn-core/src/tensor.rs:259-268): the
 * deterministic fill the reference uses for every materialised param
 * (lower.rs:117-127) and test input.  Host-only. */
int catnn_tensor_lcg(uint64_t seed, float *out, int64_t n);
/* `Tensor::checksum` (tensor.rs:279-288): FNV-1a over the f32 bit patterns.
 * Host-only. */
int catnn_tensor_checksum(const float *data, int64_t n, uint64_t *out);

/* One entry of `IrNode.params: IndexMap<String, Tensor>` (ir.rs:22-23). */
typedef struct catnn_param {
    const char *port;
    catnn_tensor value;
} catnn_param;

/* `IrNode { id, name, op, output_ty, params }` (crates/catnn-compile/src/ir.rs:17-24). */
typedef struct catnn_node {
    uint32_t id;
    const char *name;
    catnn_op op;
    catnn_tensor output_ty;
    const catnn_param *params;
    int32_t n_params;
} catnn_node;

/* ------------------------------------------------------------ the arena */
/* `BufferReq` (crates/catnn-compile/src/schedule.rs:61-70); lifetimes are
 * inclusive logical ticks. */
typedef struct catnn_buffer_req {
    const char *id;
    uint64_t bytes;
    uint64_t live_from;
    uint64_t live_to;
    int32_t checkpoint;
} catnn_buffer_req;

#define CATNN_ID_CAP 128

/* `ArenaAlloc` (schedule.rs:36-43). */
typedef struct catnn_arena_alloc {
    char id[CATNN_ID_CAP];
    uint64_t bytes;
    uint64_t offset;
    uint64_t live_from;
    uint64_t live_to;
} catnn_arena_alloc;

/* First-fit placement with aliased lifetimes; replaces `place_arena`
 * (schedule.rs:79-116).  `out` has room for `n` entries and receives them
 * in placement order.  Host-only (no GPU needed).  Overflow of `cap`
 * returns CATNN_ERR_FIBRATION naming the buffer. */
int catnn_place_arena(const catnn_buffer_req *reqs, int32_t n, uint64_t cap,
                      catnn_arena_alloc *out);

/* `arena_conflict` (schedule.rs:123-136): sets *conflict to 1 and the pair
 * (i, j) when two simultaneously live allocations overlap, else 0. */
int catnn_arena_conflict(const catnn_arena_alloc *allocs, int32_t n,
                         int32_t *conflict, int32_t *i, int32_t *j);

/* ------------------------------------------------------------ the graph */
/* `IrGraph { name, nodes, edges, inputs, outputs }` (ir.rs:35-41), built on
 * the host.  Host-only (no GPU needed). */
typedef struct catnn_graph catnn_graph;

int catnn_graph_new(const char *name, catnn_graph **out);
int catnn_graph_free(catnn_graph *g);
/* Copies the node, its name and its params. */
int catnn_graph_add_node(catnn_graph *g, const catnn_node *node);
/* `IrEdge { src, dst, src_port, dst_port }` (ir.rs:26-32).  Insertion order
 * fixes the order of a node's inputs (`preds`, ir.rs:58-60). */
int catnn_graph_add_edge(catnn_graph *g, uint32_t src, uint32_t dst,
                         const char *src_port, const char *dst_port);
int catnn_graph_add_input(catnn_graph *g, uint32_t id);
int catnn_graph_add_output(catnn_graph *g, uint32_t id);
/* `Realization.fusions` entry (FusionGroup, realization.rs:40-45): the named
 * ops run as one kernel when they are placed on the same device. */
int catnn_graph_add_fusion(catnn_graph *g, const char *const *op_names, int32_t n);
/* Builds a graph from the reference's serde JSON of `IrGraph`
 * (crates/catnn-compile/src/ir.rs:13-41 serialised with serde_json, as the
 * control plane ships it, dist.rs), replacing serde_json::from_slice on the
 * member side.  A parameter whose "data" is [] takes its numel floats from
 * `blob` (node order, then port order; blob_floats must match exactly), so
 * large parameter sets need not pass through the 64 MiB frame.  Also reads
 * "causal": true inside "attention" and a top-level "fusions" list.  Parse
 * errors are CATNN_ERR_PARSE with the byte offset. */
int catnn_graph_from_json(const char *json, uint64_t len, const float *blob, uint64_t blob_floats,
                          catnn_graph **out);
/* The inverse (serde_json::to_vec of the same IrGraph): writes the JSON to
 * buf (NUL-terminated when cap > *len; call with buf = NULL for the size)
 * and, unless inline_params, every parameter to `blob` with "data": [].
 * *blob_floats receives the blob length. */
int catnn_graph_to_json(const catnn_graph *g, int32_t inline_params, char *buf, uint64_t cap,
                        uint64_t *len, float *blob, uint64_t blob_cap, uint64_t *blob_floats);
/* Kahn order as `IrGraph::topo` (ir.rs:67-92); cycles → CATNN_ERR_WIRING. */
int catnn_graph_topo(const catnn_graph *g, uint32_t *order, int32_t cap, int32_t *n);

/* ------------------------------------------------------------ the device */
typedef struct catnn_hip_device catnn_hip_device;

int catnn_hip_device_count(int32_t *n);
/* Opens GPU `ordinal`, creates its stream.  Fails with CATNN_ERR_DEVICE
 * when no GPU is present: there is no CPU fallback. */
int catnn_hip_open(int32_t ordinal, catnn_hip_device **out);
int catnn_hip_close(catnn_hip_device *dev);
int catnn_hip_sync(catnn_hip_device *dev);
/* Device name and HBM size, for the MI355X region profile. */
int catnn_hip_device_info(catnn_hip_device *dev, char *name, int32_t cap,
                          uint64_t *hbm_bytes, int32_t *cu_count);

/* One hipMalloc backing the device's buffer region.  Replaces any earlier
 * arena (all bindings are dropped). */
int catnn_hip_arena_reserve(catnn_hip_device *dev, uint64_t bytes);
/* Bind `buffer_id` ("act:{node}", "param:{node}:{port}", …, as
 * pipeline.rs:319-379) to arena[offset, offset+bytes). */
int catnn_hip_bind(catnn_hip_device *dev, const char *buffer_id,
                   uint64_t offset, uint64_t bytes);
int catnn_hip_buffer_ptr(catnn_hip_device *dev, const char *buffer_id,
                         void **dptr, uint64_t *bytes);
int catnn_hip_upload(catnn_hip_device *dev, const char *buffer_id,
                     const void *host, uint64_t bytes);
int catnn_hip_download(catnn_hip_device *dev, const char *buffer_id,
                       void *host, uint64_t bytes);

/* Plain device memory outside the arena (test and bench plumbing). */
int catnn_hip_alloc(catnn_hip_device *dev, uint64_t bytes, void **dptr);
int catnn_hip_free(catnn_hip_device *dev, void *dptr);
int catnn_hip_h2d(catnn_hip_device *dev, void *dst, const void *src, uint64_t bytes);
int catnn_hip_d2h(catnn_hip_device *dev, void *dst, const void *src, uint64_t bytes);
int catnn_hip_memset(catnn_hip_device *dev, void *dst, int32_t value, uint64_t bytes);

/* Stream-ordered timer on the device's stream (hipEvent pair). */
int catnn_hip_timer_start(catnn_hip_device *dev);
int catnn_hip_timer_stop(catnn_hip_device *dev, float *ms);

/* ------------------------------------------------------- describe() */
/* One kernel launch of a node, with the kernel's resources as built: the
 * counts come from this build's gfx950 code objects (AMDGPU metadata note
 * and symbol table), read at build time. */
#define CATNN_KERNEL_NAME_MAX 256
typedef struct catnn_kernel_launch {
    char kernel[CATNN_KERNEL_NAME_MAX]; /* mangled kernel symbol */
    uint32_t grid[3];                   /* workgroups */
    uint32_t block[3];                  /* work-items per workgroup */
    uint64_t dynamic_lds_bytes;
    uint64_t code_bytes;                /* the kernel's function symbol */
    uint32_t vgprs;                     /* unified VGPR + AGPR registers per lane */
    uint32_t agprs, sgprs;              /* the AGPR part of vgprs; SGPRs */
    uint64_t static_lds_bytes;          /* group segment */
    uint64_t kernarg_bytes;             /* kernel-argument segment */
    uint64_t scratch_bytes_per_lane;    /* private segment */
} catnn_kernel_launch;

/* `KernelResource` (crates/catnn-compile/src/kernel/resource.rs:28-45) of
 * a node on this backend, aggregated over its launches. */
typedef struct catnn_kernel_resource {
    uint64_t code_bytes;           /* sum over the distinct kernels */
    int32_t code_estimated;        /* 0: measured from the code objects */
    uint32_t registers_per_thread; /* largest unified VGPR + AGPR count */
    uint64_t static_smem_bytes;    /* largest static LDS */
    uint64_t dynamic_smem_bytes;   /* largest dynamic LDS */
    uint32_t grid[3], block[3];    /* the launch with the most work-items */
    uint64_t launch_arg_bytes;     /* largest kernel-argument segment */
    uint64_t temp_bytes;           /* device scratch beyond the output */
    int32_t n_launches;
} catnn_kernel_resource;

/* Replaces kernel::resource::describe (resource.rs:155-186) for the HIP
 * backend: the launches `node` makes on inputs of the given types (as an
 * installed graph runs it; params need types only), the first `cap` of
 * them written to `launches`.  Host-only (no GPU needed).  Shape errors as
 * catnn_hip_run_kernel; unsupported ops → CATNN_ERR_UNSUPPORTED. */
int catnn_hip_describe(const catnn_node *node, const catnn_tensor *in_types, int32_t n_in,
                       catnn_kernel_resource *out, catnn_kernel_launch *launches, int32_t cap);
/* Every kernel of the build (resources only; block[0] = the largest
 * workgroup it accepts).  Host-only. */
int catnn_hip_kernel_table_size(int32_t *n);
int catnn_hip_kernel_table_entry(int32_t i, catnn_kernel_launch *out);

/* ---------------------------------------------------- the handler seam */
/* Drop-in for `DeviceHandler::run_kernel` (handler.rs:34-57) with
 * host tensors in and out: params ride inside `node` (as the reference
 * clones them per call, coord.rs:320-323), inputs are the node's preds in
 * edge order.  `out->data` must hold the output's numel floats; dims, rank
 * and dtype are written.  Records KernelStart/KernelEnd events. */
int catnn_hip_run_kernel(catnn_hip_device *dev, const catnn_node *node,
                         const catnn_tensor *inputs, int32_t n_inputs,
                         catnn_tensor *out);

/* Drop-in for `adjoint_of(node, inputs, output, dy) -> Adjoint { dx,
 * dparams }` (crates/catnn-compile/src/kernel/adjoint.rs:762-951), the seam
 * the training wave calls at crates/catnn-rt/src/coord.rs:413, with host
 * tensors: `dx[i]` receives the cotangent of inputs[i] (n_inputs entries)
 * and `dparams[j]` that of the node's j-th param in IndexMap order
 * (n_dparams == node->n_params); each must hold the value's numel floats,
 * and dims, rank and dtype are written.  The forward value is recomputed on
 * the device from `inputs` (as attention_backward recomputes its forward,
 * adjoint.rs:582-722), so `output` may be NULL and is not read.  Ops as the
 * training step executes them at CATNN_PREC_FP32 (the reference's adjoints
 * are fp32 throughout); the one-node plan of a node shape is built once per
 * device and reused (up to 16 shapes, 16 GiB, least recently used first);
 * a Router → CATNN_ERR_UNLAWFUL (adjoint.rs:915-920); others →
 * CATNN_ERR_UNSUPPORTED; no inputs → CATNN_ERR_WIRING
 * (adjoint.rs:768-770). */
int catnn_hip_run_adjoint(catnn_hip_device *dev, const catnn_node *node,
                          const catnn_tensor *inputs, int32_t n_inputs,
                          const catnn_tensor *output, const catnn_tensor *dy,
                          catnn_tensor *dx, catnn_tensor *dparams, int32_t n_dparams);

/* Device-resident variant: inputs, output and params are arena buffer ids
 * (params bound as "param:{node.name}:{port}"; the node's params need only
 * dims here, data may be NULL).  `in_types` gives each input's type (data
 * ignored), as the Tensors of run_kernel do.  `fused_act` applies a
 * following Relu (2) or Gelu (3) from a FusionGroup in the Linear epilogue;
 * `residual_id` (or NULL) adds a following ResidualAdd's other operand in
 * the epilogue.  Scratch (attention q/k/v, MoE permutation) comes from a
 * per-device workspace. */
int catnn_hip_run_node(catnn_hip_device *dev, const catnn_node *node,
                       const char *const *in_ids, const catnn_tensor *in_types,
                       int32_t n_in, const char *out_id, int32_t fused_act,
                       const char *residual_id);

/* ------------------------------------------------------- the program */
/* A graph installed on a device: arena planned by catnn_place_arena over
 * forward lifetimes (act:{node} live from its topo index to its last
 * consumer's, params live throughout), reserved with one hipMalloc, params
 * uploaded once.  Replaces `eval_graph_cpu` (crates/catnn-compile/src/lib.rs:48-68)
 * for a graph placed on this device. */
typedef struct catnn_hip_program catnn_hip_program;

int catnn_hip_install(catnn_hip_device *dev, const catnn_graph *g,
                      catnn_hip_program **out);
int catnn_hip_program_free(catnn_hip_program *p);
/* Host input bound to every graph input node; host output of the last
 * output node (lib.rs:57-67). */
int catnn_hip_forward(catnn_hip_program *p, const catnn_tensor *input,
                      catnn_tensor *output);
/* Same, with the input already in the program's input buffer and the
 * output left in the output buffer (no host copies, no sync).  An Embedding
 * that meets an id ≥ vocab (ShapeMismatch in moe::embedding, moe.rs:38-40)
 * is reported by the next call that synchronises the program:
 * catnn_hip_forward, catnn_hip_program_get_value or catnn_hip_program_check. */
int catnn_hip_forward_resident(catnn_hip_program *p);
/* Waits for the program's enqueued forwards; CATNN_ERR_SHAPE_MISMATCH if one
 * of them met a token id ≥ vocab. */
int catnn_hip_program_check(catnn_hip_program *p);
/* Device buffers of the program's input and output. */
int catnn_hip_program_io(catnn_hip_program *p, void **in_dptr, uint64_t *in_bytes,
                         void **out_dptr, uint64_t *out_bytes);
/* The program's arena plan (one entry per placed buffer). */
int catnn_hip_program_arena(catnn_hip_program *p, catnn_arena_alloc *out,
                            int32_t cap, int32_t *n, uint64_t *reserved_bytes);

/* Per-step device timing: while enabled, every forward records a hipEvent
 * before each executed step and after the last, on the program's stream
 * (no extra synchronisation).  `catnn_hip_program_timings` waits for the
 * recorded forwards and returns, per step, its node name, the number of
 * timed calls and the summed device milliseconds.  Enabling resets the
 * sums.  (The reference's note_kernel, handler.rs:61-79, records host
 * wall-clock spans; these are the device's.) */
typedef struct catnn_step_timing {
    char name[CATNN_ID_CAP];
    int32_t kind;       /* enum catnn_op_kind of the executed node */
    int32_t calls;
    double total_ms;
} catnn_step_timing;
int catnn_hip_program_profile(catnn_hip_program *p, int32_t enable);
int catnn_hip_program_timings(catnn_hip_program *p, catnn_step_timing *out,
                              int32_t cap, int32_t *n);

/* --------------------------------------------------- placement target */
/* The new placement target in H.  A Realization places each IR node on a
 * cluster device (`Placement.assign`, crates/catnn-core/src/architecture/
 * realization.rs:13-31); a device of kind Gpu whose architecture is gfx950
 * gets the HIP kernel backend (catnn_hip_kernels_for), and the runtime runs
 * that device's stage of the graph here (catnn_hip_install_placed). */

/* KernelBackend (realization.rs:49-55, declaration order) with the new
 * variant last. */
enum catnn_kernel_backend {
    CATNN_BACKEND_CPU_RUST = 0, CATNN_BACKEND_WGSL = 1, CATNN_BACKEND_REFERENCE = 2,
    CATNN_BACKEND_CUDA_SM121 = 3, CATNN_BACKEND_HIP = 4
};
/* DeviceKind (crates/catnn-core/src/architecture/hardware.rs:13-17). */
enum catnn_device_kind { CATNN_DEVICE_CPU = 0, CATNN_DEVICE_GPU = 1, CATNN_DEVICE_ACCELERATOR = 2 };

/* One device of the cluster: `Device { id, kind, .. }` (hardware.rs:39-49)
 * plus the GPU architecture the device reports ("gfx950" for MI355X; NULL or
 * "" for none). */
typedef struct catnn_cluster_device {
    const char *id;
    int32_t kind;      /* enum catnn_device_kind */
    const char *arch;
} catnn_cluster_device;

/* One entry of `Placement.assign`: op name → device id. */
typedef struct catnn_placement_entry {
    const char *op;
    const char *device;
} catnn_placement_entry;

/* `KernelChoice { op, backend }` (realization.rs:57-61). */
typedef struct catnn_kernel_choice {
    char op[CATNN_ID_CAP];
    int32_t backend;   /* enum catnn_kernel_backend */
} catnn_kernel_choice;

/* kernels_for (crates/catnn-compile/src/place.rs:152-166) with the HIP arm:
 * for every node in IndexMap order, the backend of the device its placement
 * names — Gpu with arch "gfx950" → CATNN_BACKEND_HIP, other Gpu or
 * Accelerator → CATNN_BACKEND_WGSL, anything else (Cpu, an unplaced node, an
 * unknown device) → CATNN_BACKEND_CPU_RUST.  Writes the first `cap` choices
 * and sets *n to the node count.  Host-only. */
int catnn_hip_kernels_for(const catnn_graph *g, const catnn_placement_entry *assign, int32_t n_assign,
                          const catnn_cluster_device *devices, int32_t n_devices,
                          catnn_kernel_choice *out, int32_t cap, int32_t *n);

/* `MemoryRegion` (crates/catnn-core/src/architecture/memory.rs:79-88) and
 * `DeviceMemory { code, buffer, scratch }` (memory.rs:95-100). */
typedef struct catnn_memory_region {
    uint64_t bytes;
    double bandwidth_bps;
    double latency_s;
    char provenance[256];
} catnn_memory_region;
typedef struct catnn_device_memory {
    catnn_memory_region code, buffer, scratch;
} catnn_device_memory;

/* The MI355X region profile of H, the counterpart of DeviceMemory::
 * dgx_spark (memory.rs:136-175): buffer = the device's HBM3E (its reported
 * size; 8 TB/s published), scratch = the 160 KiB of LDS per CU (gfx950),
 * code = the bytes of this library's gfx950 kernels (measured from its code
 * objects at build time).  `dev` may be NULL: then the published 288 GB is
 * used for the buffer and nothing touches a GPU. */
int catnn_hip_device_memory(catnn_hip_device *dev, catnn_device_memory *out);

/* Installs the stage of `g` placed on `device_id` — the nodes whose
 * placement (assign; absent: default_device, as forward_device reads it,
 * crates/catnn-rt/src/coord.rs:629) names it.  A value produced on another
 * device and read here enters as the input port "{producer}#recv" (the
 * buffer act:{producer}#recv of schedule_device, pipeline.rs:319-327); a
 * local value read elsewhere, and a graph output placed here, is an output
 * port.  No node placed there → CATNN_ERR_UNKNOWN_REALIZATION.  The stage
 * is an installed program (one hipMalloc arena; its activations are not
 * aliased, since its steps run as their inputs arrive). */
int catnn_hip_install_placed(catnn_hip_device *dev, const catnn_graph *g, const catnn_placement_entry *assign,
                             int32_t n_assign, const char *device_id, const char *default_device,
                             catnn_hip_program **out);
/* The names of a program's input and output ports, in node order. */
int catnn_hip_program_ports(catnn_hip_program *p, char (*in_names)[CATNN_ID_CAP], int32_t in_cap, int32_t *n_in,
                            char (*out_names)[CATNN_ID_CAP], int32_t out_cap, int32_t *n_out);
/* Starts a forward pass: no value is present, no step has run. */
int catnn_hip_program_new_pass(catnn_hip_program *p);
/* Delivers the value of input port `name` (a graph input placed here, or a
 * "#recv" port) for this pass; unknown name → CATNN_ERR_UNKNOWN_PORT. */
int catnn_hip_program_set_value(catnn_hip_program *p, const char *name, const catnn_tensor *value);
/* One forward wave (forward_device, coord.rs:622-676): every step not yet run
 * in this pass whose inputs are all present runs, in topo order; *fired (or
 * NULL) receives their number — 0 when the stage is quiescent. */
int catnn_hip_forward_wave(catnn_hip_program *p, int32_t *fired);
/* The value of output port `name` (after the wave that computed it; else
 * CATNN_ERR_WIRING), copied to the host, for fanout to other devices. */
int catnn_hip_program_get_value(catnn_hip_program *p, const char *name, catnn_tensor *out);

/* ------------------------------------------------------------ training */
/* One training step of an IrGraph on this device: replaces
 * pipeline::reference_train (crates/catnn-compile/src/pipeline.rs:476-547)
 * for one step with MSE (kernel/adjoint.rs:106-119) and SGD (Sgd::put,
 * crates/catnn-core/src/lens/optim.rs:32-42), i.e. the adjoint_of,
 * rematerialisation and apply_update seams of the training wave
 * (crates/catnn-rt/src/coord.rs:413, :470, :481), which bypass the handler
 * in the reference.  Executable ops: Identity, Linear/MatMul, Relu, Gelu,
 * LayerNorm, Add/ResidualAdd (same length), Attention (causal flag
 * honoured), MoE, SwiGlu, LmHead, RmsNorm, Mix, Mul, Softmax (last axis), Embedding
 * (its ids, when a graph
 * input, are checked against the vocabulary at set_batch).  The loss is loss_and_grad's (pipeline.rs:
 * 430-451): cross-entropy against class ids (adjoint.rs:123-145) when the
 * output node is an LmHead (TrainTarget::Classes), else MSE.  GEMM operands are bf16 (bf16 MFMA, fp32 accumulation);
 * master weights, the residual stream, norms, router and accumulation are
 * fp32.  All buffers live in one hipMalloc arena planned by place_arena on
 * the reference's training ticks (pipeline.rs:280-284). */
typedef struct catnn_hip_trainer catnn_hip_trainer;

int catnn_hip_train_install(catnn_hip_device *dev, const catnn_graph *g, float lr,
                            catnn_hip_trainer **out);
/* The update morphism (OptimizerKind, crates/catnn-core/src/lens/optim.rs:
 * 142-145; chosen by TrainOptions.opt and applied by apply_update,
 * crates/catnn-compile/src/pipeline.rs:455-472). */
enum { CATNN_OPT_SGD = 0, CATNN_OPT_ADAM = 1 };
/* As catnn_hip_train_install with the optimizer named: CATNN_OPT_SGD is
 * Sgd::put (optim.rs:32-42), CATNN_OPT_ADAM is Adam::put (optim.rs:95-118)
 * with Adam::default's β₁ 0.9, β₂ 0.999, eps 1e-8 and the given lr, its
 * moments m, v resident in the arena as "adam:{node}:{port}:m|v"
 * (pipeline.rs:366-376), zero at install and after train_reset.  Unknown
 * optimizer: CATNN_ERR_INVALID_ARGUMENT. */
int catnn_hip_train_install_opt(catnn_hip_device *dev, const catnn_graph *g, int32_t optimizer,
                                float lr, catnn_hip_trainer **out);
/* GEMM precision of a trainer.  CATNN_PREC_BF16 (catnn_hip_train_install and
 * _opt): bf16 MFMA operands with fp32 accumulation as described above — the
 * mixed-precision training of the benchmark's bf16 configuration.
 * CATNN_PREC_FP32: every GEMM of the step on six-part split operands (each
 * fp32 value as three bf16 parts, the six product terms above 2⁻²⁴ summed
 * by the bf16 matrix cores with fp32 accumulation), every tape and
 * cotangent fp32: the fp32 algorithm of reference_train to fp32 rounding,
 * for fp32 graphs.  Other values: CATNN_ERR_INVALID_ARGUMENT. */
enum { CATNN_PREC_BF16 = 0, CATNN_PREC_FP32 = 1 };
/* The options of a trainer.  `arena_cap` (0: the device's memory) caps the
 * training arena, the buffer region of schedule (schedule.rs:149-212): when
 * the plan misses it, the activation with the largest bytes × lifetime is
 * checkpointed — its buffer ends at its last forward read and a copy
 * "act:{id}#recomp" lives from its first backward read, where its producer
 * runs again (rematerialisation, coord.rs:441-470) — and placement is
 * retried, as schedule() does for one buffer, until the plan fits; nothing
 * left to checkpoint → CATNN_ERR_FIBRATION.  Checkpointed steps give the
 * same bits as uncheckpointed ones. */
typedef struct catnn_train_options {
    int32_t optimizer;   /* CATNN_OPT_SGD or CATNN_OPT_ADAM */
    float lr;
    int32_t precision;   /* CATNN_PREC_BF16 or CATNN_PREC_FP32 */
    uint64_t arena_cap;
} catnn_train_options;
int catnn_hip_train_install_ex(catnn_hip_device *dev, const catnn_graph *g, const catnn_train_options *opts,
                               catnn_hip_trainer **out);
/* The values the plan checkpointed ("act:{node id}"), as DeviceStage.
 * checkpointed lists them (pipeline.rs:385-396); *n receives their number. */
int catnn_hip_train_checkpointed(catnn_hip_trainer *t, char (*ids)[CATNN_ID_CAP], int32_t cap, int32_t *n);
int catnn_hip_train_free(catnn_hip_trainer *t);
/* Upload the batch: `input` is bound to every graph input, `target` is the
 * MSE target of the last output. */
int catnn_hip_train_set_batch(catnn_hip_trainer *t, const catnn_tensor *input,
                              const catnn_tensor *target);
/* The batch of a trainer whose output is an LmHead: `input` as above and
 * one class id per output row (`n` = rows); a wrong count or an id ≥ vocab
 * → CATNN_ERR_SHAPE_MISMATCH, as cross_entropy refuses them
 * (adjoint.rs:126-136).  catnn_hip_train_set_batch on such a trainer, or
 * this call on another, → CATNN_ERR_INVALID_ARGUMENT. */
int catnn_hip_train_set_batch_classes(catnn_hip_trainer *t, const catnn_tensor *input,
                                      const uint32_t *ids, int64_t n);
/* forward, loss, backward, SGD on the resident batch; `loss` (or NULL:
 * no synchronisation) receives the step's MSE before the update. */
int catnn_hip_train_step(catnn_hip_trainer *t, float *loss);
/* Restores every parameter to the value it had at install (the host copy
 * kept by the trainer), e.g. to time many steps from the same start.  Not
 * part of reference_train; asynchronous on the device stream. */
int catnn_hip_train_reset(catnn_hip_trainer *t);
/* fp32 master weight / last gradient of param `port` of node `node_id`
 * (Attention's wq, wk, wv are read out of the packed projection). */
int catnn_hip_train_read_param(catnn_hip_trainer *t, uint32_t node_id, const char *port,
                               float *host, int64_t n);
int catnn_hip_train_read_grad(catnn_hip_trainer *t, uint32_t node_id, const char *port,
                              float *host, int64_t n);
/* Adam moment `which` (0: m, 1: v) of param `port` of node `node_id`;
 * CATNN_ERR_UNSUPPORTED on an SGD trainer. */
int catnn_hip_train_read_moment(catnn_hip_trainer *t, uint32_t node_id, const char *port,
                                int32_t which, float *host, int64_t n);
/* AdamState.t: the number of Adam steps taken since install or reset. */
int catnn_hip_train_adam_step(catnn_hip_trainer *t, uint64_t *step);
/* Forward value of node `node_id` from the last step. */
int catnn_hip_train_read_value(catnn_hip_trainer *t, uint32_t node_id, float *host, int64_t n);
/* Expert indices [T, top_k] chosen by MoE node `node_id` in the last step. */
int catnn_hip_train_read_routing(catnn_hip_trainer *t, uint32_t node_id, int32_t *idx, int64_t n);
int catnn_hip_train_arena(catnn_hip_trainer *t, catnn_arena_alloc *out, int32_t cap, int32_t *n,
                          uint64_t *reserved_bytes);

/* ------------------------------------------------------------- events */
/* Sheaf events (crates/catnn-rt/src/sheaf.rs:55-79) of the handler seams,
 * as DeviceHandler::run_kernel and note_kernel record them
 * (crates/catnn-rt/src/handler.rs:34-79): KernelStart / KernelEnd around
 * each node that catnn_hip_run_kernel or catnn_hip_run_node executes, and
 * "{name}.bwd" around each catnn_hip_run_adjoint (coord.rs:412).  Times are
 * the device's: each event is a hipEvent recorded on the device's stream
 * when the call enqueues its work, resolved to ns since catnn_hip_open when
 * the events are read (strictly increasing, as handler.rs:47).  The
 * KernelEnd checksum is FNV-1a over the output's f32 bits
 * (tensor.rs:279-288); for the adjoint span it is that of dy, as
 * coord.rs:412 passes it. */
enum catnn_event_kind {
    CATNN_EV_KERNEL_START = 0, CATNN_EV_KERNEL_END = 1,
    CATNN_EV_TRANSFER_START = 2, CATNN_EV_TRANSFER_END = 3
};
typedef struct catnn_event {
    uint64_t t_ns;
    char op[CATNN_ID_CAP];
    int32_t kind;
    uint64_t checksum;
} catnn_event;
/* Waits for the device work the recorded events stamp, then copies them. */
int catnn_hip_events(catnn_hip_device *dev, catnn_event *buf, int32_t cap, int32_t *n);
/* catnn_hip_run_node's KernelEnd checksum needs the output on the host: a
 * device-to-host copy and a stream synchronisation per node.  On by
 * default; with `enable` = 0 run_node records checksum 0 and does not
 * synchronise. */
int catnn_hip_trace_checksums(catnn_hip_device *dev, int32_t enable);
int catnn_hip_clear_events(catnn_hip_device *dev);

/* ------------------------------------------------ kernels on raw buffers */
/* These are the kernels the seams above dispatch to, exposed on device
 * pointers for tests and benchmarks.  All tensors are row-major f32 in
 * device memory; they run on the device's stream and return without
 * synchronising. */

/* y[m,n] = act(x[m,k]·w[k,n] + b[n]) + r[m,n]; b and r may be NULL.
 * Replaces cpu::linear (cpu.rs:135-184) followed by cpu::relu / cpu::gelu
 * (cpu.rs:14-29) and cpu::add (cpu.rs:80-98).  act: 0 none, 2 relu, 3 gelu
 * (the OpenOp discriminants). */
int catnn_hip_linear_f32(catnn_hip_device *dev, const float *x, const float *w,
                         const float *b, const float *r, float *y,
                         int64_t m, int64_t k, int64_t n, int32_t act);

/* C[m,n] (+)= Σ_k A[m,k]·B[n,k] on bf16 operands (raw bit patterns, both
 * k-contiguous) with fp32 accumulation: the kernel behind every GEMM of the
 * training step (the bf16 counterpart of linear_backward's products,
 * adjoint.rs:35-61), exposed for tests and benchmarks.  tile_cfg: -1
 * automatic, or a fixed tile configuration: 0, 2, 7, 9, 10, 11 or 12
 * (gemm_bf16.hip; 7, 9, 10, 11 and 12 stage k chunks straight into LDS and
 * take 16-byte aligned rows, other launches given them run as 2; 11 is the
 * 256 × 256 ping-pong tile, 12 the same with the last round of tiles split
 * along k over every CU — the stream-K scratch is the device's, allocated
 * on first use). */
int catnn_hip_gemm_bf16_nt(catnn_hip_device *dev, const uint16_t *a, int64_t lda, const uint16_t *b,
                           int64_t ldb, float *c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                           int32_t accumulate, int32_t tile_cfg);

/* apply_update (crates/catnn-compile/src/pipeline.rs:455-472, the seam
 * coord.rs:481 calls) on n values in device memory, in place.
 * catnn_hip_sgd_f32 replaces Sgd::put (lens/optim.rs:32-42): p −= lr·g.
 * catnn_hip_adam_f32 replaces Adam::put (optim.rs:95-118) with Adam's
 * default β₁, β₂, eps: `t` is AdamState.t before the step (0 for a fresh
 * state), the step taken is t + 1, and m, v are updated in place.  Both are
 * bit-identical to the reference for the same inputs (every operation
 * rounded separately, in the reference's order). */
int catnn_hip_sgd_f32(catnn_hip_device *dev, float *p, const float *g, int64_t n, float lr);
int catnn_hip_adam_f32(catnn_hip_device *dev, float *p, const float *g, float *m, float *v,
                       int64_t n, uint64_t t, float lr);

/* Replaces cpu::relu / cpu::gelu (cpu.rs:14-29) as standalone passes. */
int catnn_hip_act_f32(catnn_hip_device *dev, const float *x, float *y,
                      int64_t n, int32_t act);
/* Replaces cpu::add (cpu.rs:80-98): same-length add when nb == na, bias
 * broadcast over the last dim (length nb) otherwise. */
int catnn_hip_add_f32(catnn_hip_device *dev, const float *a, const float *b,
                      float *y, int64_t na, int64_t nb);
/* Replaces cpu::mul (cpu.rs:100-109). */
int catnn_hip_mul_f32(catnn_hip_device *dev, const float *a, const float *b,
                      float *y, int64_t n);
/* Replaces cpu::layer_norm (cpu.rs:54-78). */
int catnn_hip_layer_norm_f32(catnn_hip_device *dev, const float *x,
                             const float *gamma, const float *beta, float *y,
                             int64_t rows, int64_t cols, float eps);
/* Replaces cpu::softmax_last (cpu.rs:31-52). */
int catnn_hip_softmax_f32(catnn_hip_device *dev, const float *x, float *y,
                          int64_t rows, int64_t cols);
/* The score/softmax/PV core of cpu::attention (cpu.rs:252-295) on
 * projected q, k, v [B,S,D] (head h at columns h·dh..(h+1)·dh):
 * ctx = softmax(q·kᵀ/√dh)·v per (b,h), causal when `causal` != 0
 * (masking as moe.rs:105-121). */
int catnn_hip_attention_core_f32(catnn_hip_device *dev, const float *q,
                                 const float *k, const float *v, float *ctx,
                                 int64_t batch, int64_t seq, int64_t d_model,
                                 int64_t n_heads, int64_t d_head, int32_t causal);

/* MoE router, replaces moe::route (crates/catnn-compile/src/kernel/moe.rs:177-195)
 * with lens::moe::topk_softmax (crates/catnn-core/src/lens/moe.rs:175-187):
 * logits[t,e] = Σ_p x[t,p]·gate[p,e] in sequential p order without fused
 * multiply-add (bit-equal to cpu::linear_seq, cpu.rs:115-126); idx[t,k]
 * = k-th expert by descending logit, ties to the lower id; w[t,k] =
 * exp(l−max)/max(Σ,1e-30).  Any output pointer may be NULL. */
int catnn_hip_moe_route_f32(catnn_hip_device *dev, const float *x, const float *gate,
                            int64_t tokens, int64_t hidden, int64_t n_experts,
                            int64_t top_k, int32_t *idx, float *w, float *logits);

/* Token permutation (no reference counterpart: the reference loops over
 * tokens, moe.rs:207-221).  Stable counting sort of the flattened slots
 * s = t·top_k + k by expert id: counts[e]; offsets[e] = Σ_{e'<e} counts[e']
 * (length n_experts+1); slot_of_pos[offsets[e] + r] = the r-th slot, in
 * ascending s, routed to e; pos_of_slot is its inverse. */
int catnn_hip_moe_permute(catnn_hip_device *dev, const int32_t *idx,
                          int64_t tokens, int64_t top_k, int64_t n_experts,
                          int32_t *counts, int32_t *offsets,
                          int32_t *slot_of_pos, int32_t *pos_of_slot);

/* Whole MoE layer, replaces moe::moe (moe.rs:197-223):
 * out[t] = Σ_{k ascending} w[t,k]·swiglu_{idx[t,k]}(x_t) with
 * swiglu(x) = (silu(x·w1) ⊙ (x·w3))·w2 (moe.rs:159-174).  w1s, w3s, w2s
 * are arrays of n_experts device pointers ([hidden,inter], [hidden,inter],
 * [inter,hidden]).  Workspace is allocated on first use and kept per device.
 * idx/w/counts may be NULL; if given they receive the routing. */
int catnn_hip_moe_f32(catnn_hip_device *dev, const float *x, const float *gate,
                      const float *const *w1s, const float *const *w3s,
                      const float *const *w2s, int64_t tokens, int64_t hidden,
                      int64_t intermediate, int64_t n_experts, int64_t top_k,
                      float *out, int32_t *idx, float *w, int32_t *counts);

/* Allocation-free variant of catnn_hip_moe_f32 (same arguments, same
 * results bit for bit).  No counterpart in the reference: it is for callers
 * that cannot allocate device memory — code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  It calls no hipMalloc,
 * hipFree or allocating library routine; its workspace (routing, the
 * permutation and the per-slot expert activations, the layout of
 * catnn_hip_moe_f32) lives in a fixed device array of
 * CATNN_MOE_NOALLOC_SCRATCH_BYTES that each GPU holds from library load to
 * process exit.  A call needing more (about tokens·top_k·4·(intermediate +
 * hidden + 4) bytes plus a few KiB; e.g. up to ~3,600 tokens at hidden 1024,
 * intermediate 3584, top-2) fails with CATNN_ERR_SHAPE_MISMATCH before
 * launching anything.  Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (two devices handles or two threads) race; calls
 * on one device handle are ordered by its stream. */
#define CATNN_MOE_NOALLOC_SCRATCH_BYTES (128ull << 20)
int catnn_hip_moe_f32_noalloc(catnn_hip_device *dev, const float *x, const float *gate,
                              const float *const *w1s, const float *const *w3s,
                              const float *const *w2s, int64_t tokens, int64_t hidden,
                              int64_t intermediate, int64_t n_experts, int64_t top_k, float *out,
                              int32_t *idx, float *w, int32_t *counts);

#ifdef __cplusplus
}
#endif

#endif /* CATNN_HIP_H */
