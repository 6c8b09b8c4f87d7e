"""The Mixtral decoder ops on the GPU — RmsNorm, Embedding, GqaAttention
(RoPE, grouped K/V heads, sliding window), SwiGlu, LmHead, Router and Mix —
node by node through the run_kernel seam and as whole Mixtral graphs,
against the oracle's restatement of moe.rs / deepseek.rs (fp32, rel L2 1e-4;
the embedding gather is bit-exact)."""
import numpy as np
import pytest

import oracle
from catnn_amd import (CatError, CGraph, DeviceHandler, IrGraph, IrNode, OpenOp, Program, Tensor,
                       TensorType, configs)
from catnn_amd.configs import MixtralShape
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _t(a):
    return Tensor.from_numpy(np.ascontiguousarray(a, np.float32))


def _run(device, node, ins):
    got = DeviceHandler(device).run_kernel(node, [_t(a) for a in ins]).numpy()
    want = oracle.eval_node(node, [np.asarray(a, np.float32) for a in ins])
    err = rel_l2(got, want)
    print(f"{node.name}: rel_l2 {err:.2e}", flush=True)
    assert got.shape == want.shape
    return got, want, err


@pytest.mark.parametrize("rows,cols", [(3, 32), (5, 33), (17, 4096), (4, 4100), (2, 8192), (1, 1)])
def test_rms_norm(device, rows, cols):
    r = np.random.default_rng(cols)
    x = r.standard_normal((rows, cols)) * 3
    node = IrNode(1, "rms", OpenOp.rms_norm(10), TensorType.f32([rows, cols]),
                  {"w": _t(1 + 0.1 * r.standard_normal(cols))})
    assert _run(device, node, [x])[2] < TOL


def test_embedding_is_an_exact_gather(device):
    r = np.random.default_rng(1)
    table = r.standard_normal((50, 12)).astype(np.float32)
    ids = np.array([[0, 49, 1.5, 2.5], [-3, np.nan, 48.4999, 7]], np.float32)
    node = IrNode(1, "emb", OpenOp.embedding(50, 12), TensorType.f32([2, 4, 12]), {"w": _t(table)})
    got, want, _ = _run(device, node, [ids])
    assert got.shape == (2, 4, 12) and np.array_equal(got, want)
    # A rank-1 id list gives [n, hidden]; 16-byte rows take the vector path.
    node = IrNode(1, "emb", OpenOp.embedding(50, 16), TensorType.f32([300, 16]),
                  {"w": _t(r.standard_normal((50, 16)))})
    got, want, _ = _run(device, node, [r.integers(0, 50, 300)])
    assert got.shape == (300, 16) and np.array_equal(got, want)


@pytest.mark.parametrize("n", [1, 7, 64])
def test_embedding_1024_wide_rows(device, n):
    # hidden 1024 takes the two-tokens-per-wavefront kernel; odd counts
    # leave the last wavefront one token.
    r = np.random.default_rng(n)
    table = r.standard_normal((300, 1024)).astype(np.float32)
    ids = r.integers(0, 300, n).astype(np.float32)
    for j, v in enumerate([-3.0, np.nan, 2.5, 298.5, 0.49][: (n + 2) // 3]):
        ids[3 * j] = v  # negative and NaN → 0, halves round away from zero
    node = IrNode(1, "emb", OpenOp.embedding(300, 1024), TensorType.f32([n, 1024]), {"w": _t(table)})
    got, want, _ = _run(device, node, [ids])
    assert got.shape == (n, 1024) and np.array_equal(got, want)


@pytest.mark.parametrize("bad_at", [0, 1, 2])
def test_embedding_1024_wide_rows_reject_an_id_past_the_vocabulary(device, bad_at):
    table = np.zeros((10, 1024), np.float32)
    node = IrNode(1, "emb", OpenOp.embedding(10, 1024), TensorType.f32([3, 1024]), {"w": _t(table)})
    ids = np.array([1.0, 2.0, 3.0], np.float32)
    ids[bad_at] = 10.0
    with pytest.raises(CatError) as e:
        DeviceHandler(device).run_kernel(node, [_t(ids)])
    assert e.value.kind == "ShapeMismatch"
    assert DeviceHandler(device).run_kernel(node, [_t([9.0])]).numpy().shape == (1, 1024)


def test_embedding_rejects_an_id_past_the_vocabulary(device):
    node = IrNode(1, "emb", OpenOp.embedding(10, 4), TensorType.f32([3, 4]),
                  {"w": _t(np.zeros((10, 4)))})
    with pytest.raises(CatError) as e:
        DeviceHandler(device).run_kernel(node, [_t([1.0, 9.5, 2.0])])  # 9.5 rounds to 10
    assert e.value.kind == "ShapeMismatch"
    # the device stays usable
    assert DeviceHandler(device).run_kernel(node, [_t([9.4])]).numpy().shape == (1, 4)


def _gqa_node(r, d, nh, nkv, hd, window, theta=10000, scale=1.0):
    kv = nkv * hd
    p = {"wq": _t(r.standard_normal((d, nh * hd)) * scale / np.sqrt(d)),
         "wk": _t(r.standard_normal((d, kv)) * scale / np.sqrt(d)),
         "wv": _t(r.standard_normal((d, kv)) / np.sqrt(d)),
         "wo": _t(r.standard_normal((nh * hd, d)) / np.sqrt(nh * hd))}
    return IrNode(1, f"gqa{nh}x{nkv}x{hd}w{window}", OpenOp.gqa_attention(nh, nkv, hd, d, window, theta),
                  TensorType.f32([1, 1, d]), p)


@pytest.mark.parametrize("B,S,nh,nkv,hd,window", [
    (2, 9, 4, 2, 8, None),       # Mixtral-tiny shape, generic core
    (2, 9, 4, 1, 8, 3),          # one K/V head, window 3
    (1, 7, 2, 2, 6, 1),          # window 1: each query sees itself
    (2, 200, 8, 2, 64, None),    # MFMA core, 4 query heads per K/V head
    (1, 300, 4, 4, 64, 100),     # MFMA core with a window across tile edges
    (1, 130, 4, 2, 64, 128),     # window one tile wide
    (1, 37, 2, 1, 10, 5),        # head_dim not a multiple of 4
    (2, 150, 4, 2, 32, None),    # MFMA core, head_dim 32
    (1, 200, 4, 1, 128, 70),     # MFMA core, head_dim 128, window
])
def test_gqa_attention(device, B, S, nh, nkv, hd, window):
    r = np.random.default_rng(S * 31 + hd)
    d = nh * hd
    node = _gqa_node(r, d, nh, nkv, hd, window, scale=2.0)
    x = r.standard_normal((B, S, d))
    assert _run(device, node, [x])[2] < TOL


def test_gqa_long_positions_rotate_like_the_f64_table(device):
    # Positions up to 2047 at θ = 1e6: the RoPE angles come from the f64 table.
    r = np.random.default_rng(5)
    node = _gqa_node(r, 128, 2, 1, 64, 512, theta=1000000)
    assert _run(device, node, [r.standard_normal((1, 2048, 128))])[2] < TOL


@pytest.mark.parametrize("T,H,I", [(8, 32, 64), (300, 96, 200), (1024, 256, 704), (37, 100, 52)])
def test_swiglu(device, T, H, I):
    r = np.random.default_rng(T)
    node = IrNode(1, "swiglu", OpenOp.swiglu(H, I), TensorType.f32([T, H]),
                  {"w1": _t(r.standard_normal((H, I)) / np.sqrt(H)),
                   "w3": _t(r.standard_normal((H, I)) / np.sqrt(H)),
                   "w2": _t(r.standard_normal((I, H)) / np.sqrt(I))})
    assert _run(device, node, [r.standard_normal((T, H))])[2] < TOL


@pytest.mark.parametrize("B,S,H,V", [(2, 4, 32, 32), (1, 33, 40, 1001), (2, 128, 256, 4096)])
def test_lm_head(device, B, S, H, V):
    r = np.random.default_rng(V)
    node = IrNode(1, "lm_head", OpenOp.lm_head(H, V), TensorType.f32([B, S, V]),
                  {"w": _t(r.standard_normal((V, H)) / np.sqrt(H))})
    got, _, err = _run(device, node, [r.standard_normal((B, S, H))])
    assert got.shape == (B, S, V) and err < TOL


def test_router_and_mix(device):
    r = np.random.default_rng(9)
    a, b = r.standard_normal((3, 5, 7)), r.standard_normal((3, 5, 7))
    ty = TensorType.f32([3, 5, 7])
    got, want, _ = _run(device, IrNode(1, "router", OpenOp.router(4, 2), ty), [a])
    assert np.array_equal(got, want)
    assert _run(device, IrNode(1, "mix0", OpenOp.mix(), ty), [a, b])[2] < 1e-6
    node = IrNode(1, "mix", OpenOp.mix(), ty, {"gate": _t([1.25])})
    assert _run(device, node, [a, b])[2] < 1e-6
    with pytest.raises(CatError) as e:
        DeviceHandler(device).run_kernel(node, [_t(a)])
    assert e.value.kind == "Wiring"
    with pytest.raises(CatError) as e:
        DeviceHandler(device).run_kernel(node, [_t(a), _t(b[:2])])
    assert e.value.kind == "ShapeMismatch"


def test_decoder_shape_errors(device):
    h = DeviceHandler(device)
    r = np.random.default_rng(2)
    with pytest.raises(CatError) as e:  # n_heads not a multiple of n_kv_heads
        h.run_kernel(_gqa_node(r, 24, 3, 2, 8, None), [_t(np.zeros((1, 4, 24)))])
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(CatError) as e:  # gqa needs [B,S,H]
        h.run_kernel(_gqa_node(r, 16, 2, 2, 8, None), [_t(np.zeros((4, 16)))])
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(CatError) as e:  # rmsnorm weight length
        h.run_kernel(IrNode(1, "rms", OpenOp.rms_norm(1), TensorType.f32([2, 8]), {"w": _t(np.ones(7))}),
                     [_t(np.zeros((2, 8)))])
    assert e.value.kind == "ShapeMismatch"


def _check_graph(device, g, x, tol=TOL):
    prog = Program(device, g)
    got = prog.forward(x).numpy()
    want = oracle.eval_graph(g, x.numpy())
    err = rel_l2(got, want)
    print(f"{g.name}: rel_l2 {err:.2e} max_abs {np.max(np.abs(got - want)):.2e}", flush=True)
    assert got.shape == want.shape and err < tol
    prog.free()
    return got


def test_mixtral_tiny_graph(device):
    # MixtralConfig::tiny on batch 2, seq 4 (the reference's moe.rs:477-485 case)
    w = configs.mixtral(2, 4)
    got = _check_graph(device, w.graph, w.x)
    assert got.shape == (2, 4, 32)
    # the same graph through the serde-JSON ingest
    prog = Program(device, CGraph.from_ir(w.graph))
    assert np.array_equal(prog.forward(w.x).numpy(), got)
    prog.free()


def test_mixtral_graph_on_the_mfma_core(device):
    shape = MixtralShape(vocab=512, hidden=256, inter=512, layers=2, heads=4, kv_heads=2, experts=4,
                         top_k=2, sliding_window=96)
    w = configs.mixtral(2, 160, shape)
    _check_graph(device, w.graph, w.x)


def test_residual_folds_into_gqa_and_swiglu(device):
    # x → rms → gqa → (+x) → rms → swiglu → (+res1): the adds fold into the
    # output-projection GEMMs.
    r = np.random.default_rng(12)
    d, S = 64, 40
    ty = TensorType.f32([2, S, d])
    g = IrGraph("pre_norm_block")
    g.add_node(IrNode(0, "in", OpenOp.identity(), ty))
    g.add_node(IrNode(1, "rms1", OpenOp.rms_norm(10), ty, {"w": _t(np.ones(d))}))
    node = _gqa_node(r, d, 4, 2, 16, 16)
    node.id, node.name, node.output_ty = 2, "gqa", ty
    g.add_node(node)
    g.add_node(IrNode(3, "res1", OpenOp.residual_add(), ty))
    g.add_node(IrNode(4, "rms2", OpenOp.rms_norm(10), ty, {"w": _t(np.ones(d))}))
    g.add_node(IrNode(5, "ffn", OpenOp.swiglu(d, 128), ty,
                      {"w1": _t(r.standard_normal((d, 128)) / 8), "w3": _t(r.standard_normal((d, 128)) / 8),
                       "w2": _t(r.standard_normal((128, d)) / 11)}))
    g.add_node(IrNode(6, "res2", OpenOp.residual_add(), ty))
    for s_, d_ in [(0, 1), (1, 2), (0, 3), (2, 3), (3, 4), (4, 5), (3, 6), (5, 6)]:
        g.add_edge(s_, d_)
    g.inputs.append(0)
    g.outputs.append(6)
    _check_graph(device, g, _t(r.standard_normal((2, S, d))))


def _mixtral_reference_graph(cfg, w, B, S):
    """moe::forward (moe.rs:288-322) as an IrGraph: embed → per layer
    rms_attn → gqa → ResidualAdd(x, ·) → rms_moe → moe → ResidualAdd(x, ·) →
    final_norm → lm_head, holding MixtralWeights::seeded's tensors."""
    h, hd = cfg.hidden, cfg.head_dim()
    eps_e6 = int(np.float32(cfg.eps) * np.float32(1e6))
    ty = TensorType.f32([B, S, h])
    g = IrGraph("mixtral_tiny_reference")
    g.add_node(IrNode(0, "tokens", OpenOp.identity(), TensorType.f32([B, S])))
    g.add_node(IrNode(1, "embed", OpenOp.embedding(cfg.vocab, h), ty, {"w": _t(w["embed"])}))
    g.add_edge(0, 1)
    x, nid = 1, 2
    for li, L in enumerate(w["layers"]):
        g.add_node(IrNode(nid, f"L{li}.rms_attn", OpenOp.rms_norm(eps_e6), ty, {"w": _t(L["rms_attn"])}))
        g.add_node(IrNode(nid + 1, f"L{li}.gqa",
                          OpenOp.gqa_attention(cfg.heads, cfg.kv_heads, hd, h, cfg.sliding_window,
                                               int(cfg.rope_theta)), ty,
                          {p: _t(L[p]) for p in ("wq", "wk", "wv", "wo")}))
        g.add_node(IrNode(nid + 2, f"L{li}.res_attn", OpenOp.residual_add(), ty))
        moe_p = {"gate": _t(L["gate"])}
        for e, (w1, w3, w2) in enumerate(L["experts"]):
            moe_p.update({f"e{e}.w1": _t(w1), f"e{e}.w3": _t(w3), f"e{e}.w2": _t(w2)})
        g.add_node(IrNode(nid + 3, f"L{li}.rms_moe", OpenOp.rms_norm(eps_e6), ty, {"w": _t(L["rms_moe"])}))
        g.add_node(IrNode(nid + 4, f"L{li}.moe", OpenOp.moe(cfg.experts, cfg.top_k, h, cfg.inter), ty, moe_p))
        g.add_node(IrNode(nid + 5, f"L{li}.res_moe", OpenOp.residual_add(), ty))
        for a, b in ((x, nid), (nid, nid + 1), (x, nid + 2), (nid + 1, nid + 2), (nid + 2, nid + 3),
                     (nid + 3, nid + 4), (nid + 2, nid + 5), (nid + 4, nid + 5)):
            g.add_edge(a, b)
        x, nid = nid + 5, nid + 6
    g.add_node(IrNode(nid, "final_norm", OpenOp.rms_norm(eps_e6), ty, {"w": _t(w["final_norm"])}))
    g.add_node(IrNode(nid + 1, "lm_head", OpenOp.lm_head(h, cfg.vocab), TensorType.f32([B, S, cfg.vocab]),
                      {"w": _t(w["lm_head"])}))
    g.add_edge(x, nid)
    g.add_edge(nid, nid + 1)
    g.inputs, g.outputs = [0], [nid + 1]
    return g


@pytest.mark.parametrize("seed", [7, 123])
def test_mixtral_tiny_known_answer(device, seed):
    # The reference's Mixtral-tiny test (moe.rs:476-485): MixtralConfig::tiny,
    # MixtralWeights::seeded(seed), tokens 1..8 as batch 2 × seq 4.  The same
    # weights and tokens run as an IrGraph with ResidualAdd nodes on the GPU
    # and are held to the reference's own bound against moe::forward (max |Δ|
    # < 2e-4) and to the fp32 bar (rel L2 1e-4).
    cfg = oracle.MixtralConfig()
    w = oracle.mixtral_weights_seeded(cfg, seed)
    toks = [1, 2, 3, 4, 5, 6, 7, 8]
    want = oracle.mixtral_forward(cfg, w, toks, 2, 4)
    g = _mixtral_reference_graph(cfg, w, 2, 4)
    prog = Program(device, g)
    got = prog.forward(Tensor(TensorType.f32([2, 4]), np.asarray(toks, np.float32))).numpy()
    prog.free()
    err, mx = rel_l2(got, want), float(np.abs(got - want).max())
    print(f"mixtral-tiny seed {seed}: rel_l2 {err:.2e}, max |Δ| {mx:.2e}", flush=True)
    assert got.shape == (2, 4, cfg.vocab)
    assert mx < 2e-4 and err < TOL
    assert rel_l2(got, oracle.eval_graph(g, np.asarray(toks, np.float32).reshape(2, 4))) < TOL


def test_program_reports_an_out_of_range_token_after_the_forward(device):
    # A program checks its embeddings' flag once, when it next synchronises
    # (no mid-graph stall); the next good forward runs clean.
    w = configs.mixtral(batch=2, seq=4)
    prog = Program(device, w.graph)
    good = prog.forward(w.x).numpy()
    bad = w.x.numpy().copy()
    bad[1, 2] = 32.0  # = vocab
    with pytest.raises(CatError) as e:
        prog.forward(Tensor(w.x.ty, bad.reshape(-1)))
    assert e.value.kind == "ShapeMismatch"
    assert np.array_equal(prog.forward(w.x).numpy(), good)
    # the resident path: ids already in the input buffer, reported by check()
    import ctypes
    from catnn_amd._lib import check, lib
    io = prog.io()
    check(lib.catnn_hip_h2d(device.handle, ctypes.c_void_p(io.in_ptr), bad.ctypes.data_as(ctypes.c_void_p),
                            bad.nbytes))
    prog.forward_resident()
    with pytest.raises(CatError) as e:
        prog.check()
    assert e.value.kind == "ShapeMismatch"
    prog.check()  # reported once
    prog.free()
