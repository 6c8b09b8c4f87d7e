"""Pins the CPU oracle (oracle/catnn_oracle.cpp) before anything is checked
against it.  Each check is independent of the oracle's own formula: the
reference's known-answer tests, float64 library routines (torch, scipy),
brute force in Python integers or float32 numpy, and invariants — chosen so
that a dropped term, a wrong sign, a transposed operand or a wrong index
fails one of them.
"""
import math

import numpy as np
import pytest
import scipy.special
import torch

import oracle
from conftest import rel_l2

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- tensor.rs

def _lcg_bruteforce(n, seed):
    # Tensor::lcg with Python integers: state = max(seed,1); state = state*a + 1
    # mod 2^64; (state >> 33) as u32 as f32 / u32::MAX as f32 * 2 - 1.
    state = max(seed, 1)
    out = []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1) % 2**64
        unit = np.float32(state >> 33) / np.float32(2**32 - 1)
        out.append(np.float32(unit * np.float32(2.0) - np.float32(1.0)))
    return np.array(out, np.float32)


@pytest.mark.parametrize("seed", [0, 1, 7, 42, 2**63 + 5])
def test_lcg_matches_integer_bruteforce(seed):
    got = oracle.lcg(257, seed)
    assert np.array_equal(got, _lcg_bruteforce(257, seed))


def test_lcg_is_stable_and_nonpositive():
    # tensor.rs:310-315 (stable), and finding F4: values lie in [-1, 0).
    a, b = oracle.lcg(4, 7), oracle.lcg(4, 7)
    assert np.array_equal(a, b)
    big = oracle.lcg(100_000, 99)
    assert big.min() >= -1.0 and big.max() < 0.0


def test_checksum_is_fnv1a_over_f32_bits():
    x = RNG.standard_normal(37).astype(np.float32)
    h = 0xCBF29CE484222325
    for bits in x.view(np.uint32):
        h ^= int(bits)
        h = (h * 0x100000001B3) % 2**64
    assert oracle.checksum(x) == h


# ------------------------------------------------------------------ cpu.rs

def test_relu_known_answer():
    # cpu.rs:318-322
    assert oracle.relu(np.array([-1.0, 0.0, 2.0, -0.5])).tolist() == [0.0, 0.0, 2.0, 0.0]


def test_gelu_matches_torch_tanh_gelu_float64():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    want = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    got = oracle.gelu(x)
    assert np.max(np.abs(got - want)) < 2e-6
    # and it is the tanh form, not the erf form (they differ by ~1e-3 near |x|≈2)
    erf = torch.nn.functional.gelu(torch.from_numpy(x).double()).numpy()
    assert np.max(np.abs(got - erf)) > 1e-4


def test_softmax_matches_scipy_and_rows_sum_to_one():
    x = (RNG.standard_normal((33, 129)) * 5).astype(np.float32)
    got = oracle.softmax_last(x)
    want = scipy.special.softmax(x.astype(np.float64), axis=-1)
    assert np.max(np.abs(got - want)) < 1e-6
    assert np.allclose(got.sum(-1), 1.0, atol=1e-5)
    assert np.array_equal(oracle.softmax_last(x, reference=True), got)


def test_softmax_handles_large_logits():
    x = np.array([[1000.0, 1000.0, -1000.0]], np.float32)
    got = oracle.softmax_last(x)
    assert np.allclose(got, [[0.5, 0.5, 0.0]])


def test_layer_norm_matches_torch_float64():
    x = (RNG.standard_normal((17, 96)) * 3 + 1).astype(np.float32)
    g = RNG.standard_normal(96).astype(np.float32)
    b = RNG.standard_normal(96).astype(np.float32)
    got = oracle.layer_norm(x, g, b, 1e-6)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (96,),
                                          torch.from_numpy(g).double(),
                                          torch.from_numpy(b).double(), eps=1e-6).numpy()
    assert np.max(np.abs(got - want)) < 2e-5
    assert np.array_equal(oracle.layer_norm(x, g, b, 1e-6, reference=True), got)


def test_layer_norm_constant_row_gives_beta():
    x = np.full((2, 8), 3.25, np.float32)
    b = np.arange(8, dtype=np.float32)
    assert np.array_equal(oracle.layer_norm(x, np.ones(8, np.float32), b, 1e-6),
                          np.tile(b, (2, 1)))


def test_add_same_length_and_bias_broadcast():
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    assert oracle.add(a, np.ones((2, 3), np.float32)).tolist() == [[1, 2, 3], [4, 5, 6]]
    assert oracle.add(a, np.array([10, 20, 30], np.float32)).tolist() == [[10, 21, 32],
                                                                           [13, 24, 35]]
    with pytest.raises(ValueError):
        oracle.add(a, np.ones(4, np.float32))


def test_linear_identity_known_answer():
    # cpu.rs:324-329
    y = oracle.linear(np.array([[1.0, 2.0]]), np.eye(2, dtype=np.float32))
    assert y.tolist() == [[1.0, 2.0]]


def test_linear_seq_is_bit_exact_sequential_float32():
    x = RNG.standard_normal((7, 45)).astype(np.float32)
    w = RNG.standard_normal((45, 13)).astype(np.float32)
    s = np.zeros((7, 13), np.float32)
    for p in range(45):  # float32 numpy: separate multiply and add, p ascending
        s = s + x[:, p:p + 1] * w[p:p + 1, :]
    assert np.array_equal(oracle.linear_seq(x, w), s)
    b = RNG.standard_normal(13).astype(np.float32)
    assert np.array_equal(oracle.linear_seq(x, w, b), s + b)


@pytest.mark.parametrize("m,k,n", [(4, 16, 8), (9, 37, 5), (3, 8, 1), (1, 1000, 33)])
def test_linear_variants_match_float64(m, k, n):
    x = RNG.standard_normal((m, k)).astype(np.float32)
    w = RNG.standard_normal((k, n)).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64) + b
    for fn in (oracle.linear, oracle.linear_seq, oracle.ref_linear):
        assert rel_l2(fn(x, w, b), want) < 1e-6
    # a transposed weight must not pass
    if k == n:
        assert rel_l2(oracle.linear(x, w.T.copy(), b), want) > 1e-2


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 8, 16, 4), (1, 33, 64, 2)])
def test_attention_matches_torch_sdpa_float64(causal, shape):
    B, S, D, H = shape
    dh = D // H
    x = RNG.standard_normal((B, S, D)).astype(np.float32)
    ws = [(RNG.standard_normal((D, D)) / math.sqrt(D)).astype(np.float32) for _ in range(4)]
    got = oracle.attention(x, *ws, H, dh, causal=causal)
    X = torch.from_numpy(x).double()
    q, k, v = [(X @ torch.from_numpy(w).double()).view(B, S, H, dh).transpose(1, 2) for w in ws[:3]]
    ctx = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)
    want = (ctx.transpose(1, 2).reshape(B, S, D) @ torch.from_numpy(ws[3]).double()).numpy()
    assert rel_l2(got, want) < 1e-5
    if causal:  # the first query sees only itself: its context is v_0
        noncausal = oracle.attention(x, *ws, H, dh, causal=False)
        assert rel_l2(got, noncausal) > 1e-3


# ------------------------------------------------------------------ moe.rs

def test_topk_softmax_known_answer():
    # lens/moe.rs:208-213
    idx, w = oracle.topk_softmax(np.array([1.0, 3.0, 0.0, 2.0]), 2)
    assert idx.tolist() == [1, 3]
    e = math.exp(-1.0)
    assert np.allclose(w, [1 / (1 + e), e / (1 + e)], atol=1e-7)
    assert abs(w.sum() - 1.0) < 1e-6


def test_topk_ties_go_to_the_lower_expert():
    idx, w = oracle.topk_softmax(np.array([0.5, 2.0, 2.0, 2.0, -1.0]), 3)
    assert idx.tolist() == [1, 2, 3]
    assert np.allclose(w, 1 / 3, atol=1e-7)


def test_topk_matches_stable_argsort_bruteforce():
    for _ in range(200):
        E = int(RNG.integers(2, 17))
        k = int(RNG.integers(1, E + 1))
        logits = RNG.integers(-3, 4, E).astype(np.float32)  # many ties
        idx, w = oracle.topk_softmax(logits, k)
        want = np.argsort(-logits.astype(np.float64), kind="stable")[:k]
        assert idx.tolist() == want.tolist()
        ex = np.exp(logits[want].astype(np.float64) - logits[want].max())
        assert np.allclose(w, ex / ex.sum(), atol=1e-6)


def test_route_bruteforce():
    T, H, E, k = 50, 24, 6, 2
    x = RNG.standard_normal((T, H)).astype(np.float32)
    gate = RNG.standard_normal((H, E)).astype(np.float32)
    idx, w, logits = oracle.route(x, gate, k)
    assert np.array_equal(logits, oracle.linear_seq(x, gate))
    for t in range(T):
        want = np.argsort(-logits[t].astype(np.float64), kind="stable")[:k]
        assert idx[t].tolist() == want.tolist()
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


def _swiglu64(x, w1, w3, w2):
    x, w1, w3, w2 = (np.asarray(a, np.float64) for a in (x, w1, w3, w2))
    a, c = x @ w1, x @ w3
    return (a / (1 + np.exp(-a)) * c) @ w2


def test_swiglu_matches_float64_and_reference_loop():
    T, H, I = 5, 16, 40
    x = RNG.standard_normal((T, H)).astype(np.float32)
    w1, w3 = (RNG.standard_normal((H, I)).astype(np.float32) * 0.3 for _ in range(2))
    w2 = RNG.standard_normal((I, H)).astype(np.float32) * 0.3
    got = oracle.swiglu(x, w1, w3, w2)
    assert rel_l2(got, _swiglu64(x, w1, w3, w2)) < 1e-6
    # moe::reference::swiglu accumulates in the same order: identical bits
    assert np.array_equal(oracle.swiglu(x, w1, w3, w2, reference=True), got)
    # swapping w1 and w3 (gate and up) changes the result
    assert rel_l2(oracle.swiglu(x, w3, w1, w2), got) > 1e-2


def _moe_inputs(T=40, H=16, I=24, E=5, seed=0):
    r = np.random.default_rng(seed)
    x = r.standard_normal((T, H)).astype(np.float32)
    gate = r.standard_normal((H, E)).astype(np.float32)
    w1 = (r.standard_normal((E, H, I)) * 0.3).astype(np.float32)
    w3 = (r.standard_normal((E, H, I)) * 0.3).astype(np.float32)
    w2 = (r.standard_normal((E, I, H)) * 0.3).astype(np.float32)
    return x, gate, w1, w3, w2


def test_moe_matches_dense_float64_bruteforce():
    x, gate, w1, w3, w2 = _moe_inputs()
    k = 2
    got = oracle.moe(x, gate, w1, w3, w2, k)
    idx, w, _ = oracle.route(x, gate, k)
    want = np.zeros(x.shape)
    for t in range(x.shape[0]):
        for j in range(k):
            e = idx[t, j]
            want[t] += w[t, j] * _swiglu64(x[t:t + 1], w1[e], w3[e], w2[e])[0]
    assert rel_l2(got, want) < 1e-6
    assert np.array_equal(oracle.moe(x, gate, w1, w3, w2, k, reference=True), got)
    sub = oracle.moe(x, gate, w1, w3, w2, k, tokens=[3, 17])
    assert np.array_equal(sub[[3, 17]], got[[3, 17]])
    assert not sub[0].any()


def test_moe_permute_is_a_stable_bijection():
    T, k, E = 300, 2, 7
    idx = RNG.integers(0, E, (T, k)).astype(np.int32)
    counts, offsets, sop, pos = oracle.moe_permute(idx, E)
    flat = idx.reshape(-1)
    assert counts.tolist() == np.bincount(flat, minlength=E).tolist()
    assert offsets.tolist() == [0] + np.cumsum(counts).tolist()
    assert sorted(sop.tolist()) == list(range(T * k))
    assert np.array_equal(sop[pos], np.arange(T * k))
    assert np.array_equal(flat[sop], np.sort(flat, kind="stable"))
    # stable: the slots of one expert appear in ascending order
    assert np.array_equal(sop, np.argsort(flat, kind="stable"))
    with pytest.raises(ValueError):
        oracle.moe_permute(np.array([[0, E]], np.int32), E)


# ------------------------------------------------------------- schedule.rs

def test_place_arena_reference_aliasing_case():
    # schedule.rs:479-489: disjoint lifetimes share offset 0 even with cap 8
    off, _ = oracle.place_arena([(8, 0, 1), (8, 2, 3)], 8)
    assert off.tolist() == [0, 0]


def test_place_arena_overflow_and_conflict_detection():
    with pytest.raises(OverflowError):
        oracle.place_arena([(8, 0, 2), (8, 1, 3)], 8)
    # schedule.rs:492-498
    assert oracle.arena_conflict([8, 8], [0, 4], [0, 1], [2, 3])
    assert not oracle.arena_conflict([8, 8], [0, 8], [0, 1], [2, 3])


def test_place_arena_random_plans_are_conflict_free_first_fit():
    for trial in range(100):
        n = int(RNG.integers(1, 25))
        reqs = []
        for _ in range(n):
            a = int(RNG.integers(0, 10))
            reqs.append((int(RNG.integers(1, 100)), a, a + int(RNG.integers(0, 5))))
        off, order = oracle.place_arena(reqs, 10**9)
        b = [r[0] for r in reqs]
        assert not oracle.arena_conflict(b, off, [r[1] for r in reqs], [r[2] for r in reqs])
        # first fit: no buffer could sit lower given those placed before it
        placed = []
        for i in order:
            lo = 0
            busy = sorted((off[j], off[j] + b[j]) for j in placed
                          if reqs[j][1] <= reqs[i][2] and reqs[i][1] <= reqs[j][2])
            for s, e in busy:
                if s >= lo + b[i]:
                    break
                lo = max(lo, e)
            assert off[i] == lo
            placed.append(i)


# ----------------------------------------------------------------- graphs

def test_eval_graph_cpu_matches_reference_on_lcg_mlp():
    # lib.rs:99-107: mlp_spec(4,16,32,8), input lcg seed 42, max_abs < 1e-4
    import catnn_amd
    from catnn_amd import Tensor, TensorType

    g = catnn_amd.lower_architecture(catnn_amd.mlp_spec(4, 16, 32, 8))
    x = Tensor.lcg(TensorType.f32([4, 16]), 42).numpy()
    a = oracle.eval_graph(g, x)
    b = oracle.eval_graph(g, x, reference=True)
    assert np.max(np.abs(a - b)) < 1e-4
    assert a.shape == (4, 8)
    want = x.astype(np.float64)
    for nid in (1, 3):
        p = g.nodes[nid].params
        want = want @ p["w"].numpy() + p["b"].numpy()
        if nid == 1:
            want = np.maximum(want, 0)
    assert rel_l2(a, want) < 1e-6


def test_topo_restatement_matches_reference_chain():
    # ir.rs:104-134
    import catnn_amd

    g = catnn_amd.IrGraph("t")
    g.add_node(catnn_amd.IrNode(0, "a", catnn_amd.OpenOp.identity(), catnn_amd.TensorType.f32([2])))
    g.add_node(catnn_amd.IrNode(1, "b", catnn_amd.OpenOp.relu(), catnn_amd.TensorType.f32([2])))
    g.add_edge(0, 1)
    assert oracle.topo(g) == [0, 1]
