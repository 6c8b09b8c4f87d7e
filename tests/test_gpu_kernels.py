"""Kernel parity on the GPU, through the C ABI, against the pinned oracle.

Bar: routing indices, logits, permutations and counts bit-exact; fp32
values within 1e-4 relative L2 of the oracle's restatement of the
reference CPU kernels, with the observed error
printed.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from catnn_amd import CatError
from catnn_amd import device as D
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4  # fp32 relative L2 (north star)
RNG = np.random.default_rng(2024)


def _put(dev, a):
    return dev.put(np.ascontiguousarray(a))


def _get(buf, shape, dtype=np.float32):
    return buf.download(shape, dtype)


LINEAR_CASES = [
    (256, 784, 512, 2, True, False),    # config 1 fc1 (+relu)
    (256, 512, 10, 0, True, False),     # config 1 fc3, N % 4 != 0
    (5, 7, 3, 0, False, False),         # odd everything (scalar path)
    (130, 100, 70, 3, True, True),      # ragged tiles, gelu, residual
    (1, 1, 1, 2, True, True),
    (300, 64, 96, 3, False, True),
    (1000, 1024, 1000, 3, True, True),
    (129, 257, 255, 0, True, False),
]


@pytest.mark.parametrize("m,k,n,act,bias,res", LINEAR_CASES)
def test_linear_matches_oracle(device, m, k, n, act, bias, res):
    x = RNG.standard_normal((m, k)).astype(np.float32)
    w = (RNG.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32) if bias else None
    r = RNG.standard_normal((m, n)).astype(np.float32) if res else None
    want = oracle.linear(x, w, b)
    if act == 2:
        want = oracle.relu(want)
    if act == 3:
        want = oracle.gelu(want)
    if res:
        want = oracle.add(r, want)
    dx, dw, dy = _put(device, x), _put(device, w), device.alloc(m * n * 4)
    db = _put(device, b) if bias else None
    dr = _put(device, r) if res else None
    D.linear(device, dx, dw, db, dr, dy, m, k, n, act)
    got = _get(dy, (m, n))
    err = rel_l2(got, want)
    print(f"linear m={m} k={k} n={n} act={act}: rel_l2={err:.2e}")
    assert err < TOL
    # also within tolerance of the naïve reference::linear
    want_ref = oracle.ref_linear(x, w, b)
    if act == 0 and not res:
        assert rel_l2(got, want_ref) < TOL


def _bf16_bits(a):
    """Round to bf16 (ties to even) and return (uint16 bits, float64 value)."""
    import oracle_bf16

    v = oracle_bf16.bf16_round(a)
    return (v.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16), v


GEMM_BF16_CASES = [
    (1, 1, 1), (5, 7, 3), (130, 100, 70), (129, 257, 255), (300, 64, 520),
    (256, 512, 384), (1024, 1024, 1024), (200, 3 * 784, 10),
    # 16-byte rows with a partial last k chunk, and k below one chunk
    (129, 257, 264), (77, 130, 136), (300, 200, 40), (513, 385, 1000),
]


@pytest.mark.parametrize("tile_cfg", [0, 2, 7, 9, 10, 11, 12])
@pytest.mark.parametrize("m,n,k", GEMM_BF16_CASES)
def test_gemm_bf16_matches_float64(device, m, n, k, tile_cfg):
    # bf16 operands, fp32 accumulation: only the accumulation rounds.
    a_bits, a = _bf16_bits(RNG.standard_normal((m, k)))
    b_bits, b = _bf16_bits(RNG.standard_normal((n, k)))
    c0 = RNG.standard_normal((m, n)).astype(np.float32)
    want = a @ b.T
    da, db, dc = _put(device, a_bits), _put(device, b_bits), _put(device, c0)
    D.gemm_bf16_nt(device, da, k, db, k, dc, n, m, n, k, accumulate=False, tile_cfg=tile_cfg)
    got = _get(dc, (m, n))
    err = rel_l2(got, want)
    print(f"gemm_bf16 m={m} n={n} k={k} cfg={tile_cfg}: rel_l2={err:.2e}")
    assert err < 1e-6
    D.gemm_bf16_nt(device, da, k, db, k, dc, n, m, n, k, accumulate=True, tile_cfg=tile_cfg)
    assert rel_l2(_get(dc, (m, n)), 2 * want) < 1e-6


def test_gemm_bf16_strided_operands(device):
    # Leading dimensions larger than k (the split-bf16 operands' hi part).
    m, n, k = 190, 150, 96
    a_bits, a = _bf16_bits(RNG.standard_normal((m, 3 * k)))
    b_bits, b = _bf16_bits(RNG.standard_normal((n, 3 * k)))
    dc = device.alloc(m * 200 * 4)
    D.gemm_bf16_nt(device, _put(device, a_bits), 3 * k, _put(device, b_bits), 3 * k, dc, 200, m, n, k)
    got = _get(dc, (m, 200))[:, :n]
    assert rel_l2(got, a[:, :k] @ b[:, :k].T) < 1e-6
    with pytest.raises(CatError) as e:
        D.gemm_bf16_nt(device, dc, 4, dc, 4, dc, 4, 4, 4, 8)
    assert e.value.kind == "ShapeMismatch"


def test_linear_empty_and_bad_act(device):
    dx = device.alloc(64)
    D.linear(device, dx, dx, None, None, dx, 0, 4, 4, 0)  # M = 0: nothing to do
    with pytest.raises(CatError) as e:
        D.linear(device, dx, dx, None, None, dx, 1, 4, 4, 7)
    assert e.value.kind == "InvalidArgument"


def test_activations_and_adds(device):
    x = (RNG.standard_normal(10_001) * 4).astype(np.float32)
    dx, dy = _put(device, x), device.alloc(x.nbytes)
    D.act(device, dx, dy, x.size, 2)
    assert np.array_equal(_get(dy, x.shape), oracle.relu(x))
    D.act(device, dx, dy, x.size, 3)
    assert rel_l2(_get(dy, x.shape), oracle.gelu(x)) < 1e-6
    a = RNG.standard_normal((37, 12)).astype(np.float32)
    b = RNG.standard_normal((37, 12)).astype(np.float32)
    bias = RNG.standard_normal(12).astype(np.float32)
    da, db, dbias, dout = _put(device, a), _put(device, b), _put(device, bias), device.alloc(a.nbytes)
    D.add(device, da, db, dout, a.size, b.size)
    assert np.array_equal(_get(dout, a.shape), oracle.add(a, b))
    D.add(device, da, dbias, dout, a.size, bias.size)
    assert np.array_equal(_get(dout, a.shape), oracle.add(a, bias))


@pytest.mark.parametrize("rows,cols", [(8192, 1024), (4097, 1024), (4096, 768), (33, 96), (5, 4), (7, 7), (3, 4096),
                                       (2, 5000)])
def test_layer_norm_and_softmax_match_oracle(device, rows, cols):
    x = (RNG.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
    g = RNG.standard_normal(cols).astype(np.float32)
    b = RNG.standard_normal(cols).astype(np.float32)
    dx, dg, db, dy = _put(device, x), _put(device, g), _put(device, b), device.alloc(x.nbytes)
    D.layer_norm(device, dx, dg, db, dy, rows, cols, 1e-6)
    e1 = rel_l2(_get(dy, x.shape), oracle.layer_norm(x, g, b, 1e-6))
    D.softmax(device, dx, dy, rows, cols)
    e2 = rel_l2(_get(dy, x.shape), oracle.softmax_last(x))
    print(f"rows={rows} cols={cols}: layer_norm {e1:.2e} softmax {e2:.2e}")
    assert e1 < TOL and e2 < TOL


ATTN_CASES = [
    (2, 8, 4, 4),      # the reference's demo block shape (d_head 4: generic kernel)
    (2, 256, 4, 64),   # MFMA kernel
    (1, 100, 2, 64),   # ragged sequence
    (1, 1, 1, 64),
    (2, 300, 3, 64),
    (1, 130, 2, 32),   # MFMA kernel, d_head 32
    (2, 200, 2, 128),  # MFMA kernel, d_head 128 (one block per CU)
    (1, 65, 3, 128),
    (1, 96, 2, 48),    # generic kernel
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,S,H,dh", ATTN_CASES)
def test_attention_core_matches_float64(device, B, S, H, dh, causal):
    Dm = H * dh
    q, k, v = (RNG.standard_normal((B, S, Dm)).astype(np.float32) for _ in range(3))
    dq, dk, dv, do = _put(device, q), _put(device, k), _put(device, v), device.alloc(q.nbytes)
    D.attention_core(device, dq, dk, dv, do, B, S, Dm, H, dh, causal)
    got = _get(do, q.shape)
    tq, tk, tv = (torch.from_numpy(a).double().view(B, S, H, dh).transpose(1, 2) for a in (q, k, v))
    want = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal)
    want = want.transpose(1, 2).reshape(B, S, Dm).numpy()
    err = rel_l2(got, want)
    print(f"attention B={B} S={S} H={H} dh={dh} causal={causal}: rel_l2={err:.2e}")
    assert err < TOL


@pytest.mark.parametrize("T,H,E,k", [(1000, 1024, 8, 2), (37, 100, 5, 3), (4096, 64, 64, 4),
                                     (1, 8, 2, 2),
                                     (50, 30, 4, 2),          # H % 4 != 0: the LDS-staged kernel
                                     (300, 1000, 64, 2),      # gate staged in several chunks
                                     (20, 200, 256, 8),
                                     (500, 256, 16, 4),       # direct-to-LDS staging, 16 tokens a block
                                     (300, 128, 4, 1)])       # … 64 tokens a block
def test_route_is_bit_exact(device, T, H, E, k):
    x = RNG.standard_normal((T, H)).astype(np.float32)
    gate = (RNG.standard_normal((H, E)) * math.sqrt(0.5)).astype(np.float32)
    idx_w, w_w, lg_w = oracle.route(x, gate, k)
    dx, dg = _put(device, x), _put(device, gate)
    didx, dw, dlg = device.alloc(T * k * 4), device.alloc(T * k * 4), device.alloc(T * E * 4)
    D.moe_route(device, dx, dg, T, H, E, k, didx, dw, dlg)
    assert np.array_equal(_get(dlg, (T, E)), lg_w), "logits must be bit-exact"
    assert np.array_equal(_get(didx, (T, k), np.int32), idx_w), "indices must be bit-exact"
    assert np.max(np.abs(_get(dw, (T, k)) - w_w)) < 1e-6


@pytest.mark.parametrize("E,k", [(6, 3), (8, 4), (64, 8)])  # one thread per token; lane groups (8, 64)
def test_route_ties_prefer_lower_expert(device, E, k):
    # Duplicated gate columns make equal logits: the selection must take the
    # lower expert first, as the stable descending order of the reference.
    T, H = 64, 32
    x = RNG.standard_normal((T, H)).astype(np.float32)
    base = RNG.standard_normal((H, 3)).astype(np.float32)
    gate = np.tile(np.concatenate([base[:, :1], base, base[:, 1:]], 1), (1, E))[:, :E].copy()
    idx_w, _, _ = oracle.route(x, gate, k)
    dx, dg, didx = _put(device, x), _put(device, gate), device.alloc(T * k * 4)
    D.moe_route(device, dx, dg, T, H, E, k, didx, None, None)
    assert np.array_equal(_get(didx, (T, k), np.int32), idx_w)


@pytest.mark.parametrize("T,k,E,mode", [(10_000, 2, 8, "random"), (5000, 2, 8, "one"),
                                        (3000, 4, 64, "random"), (1, 1, 1, "random"),
                                        (2049, 2, 3, "skew")])
def test_permutation_is_bit_exact(device, T, k, E, mode):
    if mode == "one":
        idx = np.full((T, k), E - 1, np.int32)
    elif mode == "skew":
        idx = np.minimum(RNG.geometric(0.7, (T, k)) - 1, E - 1).astype(np.int32)
    else:
        idx = RNG.integers(0, E, (T, k)).astype(np.int32)
    counts, offsets, sop, pos = oracle.moe_permute(idx, E)
    di = _put(device, idx)
    dc, do = device.alloc(E * 4), device.alloc((E + 1) * 4)
    ds, dp = device.alloc(T * k * 4), device.alloc(T * k * 4)
    D.moe_permute(device, di, T, k, E, dc, do, ds, dp)
    assert np.array_equal(_get(dc, E, np.int32), counts)
    assert np.array_equal(_get(do, E + 1, np.int32), offsets)
    assert np.array_equal(_get(ds, T * k, np.int32), sop)
    assert np.array_equal(_get(dp, T * k, np.int32), pos)


def test_permutation_rejects_bad_ids(device):
    idx = np.array([[0, 1], [2, 9]], np.int32)
    di, dc, do = _put(device, idx), device.alloc(16), device.alloc(20)
    ds, dp = device.alloc(16), device.alloc(16)
    with pytest.raises(CatError) as e:
        D.moe_permute(device, di, 2, 2, 4, dc, do, ds, dp)
    assert e.value.kind == "ShapeMismatch"


# (300, 100, 52) and (257, 36, 20): 16-byte rows whose K is not a multiple of
# 16, so the direct-to-LDS expert GEMMs (dual gate/up and down) end on a
# partial chunk loaded through registers.
@pytest.mark.parametrize("T,H,I,E,k", [(300, 128, 96, 4, 2), (64, 100, 50, 3, 2), (513, 256, 512, 8, 2),
                                       (7, 64, 64, 8, 8), (300, 100, 52, 4, 2), (257, 36, 20, 8, 2)])
def test_moe_layer_matches_oracle(device, T, H, I, E, k):
    r = np.random.default_rng(T + H)
    x = r.standard_normal((T, H)).astype(np.float32)
    gate = (r.standard_normal((H, E)) * math.sqrt(0.5)).astype(np.float32)
    w1 = (r.standard_normal((E, H, I)) * math.sqrt(0.02)).astype(np.float32)
    w3 = (r.standard_normal((E, H, I)) * math.sqrt(0.02)).astype(np.float32)
    w2 = (r.standard_normal((E, I, H)) * math.sqrt(0.02)).astype(np.float32)
    want = oracle.moe(x, gate, w1, w3, w2, k)
    idx_w, w_w, _ = oracle.route(x, gate, k)
    dx, dg = _put(device, x), _put(device, gate)
    d1 = [_put(device, w1[e]) for e in range(E)]
    d3 = [_put(device, w3[e]) for e in range(E)]
    d2 = [_put(device, w2[e]) for e in range(E)]
    dout, didx, dw, dc = device.alloc(x.nbytes), device.alloc(T * k * 4), device.alloc(T * k * 4), device.alloc(E * 4)
    D.moe(device, dx, dg, d1, d3, d2, T, H, I, E, k, dout, didx, dw, dc)
    got = _get(dout, x.shape)
    err = rel_l2(got, want)
    print(f"moe T={T} H={H} I={I} E={E} k={k}: rel_l2={err:.2e}")
    assert np.array_equal(_get(didx, (T, k), np.int32), idx_w)
    assert np.array_equal(_get(dc, E, np.int32), np.bincount(idx_w.reshape(-1), minlength=E))
    assert err < TOL
    assert rel_l2(got, oracle.moe(x, gate, w1, w3, w2, k, reference=True)) < TOL
