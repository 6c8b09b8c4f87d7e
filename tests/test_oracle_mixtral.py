"""Pins the oracle's restatement of the Mixtral-tiny ops (moe.rs:17-136,
:325-333, deepseek.rs:229-239) against float64 torch/numpy derivations
written independently of the reference's loop order, and against special
cases the mathematics fixes."""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_l2

RNG = np.random.default_rng(7)


def test_rmsnorm_known_answer_and_float64():
    y = oracle.rmsnorm(np.array([[3.0, 4.0]]), np.array([1.0, 2.0]), 0.0)
    r = 1.0 / np.sqrt(12.5)
    assert np.allclose(y, [[3 * r, 8 * r]], rtol=1e-6)
    x = RNG.standard_normal((5, 33)).astype(np.float32)
    w = RNG.standard_normal(33).astype(np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert rel_l2(oracle.rmsnorm(x, w, 1e-6), want) < 1e-6


def test_embedding_rounds_half_away_from_zero_and_rejects_out_of_range():
    table = np.arange(12, dtype=np.float32).reshape(4, 3)
    y = oracle.embedding(np.array([[0.4, 1.5], [2.5, -3.0]], np.float32), table)
    assert y.shape == (2, 2, 3)
    assert y[0, 0].tolist() == [0, 1, 2] and y[0, 1].tolist() == [6, 7, 8]   # 1.5 → 2
    assert y[1, 0].tolist() == [9, 10, 11] and y[1, 1].tolist() == [0, 1, 2]  # 2.5 → 3, −3 → 0
    with pytest.raises(ValueError):
        oracle.embedding(np.array([3.6], np.float32), table)  # rounds to 4 = vocab


def _rope64(t, theta):
    """RoPE as a complex rotation of interleaved pairs, float64."""
    B, S, Hh, hd = t.shape
    i = torch.arange(hd // 2, dtype=torch.float64)
    freq = 1.0 / theta ** (2.0 * i / hd)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * freq[None, :]
    z = torch.view_as_complex(t.reshape(B, S, Hh, hd // 2, 2).contiguous())
    z = z * torch.polar(torch.ones_like(ang), ang)[None, :, None, :]
    return torch.view_as_real(z).reshape(B, S, Hh, hd)


def _gqa64(x, wq, wk, wv, wo, nh, nkv, hd, theta, window):
    B, S, D = x.shape
    X = torch.tensor(x, dtype=torch.float64)
    q = (X @ torch.tensor(wq, dtype=torch.float64)).reshape(B, S, nh, hd)
    k = (X @ torch.tensor(wk, dtype=torch.float64)).reshape(B, S, nkv, hd)
    v = (X @ torch.tensor(wv, dtype=torch.float64)).reshape(B, S, nkv, hd)
    q, k = _rope64(q, theta), _rope64(k, theta)
    rep = nh // nkv
    k = k.repeat_interleave(rep, dim=2)
    v = v.repeat_interleave(rep, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", q, k) / np.sqrt(hd)
    i = torch.arange(S)[:, None]
    j = torch.arange(S)[None, :]
    ok = j <= i
    if window is not None:
        ok &= j >= i - (window - 1)
    s = s.masked_fill(~ok, float("-inf"))
    ctx = torch.einsum("bhij,bjhd->bihd", torch.softmax(s, -1), v).reshape(B, S, D)
    return (ctx @ torch.tensor(wo, dtype=torch.float64)).numpy()


@pytest.mark.parametrize("nh,nkv,window", [(4, 2, None), (4, 4, None), (4, 1, 3), (2, 2, 1)])
def test_gqa_matches_float64(nh, nkv, window):
    B, S, hd = 2, 9, 8
    D = nh * hd
    x = RNG.standard_normal((B, S, D)).astype(np.float32)
    wq = (RNG.standard_normal((D, D)) / np.sqrt(D)).astype(np.float32)
    wk = (RNG.standard_normal((D, nkv * hd)) / np.sqrt(D)).astype(np.float32)
    wv = (RNG.standard_normal((D, nkv * hd)) / np.sqrt(D)).astype(np.float32)
    wo = (RNG.standard_normal((D, D)) / np.sqrt(D)).astype(np.float32)
    got = oracle.gqa(x, wq, wk, wv, wo, nh, nkv, hd, 10000.0, window)
    assert rel_l2(got, _gqa64(x, wq, wk, wv, wo, nh, nkv, hd, 10000.0, window)) < 1e-5
    if window == 1:
        # Each query sees only itself: ctx = v, whatever q and k are.
        v = x.astype(np.float64) @ wv.astype(np.float64)
        assert rel_l2(got, v @ wo.astype(np.float64)) < 1e-5


def test_rope_pairs_are_interleaved():
    # A half-split pairing (i, i + hd/2) would fail this: rotate one vector by hand.
    hd, theta = 4, 10000.0
    q = np.array([1.0, 2.0, 3.0, 4.0])
    pos = 3
    want = q.copy()
    for i in range(hd // 2):
        a = pos / theta ** (2 * i / hd)
        want[2 * i], want[2 * i + 1] = q[2 * i] * np.cos(a) - q[2 * i + 1] * np.sin(a), \
            q[2 * i] * np.sin(a) + q[2 * i + 1] * np.cos(a)
    got = _rope64(torch.tensor(q).reshape(1, 1, 1, 4).repeat(1, pos + 1, 1, 1), theta)[0, pos, 0].numpy()
    assert np.allclose(got, want)


def test_lm_head_and_mix():
    x = RNG.standard_normal((2, 3, 8)).astype(np.float32)
    w = RNG.standard_normal((11, 8)).astype(np.float32)
    assert rel_l2(oracle.lm_head(x, w), x.astype(np.float64) @ w.astype(np.float64).T) < 1e-6
    a, b = RNG.standard_normal(7).astype(np.float32), RNG.standard_normal(7).astype(np.float32)
    assert np.allclose(oracle.mix(a, b, 0.0), 0.5 * a + 0.5 * b, rtol=1e-6)
    s = 1 / (1 + np.exp(-1.5))
    assert np.allclose(oracle.mix(a, b, 1.5), s * a + (1 - s) * b, rtol=1e-6)
