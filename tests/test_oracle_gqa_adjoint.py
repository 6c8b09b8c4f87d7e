"""Pins the oracle's restatement of gqa_backward (adjoint.rs:287-440, the
GqaAttention arm of adjoint_of at adjoint.rs:862-883) against float64 torch
autograd of an independent derivation of the forward: RoPE as a complex
rotation of interleaved pairs, K/V heads repeated per group, an explicit
causal window mask."""
import numpy as np
import pytest
import torch

import oracle_train as ot
from catnn_amd import IrNode, OpenOp, Tensor, TensorType
from conftest import rel_l2

RNG = np.random.default_rng(321)
T64 = torch.float64


def _rope64(t, theta):
    B, S, Hh, hd = t.shape
    i = torch.arange(hd // 2, dtype=T64)
    ang = torch.arange(S, dtype=T64)[:, None] * (1.0 / theta ** (2.0 * i / hd))[None, :]
    z = torch.view_as_complex(t.reshape(B, S, Hh, hd // 2, 2).contiguous())
    return torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)[None, :, None, :]).reshape(B, S, Hh, hd)


def _gqa64(X, Wq, Wk, Wv, Wo, nh, nkv, hd, theta, window, rope=True):
    B, S, D = X.shape
    q = (X @ Wq).reshape(B, S, nh, hd)
    k = (X @ Wk).reshape(B, S, nkv, hd)
    v = (X @ Wv).reshape(B, S, nkv, hd)
    if rope:
        q, k = _rope64(q, theta), _rope64(k, theta)
    k = k.repeat_interleave(nh // nkv, dim=2)
    v = v.repeat_interleave(nh // nkv, dim=2)
    s = (q.permute(0, 2, 1, 3) @ k.permute(0, 2, 3, 1)) / np.sqrt(hd)
    i, j = torch.arange(S)[:, None], torch.arange(S)[None, :]
    ok = j <= i
    if window is not None:
        ok &= j >= i - (window - 1)
    p = torch.softmax(s.masked_fill(~ok, float("-inf")), -1)
    ctx = (p @ v.permute(0, 2, 1, 3)).permute(0, 2, 1, 3).reshape(B, S, nh * hd)
    return ctx @ Wo


def _case(nh, nkv, hd, B=2, S=11):
    D = nh * hd
    x = RNG.standard_normal((B, S, D)).astype(np.float32)
    ws = [(RNG.standard_normal(sh) / np.sqrt(D)).astype(np.float32)
          for sh in ((D, D), (D, nkv * hd), (D, nkv * hd), (D, D))]
    dy = RNG.standard_normal((B, S, D)).astype(np.float32)
    return x, ws, dy


def _autograd(x, ws, dy, nh, nkv, hd, theta, window, rope=True):
    X, *W = [torch.tensor(a.astype(np.float64), requires_grad=True) for a in (x, *ws)]
    _gqa64(X, *W, nh, nkv, hd, theta, window, rope).backward(torch.tensor(dy.astype(np.float64)))
    return [X.grad.numpy()] + [w.grad.numpy() for w in W]


@pytest.mark.parametrize("nh,nkv,hd,theta,window", [(4, 2, 8, 10000.0, None), (4, 1, 8, 10000.0, 3),
                                                    (2, 2, 6, 1e6, 1), (4, 4, 4, 10000.0, None),
                                                    (6, 2, 8, 500.0, 5)])
def test_gqa_backward_matches_autograd(nh, nkv, hd, theta, window):
    x, ws, dy = _case(nh, nkv, hd)
    got = ot.gqa_backward(x, *ws, nh, nkv, hd, theta, window, dy)
    want = _autograd(x, ws, dy, nh, nkv, hd, theta, window)
    for name, g, w in zip(("dx", "dwq", "dwk", "dwv", "dwo"), got, want):
        e = rel_l2(g, w)
        assert e < 1e-4, (name, e)
    # A mistake in the rotation's adjoint or the window must not pass: the
    # same gradients without RoPE, or without the window, are far off.
    if window != 1:  # (window 1: dwq = dwk = 0 with or without RoPE)
        no_rope = _autograd(x, ws, dy, nh, nkv, hd, theta, window, rope=False)
        assert rel_l2(got[1], no_rope[1]) > 1e-2 and rel_l2(got[2], no_rope[2]) > 1e-2
    if window is not None and window > 1:
        no_win = _autograd(x, ws, dy, nh, nkv, hd, theta, None)
        assert rel_l2(got[0], no_win[0]) > 1e-2


def test_gqa_adjoint_of_arm_and_window_one():
    # adjoint_of's GqaAttention arm passes the fields through; with window 1
    # every query attends only itself, so the softmax adjoint vanishes: dwq and
    # dwk are zero and dx flows through v alone.
    nh, nkv, hd = 2, 1, 4
    x, ws, dy = _case(nh, nkv, hd, B=1, S=6)
    P = {n: Tensor.from_numpy(w) for n, w in zip(("wq", "wk", "wv", "wo"), ws)}
    node = IrNode(1, "gqa", OpenOp.gqa_attention(nh, nkv, hd, nh * hd, 1, 10000), TensorType.f32(list(x.shape)), P)
    (dx,), dp = ot.adjoint_of(node, [x], None, dy)
    assert set(dp) == {"wq", "wk", "wv", "wo"}
    assert np.abs(dp["wq"]).max() == 0 and np.abs(dp["wk"]).max() == 0
    v_path = (dy.astype(np.float64) @ ws[3].astype(np.float64).T).reshape(1, 6, nh, hd).sum(2)
    want_dx = v_path.reshape(6, hd) @ ws[2].astype(np.float64).T
    assert rel_l2(dx.reshape(6, -1), want_dx) < 1e-5
