"""Pins the oracle's rmsnorm_backward (crates/catnn-compile/src/kernel/
adjoint.rs:147-198), mix_backward (kernel/deepseek.rs:241-258) and
embedding_backward (adjoint.rs:187-197; the last two at the end) on the CPU.  rmsnorm_backward against central finite differences of
L = ⟨dy, rmsnorm(x, w)⟩ in float64 (independent of the closed form: a
dropped term, a wrong power or a swapped operand fails it), and against
the closed form dx = inv·(w⊙dy) − x·inv³·Σ(w⊙dy⊙x)/n, dw = Σ_rows dy⊙x·inv."""
import numpy as np
import pytest

import oracle_train as ot
from conftest import rel_l2


def _rms64(x, w, eps):
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return x * inv * w


@pytest.mark.parametrize("rows,cols", [(3, 5), (4, 16)])
def test_against_finite_differences(rows, cols):
    r = np.random.default_rng(cols)
    eps = 1e-5
    x = r.standard_normal((rows, cols))
    w = 1 + 0.3 * r.standard_normal(cols)
    dy = r.standard_normal((rows, cols))
    dx, dw = ot.rmsnorm_backward(x.astype(np.float32), w.astype(np.float32), dy.astype(np.float32), eps)
    h = 1e-6
    fx = np.zeros_like(x)
    for idx in np.ndindex(*x.shape):
        e = np.zeros_like(x)
        e[idx] = h
        fx[idx] = ((dy * _rms64(x + e, w, eps)).sum() - (dy * _rms64(x - e, w, eps)).sum()) / (2 * h)
    fw = np.zeros_like(w)
    for i in range(cols):
        e = np.zeros_like(w)
        e[i] = h
        fw[i] = ((dy * _rms64(x, w + e, eps)).sum() - (dy * _rms64(x, w - e, eps)).sum()) / (2 * h)
    assert rel_l2(dx, fx) < 1e-5
    assert rel_l2(dw, fw) < 1e-5


def test_against_closed_form_at_width_4096():
    r = np.random.default_rng(1)
    rows, cols, eps = 8, 4096, 1e-5
    x = r.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    dy = r.standard_normal((rows, cols)).astype(np.float32)
    dx, dw = ot.rmsnorm_backward(x, w, dy, eps)
    x64, w64, d64 = x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64)
    inv = 1.0 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)
    want_dx = inv * w64 * d64 - x64 * inv ** 3 * (w64 * d64 * x64).sum(axis=1, keepdims=True) / cols
    assert rel_l2(dx, want_dx) < 1e-5
    assert rel_l2(dw, (d64 * x64 * inv).sum(axis=0)) < 1e-5


def test_mix_backward_against_float64():
    # deepseek.rs:241-258: da = σ·dy, db = (1 − σ)·dy, dg = σ(1 − σ)·Σ(a − b)·dy.
    r = np.random.default_rng(5)
    a, b, dy = (r.standard_normal(1000).astype(np.float32) for _ in range(3))
    g = 0.7
    da, db, dg = ot.mix_backward(a, b, g, dy)
    s = 1 / (1 + np.exp(-np.float64(np.float32(g))))
    assert rel_l2(da, s * dy) < 1e-6 and rel_l2(db, (1 - s) * dy) < 1e-6
    want = s * (1 - s) * ((a.astype(np.float64) - b) * dy).sum()
    assert abs(dg - want) < 1e-5 * max(1.0, abs(want))
    # finite differences of ⟨dy, σ(g)a + (1 − σ(g))b⟩ in the gate
    f = lambda gg: (dy.astype(np.float64) * (a / (1 + np.exp(-gg)) + b * (1 - 1 / (1 + np.exp(-gg))))).sum()
    h = 1e-6
    assert abs(dg - (f(np.float64(np.float32(g)) + h) - f(np.float64(np.float32(g)) - h)) / (2 * h)) < 1e-4


def test_embedding_backward_known_answer():
    # adjoint.rs:187-197 with the ids converted as adjoint.rs:845 does:
    # 1.5 → 2, −3 → 0, NaN → 0; rows add in token order.
    dy = np.arange(5 * 3, dtype=np.float32).reshape(5, 3)
    ids = np.array([0, 2, 1.5, -3, np.nan], np.float32)
    dw = ot.embedding_backward(ids, (4, 3), dy)
    want = np.zeros((4, 3), np.float32)
    for t, v in enumerate([0, 2, 2, 0, 0]):
        want[v] += dy[t]
    assert np.array_equal(dw, want)
