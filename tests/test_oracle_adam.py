"""Pins the oracle's Adam::put (crates/catnn-core/src/lens/optim.rs:95-118)
and its f32::powi, on the CPU:

  * the reference's own known answer, adam_first_step_matches_closed_form
    (optim.rs:178-193);
  * the first step from a zero state, which the mathematics fixes:
    m̂ = g and v̂ = g² up to rounding, so p' = p − lr·g/(|g| + eps) ≈ p − lr·sign(g);
  * several steps against the textbook algorithm in float64 (a dropped bias
    correction, swapped betas or a missing square fails it);
  * a zero gradient on a zero state leaves p unchanged;
  * powi on exactly representable cases and against float64 pow.
"""
import numpy as np
import pytest

import oracle_train as ot

# Adam::default's constants as the f32 values the reference computes with.
B1, B2, EPS = (float(np.float32(c)) for c in (0.9, 0.999, 1e-8))


def _textbook(p, gs, lr):
    """Adam (Kingma & Ba, Algorithm 1) in float64 over the gradients gs."""
    p = p.astype(np.float64)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t, g in enumerate(gs, start=1):
        g = g.astype(np.float64)
        m = B1 * m + (1 - B1) * g
        v = B2 * v + (1 - B2) * g * g
        mhat = m / (1 - B1 ** t)
        vhat = v / (1 - B2 ** t)
        p = p - lr * mhat / (np.sqrt(vhat) + EPS)
    return p, m, v


def test_reference_known_answer():
    # optim.rs:178-193: p = 0, g = 1, lr 0.1 → −0.1·m̂/(√v̂ + 1e-8), t = 1.
    st = ot.AdamState((1,))
    q = ot.adam(np.zeros(1, np.float32), np.ones(1, np.float32), st, 0.1)
    m, v = np.float32(0.1), np.float32(0.001)
    mhat = m / (np.float32(1.0) - np.float32(0.9))
    vhat = v / (np.float32(1.0) - np.float32(0.999))
    expect = np.float32(0.0) - np.float32(0.1) * mhat / (np.sqrt(vhat) + np.float32(1e-8))
    assert abs(float(q[0]) - float(expect)) < 1e-6
    assert st.t == 1
    assert st.m[0] == np.float32(1.0) - np.float32(0.9)  # (1−β₁)·g with 1−β₁ rounded in f32


def test_first_step_moves_by_lr_times_sign():
    rng = np.random.default_rng(1)
    p = rng.standard_normal(4096).astype(np.float32)
    g = (rng.choice([-1, 1], 4096) * 10.0 ** rng.uniform(-2, 1, 4096)).astype(np.float32)
    st = ot.AdamState(p.shape)
    lr = 1e-3
    q = ot.adam(p, g, st, lr)
    step = (p.astype(np.float64) - q) / lr
    assert np.allclose(step, np.sign(g), rtol=0, atol=2e-3)  # p's own f32 rounding at |p| ≤ 4
    # Moments after one step: (1−β₁)g and ((1−β₂)g)g, rounded in f32.
    assert np.array_equal(st.m, np.float32(1 - np.float32(B1)) * g)
    assert np.allclose(st.v, (1 - B2) * g.astype(np.float64) ** 2, rtol=2e-6, atol=0)


def test_several_steps_follow_float64_textbook():
    rng = np.random.default_rng(2)
    p = rng.standard_normal(2048).astype(np.float32)
    gs = [rng.standard_normal(2048).astype(np.float32) for _ in range(6)]
    st = ot.AdamState(p.shape)
    q = p.copy()
    for g in gs:
        q = ot.adam(q, g, st, 1e-2)
    pw, mw, vw = _textbook(p, gs, 1e-2)
    assert st.t == 6
    assert np.abs(q - pw).max() < 1e-5
    assert np.allclose(st.m, mw, rtol=1e-5, atol=1e-7)
    assert np.allclose(st.v, vw, rtol=1e-5, atol=1e-9)


def test_zero_gradient_on_zero_state_is_identity():
    p = np.array([3.0, -4.0, 0.0], np.float32)
    st = ot.AdamState(p.shape)
    assert np.array_equal(ot.adam(p, np.zeros(3, np.float32), st, 0.1), p)


def test_state_continues_from_given_t():
    # A state at t = 4 takes the fifth step's bias corrections.
    rng = np.random.default_rng(3)
    p = rng.standard_normal(64).astype(np.float32)
    gs = [rng.standard_normal(64).astype(np.float32) for _ in range(5)]
    st = ot.AdamState(p.shape)
    q = p.copy()
    for g in gs[:4]:
        q = ot.adam(q, g, st, 1e-2)
    st2 = ot.AdamState(p.shape)
    st2.m, st2.v, st2.t = st.m.copy(), st.v.copy(), 4
    a = ot.adam(q, gs[4], st, 1e-2)
    b = ot.adam(q, gs[4], st2, 1e-2)
    assert np.array_equal(a, b) and st.t == st2.t == 5


@pytest.mark.parametrize("b,t,want", [(2.0, 10, 1024.0), (0.5, 3, 0.125), (2.0, -2, 0.25),
                                      (3.0, 0, 1.0), (-2.0, 5, -32.0), (1.5, 2, 2.25)])
def test_powi_exact_cases(b, t, want):
    assert ot.powi(b, t) == np.float32(want)


@pytest.mark.parametrize("b", [0.9, 0.999])
def test_powi_against_float64(b):
    bf = float(np.float32(b))  # the f32 base, exactly
    for t in (1, 2, 7, 100, 1000, 12345):
        if bf ** t < 2.0 ** -126:
            continue  # below the normal f32 range
        got = float(ot.powi(b, t))
        want = bf ** t
        # binary exponentiation: at most ~2·log2(t) roundings, each amplified
        # by the later squarings, i.e. a relative error within t·2⁻²³.
        assert abs(got - want) <= max(t, 4) * 2.0 ** -23 * want, (b, t, got, want)
