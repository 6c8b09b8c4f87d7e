"""catnn_hip_moe_f32_noalloc, the allocation-free MoE entry point, against
catnn_hip_moe_f32 (the entry point it mirrors) through the C ABI: two calls
in a row on the same GPU, the second with fewer tokens, so the second call
runs on scratch that still holds the first call's contents.  Outputs,
expert indices, weights and counts must be bit-identical to the allocating
entry point's, and the output within 1e-4 of the oracle's moe::moe."""
import math

import numpy as np
import pytest

import oracle
from catnn_amd import CatError
from catnn_amd import device as D
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _layer(device, T, H, I, E, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((T, H)).astype(np.float32)
    gate = (r.standard_normal((H, E)) * math.sqrt(0.5)).astype(np.float32)
    w1 = (r.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    w3 = (r.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    w2 = (r.standard_normal((E, I, H)) * 0.05).astype(np.float32)
    dev = dict(x=device.put(x), gate=device.put(gate),
               w1=[device.put(w1[e]) for e in range(E)], w3=[device.put(w3[e]) for e in range(E)],
               w2=[device.put(w2[e]) for e in range(E)])
    return (x, gate, w1, w3, w2), dev


def _run(device, fn, d, T, H, I, E, k):
    out, idx = device.alloc(T * H * 4), device.alloc(T * k * 4)
    w, counts = device.alloc(T * k * 4), device.alloc(E * 4)
    fn(device, d["x"], d["gate"], d["w1"], d["w3"], d["w2"], T, H, I, E, k, out, idx, w, counts)
    device.sync()
    return (out.download((T, H), np.float32), idx.download((T, k), np.int32),
            w.download((T, k), np.float32), counts.download(E, np.int32))


@pytest.mark.parametrize("calls", [[(700, 256, 512, 8, 2), (129, 256, 512, 8, 2)],
                                   [(1500, 1024, 3584, 8, 2), (300, 128, 96, 4, 2)]])
def test_noalloc_moe_matches_the_allocating_entry_point(device, calls):
    for i, (T, H, I, E, k) in enumerate(calls):
        print(f"[noalloc] call {i}: T={T} H={H} I={I} E={E} k={k}", flush=True)
        host, d = _layer(device, T, H, I, E, seed=T + 31 * i)
        got = _run(device, D.moe_noalloc, d, T, H, I, E, k)
        ref = _run(device, D.moe, d, T, H, I, E, k)
        for a, b, what in zip(got, ref, ("out", "idx", "w", "counts")):
            assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32)), what
        sample = min(T, 64)
        want = oracle.moe(*host, k, tokens=np.arange(sample))
        assert rel_l2(got[0][:sample], want[:sample]) < 1e-4


def test_noalloc_moe_refuses_more_than_its_scratch(device):
    # The size check runs on the host before any launch; nothing is read.
    T, H, I, E, k = 100_000, 1024, 3584, 8, 2
    small = device.alloc(256)
    with pytest.raises(CatError) as e:
        D.moe_noalloc(device, small, small, [small] * E, [small] * E, [small] * E, T, H, I, E, k,
                      small)
    assert e.value.kind == "ShapeMismatch" and "exceeds the fixed scratch" in str(e.value)
