"""bench.py's device-side input generator against the oracle's SplitMix64 fill (CPU torch, small sizes).

The bench may not use the oracle for its inputs, so it restates the generator in torch int64 arithmetic; these tests
pin that restatement: uniform draws bit for bit, Box-Muller normals to within one f32 ulp (the f64 log / cos of torch
and of the C library may differ in the last double bit, which rarely moves the f32 rounding), bf16 as RNE of the f32
sample.
"""
import numpy as np
import pytest

import bench
import oracle as O

torch = pytest.importorskip("torch")


def _oracle(n, seed, dist, a, b, dt):
    t = O.fill((n,), (1,), dt, seed, dist, a, b)
    return t.buf


@pytest.mark.parametrize("seed", [0, 1, 3, 17, 2**63 + 5])
def test_uniform_matches_oracle_bitwise(seed):
    got = bench.synth(torch, (1000,), seed, "uniform", -1.0, 1.0, torch.float32, dev="cpu").numpy()
    want = _oracle(1000, seed, "uniform", -1.0, 1.0, O.F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", [0, 1, 3])
def test_normal_matches_oracle(seed):
    got = bench.synth(torch, (4000,), seed, "normal", 0.0, 0.02, torch.float32, dev="cpu").numpy()
    want = _oracle(4000, seed, "normal", 0.0, 0.02, O.F32)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert np.mean(ulps == 0) >= 0.999


def test_bf16_is_rne_of_the_f32_sample():
    got = bench.synth(torch, (3000,), 0, "normal", 0.0, 1.0, torch.bfloat16, dev="cpu")
    f32 = bench.synth(torch, (3000,), 0, "normal", 0.0, 1.0, torch.float32, dev="cpu").numpy()
    want = O.from_f32_rne(f32, O.BF16)
    assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("dist", ["uniform", "normal"])
def test_chunks_continue_the_stream(dist):
    # generated in pieces: the draw index carries across piece boundaries (two draws per normal)
    a = bench.synth(torch, (1001,), 7, dist, 0.0, 1.0, torch.float32, dev="cpu", chunk=64).numpy()
    b = bench.synth(torch, (1001,), 7, dist, 0.0, 1.0, torch.float32, dev="cpu").numpy()
    assert np.array_equal(a, b)
