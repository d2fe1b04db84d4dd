"""Shared helpers of the parity tests: seeded tensors, device round trips, tolerance checks.

Inputs come from the oracle's SplitMix64 generator (same bits on every machine); the GPU result comes
from the C ABI; the expected result from the CPU oracle on the same buffers.
"""
from __future__ import annotations

import numpy as np

import kudnn_amd as K
import oracle as O

# Tolerances: fp32 relative error <= 1e-5, judged as max|d| / max|ref|
# (a per-element relative error is ill-posed at zero crossings); bf16 1e-2 relative / 1e-2 absolute.
FP32_MAXNORM_TOL = 1e-5
BF16_RTOL = 1e-2
BF16_ATOL = 1e-2
BF16_MAXNORM_TOL = 1e-2


class Case:
    """A tensor described for both sides: the kudnn descriptor and the oracle buffer."""

    def __init__(self, dims, dt, layout=None, strides=None, seed=0, dist="uniform", lo=-1.0, hi=1.0, zero=False):
        self.desc = K.desc(dims, dt, layout, strides)
        self.dt = dt
        shape, st = self.desc.shape(), self.desc.stride()
        self.t = O.empty(shape, st, dt) if zero else O.fill(shape, st, dt, seed, dist, lo, hi)

    def clone_empty(self) -> O.Tensor:
        return O.empty(self.t.dims, self.t.strides, self.dt)

    def device(self):
        import torch

        buf = self.t.buf
        if buf.dtype == np.uint16:
            return torch.from_numpy(buf.view(np.int16).copy()).to("cuda")
        return torch.from_numpy(buf.copy()).to("cuda")


def zeros_device(case: Case):
    import torch

    n = case.t.buf.size
    return torch.zeros(n, dtype=torch.float32 if case.dt == O.F32 else torch.int16, device="cuda")


def from_device(x, dt) -> np.ndarray:
    a = x.cpu().numpy()
    return a.view(np.uint16) if dt != O.F32 else a.astype(np.float32, copy=False)


def compare(got_buf: np.ndarray, ref_buf: np.ndarray, dt: int, what: str = ""):
    """Asserts the north-star tolerance; returns (max-normalised error, bit-exact fraction)."""
    g = O.to_f32(got_buf, dt).astype(np.float64)
    r = O.to_f32(ref_buf, dt).astype(np.float64)
    assert g.shape == r.shape
    assert np.all(np.isfinite(g) == np.isfinite(r)), f"{what}: non-finite mismatch"
    fin = np.isfinite(r)
    d = np.abs(g[fin] - r[fin])
    scale = max(np.max(np.abs(r[fin])) if r[fin].size else 0.0, 1e-30)
    maxnorm = float(np.max(d) / scale) if d.size else 0.0
    exact = float(np.mean(got_buf == ref_buf)) if got_buf.size else 1.0
    if dt == O.F32:
        assert maxnorm <= FP32_MAXNORM_TOL, f"{what}: fp32 max-normalised error {maxnorm:.3e} > {FP32_MAXNORM_TOL}"
    else:
        assert maxnorm <= BF16_MAXNORM_TOL, f"{what}: max-normalised error {maxnorm:.3e} > {BF16_MAXNORM_TOL}"
        bad = d > (BF16_ATOL + BF16_RTOL * np.abs(r[fin]))
        frac = float(np.mean(bad)) if bad.size else 0.0
        # element-wise 1e-2 rel / 1e-2 abs; a handful of elements may differ by one bf16 ulp of an
        # intermediate where f32 summation order lands on the other side of a rounding boundary
        assert frac <= 1e-4, f"{what}: {np.count_nonzero(bad)} of {bad.size} elements outside 1e-2 rel/abs"
    return maxnorm, exact


def sample_rows(m: int, count: int, seed: int = 1234) -> np.ndarray:
    rng = np.random.default_rng(seed)
    fixed = [0, 1, m // 2, m - 2, m - 1]
    rest = rng.choice(m, size=max(0, min(count, m) - len(fixed)), replace=False)
    return np.unique(np.clip(np.concatenate([fixed, rest]), 0, m - 1))
