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
# f16 (not a north-star dtype): one f16 ulp is 2^-11 ~ 4.9e-4 relative; the outputs are RNE of an f32 value
F16_TOL = 2e-3


class Case:
    """A tensor described for both sides: the kudnn descriptor and the oracle buffer."""

    def __init__(self, dims, dt, layout=None, strides=None, seed=0, dist="uniform", lo=-1.0, hi=1.0, zero=False):
        self.desc = K.desc(dims, dt, layout, strides)
        self.dt = dt
        shape, st = self.desc.shape(), self.desc.stride()
        if dt in (O.S32, O.S8, O.U8) and not zero:
            # integer tensors: uniform integers in [lo, hi] from a seeded numpy generator
            t = O.empty(shape, st, dt)
            t.buf[:] = np.random.default_rng(seed).integers(int(lo), int(hi) + 1, size=t.buf.size)
            self.t = t
        else:
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
    tdt = {O.F32: torch.float32, O.S32: torch.int32, O.S8: torch.int8, O.U8: torch.uint8}.get(case.dt, torch.int16)
    return torch.zeros(n, dtype=tdt, device="cuda")


def from_device(x, dt) -> np.ndarray:
    a = x.cpu().numpy()
    if dt == O.F32:
        return a.astype(np.float32, copy=False)
    return a.view(O.storage_dtype(dt))


def compare(got_buf: np.ndarray, ref_buf: np.ndarray, dt: int, what: str = ""):
    """Asserts the north-star tolerance (bit-exact for integer outputs); returns (max-normalised error, bit-exact
    fraction)."""
    if dt in (O.S32, O.S8, O.U8):
        bad = np.nonzero(got_buf != ref_buf)[0]
        assert bad.size == 0, (f"{what}: {bad.size} of {got_buf.size} integer outputs differ, first at {bad[0]}: "
                               f"got {got_buf[bad[0]]} want {ref_buf[bad[0]]}")
        return 0.0, 1.0
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
    elif dt == O.F16:
        assert maxnorm <= F16_TOL, f"{what}: f16 max-normalised error {maxnorm:.3e} > {F16_TOL}"
        bad = d > (F16_TOL + F16_TOL * np.abs(r[fin]))
        assert float(np.mean(bad)) <= 1e-4 if bad.size else True, f"{what}: {np.count_nonzero(bad)} elements outside 2e-3"
    else:
        assert maxnorm <= BF16_MAXNORM_TOL, f"{what}: max-normalised error {maxnorm:.3e} > {BF16_MAXNORM_TOL}"
        bad = d > (BF16_ATOL + BF16_RTOL * np.abs(r[fin]))
        frac = float(np.mean(bad)) if bad.size else 0.0
        # element-wise 1e-2 rel / 1e-2 abs; a handful of elements may differ by one bf16 ulp of an
        # intermediate where f32 summation order lands on the other side of a rounding boundary
        assert frac <= 1e-4, f"{what}: {np.count_nonzero(bad)} of {bad.size} elements outside 1e-2 rel/abs"
    return maxnorm, exact


def dense_rows(t: O.Tensor, rows) -> O.Tensor:
    """Rows of a dense row-major tensor viewed as [rows, last dim]."""
    last = t.dims[-1]
    buf = t.buf.reshape(-1, last)[rows].copy().reshape(-1)
    return O.Tensor((len(rows), last), (last, 1), t.dtype, buf)


def sample_rows(m: int, count: int, seed: int = 1234) -> np.ndarray:
    rng = np.random.default_rng(seed)
    fixed = [0, 1, m // 2, m - 2, m - 1]
    rest = rng.choice(m, size=max(0, min(count, m) - len(fixed)), replace=False)
    return np.unique(np.clip(np.concatenate([fixed, rest]), 0, m - 1))
