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


def _bf16_neighbours(bits: np.ndarray):
    """The bf16 patterns one ulp above and one ulp below each finite pattern (through zero and subnormals)."""
    u = bits.astype(np.int32)
    neg = (u & 0x8000) != 0
    mag = u & 0x7FFF
    zero = mag == 0
    # towards +inf: a positive value grows, a negative one shrinks; zero steps to the smallest subnormal
    up = np.where(neg, np.where(mag == 0, 0x0001, u - 1), u + 1)
    down = np.where(neg, u + 1, np.where(zero, 0x8001, u - 1))
    return up.astype(np.uint16), down.astype(np.uint16)


class PostOpsExplainer:
    """Explains bf16 outputs that fall outside 1e-2 rel / 1e-2 abs of the oracle.

    The GPU sums in another order than the oracle, so its GEMM-stage value can land one bf16 ulp away from the
    oracle's where the f32 sum sits next to a rounding boundary; its activation can likewise land one ulp away where
    the activation's f32 value sits next to the store's boundary. Behind a residual add the cancellation can make that
    one ulp larger than 1e-2 absolute (GELU + residual at |x| > 2, where one ulp is 2^-6). An element outside the
    tolerance is accepted only if it equals, bit for bit, the oracle's own stages recomputed from the GEMM-stage value
    or from the activation's stored value moved by one bf16 ulp.

    x, w, bias: the oracle inputs of the rows checked; dims: their output shape; src: the binary operand of those rows.
    """

    def __init__(self, x, w, bias, dims, act=None, act_alpha=0.0, act_beta=0.0, binary=None, src=None, gamma=1.0):
        self.x, self.w, self.bias, self.dims = x, w, bias, tuple(dims)
        self.act = O.ACT_NONE if act is None else act
        self.act_alpha, self.act_beta = act_alpha, act_beta
        self.binary = O.BIN_NONE if binary is None else binary
        self.src, self.gamma = src, gamma
        self._c = None
        self.counts = {"gemm stage": 0, "activation stage": 0}

    def _stage0(self) -> np.ndarray:
        if self._c is None:
            n = self.dims[-1]
            c = O.empty(self.dims, tuple(int(np.prod(self.dims[i + 1:])) for i in range(len(self.dims))), O.BF16)
            O.gemm(self.x, self.w, c, self.bias)
            self._c = c.buf
            assert n == self.dims[-1]
        return self._c

    def _after_act(self, bits: np.ndarray) -> np.ndarray:
        t = O.Tensor((bits.size,), (1,), O.BF16, bits.copy())
        if self.act != O.ACT_NONE:
            O.activation(t, self.act, self.act_alpha, self.act_beta)
        return t.buf

    def _after_bin(self, bits: np.ndarray, idx: np.ndarray) -> np.ndarray:
        t = O.Tensor((bits.size,), (1,), O.BF16, bits.copy())
        if self.binary != O.BIN_NONE:
            s = O.Tensor((idx.size,), (1,), self.src.dtype, self.src.buf[idx].copy())
            O.binary(t, s, self.binary, self.gamma)
        return t.buf

    def __call__(self, idx: np.ndarray, got: np.ndarray) -> np.ndarray:
        """Boolean mask over idx: which of those elements the one-ulp moves explain (and the counts per stage)."""
        c = self._stage0()[idx]
        ok = np.zeros(idx.size, dtype=bool)
        for moved in _bf16_neighbours(c):
            hit = self._after_bin(self._after_act(moved), idx) == got
            self.counts["gemm stage"] += int(np.count_nonzero(hit & ~ok))
            ok |= hit
        if self.act != O.ACT_NONE:
            for moved in _bf16_neighbours(self._after_act(c)):
                hit = self._after_bin(moved, idx) == got
                self.counts["activation stage"] += int(np.count_nonzero(hit & ~ok))
                ok |= hit
        return ok


def explainer(dt, x, w, bias, dims, act=None, act_alpha=0.0, act_beta=0.0, binary=None, src=None, gamma=1.0):
    """A PostOpsExplainer for a bf16 output of the Linear chain (None for other output types)."""
    if dt != O.BF16:
        return None
    return PostOpsExplainer(x, w, bias, dims, act, act_alpha, act_beta, binary, src, gamma)


def compare(got_buf: np.ndarray, ref_buf: np.ndarray, dt: int, what: str = "", explain=None):
    """Asserts the north-star tolerance (bit-exact for integer outputs); returns (max-normalised error, bit-exact
    fraction).

    Non-finite oracle values must be matched in kind: NaN by NaN, +Inf by +Inf, -Inf by -Inf. bf16: every element must
    be within 1e-2 rel + 1e-2 abs, except elements that `explain` (a PostOpsExplainer) shows to be the oracle's own
    result with one intermediate moved by one bf16 ulp; their number is printed."""
    if dt in (O.S32, O.S8, O.U8):
        bad = np.nonzero(got_buf != ref_buf)[0]
        assert bad.size == 0, (f"{what}: {bad.size} of {got_buf.size} integer outputs differ, first at {bad[0]}: "
                               f"got {got_buf[bad[0]]} want {ref_buf[bad[0]]}")
        return 0.0, 1.0
    g = O.to_f32(got_buf, dt).astype(np.float64)
    r = O.to_f32(ref_buf, dt).astype(np.float64)
    assert g.shape == r.shape
    fin = np.isfinite(r)
    nan_r, nan_g = np.isnan(r), np.isnan(g)
    assert np.array_equal(nan_r, nan_g), f"{what}: NaN mismatch at {np.nonzero(nan_r != nan_g)[0][:8]}"
    inf_r = np.isinf(r)
    assert np.array_equal(inf_r, np.isinf(g)), f"{what}: Inf mismatch at {np.nonzero(inf_r != np.isinf(g))[0][:8]}"
    assert np.array_equal(np.sign(r[inf_r]), np.sign(g[inf_r])), f"{what}: an infinity has the wrong sign"
    d = np.abs(g[fin] - r[fin])
    scale = max(np.max(np.abs(r[fin])) if r[fin].size else 0.0, 1e-30)
    maxnorm = float(np.max(d) / scale) if d.size else 0.0
    exact = float(np.mean(got_buf == ref_buf)) if got_buf.size else 1.0
    if dt == O.F32:
        assert maxnorm <= FP32_MAXNORM_TOL, f"{what}: fp32 max-normalised error {maxnorm:.3e} > {FP32_MAXNORM_TOL}"
    elif dt == O.F16:
        assert maxnorm <= F16_TOL, f"{what}: f16 max-normalised error {maxnorm:.3e} > {F16_TOL}"
        bad = np.nonzero(d > (F16_TOL + F16_TOL * np.abs(r[fin])))[0]
        assert bad.size == 0, (f"{what}: {bad.size} of {got_buf.size} f16 elements outside 2e-3 rel/abs, first at "
                               f"{bad[0]}: got {g[fin][bad[0]]} want {r[fin][bad[0]]}")
    else:
        assert maxnorm <= BF16_MAXNORM_TOL, f"{what}: max-normalised error {maxnorm:.3e} > {BF16_MAXNORM_TOL}"
        bad = np.nonzero(fin)[0][d > (BF16_ATOL + BF16_RTOL * np.abs(r[fin]))]
        if bad.size:
            assert explain is not None, (f"{what}: {bad.size} of {got_buf.size} elements outside 1e-2 rel/abs, first at "
                                         f"{bad[0]}: got {g[bad[0]]} want {r[bad[0]]}")
            ok = explain(bad, got_buf[bad])
            left = bad[~ok]
            assert left.size == 0, (f"{what}: {left.size} of {bad.size} elements outside 1e-2 rel/abs are not one "
                                    f"bf16 ulp of an intermediate away, first at {left[0]}: got {g[left[0]]} "
                                    f"want {r[left[0]]}")
            print(f"{what}: {bad.size} of {got_buf.size} elements outside 1e-2 rel/abs, each the oracle with one "
                  f"intermediate moved by one bf16 ulp ({explain.counts})")
    return maxnorm, exact


def dense_rows(t: O.Tensor, rows) -> O.Tensor:
    """Rows of a dense row-major tensor viewed as [rows, last dim]."""
    last = t.dims[-1]
    buf = t.buf.reshape(-1, last)[rows].copy().reshape(-1)
    return O.Tensor((len(rows), last), (last, 1), t.dtype, buf)


def sample_rows(m: int, count: int, seed: int = 1234, band: int = 256) -> np.ndarray:
    """Rows to check of an m-row output: the edge rows, one row at a random offset inside every `band`-row band (so
    every 256-row tile row of the GEMM kernels is looked at), and random rows up to `count` in all."""
    rng = np.random.default_rng(seed)
    fixed = [0, 1, m // 2, m - 2, m - 1]
    strata = [b + int(rng.integers(0, min(band, m - b))) for b in range(0, m, band)]
    picked = np.unique(np.clip(np.array(fixed + strata), 0, m - 1))
    rest = rng.choice(m, size=max(0, min(count, m) - picked.size), replace=False)
    return np.unique(np.concatenate([picked, rest]))
