"""CPU checks of the parity helpers themselves: the non-finite matching of compare(), the one-ulp explainer of bf16
exceptions, and the stratified row sampling of the full-size tests. Mistakes are planted in oracle outputs."""
import numpy as np
import pytest

import oracle as O
from support import PostOpsExplainer, _bf16_neighbours, compare, sample_rows


def _gelu_residual_case(seed=3, M=24, Kd=64, N=40):
    rng = np.random.default_rng(seed)
    x = O.Tensor((M, Kd), (Kd, 1), O.BF16, O.from_f32_rne(rng.standard_normal(M * Kd).astype(np.float32), O.BF16))
    # weights large enough that |GEMM stage| reaches 4, where one bf16 ulp (2^-5) exceeds 1e-2 after cancellation
    w = O.Tensor((Kd, N), (1, Kd), O.BF16, O.from_f32_rne((rng.standard_normal(N * Kd) * 0.4).astype(np.float32),
                                                           O.BF16))
    r = O.Tensor((M, N), (N, 1), O.BF16, O.from_f32_rne(rng.standard_normal(M * N).astype(np.float32) * 3, O.BF16))
    y = O.empty((M, N), (N, 1), O.BF16)
    O.linear_postops(x, w, y, None, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, r)
    return x, w, r, y


def test_bf16_neighbours_step_one_ulp():
    up, down = _bf16_neighbours(np.array([0x0000, 0x8000, 0x3F80, 0xBF80, 0x7F7F], np.uint16))
    f = lambda b: O.to_f32(b, O.BF16)
    v = f(np.array([0x0000, 0x8000, 0x3F80, 0xBF80, 0x7F7F], np.uint16))
    assert np.all(f(up) > v) and np.all(f(down) < v)
    assert up[2] == 0x3F81 and down[2] == 0x3F7F and up[3] == 0xBF7F and down[3] == 0xBF81


def test_explainer_accepts_one_ulp_of_the_gemm_stage_only():
    x, w, r, y = _gelu_residual_case()
    M, N = y.dims
    # the GEMM stage of the oracle, then the same stages from a stage moved by one and by two ulps
    c = O.empty((M, N), (N, 1), O.BF16)
    O.gemm(x, w, c, None)
    big = np.nonzero(np.abs(O.to_f32(c.buf, O.BF16)) >= 4.0)[0]
    assert big.size > 0
    up, _ = _bf16_neighbours(c.buf)
    up2, _ = _bf16_neighbours(up)
    moved = {}
    for name, cs in (("one", up), ("two", up2)):
        t = O.Tensor((M * N,), (1,), O.BF16, cs.copy())
        O.activation(t, O.ACT_GELU_TANH)
        O.binary(t, O.Tensor((M * N,), (1,), O.BF16, r.buf.copy()), O.BIN_ADD)
        moved[name] = t.buf
    # plant: every element takes its one-ulp-moved value; compare() must accept with the explainer and not without
    planted = y.buf.copy()
    planted[big] = moved["one"][big]
    assert np.any(planted != y.buf)
    why = PostOpsExplainer(x, w, None, (M, N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=r)
    outside = np.abs(O.to_f32(planted, O.BF16) - O.to_f32(y.buf, O.BF16)) > 1e-2 + 1e-2 * np.abs(O.to_f32(y.buf, O.BF16))
    if outside.any():
        with pytest.raises(AssertionError):
            compare(planted, y.buf, O.BF16, "planted one ulp, no explainer")
    compare(planted, y.buf, O.BF16, "planted one ulp", explain=why)
    # two ulps is not explained
    planted2 = y.buf.copy()
    planted2[big] = moved["two"][big]
    outside2 = np.abs(O.to_f32(planted2, O.BF16) - O.to_f32(y.buf, O.BF16)) > 1e-2 + 1e-2 * np.abs(O.to_f32(y.buf, O.BF16))
    assert outside2.any()
    with pytest.raises(AssertionError, match="not one bf16 ulp"):
        compare(planted2, y.buf, O.BF16, "planted two ulps", explain=PostOpsExplainer(
            x, w, None, (M, N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=r))


def test_compare_matches_non_finite_kinds():
    ref = O.from_f32_rne(np.array([np.inf, -np.inf, np.nan, 1.0], np.float32), O.BF16)
    compare(ref.copy(), ref, O.BF16, "same")
    for i, v in ((0, -np.inf), (1, np.inf), (2, np.inf), (0, np.nan)):
        got = ref.copy()
        got[i] = O.from_f32_rne(np.array([v], np.float32), O.BF16)[0]
        with pytest.raises(AssertionError):
            compare(got, ref, O.BF16, "planted")


@pytest.mark.parametrize("m,bands", [(2048, 8), (4096, 16), (16384, 64), (300, 2)])
def test_sample_rows_cover_every_band(m, bands):
    rows = sample_rows(m, 24)
    assert set(np.unique(rows // 256)) == set(range(bands))
    assert {0, 1, m - 2, m - 1} <= set(rows.tolist())
