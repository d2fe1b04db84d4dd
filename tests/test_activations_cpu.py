"""CPU pinning of the oracle's activation kinds (all of the reference's forward table,
src/dnn/src/kudnn_eltwise.cpp:333-400) against numpy closed forms in float64, their special values and parameter
conventions, and the bf16 store rule of each kind (truncation, overflow-to-Inf first, or RNE for ELU_DST).
"""
import math

import numpy as np
import pytest

import oracle as O

XS = np.array([-7.5, -3.0, -1.0, -0.6, -0.1, 0.0, 0.05, 0.4, 1.0, 2.5, 6.0], dtype=np.float32)


def act(kind, x, alpha=0.0, beta=0.0):
    return np.array([O.act_f32(kind, float(v), alpha, beta) for v in np.ravel(x)], dtype=np.float32)


def close(got, want, rtol=4e-6, atol=1e-7):
    want = np.asarray(want, dtype=np.float64)
    assert np.allclose(got.astype(np.float64), want, rtol=rtol, atol=atol, equal_nan=True), (got, want)


def test_unary_closed_forms():
    x = XS.astype(np.float64)
    close(act(O.ACT_ABS, XS), np.abs(x))
    close(act(O.ACT_EXP, XS), np.exp(x))
    close(act(O.ACT_SQUARE, XS), x * x)
    close(act(O.ACT_TANH, XS), np.tanh(x))
    close(act(O.ACT_SIGMOID, XS), 1.0 / (1.0 + np.exp(-x)))
    pos = XS[XS > 0].astype(np.float64)
    close(act(O.ACT_LOG, XS[XS > 0]), np.log(pos))
    close(act(O.ACT_SQRT, XS[XS > 0]), np.sqrt(pos))
    # mish = x * tanh(softplus(x)); the reference's ((e^x+1)^2 - 1) / ((e^x+1)^2 + 1) cancels in f32 for very negative
    # x (relative 1e-4 at x = -7.5, absolute 5e-7)
    close(act(O.ACT_MISH, XS), x * np.tanh(np.log1p(np.exp(x))), rtol=2e-5, atol=1e-6)


def test_unary_special_values():
    assert math.isnan(O.act_f32(O.ACT_LOG, -1.0)) and O.act_f32(O.ACT_LOG, 0.0) == -math.inf
    assert math.isnan(O.act_f32(O.ACT_SQRT, -1.0))
    assert O.act_f32(O.ACT_EXP, 0.0) == 1.0 and O.act_f32(O.ACT_SIGMOID, 0.0) == 0.5
    assert O.act_f32(O.ACT_TANH, 0.0) == 0.0 and O.act_f32(O.ACT_MISH, 0.0) == 0.0
    assert O.act_f32(O.ACT_MISH, 60.0) == 60.0  # exponent capped, the ratio is 1
    # ROUND is nearbyint: ties to even
    got = act(O.ACT_ROUND, np.array([0.5, 1.5, 2.5, -0.5, -1.5, 2.4999998, 2.5000002], np.float32))
    assert got.tolist() == [0.0, 2.0, 2.0, -0.0, -2.0, 2.0, 3.0]


def test_parameterised_closed_forms():
    x = XS.astype(np.float64)
    close(act(O.ACT_LINEAR, XS, 1.5, -0.25), 1.5 * x - 0.25)
    close(act(O.ACT_POW, XS, 2.0, 3.0), 2.0 * x ** 3)
    close(act(O.ACT_POW, XS[XS > 0], 0.5, 0.5), 0.5 * np.sqrt(XS[XS > 0].astype(np.float64)))
    assert math.isnan(O.act_f32(O.ACT_POW, -2.0, 1.0, 0.5))
    close(act(O.ACT_HARDSIGMOID, XS, 0.2, 0.5), np.clip(0.2 * x + 0.5, 0.0, 1.0))
    close(act(O.ACT_HARDSWISH, XS, 1.0 / 6.0, 0.5), x * np.clip(x / 6.0 + 0.5, 0.0, 1.0))
    close(act(O.ACT_ELU, XS, 1.3), np.where(x > 0, x, 1.3 * np.expm1(x)), rtol=2e-6, atol=4e-7)
    close(act(O.ACT_ELU_DST, XS, 1.3), np.where(x > 0, x, 1.3 * np.expm1(x)))
    close(act(O.ACT_SRELU, XS, 2.0), np.log1p(np.exp(2.0 * x)) / 2.0, rtol=2e-6)


def test_parameter_conventions_and_edges():
    # CLIP: x <= alpha -> alpha, x > beta -> beta; CLIP_V2 takes beta when x >= beta (the same value)
    assert act(O.ACT_CLIP, np.array([-1.0, -0.5, 0.2, 0.7, 1.0], np.float32), -0.5, 0.7).tolist() == \
        pytest.approx([-0.5, -0.5, 0.2, 0.7, 0.7])
    assert act(O.ACT_CLIP_V2, np.array([-1.0, 0.2, 0.7, 1.0], np.float32), -0.5, 0.7).tolist() == \
        pytest.approx([-0.5, 0.2, 0.7, 0.7])
    assert math.isnan(O.act_f32(O.ACT_CLIP, math.nan, -1.0, 1.0))
    # HARDSIGMOID is minnm / maxnm: a NaN input gives 1; HARDSWISH keeps the NaN
    assert O.act_f32(O.ACT_HARDSIGMOID, math.nan, 0.2, 0.5) == 1.0
    assert math.isnan(O.act_f32(O.ACT_HARDSWISH, math.nan, 0.2, 0.5))
    # SRELU: alpha*x at or above expf's overflow bound returns x itself
    assert O.act_f32(O.ACT_SRELU, 50.0, 2.0) == 50.0
    assert O.act_f32(O.ACT_SRELU, 0.0, 2.0) == pytest.approx(math.log(2.0) / 2.0)
    # ELU's negative branch is alpha*e^x - alpha (fused)
    assert O.act_f32(O.ACT_ELU, -50.0, 2.0) == -2.0


def _bf16_act(kind, x_bits, alpha=0.0, beta=0.0):
    buf = np.array([x_bits], dtype=np.uint16)
    t = O.Tensor((1,), (1,), O.BF16, buf)
    assert O.lib().oracle_activation(t.otensor(), t.ptr(), kind, alpha, beta) == 0
    return int(buf[0])


def test_bf16_store_rule_per_kind():
    big = 0x7F7F  # largest finite bf16, 3.3895e38
    # LINEAR and POW send results at or above 0x7f7f8000 to Inf before truncating
    assert _bf16_act(O.ACT_LINEAR, big, 1.002, 0.0) == 0x7F80
    assert _bf16_act(O.ACT_LINEAR, big, -1.002, 0.0) == 0xFF80
    assert _bf16_act(O.ACT_POW, big, 1.002, 1.0) == 0x7F80
    # below the boundary every kind truncates: 1.3 * 1.0 = 1.2999999523 (0x3fa66666) -> 0x3fa6
    one = 0x3F80
    assert _bf16_act(O.ACT_LINEAR, one, 1.3, 0.0) == 0x3FA6
    assert _bf16_act(O.ACT_SQUARE, 0x3F91, 0.0, 0.0) == 0x3FA4  # 1.1328125^2 = 1.2833 (0x3fa44400)
    # ELU_DST rounds to nearest even: expm1(-1) = -0.63212055 (0xbf21d2aa) -> 0xbf22; ELU truncates -> 0xbf21
    m_one = 0xBF80
    assert _bf16_act(O.ACT_ELU_DST, m_one, 1.0) == 0xBF22
    assert _bf16_act(O.ACT_ELU, m_one, 1.0) == 0xBF21
