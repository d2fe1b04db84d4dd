"""Pins the CPU oracle (oracle/oracle.c) against known answers and independent computations.

Each check is chosen so that a plausible mistake in the oracle fails it:
  - SplitMix64: the generator's published first output for seed 0, and its mean/std as a distribution;
  - bf16 rounding: hand-picked bit patterns (ties to even both ways, the 0x7f7f8000 overflow boundary,
    +-0, +-Inf, NaN, subnormals) and truncation; f16 rounding against numpy's IEEE float16 cast;
  - activations: closed forms evaluated in float64 (numpy / math.erf), special values, saturation, and the
    |gelu_tanh - gelu_erf| <= 4.8e-4 bound;
  - GEMM: integer-valued operands (every product and partial sum exact in f32, so the result is exact in any
    summation order) against numpy int64 matmuls, for every weight layout, batch broadcast and bias kind;
    random operands against a float64 numpy matmul rounded once;
  - composed operators: the rounding points of KuDNN's separate passes (RNE after the GEMM, truncation after a
    bf16 activation, RNE after a residual op), restated in numpy on exactly representable data;
  - the reference gtest's own oracle (test/dnn/llt/gtest/src/linear_activation_gtest.cpp:24-88, bf16 sums
    accumulated in bf16) and its acceptance test (compareEle, :120-148): the oracle must pass the reference's
    own check against the reference's own oracle.
"""
import math

import numpy as np
import pytest

import oracle as O

F32, BF16, F16 = O.F32, O.BF16, O.F16


def f32(x):
    return np.float32(x)


def bits(x):
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def from_bits(u):
    return np.array([u], dtype=np.uint32).view(np.float32)[0]


def dense(dims, dt, layout="AB"):
    """Dense logical strides for a layout given by its letters (mirrors KuDNN min strides)."""
    nd = len(dims)
    order = [ord(c) - ord("A") for c in layout]  # physical position -> logical dim
    strides = [0] * nd
    run = 1
    for p in range(nd - 1, -1, -1):
        d = order[p]
        strides[d] = run
        run *= dims[d]
    strides = [0 if dims[i] == 1 else strides[i] for i in range(nd)]
    return tuple(strides)


def tensor_from(arr, dt, layout=None):
    """Tensor whose logical values are `arr` (rounded RNE into dt), stored in `layout`."""
    arr = np.asarray(arr, dtype=np.float32)
    layout = layout or "ABCDE"[: arr.ndim]
    st = dense(arr.shape, dt, layout)
    t = O.empty(arr.shape, st, dt)
    vals = O.from_f32_rne(arr, dt).reshape(arr.shape)
    view = np.lib.stride_tricks.as_strided(t.buf, shape=arr.shape, strides=[s * t.buf.itemsize for s in st])
    view[...] = vals
    return t


# ---------------------------------------------------------------------------------------------------
# inputs


def test_splitmix64_published_vector():
    # first output of SplitMix64 seeded with 0 is 0xE220A8397B1DCDAF; the oracle takes its top 53 bits
    t = O.fill((1,), (1,), F32, 0, "uniform", 0.0, 1.0)
    assert t.buf[0] == f32((0xE220A8397B1DCDAF >> 11) / 2.0**53)


def test_fill_distributions():
    n = 200_000
    u = O.fill((n,), (1,), F32, 5, "uniform", -1.0, 1.0).buf
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 0.01 and abs(u.var() - 1.0 / 3.0) < 0.01
    g = O.fill((n,), (1,), F32, 6, "normal", 0.0, 2.0).buf
    assert abs(g.mean()) < 0.02 and abs(g.std() - 2.0) < 0.02
    b = O.fill((1000,), (1,), BF16, 7, "normal", 0.0, 1.0).buf
    g32 = O.fill((1000,), (1,), F32, 7, "normal", 0.0, 1.0).buf
    assert np.array_equal(b, O.from_f32_rne(g32, BF16))  # bf16 tensors are the RNE of the f32 samples


# ---------------------------------------------------------------------------------------------------
# bf16 / f16 conversions (Service::ConvertFp32ToBf16 RNE; vml truncation; SvF32CvtBf16InfSpecial)

RNE_CASES = [
    (0x3F800000, 0x3F80),  # 1.0
    (0x3F808000, 0x3F80),  # tie, even mantissa stays
    (0x3F818000, 0x3F82),  # tie, odd mantissa rounds up
    (0x3F808001, 0x3F81),  # above the tie
    (0x3F807FFF, 0x3F80),  # below the tie
    (0xBF818000, 0xBF82),  # negative tie rounds away from zero to even
    (0x7F7F8000, 0x7F80),  # largest finite f32 above max bf16 rounds to +Inf
    (0x7F7F7FFF, 0x7F7F),
    (0x00000000, 0x0000),
    (0x80000000, 0x8000),
    (0x7F800000, 0x7F80),
    (0xFF800000, 0xFF80),
    (0x00018000, 0x0002),  # subnormal tie, odd -> up
    (0x00008000, 0x0000),  # subnormal tie, even -> stays
]


@pytest.mark.parametrize("u,want", RNE_CASES)
def test_bf16_rne_bits(u, want):
    assert O.lib().oracle_f32_to_bf16_rne(from_bits(u)) == want


def test_bf16_rne_nan_stays_quiet_nan():
    for u in (0x7FC00000, 0x7F800001, 0xFFA00000):
        h = O.lib().oracle_f32_to_bf16_rne(from_bits(u))
        assert (h & 0x7F80) == 0x7F80 and (h & 0x7F) != 0 and (h & 0x40)
        assert (h & 0x8000) == ((u >> 16) & 0x8000)


def test_bf16_rne_matches_numpy_restatement():
    x = np.random.default_rng(0).standard_normal(100_000).astype(np.float32) * 1e3
    want = O.from_f32_rne(x, BF16)
    got = np.array([O.lib().oracle_f32_to_bf16_rne(v) for v in x[:2000]], dtype=np.uint16)
    assert np.array_equal(got, want[:2000])


def test_bf16_trunc_and_inf_special():
    lib = O.lib()
    assert lib.oracle_f32_to_bf16_trunc(from_bits(0x3F81FFFF)) == 0x3F81
    assert lib.oracle_f32_to_bf16_trunc(from_bits(0xBF81FFFF)) == 0xBF81
    assert lib.oracle_f32_to_bf16_trunc_inf(from_bits(0x7F7F8000)) == 0x7F80
    assert lib.oracle_f32_to_bf16_trunc_inf(from_bits(0xFF7FFFFF)) == 0xFF80
    assert lib.oracle_f32_to_bf16_trunc_inf(from_bits(0x7F7F7FFF)) == 0x7F7F
    assert lib.oracle_f32_to_bf16_trunc_inf(from_bits(0x7FC00001)) == 0x7FC0


def test_f16_matches_ieee():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(5000) * s for s in (1e-6, 1e-3, 1.0, 1e3, 7e4)]).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, np.inf, -np.inf])])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.lib().oracle_f32_to_f16_rne(v) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)
    back = np.array([O.lib().oracle_f16_to_f32(h) for h in want], dtype=np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


# ---------------------------------------------------------------------------------------------------
# activations (vml FWD kernels)

XS = np.concatenate([np.linspace(-12, 12, 2001), [-100.0, -88.0, -87.5, 87.5, 88.0, 100.0]]).astype(np.float32)


def act(kind, x, alpha=0.0):
    x = np.asarray(x, dtype=np.float32)
    return np.array([O.act_f32(kind, float(v), alpha) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def test_relu_closed_form():
    for alpha in (0.0, 0.1, -2.0):
        y = act(O.ACT_RELU, XS, alpha)
        want = np.where(XS <= 0, XS * np.float32(alpha), XS)
        assert np.array_equal(y, want.astype(np.float32))
    assert math.copysign(1.0, O.act_f32(O.ACT_RELU, -3.0, 0.0)) == -1.0  # -3 * 0 = -0


def test_swish_closed_form_and_saturation():
    x64 = XS.astype(np.float64)
    for alpha in (1.0, 0.5, 2.0):
        y = act(O.ACT_SWISH, XS, alpha).astype(np.float64)
        want = x64 / (1.0 + np.exp(-alpha * x64))
        assert np.max(np.abs(y - want) / np.maximum(np.abs(want), 1e-30)) < 2e-6 or np.allclose(y, want, atol=1e-6)
    assert O.act_f32(O.ACT_SWISH, 0.0, 1.0) == 0.0
    assert O.act_f32(O.ACT_SWISH, -88.0, 1.0) == 0.0   # t = 88 > 87 -> sigmoid 0
    assert O.act_f32(O.ACT_SWISH, 88.0, 1.0) == 88.0   # t = -88 < -87 -> sigmoid 1
    assert O.act_f32(O.ACT_SWISH, 3.0, 0.0) == 1.5     # alpha 0 -> x/2


def test_gelu_closed_forms():
    x64 = XS.astype(np.float64)
    gt = act(O.ACT_GELU_TANH, XS).astype(np.float64)
    want_t = 0.5 * x64 * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x64 + 0.044715 * x64**3)))
    assert np.allclose(gt, want_t, rtol=2e-6, atol=2e-7)
    ge = act(O.ACT_GELU_ERF, XS).astype(np.float64)
    want_e = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in x64])
    assert np.allclose(ge, want_e, rtol=2e-6, atol=2e-7)
    assert O.act_f32(O.ACT_GELU_TANH, 0.0) == 0.0 and O.act_f32(O.ACT_GELU_ERF, 0.0) == 0.0
    assert O.act_f32(O.ACT_GELU_TANH, 30.0) == 30.0 and O.act_f32(O.ACT_GELU_TANH, -30.0) == 0.0
    assert np.max(np.abs(gt - ge)) <= 4.8e-4


# ---------------------------------------------------------------------------------------------------
# GEMM stage


def int_tensor(shape, rng, lo=-8, hi=8):
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("la,lb,lc", [("AB", "AB", "AB"), ("AB", "BA", "AB"), ("BA", "BA", "AB"), ("AB", "AB", "BA")])
def test_gemm_integer_exact_layouts(dt, la, lb, lc):
    rng = np.random.default_rng(2)
    M, K, N = 37, 53, 29
    A, B = int_tensor((M, K), rng), int_tensor((K, N), rng)
    a, b = tensor_from(A, dt, la), tensor_from(B, dt, lb)
    c = O.empty((M, N), dense((M, N), dt, lc), dt)
    O.gemm(a, b, c)
    want = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(c.logical(), O.to_f32(O.from_f32_rne(want, dt), dt).reshape(M, N))


@pytest.mark.parametrize("bias_shape", [(1, 1), (1, 24), (16, 1), (16, 24)])
def test_gemm_bias_kinds_alpha_beta(bias_shape):
    rng = np.random.default_rng(3)
    M, K, N = 16, 20, 24
    A, B, C0 = int_tensor((M, K), rng), int_tensor((K, N), rng), int_tensor((M, N), rng)
    bias = int_tensor(bias_shape, rng)
    a, b, c, x = tensor_from(A, F32), tensor_from(B, F32, "BA"), tensor_from(C0, F32), tensor_from(bias, F32)
    O.gemm(a, b, c, x, alpha=0.5, beta=2.0)
    want = 0.5 * (A.astype(np.int64) @ B.astype(np.int64)) + 2.0 * C0 + np.broadcast_to(bias, (M, N))
    np.testing.assert_array_equal(c.logical(), want.astype(np.float32))


def test_gemm_batch_broadcast():
    rng = np.random.default_rng(4)
    A = int_tensor((3, 2, 5, 7), rng)
    B = int_tensor((3, 1, 7, 6), rng)   # broadcast over dim 1
    bias = int_tensor((1, 1, 1, 6), rng)
    a, b, x = tensor_from(A, F32), tensor_from(B, F32), tensor_from(bias, F32)
    c = O.empty((3, 2, 5, 6), dense((3, 2, 5, 6), F32, "ABCD"), F32)
    O.gemm(a, b, c, x)
    want = np.matmul(A.astype(np.int64), B.astype(np.int64)) + bias
    np.testing.assert_array_equal(c.logical(), want.astype(np.float32))


def test_gemm_random_matches_float64_rounded_once():
    rng = np.random.default_rng(5)
    M, K, N = 48, 300, 40
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    a, b = tensor_from(A, F32), tensor_from(B, F32, "BA")
    c = O.empty((M, N), (N, 1), F32)
    O.gemm(a, b, c)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    got = c.logical()
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1   # double sums differ only in the last bits; one final rounding


def test_bf16_gemm_rounding_points():
    """bf16 C with bias: f32 sum + f32 bias then RNE (kudnn_gemm.cpp:208-221); without bias: bf16 alpha/beta."""
    rng = np.random.default_rng(6)
    M, K, N = 8, 16, 12
    A = (int_tensor((M, K), rng) / 8).astype(np.float32)      # exact in bf16
    B = (int_tensor((K, N), rng) / 16).astype(np.float32)
    bias = rng.standard_normal((1, N)).astype(np.float32)
    a, b, x = tensor_from(A, BF16), tensor_from(B, BF16, "BA"), tensor_from(bias, F32)
    c = O.empty((M, N), (N, 1), BF16)
    O.gemm(a, b, c, x)
    acc = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32) + bias
    np.testing.assert_array_equal(c.buf, O.from_f32_rne(acc.astype(np.float32), BF16).reshape(-1))
    # no bias: alpha is rounded to bf16 first (cblas_bgemm takes bf16 scalars)
    c2 = O.empty((M, N), (N, 1), BF16)
    O.gemm(a, b, c2, None, alpha=1.00390625)   # rounds to 1.0 in bf16 (tie to even)
    acc2 = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(c2.buf, O.from_f32_rne(acc2, BF16).reshape(-1))


# ---------------------------------------------------------------------------------------------------
# composed operators


def trunc_bf16(x):
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_linear_act_bf16_rounding_points():
    rng = np.random.default_rng(7)
    M, K, N = 10, 32, 14
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (rng.standard_normal((K, N)) * 0.2).astype(np.float32)
    a, b = tensor_from(A, BF16), tensor_from(B, BF16, "BA")
    x = tensor_from(np.zeros((1, N), np.float32), BF16)
    for kind, alpha in ((O.ACT_GELU_TANH, 0.0), (O.ACT_SWISH, 1.0), (O.ACT_GELU_ERF, 0.0), (O.ACT_RELU, 0.0)):
        c = O.empty((M, N), (N, 1), BF16)
        O.linear_act(a, b, c, x, kind, alpha)
        A_ = O.to_f32(O.from_f32_rne(A, BF16), BF16).reshape(M, K).astype(np.float64)
        B_ = O.to_f32(O.from_f32_rne(B, BF16), BF16).reshape(K, N).astype(np.float64)
        stage0 = O.to_f32(O.from_f32_rne((A_ @ B_).astype(np.float32), BF16), BF16)
        stage1 = act(kind, stage0, alpha)
        np.testing.assert_array_equal(c.buf, trunc_bf16(stage1).reshape(-1))


def test_linear_act_runs_activation_without_beta():
    # LinearActivationLayerFWD builds its activation from (kind, alpha) only (kudnn_linear_activationlayer.cpp:33):
    # LINEAR is alpha * x + 0 and HARDSIGMOID clip(alpha * x + 0, 0, 1), whereas the post-op chain applies beta.
    # Integer-valued f32 GEMM: every product and sum is exact, so the expected values are closed forms.
    rng = np.random.default_rng(9)
    M, K, N = 6, 8, 5
    A = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    a, b = tensor_from(A, F32), tensor_from(B, F32, "BA")
    G = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    c = O.empty((M, N), (N, 1), F32)
    O.linear_act(a, b, c, None, O.ACT_LINEAR, 2.0)
    np.testing.assert_array_equal(c.buf.reshape(M, N), 2.0 * G)
    O.linear_act(a, b, c, None, O.ACT_HARDSIGMOID, 0.125)
    np.testing.assert_array_equal(c.buf.reshape(M, N), np.clip(0.125 * G, 0.0, 1.0))
    y = O.empty((M, N), (N, 1), F32)
    O.linear_postops(a, b, y, None, O.ACT_LINEAR, 2.0, act_beta=0.5)
    np.testing.assert_array_equal(y.buf.reshape(M, N), 2.0 * G + 0.5)


@pytest.mark.parametrize("dt", [F32, BF16])
def test_linear_res_kinds(dt):
    rng = np.random.default_rng(8)
    M, K, N, L = 9, 12, 10, 7
    A, B = int_tensor((M, K), rng, -4, 4), int_tensor((K, N), rng, -4, 4)
    bias = int_tensor((1, N), rng)
    a, b, x = tensor_from(A, dt), tensor_from(B, dt, "BA"), tensor_from(bias, dt)
    Cw = (A.astype(np.int64) @ B.astype(np.int64) + bias).astype(np.float32)
    # RES_IDENTIAL / RES_EXT on integer data (exact)
    R = int_tensor((M, N), rng)
    for kind, gamma, want in ((O.RES_IDENTIAL, 3.0, Cw + R), (O.RES_EXT, 0.5, Cw + 0.5 * R)):
        c, lr = O.empty((M, N), (N, 1), dt), O.empty((M, N), (N, 1), dt)
        O.linear_res(a, b, c, x, tensor_from(R, dt), lr, kind, gamma)
        np.testing.assert_array_equal(c.logical(), Cw)
        np.testing.assert_array_equal(lr.logical(), O.to_f32(O.from_f32_rne(want, dt), dt).reshape(M, N))
    # RES_MUL is a matrix product C x res (kudnn_linear_res.cpp:188-190), not element-wise
    Rm = int_tensor((N, L), rng, -2, 2)
    c, lr = O.empty((M, N), (N, 1), dt), O.empty((M, L), (L, 1), dt)
    O.linear_res(a, b, c, x, tensor_from(Rm, dt), lr, O.RES_MUL, 1.0)
    want = Cw.astype(np.float64) @ Rm.astype(np.float64)
    np.testing.assert_array_equal(lr.logical(), O.to_f32(O.from_f32_rne(want.astype(np.float32), dt), dt).reshape(M, L))


def test_postops_chain_matches_composition():
    """The post-op chain equals LinearActivationLayerFWD followed by the element-wise op."""
    rng = np.random.default_rng(9)
    M, K, N = 6, 40, 9
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (rng.standard_normal((K, N)) * 0.1).astype(np.float32)
    S = rng.uniform(0.5, 1.5, (M, N)).astype(np.float32)
    a, b, s = tensor_from(A, BF16), tensor_from(B, BF16, "BA"), tensor_from(S, BF16)
    for binary in (O.BIN_ADD, O.BIN_MUL, O.BIN_EXT):
        y = O.empty((M, N), (N, 1), BF16)
        O.linear_postops(a, b, y, None, O.ACT_GELU_TANH, 0.0, binary, s, 0.25)
        c = O.empty((M, N), (N, 1), BF16)
        O.linear_act(a, b, c, None, O.ACT_GELU_TANH, 0.0)
        cv, sv = c.logical(), s.logical()
        # gamma = 0.25 is a power of two, so sv * gamma is exact and fma(sv, gamma, cv) == cv + sv * gamma
        want = {O.BIN_ADD: cv + sv, O.BIN_MUL: cv * sv, O.BIN_EXT: cv + sv * np.float32(0.25)}[binary]
        np.testing.assert_array_equal(y.buf, O.from_f32_rne(want.astype(np.float32), BF16).reshape(-1))


# ---------------------------------------------------------------------------------------------------
# the reference gtest's own oracle and acceptance test


def gtest_linear_activation_oracle(A, B, kind, dt):
    """linearActivationSimple (linear_activation_gtest.cpp:66-88): `T sum` accumulated in T (bf16 for bf16),
    then the activation of linear_activation_gtest.cpp:24-64 in T."""
    M, K = A.shape
    N = B.shape[1]
    if dt == F32:
        out = np.zeros((M, N), np.float32)
        for i in range(M):
            for j in range(N):
                s = np.float32(0)
                for k in range(K):
                    s = np.float32(s + A[i, k] * B[k, j])
                out[i, j] = s
    else:
        rt = lambda v: O.to_f32(O.from_f32_rne(np.float32([v]), BF16), BF16)[0]
        out = np.zeros((M, N), np.float32)
        for i in range(M):
            for j in range(N):
                s = np.float32(0)
                for k in range(K):
                    s = rt(np.float32(s + rt(np.float32(A[i, k] * B[k, j]))))
                out[i, j] = s
    x = out.astype(np.float64)
    if kind == O.ACT_RELU:
        y = np.maximum(x, 0.0)
    elif kind == O.ACT_SWISH:
        y = x / (1.0 + np.exp(-x))
    elif kind == O.ACT_GELU_TANH:
        y = 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x**3)))
    else:
        y = np.array([[0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in row] for row in x])
    return y.astype(np.float32)


def compare_ele(maxval, diff, dt, K):
    """compareEle (linear_activation_gtest.cpp:120-148 / matmul_gtest.cpp:162-199)."""
    eps = 1e-4 if dt == F32 else 1e-2 * K
    thr = 1e-4 if dt == F32 else eps
    e = diff / maxval if abs(maxval) > thr else diff
    return abs(e) <= eps


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("kind", [O.ACT_RELU, O.ACT_SWISH, O.ACT_GELU_TANH, O.ACT_GELU_ERF])
def test_oracle_passes_reference_gtest_check(dt, kind):
    rng = np.random.default_rng(10)
    M, K, N = 11, 20, 13   # the reference's 2-D case is 110x20x200; same K, fewer rows for a pure-Python loop
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    Bias = np.zeros((M, N), np.float32)
    a, b, x = tensor_from(A, dt), tensor_from(B, dt), tensor_from(Bias, dt)
    c = O.empty((M, N), (N, 1), dt)
    O.linear_act(a, b, c, x, kind, 1.0 if kind == O.ACT_SWISH else 0.0)
    Aq, Bq = a.logical(), b.logical()
    ref = gtest_linear_activation_oracle(Aq, Bq, kind, dt)
    maxval = float(max(Aq.max(), Bq.max()))
    got = c.logical()
    assert all(compare_ele(maxval, float(abs(g - r)), dt, K) for g, r in zip(got.ravel(), ref.ravel()))
    if dt == F32:  # the tolerance is loose; also require closeness to the f32 gtest oracle
        assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_cpu_baseline_matches_oracle():
    """The timed CPU baseline (naive loop) computes the same function as the oracle (within f32 order)."""
    rng = np.random.default_rng(11)
    M, K, N = 5, 64, 24
    X = O.from_f32_rne(rng.standard_normal((M, K)).astype(np.float32), BF16)
    W = O.from_f32_rne((rng.standard_normal((N, K)) * 0.05).astype(np.float32), BF16)
    R = O.from_f32_rne(rng.standard_normal((M, N)).astype(np.float32), BF16)
    bias = np.zeros(N, np.uint16)
    Y = np.zeros(M * N, np.uint16)
    O.cpu_baseline(BF16, M, N, K, X, W, bias, R, Y, O.ACT_GELU_TANH, 0.0, 1)
    a = O.Tensor((M, K), (K, 1), BF16, X)
    b = O.Tensor((K, N), (1, K), BF16, W)
    y = O.empty((M, N), (N, 1), BF16)
    O.linear_postops(a, b, y, O.Tensor((1, N), (0, 1), BF16, bias), O.ACT_GELU_TANH, 0.0, O.BIN_ADD,
                     O.Tensor((M, N), (N, 1), BF16, R))
    d = np.abs(O.to_f32(Y, BF16) - O.to_f32(y.buf, BF16))
    assert np.mean(d == 0) > 0.95 and d.max() <= 0.02


def test_cpu_baseline_residual_mul_matches_oracle():
    """The timed loop's multiplier form (C4: Y = (X W^T) * M2) against the oracle's BIN_MUL post-op."""
    rng = np.random.default_rng(12)
    M, K, N = 3, 96, 40
    X = O.from_f32_rne(rng.standard_normal((M, K)).astype(np.float32), BF16)
    W = O.from_f32_rne((rng.standard_normal((N, K)) * 0.05).astype(np.float32), BF16)
    R = O.from_f32_rne(rng.uniform(0.5, 1.5, (M, N)).astype(np.float32), BF16)
    Y = np.zeros(M * N, np.uint16)
    O.cpu_baseline(BF16, M, N, K, X, W, None, R, Y, O.ACT_NONE, 0.0, 1, r_mul=True)
    a = O.Tensor((M, K), (K, 1), BF16, X)
    b = O.Tensor((K, N), (1, K), BF16, W)
    y = O.empty((M, N), (N, 1), BF16)
    O.linear_postops(a, b, y, None, O.ACT_NONE, 0.0, O.BIN_MUL, O.Tensor((M, N), (N, 1), BF16, R))
    g, r = O.to_f32(Y, BF16), O.to_f32(y.buf, BF16)
    assert np.max(np.abs(g - r) / np.maximum(np.abs(r), 1e-3)) <= 2 ** -7  # one bf16 ulp of summation-order slack
