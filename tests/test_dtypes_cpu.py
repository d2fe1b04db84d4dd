"""CPU checks of the other dtype combinations: the oracle's s8 x s8 -> s32 GEMM against numpy's int64 matmul, and the
planner's choice of compute type (or refusal) for every combination of the reference's GEMM registry
(src/dnn/src/kudnn_gemm.cpp:590-601) and its widening / all-f32 fallback (ChooseImpl, :628-708). Plans are built
without a GPU; nothing here launches a kernel.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O


def _s8(rng, shape):
    return rng.integers(-128, 128, size=shape).astype(np.int8)


def _int8(rng, shape, dt):
    return _s8(rng, shape) if dt == O.S8 else rng.integers(0, 256, size=shape).astype(np.uint8)


@pytest.mark.parametrize("adt,bdt", [(O.S8, O.S8), (O.U8, O.S8), (O.S8, O.U8), (O.U8, O.U8)])
@pytest.mark.parametrize("wlayout", ["BA", "AB"])
@pytest.mark.parametrize("bias", [None, "1N", "M1", "MN"])
def test_oracle_int8_gemm_matches_int64_matmul(adt, bdt, wlayout, bias):
    # cblas_gemm_s8s8s32 / s8u8s32 / u8s8s32 / u8u8s32 with zero offsets: the exact integer sum, wrapped to int32
    rng = np.random.default_rng(7)
    M, Kd, N = 23, 301, 19
    a = _int8(rng, (M, Kd), adt)
    w = _int8(rng, (Kd, N), bdt)  # logical [K][N]
    A = O.Tensor((M, Kd), (Kd, 1), adt, a.reshape(-1).copy())
    if wlayout == "BA":
        B = O.Tensor((Kd, N), (1, Kd), bdt, w.T.reshape(-1).copy())
    else:
        B = O.Tensor((Kd, N), (N, 1), bdt, w.reshape(-1).copy())
    want = a.astype(np.int64) @ w.astype(np.int64)
    X = None
    if bias:
        bd = {"1N": (1, N), "M1": (M, 1), "MN": (M, N)}[bias]
        bv = rng.integers(-(1 << 30), 1 << 30, size=bd).astype(np.int32)
        st = (0 if bd[0] == 1 else bd[1], 0 if bd[1] == 1 else 1)
        X = O.Tensor(bd, st, O.S32, bv.reshape(-1).copy())
        want = want + bv.astype(np.int64)
    C = O.empty((M, N), (N, 1), O.S32)
    O.gemm(A, B, C, X)
    # two's-complement wrap into int32, as the integer epilogue does
    assert np.array_equal(C.buf.reshape(M, N), (want & 0xFFFFFFFF).astype(np.uint32).view(np.int32))


def test_oracle_s8_batched_broadcast():
    rng = np.random.default_rng(8)
    a = _s8(rng, (3, 2, 9, 40))
    w = _s8(rng, (1, 1, 40, 11))
    A = O.Tensor(a.shape, tuple(s // a.itemsize for s in a.strides), O.S8, a.reshape(-1).copy())
    B = O.Tensor(w.shape, (0, 0, 11, 1), O.S8, w.reshape(-1).copy())
    C = O.empty((3, 2, 9, 11), (198, 99, 11, 1), O.S32)
    O.gemm(A, B, C)
    want = np.einsum("xymk,kn->xymn", a.astype(np.int64), w[0, 0].astype(np.int64))
    assert np.array_equal(C.buf.reshape(3, 2, 9, 11), want.astype(np.int32))


def test_oracle_s8_refuses_scaled():
    A = O.Tensor((2, 2), (2, 1), O.S8, np.ones(4, np.int8))
    B = O.Tensor((2, 2), (2, 1), O.S8, np.ones(4, np.int8))
    C = O.empty((2, 2), (2, 1), O.S32)
    with pytest.raises(AssertionError):
        O.gemm(A, B, C, alpha=2.0)


def _plan(adt, bdt, cdt, biasdt=None, M=64, Kd=128, N=96, blay="BA"):
    return K.Gemm(K.desc([M, Kd], adt), K.desc([Kd, N], bdt, blay), K.desc([M, N], cdt),
                  K.desc([1, N], biasdt) if biasdt else None)


@pytest.mark.parametrize("combo,expect", [
    ((K.BF16, K.BF16, K.BF16, K.F32), "mfma_bf16"),
    ((K.BF16, K.BF16, K.F32, K.F32), "mfma_bf16"),
    ((K.F16, K.F16, K.F16, K.F16), "mfma_f16"),
    ((K.F16, K.F16, K.F32, K.F32), "mfma_f16"),
    ((K.F16, K.S8, K.F16, K.F32), "mfma_f16"),
    ((K.F16, K.U8, K.F16, K.F32), "mfma_f16"),
    ((K.S8, K.S8, K.S32, K.S32), "mfma_s8"),
    ((K.S8, K.S8, K.S32, None), "mfma_s8"),
    ((K.U8, K.S8, K.S32, K.S32), "mfma_s8"),
    ((K.S8, K.U8, K.S32, K.S32), "mfma_s8"),
    ((K.U8, K.U8, K.S32, None), "mfma_s8"),
    ((K.F32, K.F32, K.F32, K.F32), "mfma_f32"),
    ((K.S8, K.S8, K.F32, K.F32), "mfma_f32"),
    ((K.BF16, K.F16, K.F32, None), "mfma_f32"),
])
def test_planner_compute_type(combo, expect):
    p = _plan(*combo)
    assert expect in p.describe(), p.describe()


@pytest.mark.parametrize("combo,expect", [
    # ChooseImpl's all-f32 fallback (:673-705): f32 arithmetic, then ConvertFp32ToS32 / ToS8 / ToU8
    ((K.S8, K.S8, K.S8, None), "mfma_f32"),
    ((K.U8, K.U8, K.U8, None), "mfma_f32"),
    ((K.F32, K.F32, K.S32, None), "mfma_f32"),
    ((K.S8, K.S8, K.S32, K.F32), "mfma_f32"),
    ((K.S8, K.S8, K.S32, K.U8), "mfma_f32"),
    ((K.F32, K.F32, K.F32, K.S32), "mfma_f32"),
    ((K.BF16, K.BF16, K.S8, None), "mfma_bf16"),
    ((K.BF16, K.BF16, K.BF16, K.S32), "mfma_bf16"),
    ((K.F16, K.F16, K.U8, None), "mfma_f16"),
    # the wider-type match of an s8 bias into the integer GEMMs (:655-671): exact int32
    ((K.S8, K.S8, K.S32, K.S8), "mfma_s8"),
    ((K.U8, K.S8, K.S32, K.S8), "mfma_s8"),
])
def test_planner_integer_fallback_compute_type(combo, expect):
    p = _plan(*combo)
    assert expect in p.describe(), p.describe()


def test_linear_operators_refuse_integer_outputs():
    # the reference activates an integer C through ReorderLayer, and AddOps reads only floating tensors
    a, b = K.desc([64, 128], K.F32), K.desc([128, 96], K.F32, "BA")
    for cdt in (K.S8, K.U8, K.S32):
        c = K.desc([64, 96], cdt)
        with pytest.raises(K.KudnnError) as e:
            K.LinearActivation(a, b, c, None, 0.0, 0.0, K.ACT_RELU)
        assert e.value.status == K.UNSUPPORTED
        with pytest.raises(K.KudnnError) as e:
            K.LinearPostOps(a, b, c, None, act=K.ACT_RELU)
        assert e.value.status == K.UNSUPPORTED
        assert "mfma_f32" in K.LinearPostOps(a, b, c, None).describe()


_INT_RANGE = {O.S32: (-2147483648, 2147483647), O.S8: (-128, 127), O.U8: (0, 255)}


def _int_sat_expected(x, dt):
    # an independent statement of saturate-then-nearbyintf: round half to even first (numpy rint), clamp afterwards
    # (the same for every input: rounding never crosses a bound that saturation would not), NaN -> 0
    lo, hi = _INT_RANGE[dt]
    r = np.clip(np.rint(x.astype(np.float64)), lo, hi)
    r[np.isnan(x)] = 0
    return r.astype(np.int64)


@pytest.mark.parametrize("dt", [O.S32, O.S8, O.U8])
def test_oracle_int_conversion_pinned(dt):
    # ConvertFp32ToS32 / ToS8 / ToU8 (src/dnn/src/service.cpp:77-115) on a grid of quarter steps (every .5 a tie),
    # the bounds +-0.5, the f32 neighbours of +-2^31, and the non-finite inputs
    grid = np.arange(-300.0, 300.0, 0.25)
    specials = [np.nan, np.inf, -np.inf, -0.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 127.5, 128.5, 254.5, 255.5,
                256.5, -127.5, -128.5, -129.5, 8388607.5, -8388607.5, 16777217.0, 2.0 ** 31, -(2.0 ** 31),
                np.nextafter(np.float32(2.0 ** 31), np.float32(0)), np.nextafter(np.float32(-(2.0 ** 31)), np.float32(0)),
                3e9, -3e9, 1e38, -1e38]
    rnd = np.random.default_rng(11).standard_normal(2000) * np.float32(1e6)
    x = np.concatenate([grid, np.array(specials), rnd]).astype(np.float32)
    got = np.array([O.f32_to_int_sat(float(v), dt) for v in x], dtype=np.int64)
    want = _int_sat_expected(x, dt)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{x[bad[:5]]}: got {got[bad[:5]]} want {want[bad[:5]]}"
    # ties go to even, not away from zero
    assert O.f32_to_int_sat(2.5, dt) == 2 and O.f32_to_int_sat(3.5, dt) == 4


def _int_tensor(rng, dims, dt, lo, hi, layout_ba=False):
    """An integer-valued tensor of dtype dt, dense (or [K][N] stored N-major when layout_ba), and its float64 values."""
    v = rng.integers(lo, hi + 1, size=dims).astype(np.float64)

    def store(flat):
        if dt in _INT_RANGE:
            return flat.astype(O.storage_dtype(dt))
        return O.from_f32_rne(flat.astype(np.float32), dt)

    if layout_ba:
        t = O.Tensor(dims, (1, dims[0]), dt, store(v.T.reshape(-1)))
    else:
        st = [1] * len(dims)
        for i in range(len(dims) - 2, -1, -1):
            st[i] = st[i + 1] * dims[i + 1]
        t = O.Tensor(dims, tuple(st), dt, store(v.reshape(-1)))
    return t, v


@pytest.mark.parametrize("adt,bdt,cdt,xdt", [
    (O.F32, O.F32, O.S32, O.F32), (O.F32, O.F32, O.S8, None), (O.BF16, O.BF16, O.U8, O.F32),
    (O.F16, O.F16, O.S8, O.F16), (O.S8, O.S8, O.S8, None), (O.U8, O.S8, O.U8, O.S32), (O.S8, O.U8, O.S32, O.F32),
    (O.S8, O.S8, O.S32, O.U8), (O.F32, O.F32, O.F32, O.S32), (O.BF16, O.BF16, O.BF16, O.S8),
])
def test_oracle_all_f32_fallback_integer_exact(adt, bdt, cdt, xdt):
    # integer-valued operands keep every f32 partial sum exact, so alpha * AB + beta * C + bias is exact in float64;
    # alpha = beta = 0.5 put exact .5 ties in front of the conversion
    rng = np.random.default_rng(12)
    M, Kd, N = 13, 24, 11
    lo = 0 if adt == O.U8 else -8
    A, a = _int_tensor(rng, (M, Kd), adt, lo, 8)
    B, b = _int_tensor(rng, (Kd, N), bdt, 0 if bdt == O.U8 else -8, 8, layout_ba=True)
    X, x = (None, 0.0)
    if xdt is not None:
        X, x = _int_tensor(rng, (1, N), xdt, 0 if xdt == O.U8 else -60, 60)
        X = O.Tensor((1, N), (0, 1), xdt, X.buf)
    cint = cdt in _INT_RANGE
    C, c = _int_tensor(rng, (M, N), cdt, 0 if cdt == O.U8 else -100, 100)
    v = 0.5 * (a @ b) + 0.5 * c + x
    O.gemm(A, B, C, X, alpha=0.5, beta=0.5)
    if cint:
        assert np.array_equal(C.buf.reshape(M, N).astype(np.int64), _int_sat_expected(v.astype(np.float32), cdt))
        assert np.any(np.abs(v - np.trunc(v)) == 0.5), "the case has no .5 tie"
    else:
        want = O.to_f32(O.from_f32_rne(v.reshape(-1).astype(np.float32), cdt), cdt)
        assert np.array_equal(O.to_f32(C.buf, cdt), want)


def test_oracle_s8_bias_widened_exactly():
    # s8 x s8 -> s32 with an s8 bias: the integer GEMM with the bias widened (ChooseImpl's wider-type match)
    rng = np.random.default_rng(13)
    a, w = _s8(rng, (9, 700)), _s8(rng, (700, 5))
    bv = _s8(rng, (1, 5))
    A = O.Tensor((9, 700), (700, 1), O.S8, a.reshape(-1).copy())
    B = O.Tensor((700, 5), (5, 1), O.S8, w.reshape(-1).copy())
    X = O.Tensor((1, 5), (0, 1), O.S8, bv.reshape(-1).copy())
    C = O.empty((9, 5), (5, 1), O.S32)
    O.gemm(A, B, C, X)
    assert np.array_equal(C.buf.reshape(9, 5), a.astype(np.int64) @ w.astype(np.int64) + bv.astype(np.int64))


def test_u8_operands_are_packed_shifted():
    # a u8 operand runs on the s8 MFMA shifted by -128: both operands are packed (the correction terms are row sums
    # over the packed layout)
    for combo in ((K.U8, K.S8, K.S32, K.S32), (K.S8, K.U8, K.S32, None), (K.U8, K.U8, K.S32, K.S32)):
        d = _plan(*combo).describe()
        assert "mfma_s8" in d and "packA" in d and "packB" in d, d


def test_integer_gemm_only_through_gemm():
    a, b, c = K.desc([64, 128], K.S8), K.desc([128, 96], K.S8, "BA"), K.desc([64, 96], K.S32)
    with pytest.raises(K.KudnnError):
        K.LinearActivation(a, b, c, None, 0.0, 0.0, K.ACT_RELU)
    with pytest.raises(K.KudnnError):
        K.LinearPostOps(a, b, c, None, act=K.ACT_RELU)
    assert "mfma_s8" in K.LinearPostOps(a, b, c, None).describe()


def test_s8_small_m_uses_mfma_not_skinny():
    # the skinny (decode) kernels are 16-bit only; an s8 GEMM with M <= 16 runs on the 4-wave MFMA kernel
    p = _plan(K.S8, K.S8, K.S32, None, M=4, Kd=256, N=512)
    assert "mfma_s8_128x128" in p.describe(), p.describe()
    p = _plan(K.F16, K.F16, K.F16, None, M=1, Kd=256, N=512)
    assert "skinny_f16_gemv_row" in p.describe(), p.describe()
