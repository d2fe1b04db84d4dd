"""GPU parity of the other dtype combinations of the primitive (the reference's GEMM registry,
src/dnn/src/kudnn_gemm.cpp:590-601): f16 x f16 (cblas_hgemm / cblas_shgemm), f16 x s8 (W8A16: the weight converted
to f16, :341-372) and s8 x s8 -> s32 (W8A8, cblas_gemm_s8s8s32, :243-264), each on its own MFMA kernels with the same
epilogue. ChooseImpl's all-f32 fallback into integer outputs (:673-705) and integer bias / C around a float sum run on the same
kernels with an element-wise epilogue. Integer results are compared bit for bit (the fallback on integer-valued operands,
whose f32 sums are exact in any order); f16 results within 2e-3 max-normalised.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, from_device, zeros_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()


@pytest.fixture
def force_pingpong(monkeypatch):
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")


# ---------------------------------------------------------------------------------------------------
# s8 x s8 -> s32


def run_s8(M, N, Kd, wlayout="BA", bias_dims=None, seed=0, expect=None, batch=None):
    lead = list(batch) if batch else []
    x = Case(lead + [M, Kd], O.S8, seed=seed, lo=-128, hi=127)
    w = Case(lead + [Kd, N], O.S8, wlayout if not batch else None, seed=seed + 1, lo=-128, hi=127)
    c = Case(lead + [M, N], O.S32, zero=True)
    b = Case(bias_dims, O.S32, seed=seed + 2, lo=-(1 << 24), hi=1 << 24) if bias_dims else None
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc if b else None)
    if expect:
        assert expect in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device() if b else None)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref, b.t if b else None)
    compare(from_device(dc, O.S32), ref.buf, O.S32, plan.describe())
    return plan


@pytest.mark.parametrize("mnk", [(64, 64, 128), (300, 260, 256), (17, 33, 24), (5, 48, 64), (1, 70, 300), (256, 384, 1024)])
@pytest.mark.parametrize("wlayout", ["BA", "AB"])
def test_s8s8s32_shapes_layouts(mnk, wlayout):
    M, N, Kd = mnk
    run_s8(M, N, Kd, wlayout, bias_dims=[1, N], seed=200, expect="mfma_s8")


@pytest.mark.parametrize("bias", [None, "1N", "M1", "MN"])
def test_s8s8s32_bias_kinds(bias):
    M, N, Kd = 96, 80, 256
    dims = {"1N": [1, N], "M1": [M, 1], "MN": [M, N]}.get(bias)
    run_s8(M, N, Kd, bias_dims=dims, seed=210)


@pytest.mark.parametrize("mnk", [(256, 256, 128), (300, 520, 384), (40, 600, 256)])
def test_s8s8s32_pingpong(force_pingpong, mnk):
    M, N, Kd = mnk
    run_s8(M, N, Kd, bias_dims=[1, N], seed=220, expect="mfma_s8_pingpong")


def test_s8s8s32_batched_broadcast_weight():
    x = Case([3, 40, 256], O.S8, seed=230, lo=-128, hi=127)
    w = Case([1, 256, 72], O.S8, seed=231, lo=-128, hi=127)
    c = Case([3, 40, 72], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref)
    compare(from_device(dc, O.S32), ref.buf, O.S32, plan.describe())


def test_s8s8s32_extremes_exact():
    # every product at its extreme (-128 x -128 = 16384) over K = 4096: sums of 6.7e7, beyond f32's 2^24 integer range,
    # must come out exact
    M, N, Kd = 64, 64, 4096
    x = Case([M, Kd], O.S8, zero=True)
    w = Case([Kd, N], O.S8, "BA", zero=True)
    x.t.buf[:] = -128
    w.t.buf[:] = -128
    w.t.buf[::7] = 127
    c = Case([M, N], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    got = from_device(dc, O.S32).reshape(M, N)
    want = (x.t.buf.astype(np.int64).reshape(M, Kd) @ w.t.buf.astype(np.int64).reshape(N, Kd).T).astype(np.int32)
    assert np.array_equal(got, want)
    assert np.abs(want).max() > (1 << 24)


# ---------------------------------------------------------------------------------------------------
# u8 operands (cblas_gemm_s8u8s32 / u8s8s32 / u8u8s32): s8 MFMA on the operand shifted by -128, plus the shifted-out
# terms in the epilogue


def _int8_case(dims, dt, seed, layout=None):
    lo, hi = (-128, 127) if dt == O.S8 else (0, 255)
    return Case(dims, dt, layout, seed=seed, lo=lo, hi=hi)


def run_int8(M, N, Kd, adt, bdt, wlayout="BA", bias_dims=None, seed=0, expect="mfma_s8"):
    x = _int8_case([M, Kd], adt, seed)
    w = _int8_case([Kd, N], bdt, seed + 1, wlayout)
    c = Case([M, N], O.S32, zero=True)
    b = Case(bias_dims, O.S32, seed=seed + 2, lo=-(1 << 24), hi=1 << 24) if bias_dims else None
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc if b else None)
    assert expect in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device() if b else None)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref, b.t if b else None)
    compare(from_device(dc, O.S32), ref.buf, O.S32, plan.describe())


COMBOS = [(O.U8, O.S8), (O.S8, O.U8), (O.U8, O.U8)]


@pytest.mark.parametrize("adt,bdt", COMBOS)
@pytest.mark.parametrize("mnk", [(64, 64, 128), (300, 260, 256), (17, 33, 24), (1, 70, 300)])
@pytest.mark.parametrize("wlayout", ["BA", "AB"])
def test_u8_operand_gemms(adt, bdt, mnk, wlayout):
    M, N, Kd = mnk
    run_int8(M, N, Kd, adt, bdt, wlayout, bias_dims=[1, N], seed=300)


def _random_int8_cases(count=16, seed=77):
    # seeded draws over all four operand-sign combinations: M in [1, 600], N in [1, 1200], K in [4, 1500] (ragged
    # tiles, K tails that pack), weight layout and a [1, N] bias alternating
    rng = np.random.default_rng(seed)
    combos = [(O.S8, O.S8)] + COMBOS
    return [(int(rng.integers(1, 601)), int(rng.integers(1, 1201)), int(rng.integers(4, 1501)), *combos[i % 4],
             "BA" if i % 8 < 4 else "AB", i % 2 == 0) for i in range(count)]


@pytest.mark.parametrize("M,N,Kd,adt,bdt,wl,bias", _random_int8_cases())
def test_int8_random_shapes(M, N, Kd, adt, bdt, wl, bias):
    # bit-exact against the oracle's int64 sum wrapped to int32
    run_int8(M, N, Kd, adt, bdt, wl, bias_dims=[1, N] if bias else None, seed=340)


@pytest.mark.parametrize("adt,bdt", COMBOS)
@pytest.mark.parametrize("bias", [None, "M1", "MN"])
def test_u8_operand_bias_kinds(adt, bdt, bias):
    M, N, Kd = 96, 80, 256
    dims = {"M1": [M, 1], "MN": [M, N]}.get(bias)
    run_int8(M, N, Kd, adt, bdt, bias_dims=dims, seed=310)


@pytest.mark.parametrize("adt,bdt", COMBOS)
def test_u8_operand_pingpong(force_pingpong, adt, bdt):
    run_int8(300, 520, 384, adt, bdt, bias_dims=[1, 520], seed=320, expect="mfma_s8_pingpong")


@pytest.mark.parametrize("adt,bdt", COMBOS)
def test_u8_operand_batched_broadcast_weight(adt, bdt):
    # A batched (a correction vector per batch), W broadcast over the batch (one vector for all)
    x = _int8_case([3, 40, 256], adt, 330)
    w = _int8_case([1, 256, 72], bdt, 331)
    c = Case([3, 40, 72], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref)
    compare(from_device(dc, O.S32), ref.buf, O.S32, plan.describe())


def test_u8u8_extremes_exact():
    # every product 255 x 255 over K = 4096 (the constant term 128 * 128 * K and both row-sum terms at their largest)
    M, N, Kd = 64, 64, 4096
    x = Case([M, Kd], O.U8, zero=True)
    w = Case([Kd, N], O.U8, "BA", zero=True)
    x.t.buf[:] = 255
    w.t.buf[:] = 255
    w.t.buf[::5] = 0
    c = Case([M, N], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    got = from_device(dc, O.S32).reshape(M, N)
    want = (x.t.buf.astype(np.int64).reshape(M, Kd) @ w.t.buf.astype(np.int64).reshape(N, Kd).T).astype(np.int32)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------------------------------------------
# f16 x f16 and f16 x s8


@pytest.mark.parametrize("mnk", [(64, 64, 64), (300, 260, 200), (17, 33, 24), (5, 48, 64), (1, 96, 520), (4, 130, 256)])
@pytest.mark.parametrize("act", [O.ACT_RELU, O.ACT_SWISH, O.ACT_GELU_TANH, O.ACT_GELU_ERF])
def test_f16_linear_act(mnk, act):
    M, N, Kd = mnk
    x = Case([M, Kd], O.F16, seed=240)
    w = Case([Kd, N], O.F16, "BA", seed=241)
    b = Case([1, N], O.F16, seed=242, lo=-0.1, hi=0.1)
    c = Case([M, N], O.F16, zero=True)
    alpha = 0.0 if act == O.ACT_RELU else 1.0
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, alpha, 0.0, act)
    assert "f16" in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, act, alpha)
    compare(from_device(dc, O.F16), ref.buf, O.F16, plan.describe())


@pytest.mark.parametrize("mnk", [(256, 256, 64), (300, 520, 192), (40, 600, 128)])
@pytest.mark.parametrize("post", ["gelu_add", "none_f32out"])
def test_f16_pingpong(force_pingpong, mnk, post):
    M, N, Kd = mnk
    ydt = O.F32 if post == "none_f32out" else O.F16
    x = Case([M, Kd], O.F16, seed=250, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.F16, "BA", seed=251, dist="normal", lo=0.0, hi=0.05)
    y = Case([M, N], ydt, zero=True)
    s = Case([M, N], ydt, seed=252) if post == "gelu_add" else None
    act = K.ACT_GELU_TANH if post == "gelu_add" else K.ACT_UNIMPLEMENTED
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, None, act=act, binary=K.BIN_ADD if s else K.BIN_NONE,
                           src=s.desc if s else None)
    assert "f16_pingpong" in plan.describe(), plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, None, s.device() if s else None)
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, None, O.ACT_GELU_TANH if s else O.ACT_NONE, 0.0, O.BIN_ADD if s else O.BIN_NONE,
                     s.t if s else None)
    compare(from_device(dy, ydt), ref.buf, ydt, plan.describe())


@pytest.mark.parametrize("wdt", [O.S8, O.U8])
@pytest.mark.parametrize("mnk", [(64, 96, 128), (1, 200, 256), (300, 130, 72)])
def test_f16_x_8bit_weight(wdt, mnk):
    # W8A16 (GEMMWrapper<__fp16, int8_t / uint8_t, __fp16, float>): the 8-bit weight is converted to f16, bias f32
    M, N, Kd = mnk
    x = Case([M, Kd], O.F16, seed=260)
    lo, hi = (-128, 127) if wdt == O.S8 else (0, 255)
    w = Case([Kd, N], wdt, "BA", seed=261, lo=lo, hi=hi)
    b = Case([1, N], O.F32, seed=262, lo=-0.5, hi=0.5)
    c = Case([M, N], O.F16, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc)
    assert "f16" in plan.describe() and "packB" in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref, b.t)
    compare(from_device(dc, O.F16), ref.buf, O.F16, plan.describe())


def test_s8_operands_float_output():
    # integer operands into a floating output take the reference's all-f32 fallback (ChooseImpl :672-705)
    M, N, Kd = 50, 70, 96
    x = Case([M, Kd], O.S8, seed=270, lo=-128, hi=127)
    w = Case([Kd, N], O.S8, "BA", seed=271, lo=-128, hi=127)
    c = Case([M, N], O.F32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    assert "mfma_f32" in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref)
    compare(from_device(dc, O.F32), ref.buf, O.F32, plan.describe())


# ---------------------------------------------------------------------------------------------------
# ChooseImpl's all-f32 fallback into integer outputs (src/dnn/src/kudnn_gemm.cpp:673-705): f32 arithmetic, then
# ConvertFp32ToS32 / ToS8 / ToU8 (saturate, round half to even; src/dnn/src/service.cpp:77-115); and integer bias or C
# around a float sum


def _int_valued(dims, dt, seed, lo, hi, layout=None):
    """A Case of dtype dt holding uniform integers in [lo, hi] (exact in every dtype used here)."""
    c = Case(dims, dt, layout, zero=True)
    v = np.random.default_rng(seed).integers(lo, hi + 1, size=c.t.buf.size)
    if dt in (O.S32, O.S8, O.U8):
        c.t.buf[:] = v.astype(O.storage_dtype(dt))
    else:
        c.t.buf[:] = O.from_f32_rne(v.astype(np.float32), dt)
    return c


def run_fallback(M, N, Kd, adt, bdt, cdt, xdt, alpha=0.5, beta=0.5, seed=400, expect=None, span=8):
    lo = lambda dt, v: 0 if dt == O.U8 else -v
    x = _int_valued([M, Kd], adt, seed, lo(adt, span), span)
    w = _int_valued([Kd, N], bdt, seed + 1, lo(bdt, span), span, "BA")
    c = _int_valued([M, N], cdt, seed + 2, lo(cdt, 100), 100)
    b = _int_valued([1, N], xdt, seed + 3, lo(xdt, 60), 60) if xdt is not None else None
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc if b else None)
    if expect:
        assert expect in plan.describe(), plan.describe()
    dc = c.device()
    plan.run(x.device(), w.device(), dc, b.device() if b else None, alpha=alpha, beta=beta)
    torch.cuda.synchronize()
    ref = O.Tensor(c.t.dims, c.t.strides, cdt, c.t.buf.copy())
    O.gemm(x.t, w.t, ref, b.t if b else None, alpha=alpha, beta=beta)
    got = from_device(dc, cdt)
    if cdt in (O.S32, O.S8, O.U8):
        # integer-valued operands keep every f32 partial sum exact: bit-exact, whatever the summation order
        compare(got, ref.buf, cdt, plan.describe())
    else:
        assert np.array_equal(got, ref.buf), plan.describe()
    return plan, got


FALLBACK_COMBOS = [
    (O.F32, O.F32, O.S32, O.F32), (O.F32, O.F32, O.S8, None), (O.BF16, O.BF16, O.U8, O.F32),
    (O.F16, O.F16, O.S8, O.F16), (O.S8, O.S8, O.S8, None), (O.U8, O.S8, O.U8, O.S32), (O.S8, O.U8, O.S32, O.F32),
    (O.S8, O.S8, O.S32, O.U8), (O.F32, O.F32, O.F32, O.S32), (O.BF16, O.BF16, O.BF16, O.S8),
    (O.U8, O.U8, O.S8, O.BF16), (O.F16, O.S8, O.U8, None),
]


@pytest.mark.parametrize("adt,bdt,cdt,xdt", FALLBACK_COMBOS)
@pytest.mark.parametrize("mnk", [(200, 136, 96), (5, 70, 64), (33, 17, 300)])
def test_fallback_integer_exact(adt, bdt, cdt, xdt, mnk):
    # alpha = beta = 0.5 put exact .5 ties in front of the conversion; the value range saturates s8 and u8 outputs
    M, N, Kd = mnk
    plan, got = run_fallback(M, N, Kd, adt, bdt, cdt, xdt)
    if cdt in (O.S8, O.U8):
        lo, hi = (-128, 127) if cdt == O.S8 else (0, 255)
        assert np.any(got == hi), "the case does not saturate"
        if adt != O.U8 or bdt != O.U8:  # u8 x u8 sums are never negative
            assert np.any(got == lo), "the case does not saturate"


def test_fallback_pingpong_and_skinny(monkeypatch):
    # the bf16 kernels' element-wise epilogue: the ping-pong kernel (forced) and the decode kernel (M <= 16)
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    run_fallback(300, 520, 384, O.BF16, O.BF16, O.S8, O.F32, expect="pingpong")
    monkeypatch.delenv("KUDNN_HIP_FORCE_CFG")
    run_fallback(4, 520, 384, O.BF16, O.BF16, O.U8, None, expect="skinny")
    run_fallback(1, 300, 512, O.BF16, O.BF16, O.S32, O.S32, expect="skinny")


def test_s8_bias_into_exact_int32():
    # s8 x s8 -> s32 with an s8 bias: the integer GEMM (ChooseImpl's wider-type match), exact beyond 2^24
    M, N, Kd = 64, 72, 4096
    x = Case([M, Kd], O.S8, seed=410, lo=-128, hi=127)
    w = Case([Kd, N], O.S8, "BA", seed=411, lo=-128, hi=127)
    x.t.buf[: Kd * 4] = -128
    w.t.buf[: Kd * 4] = -128
    b = Case([1, N], O.S8, seed=412, lo=-128, hi=127)
    c = Case([M, N], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc)
    assert "mfma_s8" in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref, b.t)
    compare(from_device(dc, O.S32), ref.buf, O.S32, plan.describe())
    assert np.abs(ref.buf.astype(np.int64)).max() > (1 << 24)


@pytest.mark.parametrize("cdt", [O.S32, O.S8, O.U8])
def test_fallback_random_floats(cdt):
    # non-integer f32 operands: the GPU and the oracle sum in different orders, so an output may differ by one where
    # the f32 value lies within rounding of a .5 boundary; every other element is bit-exact
    M, N, Kd = 160, 200, 256
    scale = {O.S32: 3e3, O.S8: 300.0, O.U8: 600.0}[cdt]  # sums of about scale / 3 (saturating s8 and u8)
    x = Case([M, Kd], O.F32, seed=420, lo=-1.0, hi=1.0)
    w = Case([Kd, N], O.F32, "BA", seed=421, lo=-scale / 16, hi=scale / 16)
    c = Case([M, N], cdt, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref)
    f = O.empty(c.t.dims, c.t.strides, O.F32)
    O.gemm(x.t, w.t, f)
    got = from_device(dc, cdt).astype(np.int64)
    want = ref.buf.astype(np.int64)
    bad = np.nonzero(got != want)[0]
    v = f.buf.astype(np.float64)[bad]
    # f32 summation error grows with the terms, not with the result: allow 32 f32 ulps of sum |x_k w_k| (the
    # worst-case bound is K = 256 of them)
    mag = (np.abs(x.t.logical().astype(np.float64)) @ np.abs(w.t.logical().astype(np.float64))).reshape(-1)[bad]
    near_tie = np.abs(np.abs(v - np.floor(v)) - 0.5) <= 32 * 2.0 ** -24 * mag
    assert np.all(np.abs(got[bad] - want[bad]) == 1) and np.all(near_tie), (
        f"{bad.size} differences, unexplained at {bad[~near_tie][:5]}: f32 {v[~near_tie][:5]}")
    print(f"{cdt}: {bad.size} of {got.size} outputs one step apart at a .5 boundary")
    lo, hi = {O.S32: (-2147483648, 2147483647), O.S8: (-128, 127), O.U8: (0, 255)}[cdt]
    if cdt != O.S32:
        assert np.any(want == lo) and np.any(want == hi)


@pytest.mark.parametrize("cdt", [O.S32, O.S8, O.U8])
def test_integer_conversion_special_values(cdt):
    # [n, 1] x [1, 1] -> the conversion of each f32 value alone: the saturation bounds, .5 ties, +-2^31 and non-finite
    # values, bit-exact against the oracle (whose conversion is pinned on the CPU)
    vals = np.array([np.nan, np.inf, -np.inf, -0.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 127.5, 128.5, 254.5, 255.5,
                     256.5, -127.5, -128.5, -129.5, 8388607.5, 16777216.0, 2.0 ** 31, -(2.0 ** 31), 2147483520.0,
                     -2147483520.0, 3e9, -3e9, 1e38, -1e38, 0.49999997, 1.0000001, 300.25, -300.75], dtype=np.float32)
    n = vals.size
    x = Case([n, 1], O.F32, zero=True)
    x.t.buf[:] = vals
    w = Case([1, 1], O.F32, zero=True)
    w.t.buf[:] = 1.0
    c = Case([n, 1], cdt, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref)
    compare(from_device(dc, cdt), ref.buf, cdt, plan.describe())
