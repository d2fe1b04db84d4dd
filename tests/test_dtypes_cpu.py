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


@pytest.mark.parametrize("combo", [
    (K.S8, K.S8, K.S8, None),
    (K.U8, K.U8, K.U8, None),
    (K.F32, K.F32, K.S32, None),
    (K.S8, K.S8, K.S32, K.F32),
])
def test_planner_refuses_integer_outputs_other_than_s32(combo):
    with pytest.raises(K.KudnnError) as e:
        _plan(*combo)
    assert e.value.status == K.UNSUPPORTED


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
