"""GPU parity of KuDNN::Gemm's descriptor surface (src/dnn/src/kudnn_gemm.cpp:478-549, 709-807): strided descriptors
(kudnn_tensor_desc_init_strided) on src, weight and bias; batched tensors in non-standard layouts (ACB, BAC, ABDC,
ABCED ...), which the reference reorders to f32 copies before dispatch (:722-765); 5-D broadcast batches with a full
[D1, D2, D3, M, N] bias; the serial batch loop of a dst broadcast over a looped batch dim (:783-807); and the reference's
MTest sweep, common_MNK x common_Dims in its four transpose modes (test/dnn/llt/gtest/src/matmul_gtest.cpp:546-690),
as seeded cases. Every case is compared with the oracle in full.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, from_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()


_RANGES = {O.S8: (-125, 125), O.U8: (0, 255), O.S32: (-65536, 65536)}  # the gtest's generators (matmul_gtest.cpp:142-156)


def _case(dims, dt, layout=None, strides=None, seed=0, zero=False, int_valued=False):
    lo, hi = _RANGES.get(dt, (-1.0, 1.0))
    c = Case(dims, dt, layout, strides, seed=seed, lo=lo, hi=hi, zero=zero)
    if int_valued and not zero and dt in (O.F32, O.BF16, O.F16):
        # integers in [-16, 16]: every f32 partial sum of the GEMM is exact, in any order
        v = np.random.default_rng(seed).integers(-16, 17, size=c.t.buf.size).astype(np.float32)
        c.t.buf[:] = v if dt == O.F32 else O.from_f32_rne(v, dt)
    return c


def run_gemm(a, b, c, bias=None, alpha=1.0, beta=0.0, expect=None, seed=0, int_valued=False, reordered=None):
    """a, b, c, bias: (dims, dtype, layout, strides) tuples (bias may be None). Runs KuDNN::Gemm on the GPU and the
    oracle on the same inputs; returns the plan description and the GPU result. int_valued: integer-valued float
    inputs and a bit-exact comparison. reordered: the oracle's O_REORDERED_* mask (default: from the layouts)."""
    xa = _case(*a, seed=seed, int_valued=int_valued)
    xb = _case(*b, seed=seed + 1, int_valued=int_valued)
    xc = _case(*c, seed=seed + 2, zero=beta == 0.0, int_valued=int_valued)
    xx = _case(*bias, seed=seed + 3, int_valued=int_valued) if bias else None
    plan = K.Gemm(xa.desc, xb.desc, xc.desc, xx.desc if xx else None)
    d = plan.describe()
    if expect:
        assert expect in d, d
    dc = xc.device()
    plan.run(xa.device(), xb.device(), dc, xx.device() if xx else None, alpha=alpha, beta=beta)
    torch.cuda.synchronize()
    ref = O.Tensor(xc.t.dims, xc.t.strides, xc.dt, xc.t.buf.copy())
    mask = O.reordered_mask(len(a[0]), a[2], b[2], c[2], bias[2] if bias else None) if reordered is None else reordered
    O.gemm(xa.t, xb.t, ref, xx.t if xx else None, alpha=alpha, beta=beta, reordered=mask)
    got = from_device(dc, xc.dt)
    if int_valued:
        assert np.array_equal(got, ref.buf), d
    else:
        compare(got, ref.buf, xc.dt, d)
    return d, got


def T(dims, dt, layout=None, strides=None):
    return (list(dims), dt, layout, strides)


# ---------------------------------------------------------------------------------------------------
# strided descriptors

F, B = O.F32, O.BF16
M, N, KD = 72, 80, 96

STRIDED = {
    "src_row_pitch": (T([M, KD], F, "AB", [KD + 8, 1]), T([KD, N], F, "BA"), T([M, N], F), T([1, N], F)),
    "src_elem_stride": (T([M, KD], F, "AB", [2 * KD, 2]), T([KD, N], F, "BA"), T([M, N], F), None),
    "src_col_major_pitch": (T([M, KD], B, "BA", [1, M + 5]), T([KD, N], B, "BA"), T([M, N], B), T([1, N], F)),
    "wei_ab_pitch": (T([M, KD], B), T([KD, N], B, "AB", [N + 4, 1]), T([M, N], B), T([1, N], F)),
    "wei_ba_pitch": (T([M, KD], B), T([KD, N], B, "BA", [1, KD + 3]), T([M, N], B), None),
    "wei_elem_stride": (T([M, KD], F), T([KD, N], F, "AB", [3 * N, 3]), T([M, N], F), None),
    "bias_elem_stride": (T([M, KD], F), T([KD, N], F, "BA"), T([M, N], F), T([1, N], F, "AB", [2 * N, 2])),
    "bias_mn_pitch": (T([M, KD], B), T([KD, N], B, "BA"), T([M, N], B), T([M, N], F, "AB", [N + 5, 1])),
    "bias_m1_stride": (T([M, KD], F), T([KD, N], F, "BA"), T([M, N], F), T([M, 1], F, "AB", [4, 4])),
    "all_but_dst": (T([M, KD], F, "AB", [2 * KD, 2]), T([KD, N], F, "AB", [2 * N, 2]), T([M, N], F),
                    T([M, N], F, "AB", [2 * N, 2])),
    "batch_stride_gap": (T([3, M, KD], B, "ABC", [M * KD + 128, KD, 1]), T([1, KD, N], B), T([3, M, N], B),
                         T([1, 1, N], F)),
    "batch_weight_pitch": (T([2, 3, M, KD], F), T([2, 3, KD, N], F, "ABCD", [3 * KD * (N + 2), KD * (N + 2), N + 2, 1]),
                           T([2, 3, M, N], F), T([2, 1, 1, N], F)),
}


@pytest.mark.parametrize("name", list(STRIDED))
def test_strided_descriptors(name):
    a, b, c, x = STRIDED[name]
    run_gemm(a, b, c, x, alpha=0.75, beta=0.5 if name.endswith("pitch") else 0.0, seed=500)


# ---------------------------------------------------------------------------------------------------
# batched tensors in non-standard layouts (reordered to f32 by the reference before ChooseImpl)

NONSTD = {
    "src_ACB": (T([3, M, KD], F, "ACB"), T([3, KD, N], F), T([3, M, N], F), T([3, M, N], F)),
    "src_BAC": (T([3, M, KD], B, "BAC"), T([1, KD, N], B), T([3, M, N], B), T([1, 1, N], F)),
    "src_BCA": (T([3, M, KD], F, "BCA"), T([3, KD, N], F), T([3, M, N], F), None),
    "wei_ACB": (T([3, M, KD], B), T([3, KD, N], B, "ACB"), T([3, M, N], B), None),
    "wei_dst_ABDC": (T([2, 3, M, KD], B), T([2, 3, KD, N], B, "ABDC"), T([2, 3, M, N], B, "ABDC"), None),
    "dst_ABDC_beta": (T([2, 3, M, KD], F), T([2, 3, KD, N], F), T([2, 3, M, N], F, "ABDC"), T([2, 3, M, N], F)),
    "src_ACBD": (T([2, 3, M, KD], F, "ACBD"), T([2, 1, KD, N], F), T([2, 3, M, N], F), None),
    "bias_ABDC": (T([2, 3, M, KD], B), T([2, 3, KD, N], B), T([2, 3, M, N], B), T([2, 3, M, N], F, "ABDC")),
    "all_ABCED": (T([2, 3, 2, M, KD], B, "ABCED"), T([2, 3, 2, KD, N], B, "ABCED"), T([2, 3, 2, M, N], B, "ABCED"),
                  T([2, 3, 2, M, N], F, "ABCED")),
    "src_ACBDE": (T([2, 3, 2, M, KD], F, "ACBDE"), T([1, 1, 2, KD, N], F), T([2, 3, 2, M, N], F), None),
    # the reordered s8 GEMM runs in f32 (alpha / beta allowed), into s32 through the saturating conversion
    "s8_ACB_f32": (T([2, M, KD], O.S8, "ACB"), T([2, KD, N], O.S8), T([2, M, N], O.S32), T([1, 1, N], O.S32)),
}


@pytest.mark.parametrize("name", list(NONSTD))
def test_nonstandard_layouts(name):
    a, b, c, x = NONSTD[name]
    beta = 0.5 if name.endswith("beta") else 0.0
    alpha = 1.0 + 2.0 ** -10 if name == "s8_ACB_f32" else 0.75
    run_gemm(a, b, c, x, alpha=alpha, beta=beta, seed=510)


@pytest.mark.parametrize("src_layout", ["ABC", "ACB"])
def test_bf16_scalars_only_on_the_standard_path(src_layout):
    # a bf16 GEMM into bf16 without bias: in the standard layout cblas_bgemm takes alpha rounded to bf16
    # (1 + 2^-9 -> 1); with src reordered to f32 (ACB) the all-f32 fallback takes alpha as given. Integer-valued
    # inputs make the sums exact, so the results are bit-exact and the two rules give different outputs (at the
    # bf16 ties of odd sums above 256).
    alpha = 1.0 + 2.0 ** -9
    args = (T([2, M, KD], B, src_layout), T([2, KD, N], B), T([2, M, N], B), None)
    _, got = run_gemm(*args, alpha=alpha, seed=540, int_valued=True)
    # the oracle under the other rule (src flagged as reordered or not, the other way round) must differ
    xa = _case(*args[0], seed=540, int_valued=True)
    xb = _case(*args[1], seed=541, int_valued=True)
    other = Case([2, M, N], B, zero=True).t
    O.gemm(xa.t, xb.t, other, alpha=alpha, reordered=O.reordered_mask(3, src_layout) ^ O.REORDERED_A)
    assert not np.array_equal(got, other.buf), "the case does not tell the two rules apart"


# ---------------------------------------------------------------------------------------------------
# 5-D broadcast batches with a full bias, and the serial loop


@pytest.mark.parametrize("dt,bdt", [(F, F), (B, F), (B, B)])
def test_5d_broadcast_full_bias(dt, bdt):
    run_gemm(T([5, 1, 4, 20, 33], dt), T([1, 3, 4, 33, 24], dt, "ABCED"), T([5, 3, 4, 20, 24], dt),
             T([5, 3, 4, 20, 24], bdt), seed=520)
    run_gemm(T([5, 3, 1, 40, 16], dt), T([5, 1, 1, 16, 56], dt), T([5, 3, 1, 40, 56], dt), T([1, 3, 1, 40, 56], bdt),
             seed=521)


@pytest.mark.parametrize("dt", [F, B])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_serial_batch_loop(dt, beta):
    # dst broadcast over a batch dim the weight loops over: batches run in order into the same C (kudnn_gemm.cpp:783-807;
    # with beta != 0 each one reads the previous one's result)
    d, _ = run_gemm(T([1, M, KD], dt), T([4, KD, N], dt), T([1, M, N], dt), T([1, 1, N], F), beta=beta,
                    expect="serial", seed=530)
    assert "batches=4" in d
    run_gemm(T([1, 1, 1, 24, 40], dt), T([2, 3, 1, 40, 48], dt, "ABCED"), T([1, 1, 1, 24, 48], dt),
             T([1, 1, 1, 24, 48], F), beta=beta, expect="serial", seed=531)


# ---------------------------------------------------------------------------------------------------
# the reference's MTest sweep: [D1, D2, D3, M, K] x [D1, D2, D3, K, N] -> [D1, D2, D3, M, N] with a full bias, in the
# modes Matmul, MatmulTransSrc, MatmulTransWei and MatmulTransSrcWei (ABCED for a transposed operand)

COMMON_MNK = [(5, 5, 5), (20, 20, 10), (200, 100, 200)]
COMMON_DIMS = [(1, 1, 1), (1, 1, 10), (1, 1, 20), (1, 10, 10), (1, 10, 20), (5, 10, 10), (5, 10, 20)]
MODES = {"Matmul": (0, 0), "TransSrc": (1, 0), "TransWei": (0, 1), "TransSrcWei": (1, 1)}
FLOAT_CALLERS = [(B, B, B, F), (B, B, F, F), (F, F, F, F)]
OTHER_CALLERS = [(O.F16, O.F16, O.F16, O.F16), (O.F16, O.F16, F, F), (O.S8, O.S8, O.S32, O.S32), (O.F16, O.S8, O.F16, F),
                 (O.U8, O.S8, O.S32, O.S32), (O.S8, O.U8, O.S32, O.S32), (O.U8, O.U8, O.S32, O.S32),
                 (O.F16, O.U8, O.F16, F)]


def _mtest(caller, dims, mnk, mode, seed):
    (D1, D2, D3), (Mm, Nn, Kk) = dims, mnk
    ts, tw = MODES[mode]
    sdt, wdt, ddt, bdt = caller
    return run_gemm(T([D1, D2, D3, Mm, Kk], sdt, "ABCED" if ts else "ABCDE"),
                    T([D1, D2, D3, Kk, Nn], wdt, "ABCED" if tw else "ABCDE"),
                    T([D1, D2, D3, Mm, Nn], ddt, "ABCDE"), T([D1, D2, D3, Mm, Nn], bdt, "ABCDE"), seed=seed)


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("mnk", COMMON_MNK)
@pytest.mark.parametrize("dims", COMMON_DIMS)
@pytest.mark.parametrize("caller", FLOAT_CALLERS, ids=lambda c: "_".join(O.DT_NAMES[t] for t in c))
def test_mtest_float(caller, dims, mnk, mode):
    _mtest(caller, dims, mnk, mode, seed=600)


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("dims,mnk", [((1, 1, 1), (5, 5, 5)), ((1, 10, 20), (20, 20, 10)), ((5, 10, 10), (20, 20, 10)),
                                      ((1, 1, 10), (200, 100, 200))])
@pytest.mark.parametrize("caller", OTHER_CALLERS, ids=lambda c: "_".join(O.DT_NAMES[t] for t in c))
def test_mtest_other_dtypes(caller, dims, mnk, mode):
    _mtest(caller, dims, mnk, mode, seed=610)


@pytest.mark.parametrize("case", ["bf16_one_dim", "f32_two_dims"])
def test_batches_beyond_one_grid(case):
    # more batches than one launch's grid carries (65535 rows of workgroups): the run is split over the batch dims,
    # in order, as the reference loops over them (kudnn_gemm.cpp:783-807). 70000 batches of one dim are launched in
    # chunks of that dim; 3 x 30000 loops over the outer dim
    if case == "bf16_one_dim":
        dt, xd, wd, bd, cd, lay = O.BF16, [70000, 2, 16], [70000, 16, 8], [1, 1, 8], [70000, 2, 8], "ABC"
    else:
        dt, xd, wd, bd, cd, lay = O.F32, [3, 30000, 4, 32], [3, 30000, 32, 8], [1, 1, 1, 8], [3, 30000, 4, 8], "ABCD"
    x = _case(xd, dt, lay, seed=500)
    w = _case(wd, dt, lay, seed=501)
    b = _case(bd, dt, lay, seed=502)
    c = _case(cd, dt, lay, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    assert "batches=70000" in plan.describe() or "batches=90000" in plan.describe(), plan.describe()
    dc = torch.zeros(c.t.buf.size, dtype=torch.float32 if dt == O.F32 else torch.int16, device="cuda")
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(from_device(dc, dt), ref.buf, dt, plan.describe())
