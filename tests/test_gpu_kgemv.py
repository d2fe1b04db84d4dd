"""GPU parity of the K-split decode GEMV (skinny_bf16.hip kgemv_*: 2 <= M <= 16, K <= 4096, one batch). Each of its 8
waves keeps the X fragments of one K slice in registers, and the weight streams straight into the 16 x 16 x 32 MFMA.
The cases cover:
- M from 2 to 16, with K tails and slices shorter than the 16-step maximum;
- the rows dealt to the workgroups in rounds of 16 rows each: a single partial round of one quad per workgroup
  (N = 300 over 75 workgroups), one to seven whole rounds, and partial last rounds (N = 4100, 11008, 14336);
- the compact fixed-form kernel (bf16 and f32 outputs) and the generic one (beta C, f16 operands, LinearRes storing C);
- calls the kernel cannot take (batches, K > 4096), which run the row kernel instead.
Every case is checked against the oracle, and the C4 shapes also against the 16-row MFMA row kernel on the same inputs.
The planner takes the kernel for M >= 6; the tests force it (KUDNN_HIP_FORCE_CFG=23) so that M < 6 runs it too.

Reference semantics: src/dnn/src/kudnn_gemm.cpp:208-241 (the bf16 GEMM of a short M) and the post-op stages of
kudnn_linear_activationlayer.cpp:40-56, restated by the oracle.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, explainer, from_device, zeros_device
from test_gpu_gemv_rows import _run_post

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()  # fail loudly if the HIP library is missing


@pytest.fixture
def force_kgemv(monkeypatch):
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "23")


@pytest.mark.parametrize("M", [2, 6, 9, 16])
@pytest.mark.parametrize("Kd", [40, 1001, 2048, 4096])
@pytest.mark.parametrize("post", ["bias_gelu_add", "swish_f32", "gemm_beta"])
def test_kgemv_forms(force_kgemv, M, Kd, post):
    # N = 300: 75 quads of rows, one workgroup each (4 rows, 12 of the 16-row group past the range)
    got, ref, ydt, desc, why = _run_post(M, 300, Kd, post, seed=600 + M)
    assert desc.startswith("skinny_bf16_kgemv_xreg"), desc
    compare(got, ref, ydt, f"M={M} K={Kd} {post} {desc}", explain=why)


@pytest.mark.parametrize("M,N", [(16, 14336), (16, 4096), (8, 14336), (6, 4100), (4, 14336), (12, 4100), (16, 8192),
                                 (16, 11008), (10, 28672)])
def test_kgemv_decode_shapes_against_row_kernel(monkeypatch, M, N):
    # C4 (Linear then element-wise multiply, K = 4096), rows dealt in rounds of 16 per workgroup: N = 4096, 8192 and
    # 28672 in 1, 2 and 7 whole rounds; N = 14336 and 11008 in 3 and 2 whole rounds and a partial one of 8 and 11 rows
    # per workgroup; N = 4100 in one whole round and a partial one of 4 rows that the last workgroup takes. The row
    # kernel agrees on the same inputs
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "23")
    got, ref, ydt, desc, _ = _run_post(M, N, 4096, "mul", seed=620 + M)
    assert desc.startswith("skinny_bf16_kgemv_xreg"), desc
    compare(got, ref, ydt, f"C4 M={M} N={N} {desc}")
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "20")
    got2, ref2, _, desc2, _ = _run_post(M, N, 4096, "mul", seed=620 + M)
    assert desc2.startswith("skinny_bf16_16xK"), desc2
    compare(got2, ref2, ydt, f"C4 M={M} N={N} {desc2}")
    # the two sum in different orders: their bf16 GEMM stages differ by at most one ulp, and only rarely
    assert np.mean(got == got2) > 0.99


@pytest.mark.parametrize("M", [3, 16])
@pytest.mark.parametrize("post", ["bias_gelu_add", "gemm_beta"])
def test_kgemv_f16(force_kgemv, M, post):
    # f16 operands take the generic kernel and the f16 MFMA
    got, ref, ydt, desc, why = _run_post(M, 259, 4096, post, dt=O.F16, seed=640)
    assert desc.startswith("skinny_f16_kgemv_xreg"), desc
    compare(got, ref, ydt, f"f16 M={M} {post} {desc}", explain=why)


@pytest.mark.parametrize("kind", [O.RES_IDENTIAL, O.RES_EXT])
def test_kgemv_linear_res_stores_c(force_kgemv, kind):
    # LinearResFWD writes C and linearRes from the one launch (the generic epilogue's store_c)
    M, N, Kd = 7, 1000, 4096
    x = Case([M, Kd], O.BF16, seed=650, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=651, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, N], O.BF16, seed=652, lo=-0.1, hi=0.1)
    c = Case([M, N], O.BF16, zero=True)
    res = Case([M, N], O.BF16, seed=653)
    lr = Case([M, N], O.BF16, zero=True)
    plan = K.LinearRes(x.desc, w.desc, c.desc, b.desc, res.desc, lr.desc, 1.0, 0.0, 1.0, kind)
    assert plan.describe().startswith("skinny_bf16_kgemv_xreg"), plan.describe()
    dc, dlr = zeros_device(c), zeros_device(lr)
    plan.run(x.device(), w.device(), dc, b.device(), res.device(), dlr, 0.625)
    torch.cuda.synchronize()
    rc, rlr = c.clone_empty(), lr.clone_empty()
    O.linear_res(x.t, w.t, rc, b.t, res.t, rlr, kind, 0.625)
    compare(from_device(dc, O.BF16), rc.buf, O.BF16, plan.describe() + " C")
    why = explainer(O.BF16, x.t, w.t, b.t, (M, N), src=res.t, gamma=0.625,
                    binary=O.BIN_ADD if kind == O.RES_IDENTIAL else O.BIN_EXT)
    compare(from_device(dlr, O.BF16), rlr.buf, O.BF16, plan.describe() + " linearRes", explain=why)


def test_kgemv_single_weight_row(force_kgemv):
    # N = 1: one workgroup, one quad of rows with three past N (the weight's row pitch is 0 in its descriptor)
    got, ref, ydt, desc, why = _run_post(5, 1, 4096, "bias_gelu_add", seed=660)
    assert desc.startswith("skinny_bf16_kgemv_xreg"), desc
    compare(got, ref, ydt, f"N=1 {desc}", explain=why)


@pytest.mark.parametrize("case", ["batched", "long_k"])
def test_kgemv_ineligible_calls_run_the_row_kernel(force_kgemv, case):
    # batches (grid y) and K > 4096 (more than 16 steps per wave) are outside the kernel: the launch takes the
    # 16-row MFMA kernel and the results stay right
    if case == "batched":
        x = Case([3, 6, 2048], O.BF16, "ABC", seed=670, dist="normal", lo=0.0, hi=1.0)
        w = Case([3, 2048, 200], O.BF16, "ACB", seed=671, dist="normal", lo=0.0, hi=0.05)
        y = Case([3, 6, 200], O.BF16, "ABC", zero=True)
    else:
        x = Case([6, 6000], O.BF16, seed=672, dist="normal", lo=0.0, hi=1.0)
        w = Case([6000, 200], O.BF16, "BA", seed=673, dist="normal", lo=0.0, hi=0.05)
        y = Case([6, 200], O.BF16, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, act=K.ACT_GELU_TANH)
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy)
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, None, O.ACT_GELU_TANH, 0.0, O.BIN_NONE, None)
    compare(from_device(dy, O.BF16), ref.buf, O.BF16, f"{case} {plan.describe()}")
