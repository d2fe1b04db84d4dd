"""GPU parity of the decode GEMV with X staged in LDS (1 <= M <= 5 by the planner, up to 8 forced through
KUDNN_HIP_FORCE_CFG=22): K blocks of 4096 and K tails, ragged weight-row counts, the compact fixed-form kernel (bf16 and
f32 tensors) and the generic kernel (beta C, batches, f16 operands), each against the oracle and against the 16-row MFMA
kernel forced through KUDNN_HIP_FORCE_CFG=20 on the same inputs. Reference semantics: src/dnn/src/kudnn_gemm.cpp:208-241
(the bf16 GEMM of a short M) and the post-op stages of kudnn_linear_activationlayer.cpp:40-56 and
kudnn_linear_postops restated by the oracle.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, explainer, from_device, zeros_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()  # fail loudly if the HIP library is missing


def _post_case(M, N, Kd, post, dt=O.BF16, seed=500):
    ydt = O.F32 if post in ("swish_f32", "gemm_beta") and dt == O.BF16 else dt
    x = Case([M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, "BA", seed=seed + 1, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, N], ydt, seed=seed + 2, lo=-0.2, hi=0.2)
    y = Case([M, N], ydt, seed=seed + 3, lo=-1.0, hi=1.0) if post == "gemm_beta" else Case([M, N], ydt, zero=True)
    s = Case([M, N], ydt, seed=seed + 4, lo=-1.0, hi=1.0)
    return x, w, b, y, s, ydt


def _run_post(M, N, Kd, post, dt=O.BF16, seed=500):
    """Runs the post-op chain `post` through the planner's kernel; returns (device output, oracle output, dtype, plan
    description, explainer)."""
    x, w, b, y, s, ydt = _post_case(M, N, Kd, post, dt, seed)
    dy = torch.from_numpy(y.t.buf.view(np.int16).copy() if ydt != O.F32 else y.t.buf.copy()).cuda()
    ref = O.Tensor(y.t.dims, y.t.strides, ydt, y.t.buf.copy())
    why = None
    if post == "bias_gelu_add":
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
        plan.run(x.device(), w.device(), dy, b.device(), s.device())
        O.linear_postops(x.t, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, s.t)
        why = explainer(ydt, x.t, w.t, b.t, (M, N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=s.t)
    elif post == "mul":
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, binary=K.BIN_MUL, src=s.desc)
        plan.run(x.device(), w.device(), dy, None, s.device())
        O.linear_postops(x.t, w.t, ref, None, O.ACT_NONE, 0.0, O.BIN_MUL, s.t)
    elif post == "swish_f32":
        plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
        plan.run(x.device(), w.device(), dy, b.device())
        O.linear_act(x.t, w.t, ref, b.t, O.ACT_SWISH, 1.0)
    else:
        plan = K.Gemm(x.desc, w.desc, y.desc, b.desc)
        plan.run(x.device(), w.device(), dy, b.device(), alpha=0.5, beta=0.25)
        O.gemm(x.t, w.t, ref, b.t, 0.5, 0.25)
    torch.cuda.synchronize()
    return from_device(dy, ydt), ref.buf, ydt, plan.describe(), why


@pytest.mark.parametrize("M", [2, 3, 4, 5])
@pytest.mark.parametrize("Kd", [40, 1001, 4104, 9000])
@pytest.mark.parametrize("post", ["bias_gelu_add", "swish_f32", "gemm_beta"])
def test_gemv_rows_forms(M, Kd, post):
    # N = 300 leaves the last 8-row workgroup with 4 rows past N; K = 4104 and 9000 cross the 4096-element staging
    # block (a second and third block, the last one ragged); K = 40 and 1001 end inside the first block (1001 packs)
    N = 300
    got, ref, ydt, desc, why = _run_post(M, N, Kd, post)
    assert desc.startswith("skinny_bf16_gemv_rows_xlds"), desc
    compare(got, ref, ydt, f"M={M} K={Kd} {post} {desc}", explain=why)


@pytest.mark.parametrize("M", [6, 8])
def test_gemv_rows_forced_wider(monkeypatch, M):
    # up to 8 rows of X when forced
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "22")
    for post in ("bias_gelu_add", "gemm_beta"):
        got, ref, ydt, desc, why = _run_post(M, 517, 4104, post, seed=520)
        assert desc.startswith("skinny_bf16_gemv_rows_xlds"), desc
        compare(got, ref, ydt, f"M={M} {post} {desc}", explain=why)


@pytest.mark.parametrize("M,N", [(4, 4096), (4, 14336), (2, 14336), (2, 4100), (5, 4100), (1, 14336), (1, 4100)])
def test_gemv_rows_decode_shapes_against_row_kernel(monkeypatch, M, N):
    # C4 (Linear then element-wise multiply, K = 4096) and a ragged N, in 8-wave workgroups (M = 2 below 10240 rows,
    # M >= 3) and 4-wave ones (M = 1, M = 2 from 10240 rows on): the GEMV and the 16-row MFMA kernel agree with the
    # oracle on the same inputs (the MFMA kernel takes M >= 2 only)
    got, ref, ydt, desc, _ = _run_post(M, N, 4096, "mul", seed=530)
    assert desc.startswith("skinny_bf16_gemv_row"), desc
    compare(got, ref, ydt, f"C4 M={M} N={N} {desc}")
    if M == 1:
        return
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "20")
    got2, ref2, _, desc2, _ = _run_post(M, N, 4096, "mul", seed=530)
    assert desc2.startswith("skinny_bf16_16xK"), desc2
    compare(got2, ref2, ydt, f"C4 M={M} N={N} {desc2}")
    # the two sum in different orders: their bf16 GEMM stages differ by at most one ulp, and only rarely
    assert np.mean(got == got2) > 0.99


@pytest.mark.parametrize("batch,M,wbatch,expect", [(3, 3, 3, "skinny_bf16_gemv_rows_xlds M=3 N=130 K=4200 batches=3"),
                                                   (2, 2, 1, "skinny_bf16_gemv_rows_xlds M=4 N=130 K=4200 batches=1"),
                                                   (3, 1, 3, "skinny_bf16_gemv_row M=1 N=130 K=4200 batches=3")])
def test_gemv_rows_batched(batch, M, wbatch, expect):
    # batches of M rows against a per-batch weight (the generic kernel, batches on grid y; M = 1 in 4-wave workgroups),
    # and against one broadcast weight (the batches fold into M: one launch of the compact kernel)
    Kd, N = 4200, 130
    x = Case([batch, M, Kd], O.BF16, "ABC", seed=540, dist="normal", lo=0.0, hi=1.0)
    w = Case([wbatch, Kd, N], O.BF16, "ACB", seed=541, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, 1, N], O.BF16, "ABC", seed=542, lo=-0.1, hi=0.1)
    c = Case([batch, M, N], O.BF16, "ABC", zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    assert plan.describe().startswith(expect), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(from_device(dc, O.BF16), ref.buf, O.BF16, plan.describe())


@pytest.mark.parametrize("M", [2, 5])
@pytest.mark.parametrize("post", ["bias_gelu_add", "gemm_beta"])
def test_gemv_rows_f16(M, post):
    # f16 operands take the generic kernel and v_dot2_f32_f16
    got, ref, ydt, desc, why = _run_post(M, 259, 4104, post, dt=O.F16, seed=550)
    assert desc.startswith("skinny_f16_gemv_rows_xlds"), desc
    compare(got, ref, ydt, f"f16 M={M} {post} {desc}", explain=why)
