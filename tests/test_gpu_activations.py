"""GPU parity of every forward activation kind of the reference (src/dnn/src/kudnn_eltwise.cpp:333-400) as a fused
Linear epilogue, f32 and bf16, on the 4-wave MFMA kernels, the ping-pong kernel, the M = 1 GEMV and the 2 <= M <= 16
skinny kernel, against the CPU oracle.

Kinds with a second parameter (LINEAR, POW, CLIP, CLIP_V2, HARDSIGMOID, HARDSWISH) run through the post-op chain,
which passes both parameters; LinearActivationLayerFWD passes only alpha (its activation's second parameter is 0,
kudnn_linear_activationlayer.cpp:33), which test_linear_act_drops_beta checks.
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
    K.lib()


# kind -> (alpha, beta, input range): LOG / SQRT / fractional POW take positive GEMM outputs
KINDS = {
    "abs": (O.ACT_ABS, 0.0, 0.0, "signed"),
    "exp": (O.ACT_EXP, 0.0, 0.0, "signed"),
    "linear": (O.ACT_LINEAR, 1.5, -0.25, "signed"),
    "log": (O.ACT_LOG, 0.0, 0.0, "positive"),
    "sqrt": (O.ACT_SQRT, 0.0, 0.0, "positive"),
    "square": (O.ACT_SQUARE, 0.0, 0.0, "signed"),
    "tanh": (O.ACT_TANH, 0.0, 0.0, "signed"),
    "sigmoid": (O.ACT_SIGMOID, 0.0, 0.0, "signed"),
    "pow3": (O.ACT_POW, 0.5, 3.0, "signed"),
    "pow_half": (O.ACT_POW, 2.0, 0.5, "positive"),
    "clip": (O.ACT_CLIP, -0.3, 0.4, "signed"),
    "clip_v2": (O.ACT_CLIP_V2, -0.3, 0.4, "signed"),
    "hardsigmoid": (O.ACT_HARDSIGMOID, 0.2, 0.5, "signed"),
    "hardswish": (O.ACT_HARDSWISH, 1.0 / 6.0, 0.5, "signed"),
    "elu": (O.ACT_ELU, 1.3, 0.0, "signed"),
    "elu_dst": (O.ACT_ELU_DST, 0.7, 0.0, "signed"),
    "srelu": (O.ACT_SRELU, 2.0, 0.0, "signed"),
    "mish": (O.ACT_MISH, 0.0, 0.0, "signed"),
}


def run_act(name, dt, M, N, Kd, force=None, monkeypatch=None):
    kind, alpha, beta, dom = KINDS[name]
    lo = 0.05 if dom == "positive" else -1.0
    x = Case([M, Kd], dt, seed=300, lo=lo, hi=1.0)
    w = Case([Kd, N], dt, "BA", seed=301, lo=lo, hi=1.0)
    b = Case([1, N], dt, seed=302, lo=0.0 if dom == "positive" else -0.1, hi=0.1)
    c = Case([M, N], dt, zero=True)
    dc = zeros_device(c)
    ref = c.clone_empty()
    if beta == 0.0:
        plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, alpha, 0.0, kind)
        plan.run(x.device(), w.device(), dc, b.device())
        O.linear_act(x.t, w.t, ref, b.t, kind, alpha)
    else:
        plan = K.LinearPostOps(x.desc, w.desc, c.desc, b.desc, act=kind, act_alpha=alpha, act_beta=beta)
        plan.run(x.device(), w.device(), dc, b.device())
        O.linear_postops(x.t, w.t, ref, b.t, kind, alpha, act_beta=beta)
    torch.cuda.synchronize()
    why = explainer(dt, x.t, w.t, b.t, (M, N), act=kind, act_alpha=alpha, act_beta=beta)
    compare(from_device(dc, dt), ref.buf, dt, f"{plan.describe()} {name}", explain=why)
    return plan


@pytest.mark.parametrize("name", sorted(KINDS))
@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_activation_mfma(name, dt):
    run_act(name, dt, 100, 72, 40)


@pytest.mark.parametrize("name", sorted(KINDS))
@pytest.mark.parametrize("M", [1, 4])
def test_activation_decode_kernels(name, M):
    plan = run_act(name, O.BF16, M, 200, 256)
    assert "skinny" in plan.describe()


@pytest.mark.parametrize("name", ["mish", "clip", "pow3", "elu_dst", "sqrt"])
def test_activation_pingpong(monkeypatch, name):
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    plan = run_act(name, O.BF16, 300, 260, 128)
    assert "pingpong" in plan.describe()


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_round_ties_to_even(dt):
    # integer-valued GEMM (exact in f32 on both sides) plus a bias of k + 0.5: every output is a tie
    M, N, Kd = 64, 48, 16
    x = Case([M, Kd], dt, zero=True)
    w = Case([Kd, N], dt, "BA", zero=True)
    b = Case([1, N], dt, zero=True)
    rng = np.random.default_rng(5)
    xv = rng.integers(-3, 4, size=M * Kd).astype(np.float32)
    wv = rng.integers(-3, 4, size=N * Kd).astype(np.float32)
    bv = (rng.integers(-4, 4, size=N) + 0.5).astype(np.float32)
    for case, v in ((x, xv), (w, wv), (b, bv)):
        case.t.buf[:] = O.from_f32_rne(v, dt) if dt == O.BF16 else v
    c = Case([M, N], dt, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_ROUND)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_ROUND, 0.0)
    got = from_device(dc, dt)
    assert np.array_equal(got, ref.buf), plan.describe()
    vals = O.to_f32(ref.buf, dt)
    assert np.all(vals == np.rint(vals)) and np.any(np.abs(vals) % 2 == 0)


@pytest.mark.parametrize("name", ["linear", "hardsigmoid", "pow3"])
def test_linear_act_drops_beta(name):
    # the same kinds through LinearActivationLayerFWD: the layer's beta is validated, then the activation runs with 0
    kind, alpha, beta, _ = KINDS[name]
    M, N, Kd = 64, 48, 32
    x = Case([M, Kd], O.BF16, seed=310)
    w = Case([Kd, N], O.BF16, "BA", seed=311)
    c = Case([M, N], O.BF16, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, None, alpha, beta, kind)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, None, kind, alpha)
    why = explainer(O.BF16, x.t, w.t, None, (M, N), act=kind, act_alpha=alpha)
    compare(from_device(dc, O.BF16), ref.buf, O.BF16, f"{plan.describe()} {name}", explain=why)
