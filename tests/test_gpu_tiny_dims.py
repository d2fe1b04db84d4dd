"""GPU parity at degenerate sizes: dimensions of one (whose descriptor strides are 0), K shorter than a 16-byte chunk,
and ragged dims around them, on every kernel family the planner picks for them (the skinny and GEMV kernels at
M <= 16, the k-slice and 4-wave kernels for f32, the 4-wave kernel for small 16-bit grids) and on the ping-pong kernel
forced. Reference semantics: src/dnn/src/kudnn_gemm.cpp:157-241 (the 2-D paths) and the post-op stages of
kudnn_linear_activationlayer.cpp:40-56, restated by the oracle.
"""
import itertools

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
    K.lib()  # fail loudly if the HIP library is missing


def _run(M, N, Kd, dt, wlayout, seed):
    x = Case([M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, wlayout, seed=seed + 1, dist="normal", lo=0.0, hi=0.3)
    b = Case([1, N], dt, seed=seed + 2, lo=-0.2, hi=0.2)
    c = Case([M, N], dt, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(from_device(dc, dt), ref.buf, dt, f"M={M} N={N} K={Kd} {wlayout} {plan.describe()}")
    return plan.describe()


TINY = list(itertools.product([1, 2, 3, 17], [1, 2, 3, 5], [1, 3, 8, 9]))


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("wlayout", ["BA", "AB"])
def test_tiny_dims(dt, wlayout):
    for i, (M, N, Kd) in enumerate(TINY):
        _run(M, N, Kd, dt, wlayout, 400 + i)


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("MNK", [(20480, 1, 64), (17, 1, 64), (300, 2, 128), (40, 3, 192)])
def test_tiny_n_pingpong(monkeypatch, dt, MNK):
    # N below one 8-row copy block on the ping-pong kernel (forced where the planner would not take it)
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    M, N, Kd = MNK
    assert _run(M, N, Kd, dt, "BA", 450).startswith(("mfma_bf16_pingpong", "mfma_f16_pingpong"))


@pytest.mark.parametrize("MNK", [(1, 1, 16), (3, 1, 32), (17, 2, 48), (128, 1, 1024)])
def test_tiny_n_kslice(monkeypatch, MNK):
    # the f32 k-slice kernel (forced) with one or two weight rows
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "12")
    M, N, Kd = MNK
    assert _run(M, N, Kd, O.F32, "BA", 460).startswith("mfma_f32_kslice")
