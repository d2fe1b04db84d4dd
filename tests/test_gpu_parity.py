"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on identical seeded inputs.

Small problems are checked in full. The configurations C1..C5 run at full size on the GPU. C1, C2, C3 and the C4 shapes
are checked in every output element. C5 (2.3e12 flops) is checked on a sample of output rows: rows of a GEMM are
independent, so the oracle computes exactly those rows from the matching rows of X.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, PostOpsExplainer, compare, dense_rows, explainer, from_device, sample_rows, zeros_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()  # fail loudly if the HIP library is missing


def as2d(t: O.Tensor) -> O.Tensor:
    """A broadcast-batch weight/bias [1,...,r,c] as the 2-D tensor [r,c] (same buffer)."""
    return O.Tensor(t.dims[-2:], t.strides[-2:], t.dtype, t.buf)


# ---------------------------------------------------------------------------------------------------
# small problems, checked in full


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("wlayout", ["BA", "AB"])
@pytest.mark.parametrize("mnk", [(64, 64, 64), (100, 72, 40), (300, 260, 200), (17, 33, 24), (5, 48, 64)])
@pytest.mark.parametrize("act", [O.ACT_RELU, O.ACT_SWISH, O.ACT_GELU_TANH, O.ACT_GELU_ERF])
def test_linear_act_small(dt, wlayout, mnk, act):
    M, N, Kd = mnk
    x = Case([M, Kd], dt, "AB", seed=10)
    w = Case([Kd, N], dt, wlayout, seed=11)
    b = Case([1, N], dt, "AB", seed=12, lo=-0.1, hi=0.1)
    c = Case([M, N], dt, "AB", zero=True)
    alpha = 0.0 if act == O.ACT_RELU else 1.0
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, alpha, 0.0, act)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, act, alpha)
    why = explainer(dt, x.t, w.t, b.t, (M, N), act=act, act_alpha=alpha)
    compare(from_device(dc, dt), ref.buf, dt, f"{plan.describe()}", explain=why)


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("bias_shape", [None, "1N", "M1", "MN", "11"])
def test_gemm_bias_kinds(dt, bias_shape):
    M, N, Kd = 96, 80, 72
    x = Case([M, Kd], dt, seed=20)
    w = Case([Kd, N], dt, "BA", seed=21)
    bdims = {"1N": [1, N], "M1": [M, 1], "MN": [M, N], "11": [1, 1]}.get(bias_shape)
    b = Case(bdims, dt, seed=22) if bdims else None
    c = Case([M, N], dt, seed=23)  # beta != 0 reads the old C
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc if b else None)
    dc = c.device()
    plan.run(x.device(), w.device(), dc, b.device() if b else None, alpha=0.75, beta=0.5)
    torch.cuda.synchronize()
    ref = O.Tensor(c.t.dims, c.t.strides, dt, c.t.buf.copy())
    O.gemm(x.t, w.t, ref, b.t if b else None, alpha=0.75, beta=0.5)
    compare(from_device(dc, dt), ref.buf, dt, plan.describe())


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("layouts", [("AB", "AB", "AB"), ("BA", "BA", "AB"), ("AB", "BA", "BA"), ("BA", "AB", "BA")])
def test_gemm_layouts(dt, layouts):
    la, lb, lc = layouts
    M, N, Kd = 70, 90, 56
    x = Case([M, Kd], dt, la, seed=30)
    w = Case([Kd, N], dt, lb, seed=31)
    c = Case([M, N], dt, lc, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc)
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref)
    compare(from_device(dc, dt), ref.buf, dt, plan.describe())


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("kind", [O.RES_IDENTIAL, O.RES_EXT, O.RES_MUL])
def test_linear_res(dt, kind):
    M, N, Kd, L = 64, 96, 80, 48
    x = Case([M, Kd], dt, seed=40)
    w = Case([Kd, N], dt, "BA", seed=41)
    b = Case([1, N], dt, seed=42, lo=-0.1, hi=0.1)
    c = Case([M, N], dt, zero=True)
    if kind == O.RES_MUL:
        res = Case([N, L], dt, seed=43)
        lr = Case([M, L], dt, zero=True)
    else:
        res = Case([M, N], dt, seed=43)
        lr = Case([M, N], dt, zero=True)
    gamma = 0.625
    plan = K.LinearRes(x.desc, w.desc, c.desc, b.desc, res.desc, lr.desc, 1.0, 0.0, 1.0, kind)
    dc, dlr = zeros_device(c), zeros_device(lr)
    plan.run(x.device(), w.device(), dc, b.device(), res.device(), dlr, gamma)
    torch.cuda.synchronize()
    rc, rlr = c.clone_empty(), lr.clone_empty()
    O.linear_res(x.t, w.t, rc, b.t, res.t, rlr, kind, gamma)
    compare(from_device(dc, dt), rc.buf, dt, plan.describe() + " C")
    why = None if kind == O.RES_MUL else explainer(dt, x.t, w.t, b.t, (M, N), src=res.t, gamma=gamma,
                                                   binary=O.BIN_ADD if kind == O.RES_IDENTIAL else O.BIN_EXT)
    compare(from_device(dlr, dt), rlr.buf, dt, plan.describe() + " linearRes", explain=why)


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_batched_broadcast(dt):
    # 4-D batch with broadcast weight over dim 1 and a bias broadcast over both batch dims
    x = Case([3, 2, 40, 24], dt, seed=50)
    w = Case([3, 1, 24, 56], dt, seed=51)
    b = Case([1, 1, 1, 56], dt, seed=52, lo=-0.1, hi=0.1)
    c = Case([3, 2, 40, 56], dt, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_SWISH, 1.0)
    compare(from_device(dc, dt), ref.buf, dt, plan.describe())


def test_host_pointers_staged():
    # reference-style call with host buffers: the library stages them through device memory
    dt = O.F32
    x = Case([110, 20], dt, seed=60)
    w = Case([20, 200], dt, "AB", seed=61)
    b = Case([110, 200], dt, seed=62)
    c = Case([110, 200], dt, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    out = c.clone_empty()
    plan.run(x.t.buf, w.t.buf, out.buf, b.t.buf)
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(out.buf, ref.buf, dt, plan.describe())


# ---------------------------------------------------------------------------------------------------
# BASELINE configs at full size


def test_c1_fp32_relu_full():
    x = Case([128, 1024], O.F32, seed=0)
    w = Case([1024, 1024], O.F32, "BA", seed=1)
    b = Case([1, 1024], O.F32, seed=2, lo=-0.1, hi=0.1)
    c = Case([128, 1024], O.F32, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    assert "kslice" in plan.describe(), plan.describe()
    compare(from_device(dc, O.F32), ref.buf, O.F32, "C1")


@pytest.mark.parametrize("dims", [(128, 1024, 1024), (100, 1000, 520), (1, 4096, 256), (37, 3000, 96), (16, 6000, 48),
                                  (250, 260, 2048)])
@pytest.mark.parametrize("bias", [None, "1N", "MN"])
def test_f32_kslice_shapes(dims, bias):
    # the k-slice kernel (one 16 x 32 tile per workgroup, K over its waves): ragged M and N, K tails the pack pads,
    # every bias kind, beta != 0
    M, N, Kd = dims
    x = Case([M, Kd], O.F32, seed=60)
    w = Case([Kd, N], O.F32, "BA", seed=61)
    bd = {"1N": [1, N], "MN": [M, N]}.get(bias)
    b = Case(bd, O.F32, seed=62) if bd else None
    c = Case([M, N], O.F32, seed=63)
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc if b else None)
    assert "kslice" in plan.describe(), plan.describe()
    dc = c.device()
    plan.run(x.device(), w.device(), dc, b.device() if b else None, alpha=0.75, beta=0.5)
    torch.cuda.synchronize()
    ref = O.Tensor(c.t.dims, c.t.strides, O.F32, c.t.buf.copy())
    O.gemm(x.t, w.t, ref, b.t if b else None, alpha=0.75, beta=0.5)
    compare(from_device(dc, O.F32), ref.buf, O.F32, plan.describe())


@pytest.mark.parametrize("Kd", [512, 768, 1536, 3072, 4096, 2560])
def test_f32_kslice_whole_line_forms(Kd):
    # K in whole 256-element blocks: 8 waves loading whole lines through LDS, 2, 3, 6 pairs per wave with all loads in
    # flight, 12 and 16 pairs with 6 in flight (K = 3072, 4096); K = 2560 (10 blocks) takes the 4-wave form. Edge tiles
    # in M and N
    M, N = 120, 1000
    x = Case([M, Kd], O.F32, seed=66)
    w = Case([Kd, N], O.F32, "BA", seed=67)
    b = Case([1, N], O.F32, seed=68, lo=-0.1, hi=0.1)
    c = Case([M, N], O.F32, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    assert "kslice" in plan.describe(), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(from_device(dc, O.F32), ref.buf, O.F32, plan.describe())


def test_f32_kslice_batched_and_repeatable():
    # batches in grid.y (a weight per batch); two runs give the same bits
    x = Case([3, 2, 40, 264], O.F32, seed=64)
    w = Case([3, 2, 264, 700], O.F32, seed=65)
    c = Case([3, 2, 40, 700], O.F32, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, None, 1.0, 0.0, K.ACT_SWISH)
    assert "kslice" in plan.describe(), plan.describe()
    outs = []
    for _ in range(2):
        dc = zeros_device(c)
        plan.run(x.device(), w.device(), dc)
        torch.cuda.synchronize()
        outs.append(from_device(dc, O.F32))
    assert np.array_equal(outs[0], outs[1])
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, None, O.ACT_SWISH, 1.0)
    compare(outs[0], ref.buf, O.F32, plan.describe())


def test_c2_fp32_silu_full():
    # C2 at its full size, every output element against the oracle (about 1.4e11 flops of oracle time)
    M, Kd, N = 2048, 4096, 4096
    x = Case([M, Kd], O.F32, seed=0, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.F32, "BA", seed=1, dist="normal", lo=0.0, hi=1.0 / 64)
    b = Case([1, N], O.F32, seed=2, dist="normal", lo=0.0, hi=0.02)
    c = Case([M, N], O.F32, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_SWISH, 1.0)
    maxnorm, _ = compare(from_device(dc, O.F32), ref.buf, O.F32, "C2 " + plan.describe())
    print(f"C2 all {M} x {N}: max-normalised error {maxnorm:.3e}")


def test_c3_bf16_gelu_residual_full():
    # C3 at its full size (the bench workload's shape and inputs), every output element against the oracle (about
    # 3.7e11 flops of oracle time)
    M, Kd, N = 4096, 4096, 11008
    x = Case([M, Kd], O.BF16, seed=0, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=1, dist="normal", lo=0.0, hi=0.02)
    b = Case([1, N], O.BF16, zero=True)
    r = Case([M, N], O.BF16, seed=3, dist="normal", lo=0.0, hi=1.0)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=r.desc)
    assert plan.describe().startswith("mfma_bf16_pingpong_256x256"), plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device(), r.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, r.t)
    why = PostOpsExplainer(x.t, w.t, b.t, (M, N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=r.t)
    maxnorm, exact = compare(from_device(dy, O.BF16), ref.buf, O.BF16, "C3 " + plan.describe(), explain=why)
    print(f"C3 all {M} x {N}: max-normalised error {maxnorm:.3e}, bit-exact fraction {exact:.5f}, "
          f"one-ulp exceptions {why.counts}")


def _random_gemm_cases(count=24, seed=4051):
    # seeded draws over the prefill kernels: M in [17, 2500], N in [16, 8000], K in [8, 2000] (tile counts either side
    # of the ping-pong threshold, ragged edges, K tails that pack); dtype and weight layout alternate
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(17, 2501)), int(rng.integers(16, 8001)), int(rng.integers(8, 2001)),
             O.BF16 if i % 2 == 0 else O.F32, "BA" if i % 4 < 2 else "AB") for i in range(count)]


@pytest.mark.parametrize("M,N,Kd,dt,wl", _random_gemm_cases())
def test_gemm_random_shapes(M, N, Kd, dt, wl):
    # bf16: bias + ReLU + residual add, where a 1-ULP difference of the GEMM result stays 1 ULP; f32: bias + SiLU
    x = Case([M, Kd], dt, seed=230, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, wl, seed=231, dist="normal", lo=0.0, hi=0.03)
    b = Case([1, N], dt, seed=232, lo=-0.2, hi=0.2)
    y = Case([M, N], dt, zero=True)
    rows = sample_rows(M, 12)
    dy = zeros_device(y)
    ref = O.empty((len(rows), N), (N, 1), dt)
    if dt == O.BF16:
        s = Case([M, N], dt, seed=233, lo=-1.0, hi=1.0)
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_RELU, binary=K.BIN_ADD, src=s.desc)
        plan.run(x.device(), w.device(), dy, b.device(), s.device())
        xr, sr = dense_rows(x.t, rows), dense_rows(s.t, rows)
        O.linear_postops(xr, w.t, ref, b.t, O.ACT_RELU, 0.0, O.BIN_ADD, sr)
        why = PostOpsExplainer(xr, w.t, b.t, (len(rows), N), act=O.ACT_RELU, binary=O.BIN_ADD, src=sr)
    else:
        why = None
        plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
        plan.run(x.device(), w.device(), dy, b.device())
        O.linear_act(dense_rows(x.t, rows), w.t, ref, b.t, O.ACT_SWISH, 1.0)
    torch.cuda.synchronize()
    got = from_device(dy, dt).reshape(M, N)
    _, exact = compare(got[rows].reshape(-1), ref.buf, dt, f"M={M} N={N} K={Kd} {wl} {plan.describe()}", explain=why)
    if dt == O.BF16:
        assert exact > 0.99, f"only {exact:.4f} of the elements are bit-exact"


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("N", [4096, 14336])
def test_c4_skinny_mul(M, N):
    Kd = 4096
    x = Case([M, Kd], O.BF16, seed=0, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=1, dist="normal", lo=0.0, hi=0.02)
    m2 = Case([M, N], O.BF16, seed=3, lo=0.5, hi=1.5)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, binary=K.BIN_MUL, src=m2.desc)
    assert plan.describe().startswith("skinny")
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, None, m2.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, None, O.ACT_NONE, 0.0, O.BIN_MUL, m2.t)
    compare(from_device(dy, O.BF16), ref.buf, O.BF16, f"C4 M={M} N={N}")


@pytest.mark.parametrize("M,N,Kd", [(9, 4112, 2100), (12, 4096, 2304), (16, 4104, 4096), (12, 1024, 2100),
                                    (8, 8200, 2100), (7, 8192, 4096), (6, 8192, 2304)])
def test_skinny_rows_forms(monkeypatch, M, N, Kd):
    # the 16-row kernel (forced: the planner takes the K-split GEMV for these one-batch calls with K <= 4096)
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "20")
    # M > 8 with >= 256 row groups, and M = 7, 8 with >= 512, run 2-wave workgroups with the next weight block in
    # flight and X's rows loaded whole through a second LDS tile (rows m >= M read zero): an odd count of 256-element
    # K blocks (K = 2100 packs to 9 blocks, 2304 is exactly 9) ends one wave on a block with no successor; N not a
    # multiple of 16 leaves a ragged last row group. N = 1024 (64 row groups) stays on the 16-wave form, M = 6 on the
    # 8-wave form.
    # The chain is bias + ReLU + add: a 1-ULP difference of the bf16 GEMM result (f32 summation order) stays 1 ULP,
    # where GELU's extra rounding could double it; a lost or repeated K block would move almost every element.
    x = Case([M, Kd], O.BF16, seed=210, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=211, dist="normal", lo=0.0, hi=0.03)
    b = Case([1, N], O.BF16, seed=212, lo=-0.2, hi=0.2)
    s = Case([M, N], O.BF16, seed=213, lo=-1.0, hi=1.0)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_RELU, binary=K.BIN_ADD, src=s.desc)
    assert plan.describe().startswith("skinny_bf16_16xK"), plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device(), s.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0, O.BIN_ADD, s.t)
    why = explainer(O.BF16, x.t, w.t, b.t, (M, N), act=O.ACT_RELU, binary=O.BIN_ADD, src=s.t)
    _, exact = compare(from_device(dy, O.BF16), ref.buf, O.BF16, f"skinny M={M} N={N} K={Kd} {plan.describe()}",
                       explain=why)
    assert exact > 0.99, f"only {exact:.4f} of the elements are bit-exact"


def _random_skinny_shapes(count=20, seed=2024):
    # seeded (M, N, K) draws over the decode kernels: M in [2, 16] (both sides of M > 8), N in [16, 10000] (row-group
    # counts either side of 256 and 512), K in [8, 3000] (K tails that pack, odd and even K-block counts)
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(2, 17)), int(rng.integers(16, 10001)), int(rng.integers(8, 3001))) for _ in range(count)]


@pytest.mark.parametrize("M,N,Kd", _random_skinny_shapes())
def test_skinny_random_shapes(M, N, Kd):
    x = Case([M, Kd], O.BF16, seed=220, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=221, dist="normal", lo=0.0, hi=0.03)
    b = Case([1, N], O.BF16, seed=222, lo=-0.2, hi=0.2)
    s = Case([M, N], O.BF16, seed=223, lo=-1.0, hi=1.0)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_RELU, binary=K.BIN_ADD, src=s.desc)
    assert plan.describe().startswith("skinny"), plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device(), s.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0, O.BIN_ADD, s.t)
    why = explainer(O.BF16, x.t, w.t, b.t, (M, N), act=O.ACT_RELU, binary=O.BIN_ADD, src=s.t)
    _, exact = compare(from_device(dy, O.BF16), ref.buf, O.BF16, f"skinny M={M} N={N} K={Kd} {plan.describe()}",
                       explain=why)
    assert exact > 0.99, f"only {exact:.4f} of the elements are bit-exact"


@pytest.mark.parametrize("Kd", [40, 1001, 1024, 2048, 4096, 9000])
@pytest.mark.parametrize("post", ["bias_gelu_add", "swish_f32", "gemm_beta"])
def test_m1_row_gemv(Kd, post):
    # M = 1 takes the row-per-wave GEMV: K blocks of 512 chunks, a K tail (K % 8 != 0 packs the operands with zero
    # padding), every epilogue option through the generic per-element path
    N = 300
    ydt = O.F32 if post in ("swish_f32", "gemm_beta") else O.BF16
    x = Case([1, Kd], O.BF16, seed=200, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=201, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, N], ydt, seed=202, lo=-0.2, hi=0.2)
    y = Case([1, N], ydt, seed=203, lo=-1.0, hi=1.0) if post == "gemm_beta" else Case([1, N], ydt, zero=True)
    dy = torch.from_numpy(y.t.buf.view(np.int16).copy() if ydt != O.F32 else y.t.buf.copy()).cuda()
    ref = O.Tensor(y.t.dims, y.t.strides, ydt, y.t.buf.copy())
    if post == "bias_gelu_add":
        s = Case([1, N], ydt, seed=204, lo=-1.0, hi=1.0)
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
        plan.run(x.device(), w.device(), dy, b.device(), s.device())
        O.linear_postops(x.t, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, s.t)
        why = explainer(ydt, x.t, w.t, b.t, (1, N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=s.t)
    elif post == "swish_f32":
        plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
        plan.run(x.device(), w.device(), dy, b.device())
        O.linear_act(x.t, w.t, ref, b.t, O.ACT_SWISH, 1.0)
    else:
        plan = K.Gemm(x.desc, w.desc, y.desc, b.desc)
        plan.run(x.device(), w.device(), dy, b.device(), alpha=0.5, beta=0.25)
        O.gemm(x.t, w.t, ref, b.t, 0.5, 0.25)
    assert plan.describe().startswith("skinny")
    torch.cuda.synchronize()
    compare(from_device(dy, ydt), ref.buf, ydt, f"M=1 K={Kd} {post} {plan.describe()}",
            explain=why if post == "bias_gelu_add" else None)


def test_m1_row_gemv_batched_broadcast_weight():
    # 3 batches of one row each against one K-major weight (packed once, batch stride 0)
    Kd, N = 640, 200
    x = Case([3, 1, Kd], O.BF16, "ABC", seed=210, dist="normal", lo=0.0, hi=1.0)
    w = Case([1, Kd, N], O.BF16, "ABC", seed=211, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, 1, N], O.BF16, "ABC", seed=212, lo=-0.1, hi=0.1)
    c = Case([3, 1, N], O.BF16, "ABC", zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(from_device(dc, O.BF16), ref.buf, O.BF16, plan.describe())


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("mnk", [(128, 1024, 1024), (100, 200, 2048), (64, 70, 512)])
@pytest.mark.parametrize("post", ["gelu_add", "swish_mul", "gemm_beta"])
def test_split_k_small_grids(monkeypatch, dt, mnk, post):
    # grids of fewer than 128 tiles with at least 8 k-tiles run split along K: raw f32 partials in the plan's
    # workspace, then one pass that sums them in split order and applies the whole epilogue (f32 forced onto the
    # 64 x 64 kernel, which the planner gives to the k-slice kernel where that one makes 128 tiles or more; bf16 forced
    # onto the 128 x 128 kernel, which the planner replaces by the ping-pong kernel's K slices from 32 k-tiles on)
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "11" if dt == O.F32 else "3")
    M, N, Kd = mnk
    x = Case([M, Kd], dt, seed=220, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, "BA", seed=221, dist="normal", lo=0.0, hi=1.0 / 32)
    b = Case([1, N], dt, seed=222, lo=-0.2, hi=0.2)
    y = Case([M, N], dt, seed=223, lo=-1.0, hi=1.0) if post == "gemm_beta" else Case([M, N], dt, zero=True)
    dy = torch.from_numpy(y.t.buf.view(np.int16).copy() if dt != O.F32 else y.t.buf.copy()).cuda()
    ref = O.Tensor(y.t.dims, y.t.strides, dt, y.t.buf.copy())
    if post == "gemm_beta":
        plan = K.Gemm(x.desc, w.desc, y.desc, b.desc)
        plan.run(x.device(), w.device(), dy, b.device(), alpha=0.5, beta=0.25)
        O.gemm(x.t, w.t, ref, b.t, 0.5, 0.25)
    else:
        act, binary = (O.ACT_GELU_TANH, O.BIN_ADD) if post == "gelu_add" else (O.ACT_SWISH, O.BIN_MUL)
        s = Case([M, N], dt, seed=224, lo=0.5, hi=1.5)
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=act, act_alpha=1.0, binary=binary, src=s.desc)
        plan.run(x.device(), w.device(), dy, b.device(), s.device())
        O.linear_postops(x.t, w.t, ref, b.t, act, 1.0, binary, s.t)
    why = None if post == "gemm_beta" else explainer(dt, x.t, w.t, b.t, (M, N), act=act, act_alpha=1.0,
                                                     binary=binary, src=s.t)
    torch.cuda.synchronize()
    compare(from_device(dy, dt), ref.buf, dt, f"split-K {post} {plan.describe()}", explain=why)


def test_plan_workspace_across_streams(monkeypatch):
    # one plan with a workspace (split-K) run alternately on two streams: the workspace is ordered between them
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "11")  # the 64 x 64 kernel, split along K
    M, N, Kd = 128, 1024, 1024
    dt = O.F32
    xs = [Case([M, Kd], dt, seed=230 + i, dist="normal", lo=0.0, hi=1.0) for i in range(4)]
    w = Case([Kd, N], dt, "BA", seed=240, dist="normal", lo=0.0, hi=1.0 / 32)
    y = Case([M, N], dt, zero=True)
    plan = K.LinearActivation(xs[0].desc, w.desc, y.desc, None, 0.0, 0.0, K.ACT_RELU)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    dw = w.device()
    dxs = [x.device() for x in xs]
    outs = [zeros_device(y) for _ in xs]
    torch.cuda.synchronize()
    for rep in range(3):
        for i, (dx, dout) in enumerate(zip(dxs, outs)):
            plan.run(dx, dw, dout, None, stream=streams[i % 2])
    torch.cuda.synchronize()
    for x, dout in zip(xs, outs):
        ref = y.clone_empty()
        O.linear_act(x.t, w.t, ref, None, O.ACT_RELU, 0.0)
        compare(from_device(dout, dt), ref.buf, dt, f"two streams {plan.describe()}")


def test_c5_bf16_3d_silu_kmajor_rows():
    B, S, Kd, N = 8, 2048, 5120, 13824
    x = Case([B, S, Kd], O.BF16, "ABC", seed=0, dist="normal", lo=0.0, hi=1.0)
    w = Case([1, Kd, N], O.BF16, "ABC", seed=1, dist="normal", lo=0.0, hi=0.014)
    b = Case([1, 1, N], O.BF16, "ABC", seed=2, dist="normal", lo=0.0, hi=0.02)
    y = Case([B, S, N], O.BF16, "ABC", zero=True)
    plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    got = from_device(dy, O.BF16).reshape(B * S, N)
    rows = sample_rows(B * S, 24)  # 64 bands of 256 rows: one row of each, the edges, and random rows
    ref = O.empty((len(rows), N), (N, 1), O.BF16)
    O.linear_act(dense_rows(x.t, rows), as2d(w.t), ref, as2d(b.t), O.ACT_SWISH, 1.0)
    compare(got[rows].reshape(-1), ref.buf, O.BF16, "C5 " + plan.describe())
    assert len(rows) >= B * S // 256
    # the K-major weight is read in place (transposing LDS reads), not packed
    assert "kmajorB" in plan.describe() and "packB" not in plan.describe(), plan.describe()


@pytest.fixture(scope="module")
def c5_full():
    # C5 at its full size with the bench's seeds, run once; the tests below check its output batch by batch
    B, S, Kd, N = 8, 2048, 5120, 13824
    x = Case([B, S, Kd], O.BF16, "ABC", seed=0, dist="normal", lo=0.0, hi=1.0)
    w = Case([1, Kd, N], O.BF16, "ABC", seed=1, dist="normal", lo=0.0, hi=0.014)
    b = Case([1, 1, N], O.BF16, "ABC", seed=2, dist="normal", lo=0.0, hi=0.02)
    y = Case([B, S, N], O.BF16, "ABC", zero=True)
    plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    got = from_device(dy, O.BF16).reshape(B * S, N)
    return x, w, b, got, plan.describe(), (B, S, Kd, N)


@pytest.mark.parametrize("batch", range(8))
def test_c5_bf16_3d_silu_kmajor_full(c5_full, batch):
    # every output element of C5 (about 2.9e11 oracle flops per batch of 2048 rows)
    x, w, b, got, desc, (B, S, Kd, N) = c5_full
    rows = np.arange(batch * S, (batch + 1) * S)
    ref = O.empty((S, N), (N, 1), O.BF16)
    O.linear_act(dense_rows(x.t, rows), as2d(w.t), ref, as2d(b.t), O.ACT_SWISH, 1.0)
    maxnorm, exact = compare(got[rows].reshape(-1), ref.buf, O.BF16, f"C5 batch {batch} {desc}")
    print(f"C5 batch {batch}: max-normalised error {maxnorm:.3e}, bit-exact fraction {exact:.5f}")


def _kmajor_case(dt, lead, M, Kd, N, wlead, act, bias, seed):
    x = Case(lead + [M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case(wlead + [Kd, N], dt, seed=seed + 1, dist="normal", lo=0.0, hi=0.05)  # standard layout: [K][N]
    b = Case([1] * len(lead) + [1, N], dt, seed=seed + 2, lo=-0.2, hi=0.2) if bias else None
    y = Case(lead + [M, N], dt, zero=True)
    return x, w, b, y


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("shape", [([], 256, 64, 256, []), ([], 300, 640, 768, []), ([], 1000, 256, 1536, []),
                                   ([2], 260, 192, 512, [2]), ([3], 128, 128, 256, [1]), ([], 300, 640, 1160, []),
                                   ([], 256, 128, 136, []), ([2], 260, 192, 520, [2]), ([3], 128, 128, 264, [1])])
@pytest.mark.parametrize("act", [K.ACT_UNIMPLEMENTED, K.ACT_SWISH, K.ACT_GELU_TANH])
def test_kmajor_weight_in_place(monkeypatch, dt, shape, act):
    # a [K][N] weight read in place by the ping-pong kernel (M edges, N edges with 8 or 136 columns in the last tile,
    # where the copies of the last k-row run past the operand's end, batched and broadcast weights, every
    # fixed epilogue form) against the oracle, and bit for bit against the same plan with the weight packed to [N][K]:
    # both feed the MFMAs the same k groups in the same order
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    lead, M, Kd, N, wlead = shape
    x, w, b, y = _kmajor_case(dt, lead, M, Kd, N, wlead, act, act != K.ACT_UNIMPLEMENTED, 700)
    outs = []
    for packed in (False, True):
        if packed:
            monkeypatch.setenv("KUDNN_HIP_PACK_KMAJOR", "1")
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc if b else None, act=act, act_alpha=1.0)
        assert ("packB" in plan.describe()) == packed and ("kmajorB" in plan.describe()) != packed, plan.describe()
        dy = zeros_device(y)
        plan.run(x.device(), w.device(), dy, b.device() if b else None)
        torch.cuda.synchronize()
        outs.append(from_device(dy, dt))
    monkeypatch.delenv("KUDNN_HIP_PACK_KMAJOR")
    assert np.array_equal(outs[0], outs[1]), "in-place and packed K-major weights differ"
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t if b else None, act, 1.0, O.BIN_NONE, None)
    compare(outs[0], ref.buf, dt, "kmajor " + plan.describe(),
            explain=explainer(dt, x.t, w.t, b.t if b else None, tuple(y.t.dims[-2:]), act=act, act_alpha=1.0)
            if not lead and dt == O.BF16 else None)


def test_kmajor_weight_ragged_n_is_packed(monkeypatch):
    # N not a multiple of 8 splits the last 16-byte column chunk of each k-row: the weight is packed to [N][K] instead
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    x, w, b, y = _kmajor_case(O.BF16, [], 300, 640, 1156, [], K.ACT_GELU_TANH, True, 710)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, act_alpha=1.0)
    assert "packB" in plan.describe(), plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, K.ACT_GELU_TANH, 1.0, O.BIN_NONE, None)
    compare(from_device(dy, O.BF16), ref.buf, O.BF16, plan.describe())


# ---------------------------------------------------------------------------------------------------
# the 8-wave ping-pong kernel (chosen for large bf16 problems) on shapes that exercise its edges:
# partial 256-row / 256-column tiles (rows past the end read as zero), a single k-tile, many k-tiles,
# batches, and every epilogue kind


@pytest.fixture
def force_pingpong(monkeypatch):
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")


@pytest.mark.parametrize("mnk", [(256, 256, 64), (300, 520, 192), (257, 255, 64), (512, 768, 1024), (40, 600, 128)])
@pytest.mark.parametrize("post", ["none", "bias_gelu_add", "swish", "mul", "relu_ext"])
def test_pingpong_shapes_and_epilogues(force_pingpong, mnk, post):
    M, N, Kd = mnk
    dt = O.BF16
    x = Case([M, Kd], dt, seed=70, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, "BA", seed=71, dist="normal", lo=0.0, hi=0.05)
    y = Case([M, N], dt, zero=True)
    b = Case([1, N], dt, seed=72, lo=-0.1, hi=0.1) if post in ("bias_gelu_add", "relu_ext") else None
    s = Case([M, N], dt, seed=73, lo=0.5, hi=1.5) if post in ("bias_gelu_add", "mul", "relu_ext") else None
    act, aa, binary = {"none": (O.ACT_NONE, 0.0, O.BIN_NONE), "bias_gelu_add": (O.ACT_GELU_TANH, 0.0, O.BIN_ADD),
                       "swish": (O.ACT_SWISH, 1.0, O.BIN_NONE), "mul": (O.ACT_NONE, 0.0, O.BIN_MUL),
                       "relu_ext": (O.ACT_RELU, 0.0, O.BIN_EXT)}[post]
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc if b else None, act=act, act_alpha=aa, binary=binary,
                           src=s.desc if s else None)
    assert "pingpong" in plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device() if b else None, s.device() if s else None, gamma=0.75)
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t if b else None, act, aa, binary, s.t if s else None, 0.75)
    why = PostOpsExplainer(x.t, w.t, b.t if b else None, (M, N), act=act, act_alpha=aa, binary=binary,
                           src=s.t if s else None, gamma=0.75)
    compare(from_device(dy, dt), ref.buf, dt, f"{plan.describe()} {post}", explain=why)


@pytest.mark.parametrize("mnk", [(512, 512, 128), (300, 520, 192)])
@pytest.mark.parametrize("ydt", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("bias_rows", [False, True])
def test_pingpong_epilogue_forms(force_pingpong, mnk, ydt, bias_rows):
    # bf16 operands with f32 / f16 / bf16 outputs: the kernel's fixed-type forms (bf16, f32) and its generic form
    # (f16); a bias per column ([1, N]) or per row ([M, 1]); full tiles and tiles at the matrix edge
    M, N, Kd = mnk
    x = Case([M, Kd], O.BF16, seed=90, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=91, dist="normal", lo=0.0, hi=0.05)
    y = Case([M, N], ydt, zero=True)
    b = Case([M, 1] if bias_rows else [1, N], ydt, seed=92, lo=-0.2, hi=0.2)
    s = Case([M, N], ydt, seed=93, lo=-1.0, hi=1.0)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_ERF, binary=K.BIN_ADD, src=s.desc)
    assert "pingpong" in plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device(), s.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, O.ACT_GELU_ERF, 0.0, O.BIN_ADD, s.t, 1.0)
    why = PostOpsExplainer(x.t, w.t, b.t, (M, N), act=O.ACT_GELU_ERF, binary=O.BIN_ADD, src=s.t) \
        if ydt == O.BF16 else None
    compare(from_device(dy, ydt), ref.buf, ydt, f"{plan.describe()} ydt={ydt} bias_rows={bias_rows}", explain=why)


def _rounding_boundary_values(seed: int = 7, nans: bool = False) -> np.ndarray:
    """f32 bit patterns at every kind of f32 -> bf16 rounding boundary: upper halves (sign, exponent including 0 for
    denormals, top mantissa bits; random plus special ones) joined with lower halves 0, 1, 0x7fff, 0x8000 (the tie),
    0x8001 and 0xffff. That covers ties to even and to odd, the largest finite values (which round to +-Inf), +-Inf
    and, with nans, quiet and signalling NaNs with payloads in either half."""
    rng = np.random.default_rng(seed)
    special = [0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080, 0x807F, 0x7F7F, 0xFF7F, 0x7F80, 0xFF80, 0x3F80, 0x3F81,
               0xBF80, 0xBF81, 0x7FC0, 0xFFC0, 0x7FBF, 0x7F81]
    hi = np.concatenate([rng.integers(0, 1 << 16, 1500), special]).astype(np.uint32)
    lo = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    u = ((hi[:, None] << 16) | lo[None, :]).reshape(-1)
    return u if nans else u[(u & 0x7FFFFFFF) <= 0x7F800000]


@pytest.mark.parametrize("M", [3, 64])
@pytest.mark.parametrize("via", ["weight", "bias"])
def test_bf16_output_rounding_boundaries(M, via):
    # Y(bf16) = X(f32, ones) @ W(f32) + bias(f32): each output is one W value (zero bias) or one bias value (zero W),
    # so the store is the RNE of arbitrary f32 bit patterns, checked bit for bit against the oracle. NaNs go through
    # the bias only (the epilogue's f32 add keeps their payloads; the MFMA need not).
    u = _rounding_boundary_values(nans=(via == "bias"))
    N = u.size
    vals = u.view(np.float32)
    zeros = np.zeros(N, np.float32)
    x = O.Tensor((M, 1), (1, 1), O.F32, np.ones(M, np.float32))
    w = O.Tensor((1, N), (1, 1), O.F32, vals.copy() if via == "weight" else zeros)  # BA: physically [N][1]
    b = O.Tensor((1, N), (0, 1), O.F32, zeros if via == "weight" else vals.copy())  # a size-1 dim has stride 0
    ref = O.empty((M, N), (N, 1), O.BF16)
    O.linear_postops(x, w, ref, b)
    want = O.from_f32_rne(vals, O.BF16)
    # the oracle stores the RNE of each value (-0 excepted: +0 + -0 is +0)
    nz = u != 0x80000000
    assert np.array_equal(ref.buf.reshape(M, N)[0][nz], want[nz])
    assert np.count_nonzero(want != (u >> 16).astype(np.uint16)) > 1000  # many cases round away from truncation
    plan = K.LinearPostOps(K.desc([M, 1], K.F32), K.desc([1, N], K.F32, "BA"), K.desc([M, N], K.BF16),
                           K.desc([1, N], K.F32))
    dy = torch.zeros(M * N, dtype=torch.int16, device="cuda")
    dev = lambda t: torch.from_numpy(t.buf).cuda()
    plan.run(dev(x), dev(w), dy, dev(b))
    torch.cuda.synchronize()
    got = dy.cpu().numpy().view(np.uint16)
    bad = np.nonzero(got != ref.buf)[0]
    assert bad.size == 0, (f"{plan.describe()}: {bad.size} outputs differ, first value {u[bad[0] % N]:#010x} "
                           f"got {got[bad[0]]:#06x} want {ref.buf[bad[0]]:#06x}")


@pytest.mark.parametrize("kind", [O.RES_IDENTIAL, O.RES_EXT])
def test_pingpong_linear_res_stores_c(force_pingpong, kind):
    # LinearResFWD writes C and linearRes from one launch (the generic form of the epilogue)
    M, N, Kd = 300, 264, 128
    x = Case([M, Kd], O.BF16, seed=94, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=95, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, N], O.BF16, seed=96, lo=-0.1, hi=0.1)
    c = Case([M, N], O.BF16, zero=True)
    res = Case([M, N], O.BF16, seed=97)
    lr = Case([M, N], O.BF16, zero=True)
    plan = K.LinearRes(x.desc, w.desc, c.desc, b.desc, res.desc, lr.desc, 1.0, 0.0, 1.0, kind)
    assert "pingpong" in plan.describe()
    dc, dlr = zeros_device(c), zeros_device(lr)
    plan.run(x.device(), w.device(), dc, b.device(), res.device(), dlr, 0.625)
    torch.cuda.synchronize()
    rc, rlr = c.clone_empty(), lr.clone_empty()
    O.linear_res(x.t, w.t, rc, b.t, res.t, rlr, kind, 0.625)
    compare(from_device(dc, O.BF16), rc.buf, O.BF16, plan.describe() + " C")
    why = PostOpsExplainer(x.t, w.t, b.t, (M, N), binary=O.BIN_ADD if kind == O.RES_IDENTIAL else O.BIN_EXT,
                           src=res.t, gamma=0.625)
    compare(from_device(dlr, O.BF16), rlr.buf, O.BF16, plan.describe() + " linearRes", explain=why)


def test_pingpong_batched_and_strided_weight(force_pingpong):
    # 3 batches, K-major weight (packed to [N][K] by the pack kernel), bias per batch row
    dt = O.BF16
    x = Case([3, 300, 128], dt, "ABC", seed=80, dist="normal", lo=0.0, hi=1.0)
    w = Case([3, 128, 280], dt, "ABC", seed=81, dist="normal", lo=0.0, hi=0.05)
    b = Case([3, 1, 280], dt, "ABC", seed=82, lo=-0.1, hi=0.1)
    c = Case([3, 300, 280], dt, "ABC", zero=True)
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 1.0, 0.0, K.ACT_SWISH)
    assert "pingpong" in plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_SWISH, 1.0)
    compare(from_device(dc, dt), ref.buf, dt, plan.describe())


def test_c3_plan_uses_pingpong():
    dx, dw, dy = K.desc([4096, 4096], K.BF16), K.desc([4096, 11008], K.BF16, "BA"), K.desc([4096, 11008], K.BF16)
    plan = K.LinearPostOps(dx, dw, dy, K.desc([1, 11008], K.BF16), act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=dy)
    assert plan.describe().startswith("mfma_bf16_pingpong_256x256")


@pytest.mark.parametrize("shape", ["pingpong", "split_k", "gemv", "pingpong_ksplit"])
def test_hip_graph_capture_replays(monkeypatch, shape):
    # a plan's run captured into a HIP graph (after one eager run, which sizes the plan's workspace) and replayed
    # three times with eager work in between; every replay must equal the eager result bit for bit (the ping-pong
    # K-split included: its last-arriving workgroup sums the partial tiles in a fixed order)
    dt = O.BF16
    M, N, Kd = {"pingpong": (512, 512, 256), "split_k": (100, 200, 2048), "gemv": (1, 300, 1024),
                "pingpong_ksplit": (300, 520, 1024)}[shape]
    x = Case([M, Kd], dt, seed=250, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, "BA", seed=251, dist="normal", lo=0.0, hi=0.05)
    s = Case([M, N], dt, seed=252, lo=-1.0, hi=1.0)
    y = Case([M, N], dt, zero=True)
    if shape.startswith("pingpong"):
        monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    if shape == "pingpong_ksplit":
        monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")  # read at every launch: stays set for the runs
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, None, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
    if shape == "pingpong_ksplit":
        assert " split=" in plan.describe(), plan.describe()
    dx, dw, ds = x.device(), w.device(), s.device()
    eager = zeros_device(y)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        plan.run(dx, dw, eager, None, ds, stream=stream)
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, None, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, s.t)
    compare(from_device(eager, dt), ref.buf, dt, f"eager {plan.describe()}")

    out = zeros_device(y)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        plan.run(dx, dw, out, None, ds, stream=torch.cuda.current_stream())
    for rep in range(3):
        out.zero_()
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} of {plan.describe()} differs from the eager run"
        del junk


def _sampled_tensor(rows_np, dt):
    """O.Tensor of a dense [r, c] numpy block (bf16 as uint16 bits)."""
    r, c = rows_np.shape
    return O.Tensor((r, c), (c, 1), dt, np.ascontiguousarray(rows_np).reshape(-1).copy())


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("case", ["gemm_2gib_x", "skinny_2gib_w", "gemv_2gib_w"])
def test_operands_of_2_gib(case):
    # an operand of 2^31 bytes: the ping-pong GEMM (32-bit buffer offsets) hands over to the 4-wave kernel, the
    # 2 <= M <= 16 row kernel to the MFMA-layout skinny kernel, and the M = 1 GEMV takes it directly; sampled output
    # rows / columns are checked against the oracle
    dt = O.BF16
    g = torch.Generator(device="cuda").manual_seed(260)
    if case == "gemm_2gib_x":
        M, Kd, N = 131072, 8192, 256                     # X is 2^31 bytes
    else:
        M, Kd, N = (4 if case == "skinny_2gib_w" else 1), 8192, 131072  # W is 2^31 bytes
    x = torch.randn(M, Kd, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(N, Kd, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    plan = K.LinearActivation(K.desc([M, Kd], K.BF16), K.desc([Kd, N], K.BF16, "BA"), K.desc([M, N], K.BF16), None,
                              1.0, 0.0, K.ACT_SWISH)
    plan.run(x, w, y)
    torch.cuda.synchronize()
    rng = np.random.default_rng(261)
    if case == "gemm_2gib_x":
        rows = np.unique(np.concatenate([[0, M // 2, M - 1], rng.choice(M, 13, replace=False)]))
        xs = _sampled_tensor(_bits(x[torch.as_tensor(rows, device="cuda")]), dt)
        wt = _bits(w)  # [N][K] = logical [K, N] in layout BA
        ws = O.Tensor((Kd, N), (1, Kd), dt, wt.reshape(-1).copy())
        ref = O.empty((len(rows), N), (N, 1), dt)
        O.linear_act(xs, ws, ref, None, O.ACT_SWISH, 1.0)
        got = _bits(y[torch.as_tensor(rows, device="cuda")]).reshape(-1)
    else:
        cols = np.unique(np.concatenate([[0, N // 2, N - 1], rng.choice(N, 61, replace=False)]))
        xs = _sampled_tensor(_bits(x), dt)
        wsub = _bits(w[torch.as_tensor(cols, device="cuda")])      # [n][K]
        ws = O.Tensor((Kd, len(cols)), (1, Kd), dt, wsub.reshape(-1).copy())
        ref = O.empty((M, len(cols)), (len(cols), 1), dt)
        O.linear_act(xs, ws, ref, None, O.ACT_SWISH, 1.0)
        got = _bits(y[:, torch.as_tensor(cols, device="cuda")]).reshape(-1)
    compare(got, ref.buf, dt, f"{case} {plan.describe()}")


@pytest.mark.parametrize("M,Kd,expect", [(20480, 128, "mfma_bf16_pingpong"), (16, 4096, "skinny_bf16_kgemv_xreg"),
                                         (9, 256, "skinny_bf16_kgemv_xreg"), (6, 64, "skinny_bf16_kgemv_xreg"),
                                         (16, 4096, "skinny_bf16_16xK"), (9, 256, "skinny_bf16_16xK"),
                                         (6, 64, "skinny_bf16_16xK"), (16, 4104, "skinny_bf16_16xK"),
                                         (3, 64, "skinny_bf16_gemv_rows_xlds"), (5, 4104, "skinny_bf16_gemv_rows_xlds"),
                                         (1, 520, "skinny_bf16_gemv_row")])
def test_single_weight_row(monkeypatch, M, Kd, expect):
    # N = 1: the weight descriptor's row pitch is 0 (a dimension of size one), so the kernels that bound their reads by
    # a buffer range take the operand's extent from its last row, not from rows x pitch (which is 0); the 16-row
    # kernel is forced where the planner takes the K-split GEMV
    if expect == "skinny_bf16_16xK" and Kd <= 4096:
        monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "20")
    N = 1
    x = Case([M, Kd], O.BF16, seed=270, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=271, dist="normal", lo=0.0, hi=0.05)
    b = Case([1, N], O.BF16, seed=272, lo=-0.1, hi=0.1)
    c = Case([M, N], O.BF16, zero=True)
    assert w.desc.stride()[1] == 0
    plan = K.LinearActivation(x.desc, w.desc, c.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
    assert plan.describe().startswith(expect), plan.describe()
    dc = zeros_device(c)
    plan.run(x.device(), w.device(), dc, b.device())
    torch.cuda.synchronize()
    ref = c.clone_empty()
    O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    compare(from_device(dc, O.BF16), ref.buf, O.BF16, plan.describe())


def _integer_case(dims, dt, layout, seed, lo, hi):
    # integer values in [lo, hi]: every GEMM partial sum is exact in f32 (and the stage value in bf16 when |sum| <= 256)
    c = Case(dims, dt, layout, zero=True)
    v = np.random.default_rng(seed).integers(lo, hi + 1, size=c.t.buf.size).astype(np.float32)
    c.t.buf[:] = O.from_f32_rne(v, dt)
    return c


@pytest.mark.parametrize("dt,cfg,M,N,Kd", [
    (O.F32, "10", 130, 200, 64), (O.F32, "11", 70, 136, 64), (O.F32, "12", 8, 96, 64),
    (O.BF16, "4", 300, 520, 128), (O.BF16, "3", 100, 200, 64), (O.BF16, "20", 12, 300, 256),
    (O.BF16, "22", 4, 300, 256), (O.BF16, None, 1, 300, 256)])
@pytest.mark.parametrize("op", ["res_ext", "bin_ext"])
def test_ext_gamma_fma_bit_exact(monkeypatch, dt, cfg, M, N, Kd, op):
    # RES_EXT / BIN_EXT with gamma = 0.3 (not a power of two, so res * gamma is inexact): the epilogue computes
    # fmaf(res, gamma, c) with one rounding, as the oracle does (the contraction GCC applies to c + res * gamma on
    # aarch64). Integer-valued X, W and bias make the GEMM stage exact in any summation order, so the output must equal
    # the oracle bit for bit; a separate multiply and add would differ wherever the product's rounding matters.
    if cfg is not None:
        monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", cfg)
    gamma = 0.3
    hi = 1 if dt == O.BF16 else 3
    x = _integer_case([M, Kd], dt, None, 900 + M, -hi, hi)
    w = _integer_case([Kd, N], dt, "BA", 901 + M, -hi, hi)
    b = _integer_case([1, N], dt, None, 902 + M, -2, 2)
    res = Case([M, N], dt, seed=903 + M, lo=-3.0, hi=3.0)
    out = Case([M, N], dt, zero=True)
    if op == "res_ext":
        c = Case([M, N], dt, zero=True)
        plan = K.LinearRes(x.desc, w.desc, c.desc, b.desc, res.desc, out.desc, 1.0, 0.0, gamma, O.RES_EXT)
        dc, dout = zeros_device(c), zeros_device(out)
        plan.run(x.device(), w.device(), dc, b.device(), res.device(), dout, gamma)
        rc = c.clone_empty()
        ref = out.clone_empty()
        O.linear_res(x.t, w.t, rc, b.t, res.t, ref, O.RES_EXT, gamma)
    else:
        plan = K.LinearPostOps(x.desc, w.desc, out.desc, b.desc, binary=K.BIN_EXT, src=res.desc, gamma=gamma)
        dout = zeros_device(out)
        plan.run(x.device(), w.device(), dout, b.device(), res.device(), gamma=gamma)
        ref = out.clone_empty()
        O.linear_postops(x.t, w.t, ref, b.t, O.ACT_NONE, 0.0, O.BIN_EXT, res.t, gamma)
    torch.cuda.synchronize()
    family = {"10": "mfma_f32_128x128", "11": "mfma_f32_64x64", "12": "mfma_f32_kslice_16x32",
              "4": "mfma_bf16_pingpong", "3": "mfma_bf16_128x128", "20": "skinny_bf16_16xK",
              "22": "skinny_bf16_gemv_rows_xlds", None: "skinny_bf16_gemv_row"}[cfg]
    assert plan.describe().startswith(family), plan.describe()
    got = from_device(dout, dt)
    diff = np.count_nonzero(got != ref.buf)
    assert diff == 0, f"{plan.describe()}: {diff} of {got.size} outputs differ from fmaf(res, gamma, c)"
    assert np.count_nonzero(got) > got.size // 2
