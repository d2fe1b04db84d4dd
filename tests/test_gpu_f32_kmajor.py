"""GPU parity of the fp32 GEMM reading a [K][N] weight in place (gemm_mfma.hip, BKM): the reference's Matmul mode
passes the weight as [K][N] (Layout ABCDE, test/dnn/llt/gtest/src/matmul_gtest.cpp:248-257) and KML consumes it through
the layout -> transpose mapping (src/dnn/src/kudnn_gemm.cpp:478-549). The 4-wave fp32 kernels (128 x 128 and 64 x 64,
split along K on small grids) copy each k-tile of such a weight into LDS as 32 k-rows of the tile's columns and read one
float per k. The k-slice kernel of the smallest grids reads it in place too when K = 256 c (its whole-line form: 32
k-rows of the tile's 32 columns per pair of chunks, through LDS). The cases cover full and edge tiles (N a multiple of
4 but not of the tile, so the last chunks of a k-row are clamped), batched and broadcast weights, every fixed epilogue
form and the generic one (alpha, beta C, bias), the split-K instance, the k-slice kernel, and the planner's own
choice. Each runs against the oracle and, bit for bit, against the same plan
with the weight packed to [N][K] (KUDNN_HIP_PACK_KMAJOR=1): both feed the MFMAs the same k values in the same order.
Weights the kernels cannot read in place (N not a multiple of 4, K not a multiple of 32) are packed.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, dense_rows, from_device, sample_rows, zeros_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()  # fail loudly if the HIP library is missing


def _case(lead, M, Kd, N, wlead, bias, seed):
    x = Case(lead + [M, Kd], O.F32, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case(wlead + [Kd, N], O.F32, seed=seed + 1, dist="normal", lo=0.0, hi=0.05)  # standard layout: [K][N]
    b = Case([1] * len(lead) + [1, N], O.F32, seed=seed + 2, lo=-0.2, hi=0.2) if bias else None
    y = Case(lead + [M, N], O.F32, zero=True)
    return x, w, b, y


def _both(monkeypatch, make_plan, run, outcase):
    """Runs a plan with the weight in place, then with it packed; returns both outputs and the in-place plan."""
    outs, plans = [], []
    for packed in (False, True):
        if packed:
            monkeypatch.setenv("KUDNN_HIP_PACK_KMAJOR", "1")
        plan = make_plan()
        assert ("packB" in plan.describe()) == packed and ("kmajorB" in plan.describe()) != packed, plan.describe()
        dy = outcase()
        run(plan, dy)
        torch.cuda.synchronize()
        outs.append(from_device(dy, O.F32))
        plans.append(plan)
    monkeypatch.delenv("KUDNN_HIP_PACK_KMAJOR")
    assert np.array_equal(outs[0], outs[1]), "in-place and packed K-major weights differ"
    return outs[0], plans[0]


@pytest.mark.parametrize("cfg", ["10", "11"])
@pytest.mark.parametrize("shape", [([], 256, 64, 256, []), ([], 300, 640, 772, []), ([], 1000, 256, 1540, []),
                                   ([2], 260, 192, 516, [2]), ([3], 128, 128, 264, [1]), ([], 64, 32, 4, [])])
@pytest.mark.parametrize("act", [K.ACT_UNIMPLEMENTED, K.ACT_RELU, K.ACT_GELU_TANH])
def test_f32_kmajor_weight_in_place(monkeypatch, cfg, shape, act):
    # 128 x 128 (cfg 10) and 64 x 64 (cfg 11) tiles; edge tiles with 4..124 columns of the last tile inside N; N = 4
    # (one chunk, every other chunk of the tile clamped onto it)
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", cfg)
    lead, M, Kd, N, wlead = shape
    x, w, b, y = _case(lead, M, Kd, N, wlead, act != K.ACT_UNIMPLEMENTED, 800)
    dx, dw, db = x.device(), w.device(), b.device() if b else None
    got, plan = _both(monkeypatch,
                      lambda: K.LinearPostOps(x.desc, w.desc, y.desc, b.desc if b else None, act=act, act_alpha=1.0),
                      lambda p, dy: p.run(dx, dw, dy, db), lambda: zeros_device(y))
    assert plan.describe().startswith("mfma_f32_128x128" if cfg == "10" else "mfma_f32_64x64"), plan.describe()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t if b else None, act, 1.0, O.BIN_NONE, None)
    compare(got, ref.buf, O.F32, "f32 kmajor " + plan.describe())


@pytest.mark.parametrize("shape", [([], 128, 1024, 1024, []), ([], 100, 512, 1000, []), ([], 64, 3072, 1024, []),
                                   ([], 16, 4096, 4100, []), ([2], 40, 256, 700, [2]), ([3], 48, 768, 1000, [1])])
@pytest.mark.parametrize("act", [K.ACT_UNIMPLEMENTED, K.ACT_RELU])
def test_f32_kmajor_kslice_in_place(monkeypatch, shape, act):
    # the k-slice kernel's whole-line form (grids too small for 64 x 64 tiles): C1's shape in Matmul mode; K = 512,
    # 3072 and 4096 (2, 12 and 16 pairs of 32 k per wave); edge tiles (N a multiple of 4, not of 32); M = 16; batched and
    # broadcast weights
    lead, M, Kd, N, wlead = shape
    x, w, b, y = _case(lead, M, Kd, N, wlead, act != K.ACT_UNIMPLEMENTED, 860)
    dx, dw, db = x.device(), w.device(), b.device() if b else None
    got, plan = _both(monkeypatch,
                      lambda: K.LinearPostOps(x.desc, w.desc, y.desc, b.desc if b else None, act=act, act_alpha=0.0),
                      lambda p, dy: p.run(dx, dw, dy, db), lambda: zeros_device(y))
    assert plan.describe().startswith("mfma_f32_kslice"), plan.describe()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t if b else None, act, 0.0, O.BIN_NONE, None)
    compare(got, ref.buf, O.F32, "f32 kmajor kslice " + plan.describe())


def test_f32_kmajor_gemm_generic_form(monkeypatch):
    # Gemm with alpha, beta C and a full [M, N] bias: the generic epilogue
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "10")
    M, Kd, N = 384, 320, 900
    x = Case([M, Kd], O.F32, seed=820, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.F32, seed=821, dist="normal", lo=0.0, hi=0.05)
    b = Case([M, N], O.F32, seed=822, lo=-0.2, hi=0.2)
    y = Case([M, N], O.F32, seed=823, lo=-1.0, hi=1.0)
    dx, dw, db = x.device(), w.device(), b.device()
    got, plan = _both(monkeypatch, lambda: K.Gemm(x.desc, w.desc, y.desc, b.desc),
                      lambda p, dy: p.run(dx, dw, dy, db, alpha=0.5, beta=0.25),
                      lambda: torch.from_numpy(y.t.buf.copy()).cuda())
    ref = O.Tensor(y.t.dims, y.t.strides, O.F32, y.t.buf.copy())
    O.gemm(x.t, w.t, ref, b.t, 0.5, 0.25)
    compare(got, ref.buf, O.F32, "f32 kmajor gemm " + plan.describe())


def test_f32_kmajor_split_k(monkeypatch):
    # a small grid with long K: the 64 x 64 kernel splits K across workgroups (split-K slots and arrival counters)
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "11")
    M, Kd, N = 128, 2048, 256
    x, w, b, y = _case([], M, Kd, N, [], True, 830)
    dx, dw, db = x.device(), w.device(), b.device()
    got, plan = _both(monkeypatch, lambda: K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_RELU),
                      lambda p, dy: p.run(dx, dw, dy, db), lambda: zeros_device(y))
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, K.ACT_RELU, 0.0, O.BIN_NONE, None)
    compare(got, ref.buf, O.F32, "f32 kmajor split " + plan.describe())


def test_f32_kmajor_planner_choice(monkeypatch):
    # the planner reads the [K][N] weight in place on its own (no forced configuration), on a reference perf shape
    # (matmul_gtest's freParas, 4096 x 1152 x 4608 in f32) and on a 64 x 64 grid
    for (M, Kd, N), seed in (((4096, 4608, 1152), 840), ((512, 512, 1024), 845)):
        x, w, b, y = _case([], M, Kd, N, [], False, seed)
        plan = K.Gemm(x.desc, w.desc, y.desc)
        assert "kmajorB" in plan.describe() and "packB" not in plan.describe(), plan.describe()
        dy = zeros_device(y)
        plan.run(x.device(), w.device(), dy)
        torch.cuda.synchronize()
        got = from_device(dy, O.F32).reshape(M, N)
        rows = sample_rows(M, 24)  # every 256-row tile row, the edges, and random rows
        ref = O.empty((len(rows), N), (N, 1), O.F32)
        O.gemm(dense_rows(x.t, rows), w.t, ref, None, 1.0, 0.0)
        compare(got[rows].reshape(-1), ref.buf, O.F32, "f32 kmajor planner " + plan.describe())


@pytest.mark.parametrize("M,Kd,N", [(300, 640, 1158), (300, 648, 1160)])
def test_f32_kmajor_unaligned_is_packed(monkeypatch, M, Kd, N):
    # N not a multiple of 4 (a 16-byte chunk would straddle the row end) or K not a multiple of 32 (the k-tile): packed
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "10")
    x, w, b, y = _case([], M, Kd, N, [], True, 850)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, act_alpha=1.0)
    assert "packB" in plan.describe(), plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    ref = y.clone_empty()
    O.linear_postops(x.t, w.t, ref, b.t, K.ACT_GELU_TANH, 1.0, O.BIN_NONE, None)
    compare(from_device(dy, O.F32), ref.buf, O.F32, plan.describe())


def _random_f32_kmajor_shapes(count=24, seed=2026):
    # seeded (M, N, K) draws for an fp32 [K][N] weight: M in [1, 400] or [1, 4096] (the k-slice kernel's small grids,
    # 64 x 64 and 128 x 128 grids of several rounds), N a multiple of 4 in [4, 4096] (edge tiles of every width), K a multiple of
    # 32 in [32, 4096] (the k-slice kernel's whole-line K values and others, which pack), plus a few draws with N or K
    # off those multiples (packed)
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        M = int(rng.integers(1, 401 if i % 2 else 4097))
        N = 4 * int(rng.integers(1, 1025))
        Kd = 32 * int(rng.integers(1, 129)) if i % 3 else 256 * int(rng.choice([1, 2, 3, 4, 6, 8, 12, 16]))
        if i % 8 == 7:
            N += 2 if i % 16 == 7 else 0
            Kd += 8 if i % 16 == 15 else 0
        out.append((M, N, Kd))
    return out


@pytest.mark.parametrize("M,N,Kd", _random_f32_kmajor_shapes())
def test_f32_kmajor_random_shapes(M, N, Kd):
    # the planner's own choice on each draw (k-slice, 64 x 64 or 128 x 128 kernel; in place or packed) against the
    # oracle on sampled rows
    x, w, b, y = _case([], M, Kd, N, [], True, 870)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_RELU)
    inplace = N % 4 == 0 and Kd % 32 == 0 and ("kslice" not in plan.describe() or Kd in
                                                  [256 * c for c in (1, 2, 3, 4, 6, 8, 12, 16)])
    assert ("kmajorB" in plan.describe()) == inplace, plan.describe()
    dy = zeros_device(y)
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    got = from_device(dy, O.F32).reshape(M, N)
    rows = sample_rows(M, 24)
    ref = O.empty((len(rows), N), (N, 1), O.F32)
    O.linear_postops(dense_rows(x.t, rows), w.t, ref, b.t, K.ACT_RELU, 0.0, O.BIN_NONE, None)
    compare(got[rows].reshape(-1), ref.buf, O.F32, f"f32 kmajor M={M} N={N} K={Kd} {plan.describe()}")
