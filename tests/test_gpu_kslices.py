"""GPU parity of the ping-pong kernel's K slices (KUDNN_HIP_FORCE_KSLICES=S): every tile's k-tiles divided into S
slices run as separate workgroups of the data-parallel kernel, each storing its f32 sums, then one element-wise launch
adding the slices in slice order and running the epilogue. Edge tiles, uneven slices, the fixed and generic epilogue
forms, f16 operands and a K-major weight read in place, each against the oracle. Tail slices (the last partial round
of a larger grid sliced, KUDNN_HIP_FORCE_TAILSLICES=S) likewise, and against the unsliced run. Reference semantics:
src/dnn/src/kudnn_gemm.cpp:208-241 and the post-op stages of kudnn_linear_activationlayer.cpp:40-56 restated by the
oracle.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, dense_rows, explainer, from_device, sample_rows

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()  # fail loudly if the HIP library is missing


@pytest.fixture
def slices(monkeypatch):
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")  # the ping-pong kernel, also where the planner would not take it

    def force(S):
        monkeypatch.setenv("KUDNN_HIP_FORCE_KSLICES", str(S))

    return force


def _run(M, N, Kd, post, dt=O.BF16, wl="BA", seed=600):
    ydt = O.F32 if post == "gemm_beta" and dt == O.BF16 else dt
    x = Case([M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, wl, seed=seed + 1, dist="normal", lo=0.0, hi=0.03)
    b = Case([1, N], ydt, seed=seed + 2, lo=-0.2, hi=0.2)
    y = Case([M, N], ydt, seed=seed + 3, lo=-1.0, hi=1.0) if post == "gemm_beta" else Case([M, N], ydt, zero=True)
    s = Case([M, N], ydt, seed=seed + 4, lo=-1.0, hi=1.0)
    dy = torch.from_numpy(y.t.buf.view(np.int16).copy() if ydt != O.F32 else y.t.buf.copy()).cuda()
    ref = O.Tensor(y.t.dims, y.t.strides, ydt, y.t.buf.copy())
    why = None
    if post == "bias_gelu_add":
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
        plan.run(x.device(), w.device(), dy, b.device(), s.device())
        O.linear_postops(x.t, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, s.t)
        why = explainer(ydt, x.t, w.t, b.t, (M, N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=s.t)
    elif post == "relu":
        plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 0.0, 0.0, K.ACT_RELU)
        plan.run(x.device(), w.device(), dy, b.device())
        O.linear_act(x.t, w.t, ref, b.t, O.ACT_RELU, 0.0)
    else:
        plan = K.Gemm(x.desc, w.desc, y.desc, b.desc)
        plan.run(x.device(), w.device(), dy, b.device(), alpha=0.5, beta=0.25)
        O.gemm(x.t, w.t, ref, b.t, 0.5, 0.25)
    torch.cuda.synchronize()
    compare(from_device(dy, ydt), ref.buf, ydt, f"M={M} N={N} K={Kd} {post} {plan.describe()}", explain=why)
    return plan.describe()


@pytest.mark.parametrize("S", [2, 3, 5])
@pytest.mark.parametrize("post", ["bias_gelu_add", "gemm_beta"])
def test_kslices_edges(slices, S, post):
    # 600 x 700: edge tiles along both dims; K = 2048 is 32 k-tiles, so S = 3 and 5 leave a shorter last slice
    slices(S)
    desc = _run(600, 700, 2048, post)
    assert f"kslices={S}" in desc, desc


@pytest.mark.parametrize("S", [2, 4])
def test_kslices_f16_and_kmajor(slices, S):
    slices(S)
    assert f"kslices={S}" in _run(300, 512, 1024, "relu", dt=O.F16, seed=610)
    # a [K][N] weight (N a multiple of 8, K of 64) is read in place by the sliced launch too, also with an edge tile
    # along N (1152 = 4.5 tiles: the reference's performance shapes)
    for N, seed in ((512, 620), (1152, 625)):
        desc = _run(512, N, 4096, "bias_gelu_add", wl="AB", seed=seed)
        assert f"kslices={S}" in desc and "kmajorB" in desc, desc


def test_kslices_one_k_tile_each(slices):
    # as many slices as k-tiles: one k-tile per workgroup
    slices(8)
    assert "kslices=8" in _run(256, 256, 512, "bias_gelu_add", seed=630)


def test_kslices_match_unsliced(monkeypatch, slices):
    # the same inputs with and without slices: the f32 sums are added in another order, so the bf16 GEMM stages can
    # differ by one ulp, and only rarely
    outs = []
    for S in (0, 3):
        slices(S)
        M, N, Kd = 512, 768, 3072
        x = Case([M, Kd], O.BF16, seed=640, dist="normal", lo=0.0, hi=1.0)
        w = Case([Kd, N], O.BF16, "BA", seed=641, dist="normal", lo=0.0, hi=0.03)
        y = Case([M, N], O.BF16, zero=True)
        plan = K.LinearActivation(x.desc, w.desc, y.desc, None, 0.0, 0.0, K.ACT_RELU)
        assert ("kslices=3" in plan.describe()) == (S == 3), plan.describe()
        dy = torch.zeros(M * N, dtype=torch.int16, device="cuda")
        plan.run(x.device(), w.device(), dy)
        torch.cuda.synchronize()
        outs.append(from_device(dy, O.BF16))
    assert np.mean(outs[0] == outs[1]) > 0.99


@pytest.mark.parametrize("mnk,S", [((1024, 4096, 11008), 2), ((512, 4096, 14336), 4), ((256, 4096, 4096), 4),
                                   ((4096, 1152, 4608), 2)])
def test_planner_kslices(mnk, S):
    # the planner's own choice: 64 tiles x 172 k-tiles, 32 x 224, 16 x 64 and one of the reference's perf shapes
    # (80 tiles, M >= 1024); large outputs checked on sampled rows of every 256-row band
    M, N, Kd = mnk
    x = Case([M, Kd], O.BF16, seed=650, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=651, dist="normal", lo=0.0, hi=0.02)
    b = Case([1, N], O.BF16, seed=652, lo=-0.2, hi=0.2)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 0.0, 0.0, K.ACT_GELU_TANH)
    assert plan.describe().startswith("mfma_bf16_pingpong") and f"kslices={S}" in plan.describe(), plan.describe()
    dy = torch.zeros(M * N, dtype=torch.int16, device="cuda")
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    got = from_device(dy, O.BF16).reshape(M, N)
    rows = sample_rows(M, 24)
    xr = dense_rows(x.t, rows)
    ref = O.empty((len(rows), N), (N, 1), O.BF16)
    O.linear_act(xr, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0)
    why = explainer(O.BF16, xr, w.t, b.t, (len(rows), N), act=O.ACT_GELU_TANH)
    compare(got[rows].reshape(-1), ref.buf, O.BF16, plan.describe(), explain=why)


@pytest.mark.parametrize("mnk,wl,start", [((1024, 4096, 4096), "BA", "mfma_bf16_128x128"),
                                           ((256, 11008, 4096), "BA", "mfma_bf16_128x128"),
                                           ((1024, 4096, 4096), "AB", "mfma_bf16_pingpong")])
def test_planner_four_wave_or_slices(mnk, wl, start):
    # 32-64 tiles with at most 64 k-tiles: the planner's 4-wave 128 x 128 kernel when the weight is stored [N][K]; the
    # ping-pong kernel in K slices, reading the weight in place, when it is stored [K][N]
    M, N, Kd = mnk
    x = Case([M, Kd], O.BF16, seed=655, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, wl, seed=656, dist="normal", lo=0.0, hi=0.02)
    b = Case([1, N], O.BF16, seed=657, lo=-0.2, hi=0.2)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearActivation(x.desc, w.desc, y.desc, b.desc, 0.0, 0.0, K.ACT_GELU_TANH)
    desc = plan.describe()
    assert desc.startswith(start) and (("kslices=2" in desc and "kmajorB" in desc) == (wl == "AB")), desc
    dy = torch.zeros(M * N, dtype=torch.int16, device="cuda")
    plan.run(x.device(), w.device(), dy, b.device())
    torch.cuda.synchronize()
    got = from_device(dy, O.BF16).reshape(M, N)
    rows = sample_rows(M, 24)
    xr = dense_rows(x.t, rows)
    ref = O.empty((len(rows), N), (N, 1), O.BF16)
    O.linear_act(xr, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0)
    why = explainer(O.BF16, xr, w.t, b.t, (len(rows), N), act=O.ACT_GELU_TANH)
    compare(got[rows].reshape(-1), ref.buf, O.BF16, desc, explain=why)


def test_kslices_graph_replays(slices):
    # both launches captured in a HIP graph (no memset nodes): every replay, with eager work between replays, equals
    # the eager result
    slices(3)
    M, N, Kd = 300, 520, 2048
    x = Case([M, Kd], O.BF16, seed=660, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=661, dist="normal", lo=0.0, hi=0.05)
    s = Case([M, N], O.BF16, seed=662, lo=-1.0, hi=1.0)
    y = Case([M, N], O.BF16, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, None, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
    assert "kslices=3" in plan.describe(), plan.describe()
    dx, dw, ds = x.device(), w.device(), s.device()
    stream = torch.cuda.Stream()
    eager = torch.zeros(M * N, dtype=torch.int16, device="cuda")
    with torch.cuda.stream(stream):
        plan.run(dx, dw, eager, None, ds, stream=stream)
    torch.cuda.synchronize()
    out = torch.zeros(M * N, dtype=torch.int16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        plan.run(dx, dw, out, None, ds, stream=stream)  # warm: the plan's workspace exists before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            plan.run(dx, dw, out, None, ds, stream=stream)
    for r in range(3):
        out.zero_()
        plan.run(dx, dw, torch.zeros_like(eager), None, ds)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"


# ---------------------------------------------------------------------------------------------------
# tail slices: a grid of more tiles than CUs runs its full rounds as whole tiles and splits only the last partial
# round's tiles (the last tiles of the grouped tile order) into K slices, stored as 256 x 256 blocks and added by the
# reduction launch, 32 workgroups per tile


def _tail_run(monkeypatch, M, N, Kd, post, dt=O.BF16, wl="BA", seed=700, force=None):
    """Runs the chain `post` with the tail slices the planner (or KUDNN_HIP_FORCE_TAILSLICES=force) gives and with
    none; checks sampled rows of every 256-row band against the oracle and the two runs against each other (their f32
    sums are added in another order: the 16-bit GEMM stages differ by one ulp, and only rarely); returns the sliced
    plan's description."""
    ydt = O.F32 if post == "gemm_beta" and dt == O.BF16 else dt
    x = Case([M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, wl, seed=seed + 1, dist="normal", lo=0.0, hi=0.02)
    b = Case([1, N], ydt, seed=seed + 2, lo=-0.2, hi=0.2)
    y = Case([M, N], ydt, seed=seed + 3, lo=-1.0, hi=1.0) if post == "gemm_beta" else Case([M, N], ydt, zero=True)
    s = Case([M, N], ydt, seed=seed + 4, lo=-1.0, hi=1.0)
    dx, dw, db, ds = x.device(), w.device(), b.device(), s.device()
    outs, descs = [], []
    for S in (force, 0):
        if S is None:
            monkeypatch.delenv("KUDNN_HIP_FORCE_TAILSLICES", raising=False)
        else:
            monkeypatch.setenv("KUDNN_HIP_FORCE_TAILSLICES", str(S))
        dy = torch.from_numpy(y.t.buf.view(np.int16).copy() if ydt != O.F32 else y.t.buf.copy()).cuda()
        if post == "bias_gelu_add":
            plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
            plan.run(dx, dw, dy, db, ds)
        else:
            plan = K.Gemm(x.desc, w.desc, y.desc, b.desc)
            plan.run(dx, dw, dy, db, alpha=0.5, beta=0.25)
        torch.cuda.synchronize()
        outs.append(from_device(dy, ydt).reshape(M, N))
        descs.append(plan.describe())
    monkeypatch.delenv("KUDNN_HIP_FORCE_TAILSLICES", raising=False)
    assert " tail=" not in descs[1], descs[1]
    a, r = outs
    av, rv = O.to_f32(a.reshape(-1), ydt), O.to_f32(r.reshape(-1), ydt)
    if ydt == O.F32:
        # f32 outputs keep the summation order's last bits
        assert np.allclose(av, rv, rtol=1e-4, atol=1e-4), f"{descs[0]}: {np.max(np.abs(av - rv))}"
    else:
        assert np.mean(a == r) > 0.99 and np.allclose(av, rv, rtol=2e-2, atol=2e-2), \
            f"{descs[0]}: {np.count_nonzero(a != r)} outputs differ from the unsliced run"
    rows = sample_rows(M, 24)
    xr = dense_rows(x.t, rows)
    ref = O.empty((len(rows), N), (N, 1), ydt)
    if post == "bias_gelu_add":
        sr = dense_rows(s.t, rows)
        O.linear_postops(xr, w.t, ref, b.t, O.ACT_GELU_TANH, 0.0, O.BIN_ADD, sr)
        why = explainer(ydt, xr, w.t, b.t, (len(rows), N), act=O.ACT_GELU_TANH, binary=O.BIN_ADD, src=sr)
    else:
        ref.buf[:] = dense_rows(y.t, rows).buf
        O.gemm(xr, w.t, ref, b.t, 0.5, 0.25)
        why = None
    compare(a[rows].reshape(-1), ref.buf, ydt, descs[0], explain=why)
    return descs[0]


@pytest.mark.parametrize("mnk,expect", [((4352, 4096, 4096), "kslices=4 tail=16"), ((3072, 11008, 2048), "kslices=2 tail=4")])
def test_tail_slices_planner(monkeypatch, mnk, expect):
    # the planner's choice: 272 tiles (16 in the last round, 64 k-tiles: 4 slices), 516 tiles (4 left, 32 k-tiles: 2)
    M, N, Kd = mnk
    desc = _tail_run(monkeypatch, M, N, Kd, "bias_gelu_add", seed=710)
    assert desc.startswith("mfma_bf16_pingpong") and expect in desc, desc


@pytest.mark.parametrize("post", ["bias_gelu_add", "gemm_beta"])
@pytest.mark.parametrize("S", [3, 5])
def test_tail_slices_edges(monkeypatch, post, S):
    # 4300 x 4000: 17 x 16 tiles with edges along both dims among the sliced ones; K = 2048 is 32 k-tiles, so 3 and 5
    # slices leave a shorter last slice; fixed (bf16) and generic (f32 output with beta) epilogues
    desc = _tail_run(monkeypatch, 4300, 4000, 2048, post, seed=720, force=S)
    assert f"kslices={S} tail=16" in desc, desc


def test_tail_slices_f16_and_kmajor(monkeypatch):
    assert "kslices=4 tail=16" in _tail_run(monkeypatch, 4352, 4096, 1024, "bias_gelu_add", dt=O.F16, seed=730, force=4)
    # a [K][N] weight read in place (N a multiple of 8, an edge tile along N)
    desc = _tail_run(monkeypatch, 4352, 3880, 1024, "bias_gelu_add", wl="AB", seed=740, force=2)
    assert "kslices=2 tail=16" in desc and "kmajorB" in desc, desc


def test_no_tail_slices_where_they_lose():
    # C3 (176 tiles in the last round), 88 tiles left, and 18 k-tiles: whole tiles only
    for M, N, Kd in ((4096, 11008, 4096), (2048, 11008, 4096), (4096, 4608, 1152)):
        plan = K.Gemm(K.desc([M, Kd], K.BF16), K.desc([Kd, N], K.BF16, "BA"), K.desc([M, N], K.BF16))
        assert "kslices" not in plan.describe(), plan.describe()
