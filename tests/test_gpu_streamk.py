"""GPU parity of the ping-pong kernel's tail split: whole rounds of tiles data-parallel, the remaining tiles' k-iterations
divided between one workgroup per CU, a tile spanning several workgroups finished by the last to arrive (partial
accumulators through the plan's workspace, an arrival counter per tile). KUDNN_HIP_FORCE_STREAMK=1 forces the split on
small problems, so a tile gets 2, 3 or up to 64 contributors; the unforced cases are shapes whose last round would leave
CUs idle. Every epilogue form is checked against the CPU oracle, s8 bit for bit, and repeated runs of one plan check
that the counters are left ready for the next launch.
"""
import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, compare, dense_rows, explainer, from_device, sample_rows, zeros_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()


@pytest.fixture
def pingpong(monkeypatch):
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "4")
    monkeypatch.setenv("KUDNN_HIP_FORCE_KSLICES", "0")  # the tail split, not the K slices the planner prefers


def run_linear(M, N, Kd, dt=O.BF16, ydt=None, act=O.ACT_GELU_TANH, alpha=0.0, beta=0.0, bias="1N", binary=True,
               seed=0, runs=1):
    ydt = ydt or dt
    x = Case([M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, "BA", seed=seed + 1, dist="normal", lo=0.0, hi=0.05)
    bdims = {"1N": [1, N], "M1": [M, 1], "MN": [M, N], None: None}[bias]
    b = Case(bdims, ydt, seed=seed + 2, lo=-0.1, hi=0.1) if bdims else None
    s = Case([M, N], ydt, seed=seed + 3) if binary else None
    y = Case([M, N], ydt, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc if b else None, act=act, act_alpha=alpha, act_beta=beta,
                           binary=K.BIN_ADD if binary else K.BIN_NONE, src=s.desc if s else None)
    assert "pingpong" in plan.describe() and " split=" in plan.describe(), plan.describe()
    # large problems: the oracle computes a sample of rows (rows of a GEMM are independent)
    rows = sample_rows(M, 24) if M * N * Kd > (1 << 30) else None
    if rows is None:
        ref = y.clone_empty()
        O.linear_postops(x.t, w.t, ref, b.t if b else None, act, alpha, O.BIN_ADD if binary else O.BIN_NONE,
                         s.t if s else None, act_beta=beta)
    else:
        assert bias in (None, "1N")
        ref = O.empty((len(rows), N), (N, 1), ydt)
        O.linear_postops(dense_rows(x.t, rows), w.t, ref, b.t if b else None, act, alpha,
                         O.BIN_ADD if binary else O.BIN_NONE, dense_rows(s.t, rows) if s else None, act_beta=beta)
    first = None
    for r in range(runs):
        dy = zeros_device(y)
        plan.run(x.device(), w.device(), dy, b.device() if b else None, s.device() if s else None)
        torch.cuda.synchronize()
        got = from_device(dy, ydt)
        # a split tile is summed in contributor order whoever arrives last: runs agree bit for bit
        if first is None:
            first = got.copy()
        else:
            assert np.array_equal(got, first), f"{plan.describe()}: run {r} differs from run 0"
        if rows is not None:
            got = got.reshape(M, N)[rows].reshape(-1)
        xr = dense_rows(x.t, rows) if rows is not None else x.t
        sr = (dense_rows(s.t, rows) if rows is not None else s.t) if s else None
        why = explainer(ydt, xr, w.t, b.t if b else None, (len(rows) if rows is not None else M, N), act=act,
                        act_alpha=alpha, act_beta=beta, binary=O.BIN_ADD if binary else None, src=sr)
        compare(got, ref.buf, ydt, f"{plan.describe()} run {r}", explain=why)
    return plan


@pytest.mark.parametrize("mnk", [(300, 520, 384), (512, 256, 1024), (256, 768, 640), (40, 600, 256)])
def test_forced_tail_split_bf16(monkeypatch, pingpong, mnk):
    # one k-tile per workgroup at these sizes: every tile is split 2 ways or more (6 x 3 k-tiles: 3 contributors)
    monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")
    run_linear(*mnk, seed=10, runs=2)


def test_forced_tail_split_many_contributors(monkeypatch, pingpong):
    # 4 tiles x 64 k-tiles over 256 workgroups: 64 contributors per tile
    monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")
    run_linear(512, 512, 4096, seed=20, runs=2)


@pytest.mark.parametrize("form", ["f32out", "generic_act", "mn_bias", "m1_bias", "no_post"])
def test_forced_tail_split_epilogue_forms(monkeypatch, pingpong, form):
    monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")
    if form == "f32out":
        run_linear(300, 520, 384, ydt=O.F32, seed=30)
    elif form == "generic_act":
        run_linear(300, 520, 384, act=O.ACT_HARDSWISH, alpha=1.0 / 6.0, beta=0.5, seed=31)
    elif form == "mn_bias":
        run_linear(300, 520, 384, bias="MN", seed=32)
    elif form == "m1_bias":
        run_linear(300, 520, 384, bias="M1", act=O.ACT_SWISH, alpha=1.0, seed=33)
    else:
        run_linear(300, 520, 384, act=O.ACT_NONE, bias=None, binary=False, seed=34)


def test_forced_tail_split_f16(monkeypatch, pingpong):
    monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")
    run_linear(300, 520, 384, dt=O.F16, seed=40, runs=2)


def test_forced_tail_split_s8_exact(monkeypatch, pingpong):
    monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")
    M, N, Kd = 300, 520, 1024
    x = Case([M, Kd], O.S8, seed=50, lo=-128, hi=127)
    w = Case([Kd, N], O.S8, "BA", seed=51, lo=-128, hi=127)
    b = Case([1, N], O.S32, seed=52, lo=-(1 << 24), hi=1 << 24)
    c = Case([M, N], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc, b.desc)
    assert "s8_pingpong" in plan.describe() and " split=" in plan.describe(), plan.describe()
    ref = c.clone_empty()
    O.gemm(x.t, w.t, ref, b.t)
    for r in range(2):
        dc = zeros_device(c)
        plan.run(x.device(), w.device(), dc, b.device())
        torch.cuda.synchronize()
        compare(from_device(dc, O.S32), ref.buf, O.S32, f"{plan.describe()} run {r}")


def test_planner_tail_split_s8():
    # the planner's own choice on 256 CUs for an s8 GEMM (the 16-bit types take K slices instead): 64 tiles x 128
    # k-tiles of 128 bytes, 32 per CU; integer results exact on sampled rows of every 256-row band
    M, N, Kd = 1024, 4096, 16384
    x = Case([M, Kd], O.S8, seed=62, lo=-128, hi=127)
    w = Case([Kd, N], O.S8, "BA", seed=63, lo=-128, hi=127)
    c = Case([M, N], O.S32, zero=True)
    plan = K.Gemm(x.desc, w.desc, c.desc)
    assert "s8_pingpong" in plan.describe() and " split=0+64/32" in plan.describe(), plan.describe()
    rows = sample_rows(M, 24)
    ref = O.empty((len(rows), N), (N, 1), O.S32)
    O.gemm(dense_rows(x.t, rows), w.t, ref)
    for r in range(2):
        dc = zeros_device(c)
        plan.run(x.device(), w.device(), dc)
        torch.cuda.synchronize()
        got = from_device(dc, O.S32).reshape(M, N)[rows].reshape(-1)
        compare(got, ref.buf, O.S32, f"{plan.describe()} run {r}")


def test_forced_split_behind_whole_rounds(monkeypatch):
    # 16 x 24 = 384 tiles: 256 data-parallel, 128 split (the planner would not split here; forced to test the
    # data-parallel launch clearing the counters the tail launch uses)
    monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", "1")
    run_linear(4096, 6144, 2048, seed=61, runs=2)


def test_tail_split_matches_unsplit(monkeypatch, pingpong):
    # same inputs, split and unsplit: equal within the fp32 summation-order difference
    M, N, Kd = 300, 520, 2048
    x = Case([M, Kd], O.BF16, seed=70, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], O.BF16, "BA", seed=71, dist="normal", lo=0.0, hi=0.05)
    y = Case([M, N], O.F32, zero=True)
    outs = []
    for force in ("0", "1"):
        monkeypatch.setenv("KUDNN_HIP_FORCE_STREAMK", force)
        plan = K.LinearPostOps(x.desc, w.desc, y.desc, None)
        dy = zeros_device(y)
        plan.run(x.device(), w.device(), dy, None, None)
        torch.cuda.synchronize()
        outs.append(from_device(dy, O.F32).astype(np.float64))
    assert np.max(np.abs(outs[0] - outs[1])) <= 1e-5 * np.max(np.abs(outs[0]))
