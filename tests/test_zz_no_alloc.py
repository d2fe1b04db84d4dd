"""GPU test of kudnn_linear_postops_run_noalloc, the entry point that allocates nothing: through the C ABI its
results equal kudnn_linear_postops_run's bit for bit (same kernels) on calls in a row, each smaller than the one
before, with plans that use the workspace (the ping-pong kernel's K-slice sums, whole-grid or of the last partial
round only, operand packs and the 4-wave kernels' split-K partials, bf16 and f32, which it takes from its static device
scratch)."""
import ctypes

import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import Case, from_device, zeros_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()


def _run_both(M, N, Kd, seed, dt=O.BF16):
    # weight in layout AB (K-major [K][N]). bf16: the ping-pong kernel reads it in place when N is a multiple of 8 and
    # K of 64 (the plan says kmajorB); the 4-wave kernel, and K tails, pack it into the workspace (packB). f32: the
    # 4-wave kernels read it in place when N is a multiple of 4 and K of 32, the k-slice kernel for whole-line K
    x = Case([M, Kd], dt, seed=seed, dist="normal", lo=0.0, hi=1.0)
    w = Case([Kd, N], dt, "AB", seed=seed + 1, dist="normal", lo=0.0, hi=0.03)
    b = Case([1, N], dt, seed=seed + 2, lo=-0.1, hi=0.1)
    s = Case([M, N], dt, seed=seed + 3, lo=-1.0, hi=1.0)
    y = Case([M, N], dt, zero=True)
    plan = K.LinearPostOps(x.desc, w.desc, y.desc, b.desc, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=s.desc)
    dx, dw, db, ds = x.device(), w.device(), b.device(), s.device()
    want, got = zeros_device(y), zeros_device(y)
    plan.run(dx, dw, want, db, ds, gamma=1.0)
    stream = torch.cuda.current_stream().cuda_stream
    st = K.lib().kudnn_linear_postops_run_noalloc(plan.handle, dx.data_ptr(), dw.data_ptr(), got.data_ptr(),
                                                  db.data_ptr(), ds.data_ptr(), ctypes.c_float(1.0), stream)
    assert st == K.SUCCESS, K.last_error()
    torch.cuda.synchronize()
    a, r = from_device(got, dt), from_device(want, dt)
    assert np.array_equal(a, r), f"{plan.describe()}: {np.count_nonzero(a != r)} outputs differ"
    assert np.count_nonzero(a) > a.size // 2
    return plan


def test_noalloc_matches_run_on_two_calls():
    # 256 x 1024 x 2048 (ping-pong kernel, K-major weight read in place, 2 K slices), then a smaller 256 x 1024 x 512
    # (4-wave kernel split along K, packed weight), then 64 x 512 x 1000 (K tail: both operands packed with zero
    # padding); each call reuses the scratch the one before left behind
    p1 = _run_both(256, 1024, 2048, seed=500)
    assert "kslices=2" in p1.describe(), p1.describe()
    p2 = _run_both(256, 1024, 512, seed=505)
    assert p2.describe().startswith("mfma_bf16_128x128") and "packB" in p2.describe(), p2.describe()
    p3 = _run_both(64, 512, 1000, seed=510)
    assert "packA" in p3.describe()


def test_noalloc_tail_slices_then_smaller():
    # 4352 x 4096 x 4096: 272 tiles, the last round's 16 in 4 K slices (16 MB of partial blocks in the scratch), then
    # a smaller call in 2 whole-grid slices over the same scratch
    p1 = _run_both(4352, 4096, 4096, seed=520)
    assert "kslices=4 tail=16" in p1.describe(), p1.describe()
    p2 = _run_both(512, 1024, 2048, seed=525)
    assert "kslices=" in p2.describe() and "tail=" not in p2.describe(), p2.describe()


def test_noalloc_f32_kmajor_in_place(monkeypatch):
    # f32 with the [K][N] weight read in place: 128 x 256 x 2048 on the 64 x 64 kernel split along K (its partial tiles
    # and arrival counters in the scratch), then a smaller 64 x 1024 x 1024 on the k-slice kernel, which needs none
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "11")
    p1 = _run_both(128, 256, 2048, seed=530, dt=O.F32)
    assert p1.describe().startswith("mfma_f32_64x64") and "kmajorB" in p1.describe(), p1.describe()
    monkeypatch.delenv("KUDNN_HIP_FORCE_CFG")
    p2 = _run_both(64, 1024, 1024, seed=535, dt=O.F32)
    assert p2.describe().startswith("mfma_f32_kslice") and "kmajorB" in p2.describe(), p2.describe()


def test_noalloc_refuses_what_it_cannot_do():
    # a packed weight of 128 MiB exceeds the scratch: refused before anything runs (N not a multiple of 8, so the
    # K-major weight cannot be read in place)
    M, N, Kd = 64, 16388, 4096
    plan = K.LinearPostOps(K.desc([M, Kd], K.BF16), K.desc([Kd, N], K.BF16, "AB"), K.desc([M, N], K.BF16))
    assert "packB" in plan.describe(), plan.describe()
    x = torch.zeros(M * Kd, dtype=torch.int16, device="cuda")
    w = torch.zeros(Kd * N, dtype=torch.int16, device="cuda")
    y = torch.zeros(M * N, dtype=torch.int16, device="cuda")
    lib = K.lib()
    st = lib.kudnn_linear_postops_run_noalloc(plan.handle, x.data_ptr(), w.data_ptr(), y.data_ptr(), None, None,
                                              ctypes.c_float(1.0), None)
    assert st == K.UNSUPPORTED and "workspace" in K.last_error()
    # host buffers would need staging allocations
    hx = np.zeros(M * Kd, np.uint16)
    st = lib.kudnn_linear_postops_run_noalloc(plan.handle, hx.ctypes.data, w.data_ptr(), y.data_ptr(), None, None,
                                              ctypes.c_float(1.0), None)
    assert st == K.BAD_ARGUMENTS
    torch.cuda.synchronize()


def test_noalloc_refuses_slices_that_do_not_fit():
    # 2048 x 8192 x 2560: 80 tiles in 2 K slices (40 MiB of f32 sums) plus the source packed from its [K][M] layout
    # (32 MiB) exceed the 64 MiB scratch. The allocation-free entry point refuses the plan instead of running it
    # unsliced, which would change the summation order; the allocating entry point runs it sliced.
    M, N, Kd = 2048, 2560, 8192
    dx, dw, dy = K.desc([M, Kd], K.BF16, "BA"), K.desc([Kd, N], K.BF16, "AB"), K.desc([M, N], K.BF16)
    plan = K.LinearPostOps(dx, dw, dy)
    assert "kslices=2" in plan.describe() and "packA" in plan.describe(), plan.describe()
    x = torch.zeros(M * Kd, dtype=torch.int16, device="cuda")
    w = torch.zeros(Kd * N, dtype=torch.int16, device="cuda")
    y = torch.full((M * N,), 7, dtype=torch.int16, device="cuda")
    st = K.lib().kudnn_linear_postops_run_noalloc(plan.handle, x.data_ptr(), w.data_ptr(), y.data_ptr(), None, None,
                                                  ctypes.c_float(1.0), None)
    assert st == K.UNSUPPORTED and "workspace" in K.last_error(), K.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7).all()), "a refused call wrote its output"
    plan.run(x, w, y)
    torch.cuda.synchronize()
    assert not bool(y.any()), "the allocating entry point did not run the plan"
