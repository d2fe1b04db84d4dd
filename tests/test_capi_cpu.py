"""C ABI checks that need no GPU: the library loads and exports every entry point include/kudnn_hip.h
declares, descriptors get KuDNN's strides, validation follows KuDNN's rules, and the dispatcher picks the
intended kernel family for each BASELINE config. (Plan creation makes no HIP calls.)"""
import re
from pathlib import Path

import pytest

import kudnn_amd as K

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "kudnn_hip.h").read_text()
    return sorted(set(re.findall(r"KUDNN_HIP_API\s+[\w\s\*]+?\b(kudnn_\w+)\s*\(", text)))


def test_header_declares_what_the_binding_binds():
    decl = declared_symbols()
    assert len(decl) >= 30
    assert sorted(K.exported_symbols()) == decl


def test_library_exports_every_declared_symbol():
    lib = K.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert K.lib().kudnn_version().decode().startswith("kudnn-mi355x")


def test_cpp_library_exports_kudnn_classes():
    import ctypes
    import subprocess

    so = K.LIB_DIR / "libkudnn.so"
    ctypes.CDLL(str(so))
    out = subprocess.run(["nm", "-DC", "--defined-only", str(so)], capture_output=True, text=True, check=True).stdout
    for sym in ("KuDNN::Gemm::Gemm(", "KuDNN::Gemm::Run(", "KuDNN::LinearActivationLayerFWD::Run(",
                "KuDNN::LinearResFWD::Run(", "KuDNN::LinearPostOpsFWD::Run(", "KuDNN::Threading::GetMaxNumThreads()",
                "KuDNN::TensorInfo::ValidateLayout<false>", "KuDNN::Service::AlignedAlloc("):
        assert sym in out, sym


@pytest.mark.parametrize("layout,dims,strides", [
    ("AB", [3, 4], (4, 1)),
    ("BA", [3, 4], (1, 3)),
    ("AB", [1, 4], (0, 1)),
    ("ABC", [2, 3, 4], (12, 4, 1)),
    ("ACB", [2, 3, 4], (12, 1, 3)),
    ("CAB", [2, 3, 4], (3, 1, 6)),
    ("ABCED", [2, 3, 4, 5, 6], (360, 120, 30, 1, 5)),
    ("DECAB", [2, 3, 4, 5, 6], (3, 1, 6, 144, 24)),
])
def test_descriptor_min_strides(layout, dims, strides):
    d = K.desc(dims, K.F32, layout)
    assert d.stride() == strides
    assert K.lib().kudnn_tensor_desc_is_dense(d) == 1


def test_descriptor_errors():
    with pytest.raises(K.KudnnError) as e:
        K.desc([2, 3], K.F32, "ABC")
    assert e.value.status == K.BAD_ARGUMENTS
    with pytest.raises(K.KudnnError):
        K.desc([2, 3], K.DT_UNDEFINED, "AB")
    with pytest.raises(K.KudnnError):
        K.desc([4, 5], K.F32, "AB", strides=[4, 1])  # below the minimum stride
    d = K.desc([4, 5], K.F32, "AB", strides=[8, 1])
    assert K.lib().kudnn_tensor_desc_is_dense(d) == 0


def validate(a, b, c, bias=None, nt=0):
    return K.lib().kudnn_gemm_validate(a, b, c, bias, nt)


def test_gemm_validation_rules():
    F = K.F32
    a, b, c = K.desc([5, 6], F), K.desc([6, 7], F, "BA"), K.desc([5, 7], F)
    assert validate(a, b, c) == K.SUCCESS
    assert validate(a, K.desc([7, 7], F), c) == K.BAD_ARGUMENTS                    # K mismatch
    assert validate(a, b, K.desc([5, 8], F)) == K.BAD_ARGUMENTS                    # N mismatch
    assert validate(K.desc([5, 6], K.S32), b, c) == K.UNSUPPORTED                  # S32 source
    assert validate(a, b, K.desc([5, 7], F, "AB", strides=[8, 1])) == K.UNSUPPORTED  # strided destination
    assert validate(a, b, c, K.desc([2, 7], F)) == K.BAD_ARGUMENTS                 # bias rows neither 1 nor M
    assert validate(a, b, c, K.desc([5, 1], F)) == K.SUCCESS
    assert validate(a, b, c, K.desc([1, 1, 7], F)) == K.BAD_ARGUMENTS             # bias rank differs
    assert validate(a, b, c, nt=-1) == K.BAD_ARGUMENTS
    assert validate(a, b, c, nt=K.lib().kudnn_threading_get_max_num_threads() + 1) == K.BAD_ARGUMENTS
    assert validate(K.desc([1, 6], F), K.desc([6, 7], F), K.desc([1, 7], F)) == K.SUCCESS
    assert validate(K.desc([0, 6], F), b, K.desc([0, 7], F)) == K.UNSUPPORTED      # zero-size
    # batch dims: equal or 1
    a3, b3 = K.desc([4, 5, 6], F), K.desc([1, 6, 7], F)
    assert validate(a3, b3, K.desc([4, 5, 7], F)) == K.SUCCESS
    assert validate(a3, K.desc([3, 6, 7], F), K.desc([4, 5, 7], F)) == K.BAD_ARGUMENTS


def test_linear_act_validation_and_kinds():
    F = K.F32
    a, b, c = K.desc([5, 6], F), K.desc([6, 7], F), K.desc([5, 7], F)
    v = lambda kind, alpha=0.0, beta=0.0, cc=c: K.lib().kudnn_linear_act_validate(a, b, cc, None, alpha, beta, kind, 0)
    assert v(K.ACT_RELU) == K.SUCCESS
    assert v(K.ACT_TANH) == K.SUCCESS
    # every forward kind of KuDNN's eltwise table is a fused epilogue; the backward-only kinds are refused
    for kind in (K.ACT_ABS, K.ACT_EXP, K.ACT_LINEAR, K.ACT_LOG, K.ACT_ROUND, K.ACT_SQRT, K.ACT_SQUARE, K.ACT_TANH,
                 K.ACT_SIGMOID, K.ACT_POW, K.ACT_CLIP, K.ACT_CLIP_V2, K.ACT_HARDSIGMOID, K.ACT_HARDSWISH, K.ACT_ELU,
                 K.ACT_ELU_DST, K.ACT_SRELU, K.ACT_MISH):
        # CLIP's lower bound must not exceed the activation member's upper bound, which is 0 (see below)
        alpha = -1.0 if kind in (K.ACT_CLIP, K.ACT_CLIP_V2) else 1.0
        K.LinearActivation(a, b, c, None, alpha, 2.0, kind)
    exp_dst = 16
    assert v(exp_dst) == K.UNSUPPORTED
    with pytest.raises(K.KudnnError) as e:
        K.LinearActivation(a, b, c, None, 0.0, 0.0, exp_dst)
    assert e.value.status == K.UNSUPPORTED
    assert v(K.ACT_UNIMPLEMENTED) == K.UNSUPPORTED
    assert v(K.ACT_CLIP, 2.0, 1.0) == K.UNSUPPORTED  # alpha > beta
    assert v(K.ACT_SRELU, 0.0) == K.UNSUPPORTED
    assert v(K.ACT_SWISH, cc=K.desc([5, 7], K.S8)) == K.UNSUPPORTED


def test_linear_act_beta_reaches_validation_only():
    # The reference builds the layer's activation as activationlayerfwd(cInfo, cInfo, kind, alpha)
    # (kudnn_linear_activationlayer.cpp:33): that member validates with beta = 0 and runs with beta = 0, while the
    # layer's own ValidateInput sees the caller's beta.
    F = K.F32
    a, b, c = K.desc([5, 6], F), K.desc([6, 7], F), K.desc([5, 7], F)
    lib = K.lib()
    # CLIP with 0 < alpha <= beta: the static check passes, the constructor refuses (alpha > the member's beta 0)
    assert lib.kudnn_linear_act_validate(a, b, c, None, 0.5, 1.0, K.ACT_CLIP, 0) == K.SUCCESS
    with pytest.raises(K.KudnnError) as e:
        K.LinearActivation(a, b, c, None, 0.5, 1.0, K.ACT_CLIP)
    assert e.value.status == K.UNSUPPORTED and "Activation layer" in str(e.value)
    # CLIP with alpha <= 0 < ... but alpha > beta: the member passes (alpha <= 0), the layer's own check refuses
    with pytest.raises(K.KudnnError) as e:
        K.LinearActivation(a, b, c, None, -0.5, -1.0, K.ACT_CLIP)
    assert e.value.status == K.UNSUPPORTED and "LinearActivationLayerFWD" in str(e.value)
    K.LinearActivation(a, b, c, None, -0.5, 1.0, K.ACT_CLIP)


def test_batch_dim_of_output_must_match_operands():
    # src [1,M,K] x wei [4,K,N] -> dst [2,M,N] passes the reference's validation (a weight dim is compared with src's
    # only when src's is not 1) but would address 4 batches of a 2-batch output: refused at plan creation
    F = K.F32
    a, b = K.desc([1, 64, 128], F), K.desc([4, 128, 64], F)
    assert K.lib().kudnn_gemm_validate(a, b, K.desc([2, 64, 64], F), None, 0) == K.SUCCESS
    with pytest.raises(K.KudnnError) as e:
        K.Gemm(a, b, K.desc([2, 64, 64], F))
    assert e.value.status == K.BAD_ARGUMENTS
    with pytest.raises(K.KudnnError):
        K.LinearActivation(a, b, K.desc([2, 64, 64], F), K.desc([2, 1, 64], F), 0.0, 0.0, K.ACT_RELU)
    # dst batch = the operands' batch count (src broadcast) and dst batch 1 (the serial loop) stay accepted
    assert "batches=4" in K.Gemm(a, b, K.desc([4, 64, 64], F)).describe()
    assert "serial" in K.Gemm(a, b, K.desc([1, 64, 64], F)).describe()


def test_decode_kernel_rule(monkeypatch):
    # M <= 5: the GEMV with X staged in LDS (M = 1 named apart); 6 <= M <= 16, one batch, K <= 4096: the K-split GEMV
    # with X in registers; otherwise 16-row MFMA tiles (bf16 and f16)
    assert plan_of(1, 4096, 4096).describe().startswith("skinny_bf16_gemv_row ")
    for M in (2, 3, 4, 5):
        assert plan_of(M, 4096, 14336).describe().startswith("skinny_bf16_gemv_rows_xlds"), M
        assert plan_of(M, 1000, 300, K.F16).describe().startswith("skinny_f16_gemv_rows_xlds"), M
    for M in (6, 8, 16):
        assert plan_of(M, 4096, 14336).describe().startswith("skinny_bf16_kgemv_xreg"), M
        assert plan_of(M, 1000, 300, K.F16).describe().startswith("skinny_f16_kgemv_xreg"), M
    assert plan_of(16, 4104, 4096).describe().startswith("skinny_bf16_16xK")  # K > 4096
    batched = K.LinearPostOps(K.desc([2, 8, 512], K.BF16, "ABC"), K.desc([2, 512, 300], K.BF16, "ACB"),
                              K.desc([2, 8, 300], K.BF16, "ABC"))
    assert batched.describe().startswith("skinny_bf16_16xK"), batched.describe()
    # the overrides: the 16-row kernel and the K-split GEMV for 2 <= M <= 16, the staged GEMV for 2 <= M <= 8
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "20")
    assert plan_of(4, 4096, 4096).describe().startswith("skinny_bf16_16xK")
    assert plan_of(12, 4096, 4096).describe().startswith("skinny_bf16_16xK")
    assert plan_of(1, 4096, 4096).describe().startswith("skinny_bf16_gemv_row ")
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "23")
    assert plan_of(2, 4096, 4096).describe().startswith("skinny_bf16_kgemv_xreg")
    monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", "22")
    assert plan_of(8, 4096, 4096).describe().startswith("skinny_bf16_gemv_rows_xlds")
    assert plan_of(9, 4096, 4096).describe().startswith("skinny_bf16_kgemv_xreg")
    assert plan_of(64, 4096, 4096).describe().startswith("mfma_bf16")


def test_f32_kmajor_weight_rule(monkeypatch):
    # an fp32 [K][N] weight (layout AB) is read in place by the 128 x 128 and 64 x 64 kernels when N is a multiple of 4
    # and K of 32, and by the k-slice kernel for K = 256 c; otherwise, or with KUDNN_HIP_PACK_KMAJOR set, it is packed
    # to [N][K]
    def f32_plan(M, Kd, N):
        return K.Gemm(K.desc([M, Kd], K.F32), K.desc([Kd, N], K.F32, "AB"), K.desc([M, N], K.F32)).describe()
    for M, Kd, N in ((4096, 4608, 1152), (512, 512, 1024), (1024, 640, 772), (8192, 64, 4)):
        d = f32_plan(M, Kd, N)
        assert d.startswith("mfma_f32_") and "kmajorB" in d and "packB" not in d, d
    for M, Kd, N in ((1024, 640, 1158), (1024, 648, 1160), (4096, 3256, 1152)):
        d = f32_plan(M, Kd, N)
        assert "packB" in d and "kmajorB" not in d, d
    # the k-slice kernel of small grids: in place when K = 256 c, c in 1, 2, 3, 4, 6, 8, 12, 16 (C1's shape in Matmul
    # mode), packed otherwise (K = 1280)
    d = f32_plan(128, 1024, 1024)
    assert d.startswith("mfma_f32_kslice") and "kmajorB" in d and "packB" not in d, d
    d = f32_plan(128, 1280, 1024)
    assert d.startswith("mfma_f32_kslice") and "packB" in d, d
    monkeypatch.setenv("KUDNN_HIP_PACK_KMAJOR", "1")
    assert "packB" in f32_plan(512, 512, 1024)


def test_kslice_rule():
    # small 16-bit grids: the ping-pong kernel with K slices (tiles x slices <= 128, slices of >= 16 k-tiles); not at
    # 64 tiles with < 64 k-tiles (the 4-wave kernel), nor from 97 tiles on, nor for M < 1024 above 64 tiles
    for (M, N, Kd), S in {(256, 4096, 4096): 4, (256, 4096, 14336): 8, (512, 4096, 14336): 4, (1024, 4096, 11008): 2,
                          (4096, 1152, 4608): 2, (4096, 1536, 5120): 2}.items():
        d = plan_of(M, Kd, N).describe()
        assert d.startswith("mfma_bf16_pingpong") and f" kslices={S}" in d, d
        assert f" kslices={S}" in plan_of(M, Kd, N, K.F16).describe()
    for M, N, Kd in ((2048, 2048, 2048), (512, 11008, 4096), (2048, 4096, 4096), (4096, 11008, 4096)):
        assert "kslices" not in plan_of(M, Kd, N).describe(), (M, N, Kd)
    assert plan_of(2048, 2048, 2048).describe().startswith("mfma_bf16_128x128")
    assert "kslices" not in plan_of(256, 4096, 4096, K.F32).describe()
    # 32-64 tiles with at most 64 k-tiles: the 4-wave kernel when the weight is stored [N][K]; stored [K][N], the
    # ping-pong kernel reads it in place, in K slices
    for M, N, Kd in ((256, 11008, 4096), (1024, 4096, 4096), (1024, 2048, 2048), (512, 4096, 4096)):
        assert plan_of(M, Kd, N).describe().startswith("mfma_bf16_128x128"), (M, N, Kd)
        assert plan_of(M, Kd, N, K.F16).describe().startswith("mfma_f16_128x128"), (M, N, Kd)
        d = plan_of(M, Kd, N, wl="AB").describe()
        assert d.startswith("mfma_bf16_pingpong") and "kslices=" in d and "kmajorB" in d, d


def test_forced_mfma_config_keeps_decode_plans(monkeypatch):
    # a forced 4-wave or ping-pong configuration needs whole k-tiles, which only the prefill plans pack for: a
    # 16-bit plan with M <= 16 keeps its decode kernel
    for cfg in ("1", "2", "3", "4"):
        monkeypatch.setenv("KUDNN_HIP_FORCE_CFG", cfg)
        assert plan_of(4, 200, 64).describe().startswith("skinny_bf16"), cfg
        assert plan_of(64, 256, 64).describe().startswith("mfma_bf16")


def test_linear_res_validation():
    F = K.F32
    a, b, c = K.desc([5, 6], F), K.desc([6, 7], F), K.desc([5, 7], F)
    v = lambda res, lr, kind: K.lib().kudnn_linear_res_validate(a, b, c, None, res, lr, kind, 0)
    assert v(K.desc([5, 7], F), K.desc([5, 7], F), K.RES_IDENTIAL) == K.SUCCESS
    assert v(K.desc([7, 3], F), K.desc([5, 3], F), K.RES_MUL) == K.SUCCESS
    assert v(K.desc([7, 3], K.S32), K.desc([5, 3], F), K.RES_MUL) == K.UNSUPPORTED
    assert v(K.desc([6, 7], F), K.desc([5, 7], F), K.RES_EXT) == K.BAD_ARGUMENTS
    assert v(K.desc([5, 7], F), K.desc([5, 7], F), 7) == K.UNSUPPORTED


def plan_of(M, Kd, N, dt=K.BF16, wl="BA", **kw):
    return K.LinearPostOps(K.desc([M, Kd], dt), K.desc([Kd, N], dt, wl), K.desc([M, N], dt), **kw)


def test_dispatcher_choices():
    assert plan_of(4096, 4096, 11008).describe().startswith("mfma_bf16_pingpong_256x256 M=4096 N=11008 K=4096")
    for M in (1, 4, 16):
        for N in (4096, 14336):
            assert plan_of(M, 4096, N).describe().startswith("skinny_bf16")
    assert plan_of(17, 4096, 4096).describe().startswith("mfma_bf16")
    assert plan_of(2048, 4096, 4096, K.F32).describe().startswith("mfma_f32_128x128")
    assert plan_of(128, 1024, 1024, K.F32).describe().startswith("mfma_f32_kslice_16x32")
    assert plan_of(100, 2048, 200, K.F32).describe().startswith("mfma_f32_64x64")  # 49 tiles of 16 x 32: split-K
    # C5: 3-D input with a batch-broadcast K-major weight folds into one M=16384 GEMM
    p = K.LinearActivation(K.desc([8, 2048, 5120], K.BF16, "ABC"), K.desc([1, 5120, 13824], K.BF16, "ABC"),
                           K.desc([8, 2048, 13824], K.BF16, "ABC"), K.desc([1, 1, 13824], K.BF16, "ABC"), 1.0, 0.0,
                           K.ACT_SWISH)
    assert p.describe().startswith("mfma_bf16_pingpong_256x256 M=16384 N=13824 K=5120 batches=1")
    # a K not a multiple of the k-tile is packed (zero-padded)
    assert "packA" in plan_of(300, 200, 260).describe()


@pytest.mark.parametrize("M,Kd,N,cfg", [
    (512, 4096, 11008, "pingpong"),   # 2 x 43 = 86 tiles of 256 x 256: from 80 on, the ping-pong kernel
    (3072, 14336, 4096, "pingpong"),  # 192 tiles: a partial round still goes to the ping-pong kernel
    (1024, 4096, 4096, "128x128"),    # 64 tiles, 64 k-tiles: the 4-wave kernel's 256 tiles of 128 x 128
    (1024, 11008, 4096, "pingpong"),  # 64 tiles, 172 k-tiles: K slices
    (512, 14336, 4096, "pingpong"),   # 32 tiles, 224 k-tiles: K slices
    (512, 11008, 4096, "pingpong"),   # 32 tiles, 172 k-tiles: K slices
    (256, 8192, 8192, "pingpong"),    # 32 tiles, 128 k-tiles: K slices
    (2048, 2048, 2048, "128x128"),    # 64 tiles, 32 k-tiles: the 4-wave kernel fills the CUs
    (256, 256, 2048, "128x128"),      # 8 tiles, 4 k-tiles: too short to slice
])
def test_dispatch_rule(M, Kd, N, cfg):
    # the planner's measured rule (bench.py --only dispatch): ping-pong from 80 tiles of 256 x 256, or with K slices
    # on small grids (kudnn_kslice_rule), or with long K for its tail split; else 4-wave 128 x 128
    assert plan_of(M, Kd, N).describe().startswith(f"mfma_bf16_{cfg}"), plan_of(M, Kd, N).describe()
    assert plan_of(M, Kd, N, K.F16).describe().startswith(f"mfma_f16_{cfg}")


def test_run_rejects_null_pointers_without_gpu():
    p = plan_of(64, 64, 64)
    with pytest.raises(K.KudnnError) as e:
        p.run(None, None, None)
    assert e.value.status == K.NULL_POINTER


def test_threading_api_contract():
    lib = K.lib()
    mx = lib.kudnn_threading_get_max_num_threads()
    assert mx >= 1
    assert lib.kudnn_threading_set_max_num_threads(0) == mx          # ignored, old value returned
    assert lib.kudnn_threading_get_max_num_threads() == mx
