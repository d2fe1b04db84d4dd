"""ctypes binding of the CPU oracle (oracle.c). TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always as the checker or
as the timed CPU baseline; the product never imports it.

Tensors are (numpy storage buffer, descriptor) pairs: float32 storage for F32, uint16 bit patterns for
BF16/F16; descriptors carry dims and logical strides exactly like kudnn_tensor_desc.
"""
from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

_DIR = Path(__file__).resolve().parent
LIB_PATH = _DIR / "liboracle.so"

F32, F16, BF16, S32, S8, U8 = 1, 2, 3, 4, 5, 6
DT_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", S32: "s32", S8: "s8", U8: "u8"}
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SWISH, ACT_GELU_ERF = 0, 5, 20, 25, 27
# the other forward kinds (KuDNN::ActivationFunction values)
(ACT_ABS, ACT_EXP, ACT_LINEAR, ACT_LOG, ACT_ROUND, ACT_SQRT, ACT_SQUARE, ACT_TANH, ACT_SIGMOID, ACT_POW, ACT_CLIP,
 ACT_CLIP_V2, ACT_HARDSIGMOID, ACT_HARDSWISH, ACT_ELU, ACT_ELU_DST, ACT_SRELU, ACT_MISH) = (
    1, 2, 3, 4, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 19, 22, 26, 28)
RES_EXT, RES_MUL, RES_IDENTIAL = 0, 1, 2
BIN_NONE, BIN_ADD, BIN_EXT, BIN_MUL = 0, 1, 2, 3


class OTensor(ctypes.Structure):
    _fields_ = [
        ("ndims", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("dims", ctypes.c_int64 * 5),
        ("strides", ctypes.c_int64 * 5),
    ]


class OGemm(ctypes.Structure):
    _fields_ = [
        ("a", OTensor), ("b", OTensor), ("c", OTensor), ("bias", OTensor),
        ("pa", ctypes.c_void_p), ("pb", ctypes.c_void_p), ("pbias", ctypes.c_void_p), ("pc", ctypes.c_void_p),
        ("alpha", ctypes.c_float), ("beta", ctypes.c_float),
        ("reordered", ctypes.c_int32),
    ]


_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        T = ctypes.POINTER(OTensor)
        G = ctypes.POINTER(OGemm)
        sig = {
            "oracle_f32_to_bf16_rne": ([ctypes.c_float], ctypes.c_uint16),
            "oracle_f32_to_bf16_trunc": ([ctypes.c_float], ctypes.c_uint16),
            "oracle_f32_to_bf16_trunc_inf": ([ctypes.c_float], ctypes.c_uint16),
            "oracle_bf16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
            "oracle_f16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
            "oracle_f32_to_f16_rne": ([ctypes.c_float], ctypes.c_uint16),
            "oracle_f32_to_int_sat": ([ctypes.c_float, ctypes.c_int], ctypes.c_int64),
            "oracle_act_f32": ([ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_float], ctypes.c_float),
            "oracle_activation": ([T, P, ctypes.c_int, ctypes.c_float, ctypes.c_float], ctypes.c_int),
            "oracle_gemm": ([G], ctypes.c_int),
            "oracle_res_add": ([ctypes.c_int, ctypes.c_int64, P, P, P, ctypes.c_int, ctypes.c_float], ctypes.c_int),
            "oracle_binary": ([T, P, T, P, ctypes.c_int, ctypes.c_float], ctypes.c_int),
            "oracle_linear_act": ([G, ctypes.c_int, ctypes.c_float], ctypes.c_int),
            "oracle_linear_res": ([G, T, P, T, P, ctypes.c_int, ctypes.c_float], ctypes.c_int),
            "oracle_linear_postops": ([G, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int, T, P, ctypes.c_float],
                                      ctypes.c_int),
            "oracle_fill": ([P, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_double,
                             ctypes.c_double], ctypes.c_int),
            "oracle_cpu_baseline": ([ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, P, P, P, P,
                                     ctypes.c_int, P, ctypes.c_int, ctypes.c_float, ctypes.c_int], ctypes.c_int),
            "oracle_max_threads": ([], ctypes.c_int),
            "oracle_build_flags": ([], ctypes.c_char_p),
        }
        for name, (args, res) in sig.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


# ---------------------------------------------------------------------------------------------------
# tensors


def storage_dtype(dt: int):
    return {F32: np.float32, S32: np.int32, S8: np.int8, U8: np.uint8}.get(dt, np.uint16)


@dataclass
class Tensor:
    """A typed buffer plus its descriptor (dims, logical strides)."""

    dims: tuple
    strides: tuple
    dtype: int
    buf: np.ndarray  # flat storage

    @property
    def ndims(self) -> int:
        return len(self.dims)

    def otensor(self) -> OTensor:
        t = OTensor()
        t.ndims = len(self.dims)
        t.dtype = self.dtype
        for i, (d, s) in enumerate(zip(self.dims, self.strides)):
            t.dims[i] = d
            t.strides[i] = s
        return t

    def ptr(self) -> int:
        return self.buf.ctypes.data

    def logical(self) -> np.ndarray:
        """float32 array of the logical tensor (dims order)."""
        vals = to_f32(self.buf, self.dtype)
        itemsize = vals.itemsize
        view = np.lib.stride_tricks.as_strided(vals, shape=self.dims, strides=[s * itemsize for s in self.strides])
        return np.array(view, dtype=np.float32)


def extent(dims: Sequence[int], strides: Sequence[int]) -> int:
    if any(d == 0 for d in dims):
        return 0
    return 1 + sum((d - 1) * s for d, s in zip(dims, strides))


def empty(dims, strides, dt) -> Tensor:
    return Tensor(tuple(dims), tuple(strides), dt, np.zeros(extent(dims, strides), dtype=storage_dtype(dt)))


def fill(dims, strides, dt, seed: int, dist: str = "uniform", lo: float = -1.0, hi: float = 1.0) -> Tensor:
    """Seeded tensor: SplitMix64 uniform[lo,hi) or normal(mean=lo, std=hi); bf16/f16 by RNE of the f32 sample."""
    t = empty(dims, strides, dt)
    n = t.buf.size
    if n:
        lib().oracle_fill(t.ptr(), dt, n, seed, 0 if dist == "uniform" else 1, lo, hi)
    return t


def to_f32(buf: np.ndarray, dt: int) -> np.ndarray:
    if dt == F32:
        return buf.astype(np.float32, copy=False)
    if dt == BF16:
        return (buf.astype(np.uint32) << 16).view(np.float32)
    if dt == F16:
        return buf.view(np.float16).astype(np.float32)
    if dt in (S32, S8, U8):
        return buf.astype(np.float32)
    raise ValueError(dt)


def from_f32_rne(x: np.ndarray, dt: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dt == F32:
        return x.copy()
    if dt == BF16:
        u = x.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
        return r
    if dt == F16:
        return x.astype(np.float16).view(np.uint16)
    raise ValueError(dt)


# ---------------------------------------------------------------------------------------------------
# operators


def _gemm_struct(a: Tensor, b: Tensor, c: Tensor, bias: Optional[Tensor], alpha=1.0, beta=0.0) -> OGemm:
    g = OGemm()
    g.a, g.b, g.c = a.otensor(), b.otensor(), c.otensor()
    g.pa, g.pb, g.pc = a.ptr(), b.ptr(), c.ptr()
    if bias is not None:
        g.bias = bias.otensor()
        g.pbias = bias.ptr()
    g.alpha, g.beta = alpha, beta
    return g


_STANDARD_LAYOUTS = {3: "ABC", 4: "ABCD", 5: "ABCDE"}
REORDERED_A, REORDERED_B, REORDERED_C, REORDERED_BIAS = 1, 2, 4, 8  # O_REORDERED_* of oracle.h


def reordered_mask(ndims: int, la=None, lb=None, lc=None, lbias=None) -> int:
    """The tensors the reference's BatchedExtendedGemm copies to f32 before ChooseImpl (kudnn_gemm.cpp:722-765): those
    of more than two dims whose layout (a name such as "ABCED"; None = the standard order) is not ABC.., ABCD..."""
    mask = 0
    for bit, lay in ((REORDERED_A, la), (REORDERED_B, lb), (REORDERED_C, lc), (REORDERED_BIAS, lbias)):
        if ndims > 2 and lay is not None and lay != _STANDARD_LAYOUTS[ndims]:
            mask |= bit
    return mask


def gemm(a, b, c, bias=None, alpha=1.0, beta=0.0, reordered=0) -> None:
    """In place into c.buf: Gemm::Run semantics. reordered: reordered_mask() of the tensors' layouts."""
    g = _gemm_struct(a, b, c, bias, alpha, beta)
    g.reordered = reordered
    assert lib().oracle_gemm(ctypes.byref(g)) == 0


def linear_act(a, b, c, bias=None, kind=ACT_RELU, alpha=0.0) -> None:
    """LinearActivationLayerFWD::Run: the activation gets the layer's alpha; its second parameter is 0 whatever the
    layer's beta (kudnn_linear_activationlayer.cpp:33)."""
    g = _gemm_struct(a, b, c, bias)
    assert lib().oracle_linear_act(ctypes.byref(g), kind, alpha) == 0


def linear_res(a, b, c, bias, res, lr, kind=RES_IDENTIAL, gamma=1.0) -> None:
    g = _gemm_struct(a, b, c, bias)
    rt, lt = res.otensor(), lr.otensor()
    assert lib().oracle_linear_res(ctypes.byref(g), ctypes.byref(rt), res.ptr(), ctypes.byref(lt), lr.ptr(), kind,
                                   gamma) == 0


def linear_postops(a, b, y, bias=None, act=ACT_NONE, act_alpha=0.0, binary=BIN_NONE, src=None, gamma=1.0,
                   act_beta=0.0) -> None:
    g = _gemm_struct(a, b, y, bias)
    st = src.otensor() if src is not None else OTensor()
    sp = src.ptr() if src is not None else None
    assert lib().oracle_linear_postops(ctypes.byref(g), act, act_alpha, act_beta, binary, ctypes.byref(st), sp, gamma) == 0


def activation(t: Tensor, kind: int, alpha: float = 0.0, beta: float = 0.0) -> None:
    """In place over a dense tensor: the activation stage with the kind's bf16 store rule."""
    ot = t.otensor()
    assert lib().oracle_activation(ctypes.byref(ot), t.ptr(), kind, alpha, beta) == 0


def binary(y: Tensor, src: Tensor, kind: int, gamma: float = 1.0) -> None:
    """In place into y: the binary stage of the post-op chain against a same-shaped src."""
    yt, st = y.otensor(), src.otensor()
    assert lib().oracle_binary(ctypes.byref(yt), y.ptr(), ctypes.byref(st), src.ptr(), kind, gamma) == 0


def f32_to_int_sat(x: float, dt: int) -> int:
    """ConvertFp32ToS32 / ToS8 / ToU8 of one f32 value (saturate, then round half to even)."""
    return lib().oracle_f32_to_int_sat(x, dt)


def act_f32(kind: int, x: float, alpha: float = 0.0, beta: float = 0.0) -> float:
    return lib().oracle_act_f32(kind, x, alpha, beta)


def cpu_baseline(dt, M, N, K, X, W, bias, R, Y, act, act_alpha, threads, r_mul=False) -> None:
    """The reference tests' naive loop (f32 accumulation), OpenMP over rows; X[M][K], W[N][K], Y[M][N]; R (optional)
    added to, or with r_mul multiplied into, the activated result."""
    ptr = lambda t: None if t is None else t.ctypes.data
    assert lib().oracle_cpu_baseline(dt, M, N, K, ptr(X), ptr(W), ptr(bias), ptr(R), int(r_mul), ptr(Y), act,
                                     act_alpha, threads) == 0


def max_threads() -> int:
    return lib().oracle_max_threads()


def build_flags() -> str:
    """The C compiler flags liboracle.so was built with."""
    return lib().oracle_build_flags().decode()
