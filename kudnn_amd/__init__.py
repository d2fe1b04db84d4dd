"""Python (ctypes) binding of the MI355X KuDNN Linear/GEMM C ABI (``include/kudnn_hip.h``).

The product is the pair of native libraries under ``kudnn_amd/lib``; this module only binds the C ABI
the way a ctypes caller would, for the tests and the benchmark.
Pointers passed to ``run`` may be device pointers (torch CUDA/HIP tensors, the fast path) or host
pointers (staged by the library). There is no fallback: if ``libkudnn_hip.so`` is missing, ``lib()``
raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence

_PKG = Path(__file__).resolve().parent
LIB_DIR = _PKG / "lib"

MAX_DIMS = 5

# status codes (kudnn_hip.h)
SUCCESS, UNSUPPORTED, BAD_ARGUMENTS, NULL_POINTER, ALLOC_FAILED, HIP_ERROR, INTERNAL = range(7)

# element types == KuDNN::Element::TypeT
DT_UNDEFINED, F32, F16, BF16, S32, S8, U8 = range(7)
DT_SIZE = {F32: 4, F16: 2, BF16: 2, S32: 4, S8: 1, U8: 1}

# layouts == KuDNN::Layout
_LAYOUT_NAMES = [
    "UNDEFINED", "A", "AB", "BA", "ABC", "ACB", "BAC", "BCA", "CAB", "CBA",
    "ABCD", "ABDC", "ACBD", "ACDB", "ADBC", "ADCB", "BACD", "BCDA", "CDAB", "CDBA", "DCAB",
    "ABCDE", "ABCED", "ABDEC", "ACBDE", "ACDEB", "ADECB", "BACDE", "BCDEA", "CDEAB", "CDEBA", "DECAB",
]
LAYOUT = {name: i for i, name in enumerate(_LAYOUT_NAMES)}
STANDARD_LAYOUT = {1: "A", 2: "AB", 3: "ABC", 4: "ABCD", 5: "ABCDE"}

# activation kinds == KuDNN::ActivationFunction
ACT_UNIMPLEMENTED = 0
ACT_ABS = 1
ACT_EXP = 2
ACT_LINEAR = 3
ACT_LOG = 4
ACT_RELU = 5
ACT_ROUND = 6
ACT_SQRT = 7
ACT_SQUARE = 8
ACT_TANH = 9
ACT_SIGMOID = 10
ACT_POW = 11
ACT_CLIP = 12
ACT_CLIP_V2 = 13
ACT_HARDSIGMOID = 14
ACT_HARDSWISH = 15
ACT_ELU = 19
ACT_GELU_TANH = 20
ACT_ELU_DST = 22
ACT_SWISH = 25
ACT_SRELU = 26
ACT_GELU_ERF = 27
ACT_MISH = 28

# residual kinds == KuDNN::ResOpsFunction
RES_EXT, RES_MUL, RES_IDENTIAL = 0, 1, 2
# binary post-op of the post-op chain
BIN_NONE, BIN_ADD, BIN_EXT, BIN_MUL = 0, 1, 2, 3


class TensorDesc(ctypes.Structure):
    _fields_ = [
        ("ndims", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("dims", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
    ]

    def shape(self):
        return tuple(self.dims[i] for i in range(self.ndims))

    def stride(self):
        return tuple(self.strides[i] for i in range(self.ndims))


class KudnnError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status


_lib = None

_P = ctypes.c_void_p
_D = ctypes.POINTER(TensorDesc)
_SIGS = {
    "kudnn_last_error": ([], ctypes.c_char_p),
    "kudnn_version": ([], ctypes.c_char_p),
    "kudnn_stream_synchronize": ([_P], ctypes.c_int),
    "kudnn_tensor_desc_init": ([_D, ctypes.c_int32, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int32],
                               ctypes.c_int),
    "kudnn_tensor_desc_init_strided": ([_D, ctypes.c_int32, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                                        ctypes.c_int32, ctypes.POINTER(ctypes.c_int64)], ctypes.c_int),
    "kudnn_tensor_desc_is_dense": ([_D], ctypes.c_int),
    "kudnn_threading_get_max_num_threads": ([], ctypes.c_int),
    "kudnn_threading_set_max_num_threads": ([ctypes.c_int], ctypes.c_int),
    "kudnn_threading_set_fixed_num_threads": ([ctypes.c_int], ctypes.c_int),
    "kudnn_threading_set_num_threads_local": ([ctypes.c_int], ctypes.c_int),
    "kudnn_threading_should_calculate_opt_threads": ([], ctypes.c_int),
    "kudnn_threading_set_env_mode": ([ctypes.c_int], ctypes.c_int),
    "kudnn_threading_get_control_status": ([], ctypes.c_int),
    "kudnn_gemm_validate": ([_D, _D, _D, _D, ctypes.c_int], ctypes.c_int),
    "kudnn_gemm_create": ([_D, _D, _D, _D, ctypes.c_int, ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_gemm_run": ([_P, _P, _P, _P, _P, ctypes.c_float, ctypes.c_float, ctypes.c_int, _P], ctypes.c_int),
    "kudnn_gemm_clone": ([_P, ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_gemm_destroy": ([_P], ctypes.c_int),
    "kudnn_linear_act_validate": ([_D, _D, _D, _D, ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int],
                                  ctypes.c_int),
    "kudnn_linear_act_create": ([_D, _D, _D, _D, ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                 ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_linear_act_run": ([_P, _P, _P, _P, _P, ctypes.c_int, _P], ctypes.c_int),
    "kudnn_linear_act_clone": ([_P, ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_linear_act_destroy": ([_P], ctypes.c_int),
    "kudnn_linear_res_validate": ([_D, _D, _D, _D, _D, _D, ctypes.c_int, ctypes.c_int], ctypes.c_int),
    "kudnn_linear_res_create": ([_D, _D, _D, _D, _D, _D, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                 ctypes.c_int, ctypes.c_int, ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_linear_res_run": ([_P, _P, _P, _P, _P, _P, _P, ctypes.c_float, ctypes.c_int, _P], ctypes.c_int),
    "kudnn_linear_res_clone": ([_P, ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_linear_res_destroy": ([_P], ctypes.c_int),
    "kudnn_linear_postops_create": ([_D, _D, _D, _D, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int, _D,
                                     ctypes.c_float, ctypes.c_int, ctypes.POINTER(_P)], ctypes.c_int),
    "kudnn_linear_postops_run": ([_P, _P, _P, _P, _P, _P, ctypes.c_float, _P], ctypes.c_int),
    "kudnn_linear_postops_destroy": ([_P], ctypes.c_int),
    "kudnn_linear_postops_run_noalloc": ([_P, _P, _P, _P, _P, _P, ctypes.c_float, _P], ctypes.c_int),
    "kudnn_plan_describe": ([_P, ctypes.c_char_p, ctypes.c_int], ctypes.c_int),
    "kudnn_pingpong_source_digest": ([], ctypes.c_char_p),
}


def lib_path() -> Path:
    return Path(os.environ.get("KUDNN_HIP_LIB", LIB_DIR / "libkudnn_hip.so"))


def lib() -> ctypes.CDLL:
    """Loads libkudnn_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not path.exists():
            raise FileNotFoundError(f"{path} is missing: build it with `python -m kudnn_amd.build`")
        l = ctypes.CDLL(str(path))
        for name, (args, res) in _SIGS.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def last_error() -> str:
    return lib().kudnn_last_error().decode()


def check(status: int) -> None:
    if status != SUCCESS:
        raise KudnnError(status, last_error())


def layout_value(layout) -> int:
    return LAYOUT[layout] if isinstance(layout, str) else int(layout)


def desc(dims: Sequence[int], dtype: int, layout=None, strides: Optional[Sequence[int]] = None) -> TensorDesc:
    """TensorInfo(shape, type, layout[, strides]) as a POD descriptor."""
    d = TensorDesc()
    nd = len(dims)
    layout = layout if layout is not None else STANDARD_LAYOUT[nd]
    arr = (ctypes.c_int64 * MAX_DIMS)(*dims)
    if strides is None:
        check(lib().kudnn_tensor_desc_init(ctypes.byref(d), nd, arr, dtype, layout_value(layout)))
    else:
        sarr = (ctypes.c_int64 * MAX_DIMS)(*strides)
        check(lib().kudnn_tensor_desc_init_strided(ctypes.byref(d), nd, arr, dtype, layout_value(layout), sarr))
    return d


def _ref(d: Optional[TensorDesc]):
    return ctypes.byref(d) if d is not None else None


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):  # numpy array
        return x.ctypes.data
    raise TypeError(f"cannot take a pointer of {type(x)}")


def _stream(stream) -> Optional[int]:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


class _Plan:
    _destroy = ""

    def __init__(self):
        self.handle = ctypes.c_void_p()

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(512)
        check(lib().kudnn_plan_describe(self.handle, buf, 512))
        return buf.value.decode()

    def close(self):
        if self.handle:
            getattr(lib(), self._destroy)(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Gemm(_Plan):
    """KuDNN::Gemm: C = alpha * A x B + beta * C (+ bias)."""

    _destroy = "kudnn_gemm_destroy"

    def __init__(self, a: TensorDesc, b: TensorDesc, c: TensorDesc, bias: Optional[TensorDesc] = None,
                 num_threads: int = 0):
        super().__init__()
        check(lib().kudnn_gemm_create(_ref(a), _ref(b), _ref(c), _ref(bias), num_threads, ctypes.byref(self.handle)))

    def run(self, a, b, c, bias=None, alpha=1.0, beta=0.0, num_threads=0, stream=None):
        check(lib().kudnn_gemm_run(self.handle, _ptr(a), _ptr(b), _ptr(c), _ptr(bias), alpha, beta, num_threads,
                                   _stream(stream)))


class LinearActivation(_Plan):
    """KuDNN::LinearActivationLayerFWD: C = act(A x B + bias)."""

    _destroy = "kudnn_linear_act_destroy"

    def __init__(self, a, b, c, bias=None, alpha=1.0, beta=0.0, kind=ACT_RELU, num_threads=0):
        super().__init__()
        check(lib().kudnn_linear_act_create(_ref(a), _ref(b), _ref(c), _ref(bias), alpha, beta, kind, num_threads,
                                            ctypes.byref(self.handle)))

    def run(self, a, b, c, bias=None, num_threads=0, stream=None):
        check(lib().kudnn_linear_act_run(self.handle, _ptr(a), _ptr(b), _ptr(c), _ptr(bias), num_threads,
                                         _stream(stream)))


class LinearRes(_Plan):
    """KuDNN::LinearResFWD: C = A x B + bias, linearRes = C + res | C + gamma*res | C x res."""

    _destroy = "kudnn_linear_res_destroy"

    def __init__(self, a, b, c, bias, res, linear_res, alpha=1.0, beta=0.0, gamma=1.0, kind=RES_IDENTIAL,
                 num_threads=0):
        super().__init__()
        check(lib().kudnn_linear_res_create(_ref(a), _ref(b), _ref(c), _ref(bias), _ref(res), _ref(linear_res), alpha,
                                            beta, gamma, kind, num_threads, ctypes.byref(self.handle)))

    def run(self, a, b, c, bias, res, linear_res, gamma=1.0, num_threads=0, stream=None):
        check(lib().kudnn_linear_res_run(self.handle, _ptr(a), _ptr(b), _ptr(c), _ptr(bias), _ptr(res),
                                         _ptr(linear_res), gamma, num_threads, _stream(stream)))


class LinearPostOps(_Plan):
    """Linear with a fused post-op chain: Y = binary(act(A x B + bias), src)."""

    _destroy = "kudnn_linear_postops_destroy"

    def __init__(self, a, b, y, bias=None, act=ACT_UNIMPLEMENTED, act_alpha=0.0, act_beta=0.0, binary=BIN_NONE,
                 src=None, gamma=1.0, num_threads=0):
        super().__init__()
        check(lib().kudnn_linear_postops_create(_ref(a), _ref(b), _ref(y), _ref(bias), act, act_alpha, act_beta,
                                                binary, _ref(src), gamma, num_threads, ctypes.byref(self.handle)))

    def run(self, a, b, y, bias=None, src=None, gamma=1.0, stream=None):
        check(lib().kudnn_linear_postops_run(self.handle, _ptr(a), _ptr(b), _ptr(y), _ptr(bias), _ptr(src), gamma,
                                             _stream(stream)))


def synchronize(stream=None) -> None:
    check(lib().kudnn_stream_synchronize(_stream(stream)))
