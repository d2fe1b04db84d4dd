"""PyTorch-ROCm integration of the KuDNN Linear primitive: a module, a functional form, and a switch that routes
``torch.nn.functional.linear`` to it.

The reference's PyTorch fork sends ``nn.Linear`` to KuDNN after ``torch._C._set_kdnn_enabled(True)``
(docs/zh/KuDNN_development_guide.md:1748-1776). Here ``set_enabled(True)`` does the same for CUDA/HIP tensors of
float32 or bfloat16 that do not require gradients: the call goes through the C ABI
(``kudnn_linear_postops_*``) on torch's current stream. The primitive is forward-only, as KuDNN's
``LinearActivationLayerFWD`` is. Any other call (CPU tensors, other dtypes, autograd) stays with torch's own
``linear``. Enabling fails loudly if the HIP library is missing; nothing falls back to a CPU path.

Plans are built once per (M, K, N, dtypes, post-ops) and cached; a plan's kernel choice, tile configuration and
workspace are fixed at construction, as the KuDNN primitive descriptor's are. The cache holds at most
``MAX_CACHED_PLANS`` plans and drops the least recently used one beyond that (prefill with many distinct sequence
lengths would otherwise keep one device workspace per length); a dropped plan is destroyed, and its workspace freed,
once no caller holds it any more.
"""
from __future__ import annotations

import threading
from collections import OrderedDict
from typing import Optional, Tuple

import torch

from . import (ACT_ABS, ACT_CLIP, ACT_CLIP_V2, ACT_ELU, ACT_ELU_DST, ACT_EXP, ACT_GELU_ERF, ACT_GELU_TANH,
               ACT_HARDSIGMOID, ACT_HARDSWISH, ACT_LINEAR, ACT_LOG, ACT_MISH, ACT_POW, ACT_RELU, ACT_ROUND, ACT_SIGMOID,
               ACT_SQRT, ACT_SQUARE, ACT_SRELU, ACT_SWISH, ACT_TANH, ACT_UNIMPLEMENTED, BF16, BIN_ADD, BIN_EXT, BIN_MUL,
               BIN_NONE, F32, LinearPostOps, desc, lib)

# every forward kind of KuDNN's activation table; act_alpha / act_beta carry its parameters as KuDNN defines them
_ACTS = {None: ACT_UNIMPLEMENTED, "relu": ACT_RELU, "silu": ACT_SWISH, "swish": ACT_SWISH, "gelu_tanh": ACT_GELU_TANH,
         "gelu": ACT_GELU_ERF, "gelu_erf": ACT_GELU_ERF, "abs": ACT_ABS, "exp": ACT_EXP, "linear": ACT_LINEAR,
         "log": ACT_LOG, "round": ACT_ROUND, "sqrt": ACT_SQRT, "square": ACT_SQUARE, "tanh": ACT_TANH,
         "sigmoid": ACT_SIGMOID, "pow": ACT_POW, "clip": ACT_CLIP, "clip_v2": ACT_CLIP_V2, "hardsigmoid": ACT_HARDSIGMOID,
         "hardswish": ACT_HARDSWISH, "elu": ACT_ELU, "elu_dst": ACT_ELU_DST, "srelu": ACT_SRELU, "mish": ACT_MISH}
_BINS = {None: BIN_NONE, "add": BIN_ADD, "ext": BIN_EXT, "mul": BIN_MUL}
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16}

MAX_CACHED_PLANS = 64
_plans: "OrderedDict[Tuple, LinearPostOps]" = OrderedDict()
_plans_lock = threading.Lock()


def _plan(m: int, k: int, n: int, xdt: int, wdt: int, ydt: int, has_bias: bool, act: int, act_alpha: float,
          act_beta: float, binary: int) -> LinearPostOps:
    key = (m, k, n, xdt, wdt, ydt, has_bias, act, act_alpha, act_beta, binary)
    with _plans_lock:
        plan = _plans.get(key)
        if plan is not None:
            _plans.move_to_end(key)
        else:
            # X{M,K} AB; W{K,N} BA (physically [N][K], nn.Linear's weight); bias{1,N}; Y and the binary operand {M,N}
            dy = desc([m, n], ydt)
            plan = LinearPostOps(desc([m, k], xdt), desc([k, n], wdt, "BA"), dy, desc([1, n], ydt) if has_bias else None,
                                 act=act, act_alpha=act_alpha, act_beta=act_beta, binary=binary,
                                 src=dy if binary != BIN_NONE else None)
            _plans[key] = plan
            while len(_plans) > MAX_CACHED_PLANS:
                # dropped, not closed: a caller on another thread may still be running it; the plan's destructor
                # frees its workspace when the last reference goes
                _plans.popitem(last=False)
        return plan


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None, act: Optional[str] = None,
           act_alpha: Optional[float] = None, binary: Optional[str] = None, src: Optional[torch.Tensor] = None,
           gamma: float = 1.0, act_beta: float = 0.0) -> torch.Tensor:
    """y = binary(act(x @ weight.T + bias), src) on the GPU through the KuDNN C ABI.

    x: [..., K] (rows are flattened to M), weight: [N, K] (nn.Linear layout), bias: [N], src: x's leading shape + [N].
    act: None, "relu", "silu" / "swish", "gelu_tanh", "gelu" / "gelu_erf", or any other forward kind of KuDNN's table
    ("abs", "exp", "linear", "log", "round", "sqrt", "square", "tanh", "sigmoid", "pow", "clip", "clip_v2",
    "hardsigmoid", "hardswish", "elu", "elu_dst", "srelu", "mish") with KuDNN's act_alpha / act_beta. act_alpha
    defaults to 0 for relu (the negative slope) and 1 for swish. binary: None, "add", "ext" (y + gamma * src), "mul".
    The output has x's dtype.
    Every rounding point is the reference's: RNE after the bias, truncating bf16 store after the activation, RNE after
    the binary op.
    """
    if act not in _ACTS or binary not in _BINS:
        raise ValueError(f"unsupported post-op act={act!r} binary={binary!r}")
    if not (x.is_cuda and weight.is_cuda):
        raise ValueError("kudnn linear takes GPU tensors")
    if x.dtype not in _DTYPES or weight.dtype != x.dtype:
        raise ValueError(f"kudnn linear supports float32 and bfloat16 operands of one dtype, got {x.dtype}/{weight.dtype}")
    if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, weight {tuple(weight.shape)}")
    n, k = weight.shape
    lead = x.shape[:-1]
    m = 1
    for d in lead:
        m *= d
    x2 = x.reshape(m, k).contiguous()
    w = weight.contiguous()
    dt = _DTYPES[x.dtype]
    b = None
    if bias is not None:
        if bias.shape != (n,) or bias.dtype != x.dtype:
            raise ValueError("bias must be [N] of x's dtype")
        b = bias.contiguous()
    s = None
    bin_kind = _BINS[binary]
    if bin_kind != BIN_NONE:
        if src is None or tuple(src.shape) != tuple(lead) + (n,) or src.dtype != x.dtype:
            raise ValueError("src must have shape x.shape[:-1] + [N] and x's dtype")
        s = src.reshape(m, n).contiguous()
    act_kind = _ACTS[act]
    alpha = act_alpha if act_alpha is not None else (1.0 if act_kind == ACT_SWISH else 0.0)
    y = torch.empty(m, n, device=x.device, dtype=x.dtype)
    if m == 0 or n == 0:
        return y.reshape(*lead, n)
    plan = _plan(m, k, n, dt, dt, dt, b is not None, act_kind, float(alpha), float(act_beta), bin_kind)
    plan.run(x2, w, y, b, s, gamma=gamma, stream=torch.cuda.current_stream())
    return y.reshape(*lead, n)


class KudnnLinear(torch.nn.Module):
    """nn.Linear whose forward runs the KuDNN Linear primitive, with an optional fused activation and binary op.

    forward(x, src=None) = binary(act(x @ weight.T + bias), src). Forward only: the parameters are registered without
    gradients.
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = True, act: Optional[str] = None,
                 act_alpha: Optional[float] = None, binary: Optional[str] = None, gamma: float = 1.0,
                 device=None, dtype=torch.bfloat16, act_beta: float = 0.0):
        super().__init__()
        if act not in _ACTS or binary not in _BINS:
            raise ValueError(f"unsupported post-op act={act!r} binary={binary!r}")
        self.in_features, self.out_features = in_features, out_features
        self.act, self.act_alpha, self.act_beta, self.binary, self.gamma = act, act_alpha, act_beta, binary, gamma
        self.weight = torch.nn.Parameter(torch.empty(out_features, in_features, device=device, dtype=dtype),
                                         requires_grad=False)
        self.bias = torch.nn.Parameter(torch.zeros(out_features, device=device, dtype=dtype),
                                       requires_grad=False) if bias else None

    @classmethod
    def from_linear(cls, lin: torch.nn.Linear, act: Optional[str] = None, act_alpha: Optional[float] = None,
                    binary: Optional[str] = None, gamma: float = 1.0, act_beta: float = 0.0) -> "KudnnLinear":
        m = cls(lin.in_features, lin.out_features, lin.bias is not None, act, act_alpha, binary, gamma,
                device=lin.weight.device, dtype=lin.weight.dtype, act_beta=act_beta)
        with torch.no_grad():
            m.weight.copy_(lin.weight)
            if lin.bias is not None:
                m.bias.copy_(lin.bias)
        return m

    def forward(self, x: torch.Tensor, src: Optional[torch.Tensor] = None) -> torch.Tensor:
        return linear(x, self.weight, self.bias, self.act, self.act_alpha, self.binary, src, self.gamma, self.act_beta)


_torch_linear = torch.nn.functional.linear
_enabled = False


def _eligible(input, weight, bias) -> bool:
    if not (input.is_cuda and weight.is_cuda and input.dtype in _DTYPES and weight.dtype == input.dtype and
            weight.dim() == 2 and input.dim() >= 1):
        return False
    if bias is not None and (not bias.is_cuda or bias.dtype != input.dtype or bias.dim() != 1):
        return False
    # forward-only primitive: calls that autograd must record stay with torch
    return not (torch.is_grad_enabled() and
                (input.requires_grad or weight.requires_grad or (bias is not None and bias.requires_grad)))


def _routed_linear(input, weight, bias=None):
    if _enabled and _eligible(input, weight, bias):
        return linear(input, weight, bias)
    return _torch_linear(input, weight, bias)


def set_enabled(on: bool) -> None:
    """Routes torch.nn.functional.linear (and so nn.Linear) to KuDNN for eligible calls, like the reference fork's
    torch._C._set_kdnn_enabled: GPU tensors of float32 or bfloat16 whose call autograd need not record (for example
    under torch.no_grad() or torch.inference_mode()). Raises if the HIP library cannot be loaded."""
    global _enabled
    if on:
        lib()  # fail loudly when the HIP library is missing
        torch.nn.functional.linear = _routed_linear
    else:
        torch.nn.functional.linear = _torch_linear
    _enabled = bool(on)


def is_enabled() -> bool:
    return _enabled
