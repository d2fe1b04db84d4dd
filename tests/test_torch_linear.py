"""kudnn_amd.torch_linear: the PyTorch module / functional form and the nn.functional.linear switch.

CPU tests cover the routing predicate and argument checks; GPU tests compare against the CPU oracle on the same
inputs (the oracle's rounding points are the reference's; torch's own bf16 linear rounds differently).
"""
import numpy as np
import pytest

import oracle as O
from support import compare, explainer

torch = pytest.importorskip("torch")
import kudnn_amd.torch_linear as T  # noqa: E402


def _oracle_tensor(t, dt):
    a = t.detach().cpu().contiguous()
    buf = a.view(torch.int16).numpy().view(np.uint16).reshape(-1) if dt != O.F32 else a.numpy().reshape(-1).copy()
    dims = tuple(a.shape)
    strides = tuple(0 if d == 1 else s for d, s in zip(dims, a.stride()))
    return O.Tensor(dims, strides, dt, buf.copy())


def test_switch_restores_torch_linear():
    orig = torch.nn.functional.linear
    T.set_enabled(True)
    try:
        assert T.is_enabled() and torch.nn.functional.linear is not orig
    finally:
        T.set_enabled(False)
    assert torch.nn.functional.linear is orig and not T.is_enabled()


def test_cpu_and_autograd_calls_stay_with_torch():
    x = torch.randn(3, 8)
    w = torch.randn(5, 8)
    assert not T._eligible(x, w, None)  # CPU tensors
    T.set_enabled(True)
    try:
        y = torch.nn.functional.linear(x, w)  # routed back to torch's implementation
        assert torch.allclose(y, x @ w.T)
    finally:
        T.set_enabled(False)


def test_argument_checks():
    with pytest.raises(ValueError):
        T.KudnnLinear(8, 4, act="exp_dst")  # backward-only kind
    with pytest.raises(ValueError):
        T.linear(torch.randn(2, 8), torch.randn(4, 8))  # CPU tensors


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("post", [(None, None), ("relu", None), ("silu", "mul"), ("gelu_tanh", "add"), ("gelu", "ext")])
def test_linear_matches_oracle(dtype, post):
    act, binary = post
    dt = O.BF16 if dtype == torch.bfloat16 else O.F32
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 37, 96, generator=g).to(dtype).cuda()
    w = (torch.randn(80, 96, generator=g) * 0.1).to(dtype).cuda()
    b = (torch.randn(80, generator=g) * 0.1).to(dtype).cuda()
    s = torch.randn(2, 37, 80, generator=g).to(dtype).cuda() if binary else None
    y = T.linear(x, w, b, act=act, binary=binary, src=s, gamma=0.5)
    torch.cuda.synchronize()
    ox = _oracle_tensor(x.reshape(74, 96), dt)
    ow = O.Tensor((96, 80), (1, 96), dt, _oracle_tensor(w, dt).buf)  # [N][K] storage = logical [K, N] in layout BA
    ob = O.Tensor((1, 80), (0, 1), dt, _oracle_tensor(b, dt).buf)
    os_ = _oracle_tensor(s.reshape(74, 80), dt) if binary else None
    ref = O.empty((74, 80), (80, 1), dt)
    acts = {None: O.ACT_NONE, "relu": O.ACT_RELU, "silu": O.ACT_SWISH, "gelu_tanh": O.ACT_GELU_TANH, "gelu": O.ACT_GELU_ERF}
    bins = {None: O.BIN_NONE, "add": O.BIN_ADD, "mul": O.BIN_MUL, "ext": O.BIN_EXT}
    alpha = 1.0 if act == "silu" else 0.0
    O.linear_postops(ox, ow, ref, ob, acts[act], alpha, bins[binary], os_, 0.5)
    got = _oracle_tensor(y.reshape(74, 80), dt).buf
    why = explainer(dt, ox, ow, ob, (74, 80), act=acts[act], act_alpha=alpha, binary=bins[binary], src=os_, gamma=0.5)
    compare(got, ref.buf, dt, f"torch_linear {dtype} {post}", explain=why)


@pytest.mark.gpu
@pytest.mark.parametrize("act,alpha,beta,okind", [("hardswish", 1.0 / 6.0, 0.5, O.ACT_HARDSWISH),
                                                   ("clip", -0.2, 0.3, O.ACT_CLIP), ("mish", 0.0, 0.0, O.ACT_MISH),
                                                   ("pow", 0.5, 3.0, O.ACT_POW)])
def test_linear_other_activation_kinds(act, alpha, beta, okind):
    # the remaining kinds of KuDNN's table, with their act_alpha / act_beta
    g = torch.Generator().manual_seed(8)
    x = torch.randn(37, 96, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(80, 96, generator=g) * 0.1).to(torch.bfloat16).cuda()
    y = T.linear(x, w, None, act=act, act_alpha=alpha, act_beta=beta)
    torch.cuda.synchronize()
    ox = _oracle_tensor(x, O.BF16)
    ow = O.Tensor((96, 80), (1, 96), O.BF16, _oracle_tensor(w, O.BF16).buf)
    ref = O.empty((37, 80), (80, 1), O.BF16)
    O.linear_postops(ox, ow, ref, None, okind, alpha, O.BIN_NONE, None, 1.0, act_beta=beta)
    why = explainer(O.BF16, ox, ow, None, (37, 80), act=okind, act_alpha=alpha, act_beta=beta)
    compare(_oracle_tensor(y, O.BF16).buf, ref.buf, O.BF16, f"torch_linear {act}", explain=why)


@pytest.mark.gpu
def test_nn_linear_routed_under_inference_mode():
    g = torch.Generator().manual_seed(9)
    lin = torch.nn.Linear(256, 192).to(torch.bfloat16).cuda()
    x = torch.randn(5, 256, generator=g).to(torch.bfloat16).cuda()
    with torch.inference_mode():
        expect = T.linear(x, lin.weight, lin.bias)
        T.set_enabled(True)
        try:
            got = lin(x)
        finally:
            T.set_enabled(False)
    torch.cuda.synchronize()
    assert torch.equal(got, expect)
    ref = (x.float() @ lin.weight.float().T + lin.bias.float())
    assert torch.allclose(got.float(), ref, rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
def test_module_from_linear_fuses_postops():
    g = torch.Generator().manual_seed(11)
    lin = torch.nn.Linear(128, 64).to(torch.bfloat16).cuda()
    m = T.KudnnLinear.from_linear(lin, act="gelu_tanh", binary="add")
    x = torch.randn(33, 128, generator=g).to(torch.bfloat16).cuda()
    r = torch.randn(33, 64, generator=g).to(torch.bfloat16).cuda()
    y = m(x, r)
    torch.cuda.synchronize()
    ref = torch.nn.functional.gelu(x.float() @ lin.weight.float().T + lin.bias.float(), approximate="tanh") + r.float()
    assert torch.allclose(y.float(), ref, rtol=3e-2, atol=3e-2)
