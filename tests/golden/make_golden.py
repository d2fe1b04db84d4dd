"""Writes the golden fixtures of the Linear/GEMM path: linear_cases.json (manifest) + linear_cases.npz (buffers).

Run from the repository root:  python tests/golden/make_golden.py

Two kinds of case:
  * "oracle" cases: small versions of the five benchmark configurations (and the LinearResFWD kinds) with inputs
    from the oracle's SplitMix64 generator (seed and distribution in the manifest) and outputs from the CPU
    restatement. They freeze the restatement's bits, so a later change to it shows up as a fixture mismatch,
    and they give the GPU tests committed expected outputs.
  * "exact" cases: integer-valued inputs (numpy PCG64, fixed seed) whose products and partial sums are exact in
    f32 whatever the summation order; the expected outputs are computed here with int64 arithmetic, independently
    of the oracle, and the oracle must reproduce them bit for bit.

The reference's own tests hold no golden vectors (they draw inputs from time(NULL)); these fixtures are this
build's. Buffers are stored raw: float32 for F32 tensors, uint16 bit patterns for BF16 / F16.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle as O  # noqa: E402

LAYOUT_STRIDES = {  # logical-dim strides of the dense layouts used here (kudnn_tensor_info.cpp:141-325)
    "AB": lambda d: (d[1], 1),
    "BA": lambda d: (1, d[0]),
    "ABC": lambda d: (d[1] * d[2], d[2], 1),
}


def strides(dims, layout):
    """Dense strides of the layout; a dimension of size 1 has stride 0, as TensorInfo computes them."""
    return tuple(0 if d == 1 else s for d, s in zip(dims, LAYOUT_STRIDES[layout](dims)))


def tensor(spec):
    dims = tuple(spec["dims"])
    st = strides(dims, spec["layout"])
    if spec.get("zero"):
        return O.empty(dims, st, spec["dtype"])
    if "ints" in spec:
        lo, hi = spec["ints"]
        rng = np.random.default_rng(spec["seed"])
        vals = rng.integers(lo, hi + 1, size=O.extent(dims, st)).astype(np.float32)
        return O.Tensor(dims, st, spec["dtype"], O.from_f32_rne(vals, spec["dtype"]))
    return O.fill(dims, st, spec["dtype"], spec["seed"], spec.get("dist", "uniform"), spec.get("lo", -1.0),
                  spec.get("hi", 1.0))


def T(dims, dtype, layout, **kw):
    return dict(dims=list(dims), dtype=dtype, layout=layout, **kw)


def cases():
    bf, f32 = O.BF16, O.F32
    return {
        # C1: fp32 Linear + ReLU(alpha 0), nn.Linear weight (BA)
        "c1_f32_relu": dict(op="linear_act", act=O.ACT_RELU, act_alpha=0.0, tensors=dict(
            a=T([8, 32], f32, "AB", seed=100), b=T([32, 16], f32, "BA", seed=101),
            bias=T([1, 16], f32, "AB", seed=102, lo=-0.1, hi=0.1), c=T([8, 16], f32, "AB", zero=True)), out=["c"]),
        # C2: fp32 Linear + SWISH(alpha 1)
        "c2_f32_swish": dict(op="linear_act", act=O.ACT_SWISH, act_alpha=1.0, tensors=dict(
            a=T([16, 64], f32, "AB", seed=110, dist="normal", lo=0.0, hi=1.0),
            b=T([64, 24], f32, "BA", seed=111, dist="normal", lo=0.0, hi=0.125),
            bias=T([1, 24], f32, "AB", seed=112, dist="normal", lo=0.0, hi=0.02), c=T([16, 24], f32, "AB", zero=True)),
            out=["c"]),
        # C3: bf16 Linear + GELU_tanh + residual add, zero bias
        "c3_bf16_gelu_tanh_add": dict(op="linear_postops", act=O.ACT_GELU_TANH, act_alpha=0.0, binary=O.BIN_ADD,
                                      gamma=1.0, tensors=dict(
            a=T([16, 64], bf, "AB", seed=120, dist="normal", lo=0.0, hi=1.0),
            b=T([64, 40], bf, "BA", seed=121, dist="normal", lo=0.0, hi=0.02),
            bias=T([1, 40], bf, "AB", zero=True), src=T([16, 40], bf, "AB", seed=123, dist="normal", lo=0.0, hi=1.0),
            y=T([16, 40], bf, "AB", zero=True)), out=["y"]),
        # C4: bf16 decode row, Linear then element-wise multiply by M2
        "c4_bf16_mul_m1": dict(op="linear_postops", act=O.ACT_NONE, act_alpha=0.0, binary=O.BIN_MUL, gamma=1.0,
                               tensors=dict(
            a=T([1, 64], bf, "AB", seed=130, dist="normal", lo=0.0, hi=1.0),
            b=T([64, 48], bf, "BA", seed=131, dist="normal", lo=0.0, hi=0.125),
            src=T([1, 48], bf, "AB", seed=133, lo=0.5, hi=1.5), y=T([1, 48], bf, "AB", zero=True)), out=["y"]),
        # C5: bf16 3-D Linear + SWISH, K-major weight broadcast over the batch
        "c5_bf16_3d_swish_kmajor": dict(op="linear_act", act=O.ACT_SWISH, act_alpha=1.0, tensors=dict(
            a=T([2, 8, 64], bf, "ABC", seed=140, dist="normal", lo=0.0, hi=1.0),
            b=T([1, 64, 40], bf, "ABC", seed=141, dist="normal", lo=0.0, hi=0.125),
            bias=T([1, 1, 40], bf, "ABC", seed=142, dist="normal", lo=0.0, hi=0.02),
            c=T([2, 8, 40], bf, "ABC", zero=True)), out=["c"]),
        "gelu_erf_f32": dict(op="linear_act", act=O.ACT_GELU_ERF, act_alpha=0.0, tensors=dict(
            a=T([8, 48], f32, "AB", seed=150), b=T([48, 20], f32, "BA", seed=151),
            bias=T([8, 20], f32, "AB", seed=152, lo=-0.5, hi=0.5), c=T([8, 20], f32, "AB", zero=True)), out=["c"]),
        "res_ext_bf16": dict(op="linear_res", kind=O.RES_EXT, gamma=0.625, tensors=dict(
            a=T([8, 32], bf, "AB", seed=160), b=T([32, 24], bf, "BA", seed=161),
            bias=T([1, 24], bf, "AB", seed=162, lo=-0.1, hi=0.1), res=T([8, 24], bf, "AB", seed=163),
            c=T([8, 24], bf, "AB", zero=True), lr=T([8, 24], bf, "AB", zero=True)), out=["c", "lr"]),
        "res_mul_f32": dict(op="linear_res", kind=O.RES_MUL, gamma=1.0, tensors=dict(
            a=T([8, 32], f32, "AB", seed=170), b=T([32, 24], f32, "BA", seed=171),
            bias=T([1, 24], f32, "AB", seed=172, lo=-0.1, hi=0.1), res=T([24, 12], f32, "AB", seed=173),
            c=T([8, 24], f32, "AB", zero=True), lr=T([8, 12], f32, "AB", zero=True)), out=["c", "lr"]),
        # exact: integer-valued bf16 GEMM + integer bias + ReLU, K = 256 (|sums| <= 256 * 64 + 8 < 2^24)
        "exact_bf16_relu": dict(op="linear_act", act=O.ACT_RELU, act_alpha=0.0, exact=True, tensors=dict(
            a=T([24, 256], bf, "AB", seed=180, ints=[-8, 8]), b=T([256, 40], bf, "BA", seed=181, ints=[-8, 8]),
            bias=T([1, 40], bf, "AB", seed=182, ints=[-8, 8]), c=T([24, 40], bf, "AB", zero=True)), out=["c"]),
        # exact: integer-valued fp32 3-D GEMM with a K-major broadcast weight and a per-row bias
        "exact_f32_3d": dict(op="gemm", exact=True, tensors=dict(
            a=T([2, 12, 128], f32, "ABC", seed=190, ints=[-8, 8]), b=T([1, 128, 20], f32, "ABC", seed=191, ints=[-8, 8]),
            bias=T([1, 12, 1], f32, "ABC", seed=192, ints=[-100, 100]), c=T([2, 12, 20], f32, "ABC", zero=True)),
            out=["c"]),
    }


def run_oracle(case, ts):
    op = case["op"]
    if op == "gemm":
        O.gemm(ts["a"], ts["b"], ts["c"], ts.get("bias"))
    elif op == "linear_act":
        O.linear_act(ts["a"], ts["b"], ts["c"], ts.get("bias"), case["act"], case["act_alpha"])
    elif op == "linear_res":
        O.linear_res(ts["a"], ts["b"], ts["c"], ts["bias"], ts["res"], ts["lr"], case["kind"], case["gamma"])
    elif op == "linear_postops":
        O.linear_postops(ts["a"], ts["b"], ts["y"], ts.get("bias"), case["act"], case["act_alpha"], case["binary"],
                         ts.get("src"), case["gamma"])
    else:
        raise ValueError(op)


def exact_expected(case, ts):
    """int64 restatement of the exact cases (GEMM + bias, then ReLU when asked), independent of the oracle."""
    a = ts["a"].logical().astype(np.int64)
    b = ts["b"].logical().astype(np.int64)
    acc = np.matmul(a, b)  # broadcasts the batch dims
    if "bias" in ts:
        acc = acc + ts["bias"].logical().astype(np.int64)
    assert np.all(np.abs(acc) < 2 ** 24)
    dense = acc.astype(np.float32)
    if case.get("act") == O.ACT_RELU:
        # RELU with alpha 0 maps x <= 0 to x * 0: -0.0 for negative x (relu/relu.c:14-25)
        dense = np.where(acc <= 0, dense * np.float32(0.0), dense)
    out = ts["c"]
    flat = np.zeros(out.buf.size, dtype=np.float32)
    view = np.lib.stride_tricks.as_strided(flat, shape=out.dims, strides=[s * 4 for s in out.strides])
    view[...] = dense
    return O.from_f32_rne(flat, out.dtype)


def main():
    manifest, arrays = {}, {}
    for name, case in cases().items():
        ts = {k: tensor(v) for k, v in case["tensors"].items()}
        run_oracle(case, ts)
        if case.get("exact"):
            for o in case["out"]:
                want = exact_expected(case, ts)
                assert np.array_equal(ts[o].buf, want), f"{name}: oracle differs from the int64 restatement"
        for k, t in ts.items():
            arrays[f"{name}__{k}"] = t.buf
        manifest[name] = case
    (HERE / "linear_cases.json").write_text(json.dumps(manifest, indent=1) + "\n")
    np.savez_compressed(HERE / "linear_cases.npz", **arrays)
    print(f"wrote {len(manifest)} cases, {sum(a.nbytes for a in arrays.values())} bytes of buffers")


if __name__ == "__main__":
    main()
