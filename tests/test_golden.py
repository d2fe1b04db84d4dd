"""Golden fixtures of the Linear/GEMM path (tests/golden/linear_cases.{json,npz}, written by make_golden.py).

CPU: the oracle reproduces every fixture bit for bit from the stored inputs, and the integer-valued ("exact") cases
equal an int64 restatement computed here, independently of the oracle.
GPU: the HIP path, called through the C ABI, matches every fixture (exact cases bit for bit, the others to the
north-star tolerance).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import kudnn_amd as K
import oracle as O
from support import compare, from_device

GOLDEN = Path(__file__).resolve().parent / "golden"
MANIFEST = json.loads((GOLDEN / "linear_cases.json").read_text())
ARRAYS = np.load(GOLDEN / "linear_cases.npz")
LAYOUT_STRIDES = {"AB": lambda d: (d[1], 1), "BA": lambda d: (1, d[0]), "ABC": lambda d: (d[1] * d[2], d[2], 1)}


def strides(dims, layout):
    return tuple(0 if d == 1 else s for d, s in zip(dims, LAYOUT_STRIDES[layout](dims)))


def load(name, outputs_zero=True):
    """Oracle tensors of a case from the stored buffers (outputs zeroed unless asked otherwise)."""
    case = MANIFEST[name]
    ts = {}
    for k, spec in case["tensors"].items():
        dims = tuple(spec["dims"])
        buf = ARRAYS[f"{name}__{k}"].copy()
        if outputs_zero and k in case["out"]:
            buf[...] = 0
        ts[k] = O.Tensor(dims, strides(dims, spec["layout"]), spec["dtype"], buf)
    return case, ts


def run_oracle(case, ts):
    op = case["op"]
    if op == "gemm":
        O.gemm(ts["a"], ts["b"], ts["c"], ts.get("bias"))
    elif op == "linear_act":
        O.linear_act(ts["a"], ts["b"], ts["c"], ts.get("bias"), case["act"], case["act_alpha"])
    elif op == "linear_res":
        O.linear_res(ts["a"], ts["b"], ts["c"], ts["bias"], ts["res"], ts["lr"], case["kind"], case["gamma"])
    else:
        O.linear_postops(ts["a"], ts["b"], ts["y"], ts.get("bias"), case["act"], case["act_alpha"], case["binary"],
                         ts.get("src"), case["gamma"])


def test_manifest_covers_the_configs():
    ops = {c["op"] for c in MANIFEST.values()}
    assert ops == {"gemm", "linear_act", "linear_res", "linear_postops"}
    assert {n.split("_")[0] for n in MANIFEST} >= {"c1", "c2", "c3", "c4", "c5", "exact"}
    assert sum(1 for c in MANIFEST.values() if c.get("exact")) >= 2


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_oracle_reproduces_fixture(name):
    case, ts = load(name)
    run_oracle(case, ts)
    for o in case["out"]:
        assert np.array_equal(ts[o].buf, ARRAYS[f"{name}__{o}"]), f"{name}.{o}: oracle no longer matches the fixture"


@pytest.mark.parametrize("name", sorted(n for n, c in MANIFEST.items() if c.get("exact")))
def test_exact_fixture_matches_int64(name):
    case, ts = load(name, outputs_zero=False)
    a = ts["a"].logical().astype(np.int64)
    b = ts["b"].logical().astype(np.int64)
    acc = np.matmul(a, b) + ts["bias"].logical().astype(np.int64)
    assert np.all(np.abs(acc) < 2 ** 24)
    want = acc.astype(np.float32)
    if case.get("act") == O.ACT_RELU:
        want = np.where(acc <= 0, want * np.float32(0.0), want)  # x <= 0 -> x * 0 keeps the sign
    got = ts["c"].logical()
    want = O.to_f32(O.from_f32_rne(want, ts["c"].dtype), ts["c"].dtype).reshape(want.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _device(t: O.Tensor):
    import torch

    if t.buf.dtype == np.uint16:
        return torch.from_numpy(t.buf.view(np.int16).copy()).to("cuda")
    return torch.from_numpy(t.buf.copy()).to("cuda")


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_hip_matches_fixture(name):
    import torch

    case, ts = load(name)
    specs = case["tensors"]
    d = {k: K.desc(s["dims"], s["dtype"], s["layout"]) for k, s in specs.items()}
    dev = {k: _device(t) for k, t in ts.items()}
    op = case["op"]
    if op == "gemm":
        plan = K.Gemm(d["a"], d["b"], d["c"], d.get("bias"))
        plan.run(dev["a"], dev["b"], dev["c"], dev.get("bias"))
    elif op == "linear_act":
        plan = K.LinearActivation(d["a"], d["b"], d["c"], d.get("bias"), case["act_alpha"], 0.0, case["act"])
        plan.run(dev["a"], dev["b"], dev["c"], dev.get("bias"))
    elif op == "linear_res":
        plan = K.LinearRes(d["a"], d["b"], d["c"], d["bias"], d["res"], d["lr"], 1.0, 0.0, case["gamma"], case["kind"])
        plan.run(dev["a"], dev["b"], dev["c"], dev["bias"], dev["res"], dev["lr"], case["gamma"])
    else:
        plan = K.LinearPostOps(d["a"], d["b"], d["y"], d.get("bias"), act=case["act"], act_alpha=case["act_alpha"],
                               binary=case["binary"], src=d.get("src"))
        plan.run(dev["a"], dev["b"], dev["y"], dev.get("bias"), dev.get("src"), gamma=case["gamma"])
    torch.cuda.synchronize()
    for o in case["out"]:
        dt = specs[o]["dtype"]
        got = from_device(dev[o], dt)
        ref = ARRAYS[f"{name}__{o}"]
        if case.get("exact"):
            assert np.array_equal(got, ref), f"{name}.{o} ({plan.describe()}): exact case differs"
        else:
            compare(got, ref, dt, f"{name}.{o} {plan.describe()}")
