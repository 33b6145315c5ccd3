"""Committed golden fixtures (tests/golden/, written by make_golden.py from the
float64 per-token recurrence): the CPU oracle and the GPU kernels must both
reproduce them."""

import os

import numpy as np
import pytest
import torch

from oracle.decode_ref import ref_decode
from oracle.prefill_ref import ref_prefill

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bf16(a):
    return torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)


def _load(name):
    z = np.load(os.path.join(HERE, name))  # allow_pickle defaults to False
    return {k: z[k] for k in z.files}


def _decode_inputs():
    z = _load("decode_cfg1.npz")
    d = dict(q=_bf16(z["q"]), k=_bf16(z["k"]), v=_bf16(z["v"]), a=_bf16(z["a"]), b=_bf16(z["b"]),
             A_log=torch.from_numpy(z["A_log"]), dt_bias=torch.from_numpy(z["dt_bias"]),
             S=torch.from_numpy(z["S_in"]))
    return d, float(z["scale"]), torch.from_numpy(z["o"]), torch.from_numpy(z["S_out"])


def _prefill_inputs():
    z = _load("prefill_T130_H2_V32.npz")
    d = dict(q=_bf16(z["q"]), k=_bf16(z["k"]), v=_bf16(z["v"]), a=_bf16(z["a"]), b_logits=_bf16(z["b_logits"]),
             A_log=torch.from_numpy(z["A_log"]), state_in=torch.from_numpy(z["state_in"]))
    return d, torch.from_numpy(z["o"]), torch.from_numpy(z["S_out"])


def test_oracle_reproduces_decode_fixture():
    d, scale, o_exp, S_exp = _decode_inputs()
    B, H, K = d["q"].shape
    o, S = ref_decode(d["q"].reshape(B, 1, H, K), d["k"].reshape(B, 1, H, K), d["v"].reshape(B, 1, H, -1), d["S"],
                      d["A_log"], d["a"].reshape(B, 1, H), d["dt_bias"], d["b"].reshape(B, 1, H), scale)
    torch.testing.assert_close(o, o_exp, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(S, S_exp, rtol=1e-4, atol=1e-6)


def test_oracle_reproduces_prefill_fixture():
    d, o_exp, S_exp = _prefill_inputs()
    o, S = ref_prefill(d["q"], d["k"], d["v"], d["A_log"], d["a"], torch.tensor(0.0), d["b_logits"],
                       torch.ones(1, d["q"].shape[2]), state_in=d["state_in"], chunk_size=64)
    torch.testing.assert_close(o, o_exp, rtol=1e-4, atol=2e-6)
    torch.testing.assert_close(S, S_exp, rtol=1e-4, atol=2e-6)


@pytest.mark.gpu
def test_kernel_reproduces_decode_fixture(exts, dev):
    d, scale, o_exp, S_exp = _decode_inputs()
    g = {k: v.to(dev) for k, v in d.items()}
    o = torch.empty(o_exp.shape, device=dev)
    S = torch.empty_like(g["S"])
    exts["decode"].forward(g["q"], g["k"], g["v"], g["a"], g["b"], g["A_log"], g["dt_bias"], g["S"], scale, o, S)
    torch.cuda.synchronize()
    torch.testing.assert_close(o.cpu(), o_exp, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(S.cpu(), S_exp, rtol=1e-4, atol=1e-6)


@pytest.mark.gpu
def test_kernel_reproduces_prefill_fixture(exts, dev):
    from tests.helpers import assert_out_close, assert_state_close
    d, o_exp, S_exp = _prefill_inputs()
    g = {k: v.to(dev) for k, v in d.items()}
    mask = torch.ones(1, d["q"].shape[2], device=dev)
    out, S = exts["prefill"].prefill(g["q"], g["k"], g["v"], g["A_log"], g["a"], 0.0, g["b_logits"], mask,
                                     g["state_in"], 0.0)
    torch.cuda.synchronize()
    assert_out_close(out.cpu(), o_exp)
    assert_state_close(S.cpu(), S_exp)
