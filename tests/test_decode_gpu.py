"""GPU parity of the decode kernel against the CPU oracle (reference/decode_ref.py).

Calls go through the torch binding (the reference's ``decode.forward`` API) and,
in one test, straight through the C ABI with ctypes.
"""

import math

import pytest
import torch

from gdn_18646_amd import synth
from oracle.decode_ref import ref_decode
from tests.helpers import assert_out_close, assert_state_close

pytestmark = pytest.mark.gpu


def _run_kernel(exts, d, dev, scale, inplace=False):
    B, H, K = d["q"].shape
    V = d["v"].shape[-1]
    g = {k: v.to(dev) for k, v in d.items()}
    o = torch.empty(B, H, V, device=dev, dtype=torch.float32)
    S_out = g["S"] if inplace else torch.empty_like(g["S"])
    exts["decode"].forward(g["q"], g["k"], g["v"], g["a"], g["b"], g["A_log"], g["dt_bias"], g["S"], scale, o, S_out)
    torch.cuda.synchronize()
    return o.cpu(), S_out.cpu()


def _oracle(d, scale):
    B, H, K = d["q"].shape
    return ref_decode(d["q"].reshape(B, 1, H, K), d["k"].reshape(B, 1, H, K), d["v"].reshape(B, 1, H, -1),
                      d["S"], d["A_log"], d["a"].reshape(B, 1, H), d["dt_bias"], d["b"].reshape(B, 1, H), scale)


def test_decode_config1(exts, dev):
    """Brief config 1: B=1, H=4, K=V=128, seed 0."""
    d = synth.decode_inputs(1, 4, 128, 128, seed=0)
    scale = 128 ** -0.5
    o, S = _run_kernel(exts, d, dev, scale)
    o_ref, S_ref = _oracle(d, scale)
    assert_out_close(o, o_ref)
    assert_state_close(S, S_ref)
    # The kernel is fp32 end to end: hold it to fp32 rounding as well.
    assert torch.allclose(o, o_ref, atol=1e-5, rtol=1e-4)
    assert torch.allclose(S, S_ref, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("B", [1, 8, 32, 64])
def test_decode_reference_shapes(exts, dev, B):
    """The reference test's shapes and input scales (tests/test_decode.py:25-46): H=16, dv=256."""
    H, dk, dv = 16, 128, 256
    g = torch.Generator().manual_seed(100 + B)
    d = dict(q=(torch.randn(B, H, dk, generator=g) * 0.02).bfloat16(),
             k=(torch.randn(B, H, dk, generator=g) * 0.02).bfloat16(),
             v=(torch.randn(B, H, dv, generator=g) * 0.02).bfloat16(),
             a=(torch.randn(B, H, generator=g) * 0.1).bfloat16(),
             b=(torch.randn(B, H, generator=g) * 0.1).bfloat16(),
             A_log=torch.zeros(H), dt_bias=torch.zeros(H),
             S=torch.randn(B, H, dk, dv, generator=g) * 0.01)
    scale = 1.0 / math.sqrt(dk)
    o, S = _run_kernel(exts, d, dev, scale)
    o_ref, S_ref = _oracle(d, scale)
    assert torch.allclose(o, o_ref, atol=1e-6, rtol=1e-4)
    assert torch.allclose(S, S_ref, atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("dv", [32, 64, 96, 160, 384])
def test_decode_dv_shapes(exts, dev, dv):
    d = synth.decode_inputs(3, 5, 128, dv, seed=7)
    o, S = _run_kernel(exts, d, dev, 0.125)
    o_ref, S_ref = _oracle(d, 0.125)
    assert torch.allclose(o, o_ref, atol=1e-5, rtol=1e-4)
    assert torch.allclose(S, S_ref, atol=1e-6, rtol=1e-5)


def test_decode_inplace_matches_out_of_place(exts, dev):
    d = synth.decode_inputs(16, 8, 128, 128, seed=11)
    o1, S1 = _run_kernel(exts, d, dev, 0.1)
    o2, S2 = _run_kernel(exts, d, dev, 0.1, inplace=True)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)


def test_decode_config3_steps(exts, dev):
    """Brief config 3 shape (B=256, H=32, 512 MiB state in place): 3 consecutive steps vs the oracle."""
    B, H = 256, 32
    d = synth.decode_inputs(B, H, 128, 128, seed=2)
    steps = synth.decode_step_stream(3, B, H, seed=2)
    scale = 128 ** -0.5
    S_dev = d["S"].to(dev)
    A_log, dtb = d["A_log"].to(dev), d["dt_bias"].to(dev)
    o = torch.empty(B, H, 128, device=dev)
    S_ref = d["S"]
    for st in steps:
        g = {k: v.to(dev) for k, v in st.items()}
        exts["decode"].forward(g["q"], g["k"], g["v"], g["a"], g["b"], A_log, dtb, S_dev, scale, o, S_dev)
        o_ref, S_ref = ref_decode(st["q"].reshape(B, 1, H, 128), st["k"].reshape(B, 1, H, 128),
                                  st["v"].reshape(B, 1, H, 128), S_ref, d["A_log"], st["a"].reshape(B, 1, H),
                                  d["dt_bias"], st["b"].reshape(B, 1, H), scale)
        torch.cuda.synchronize()
        assert_out_close(o.cpu(), o_ref)
    assert_state_close(S_dev.cpu(), S_ref, tol=1e-5)


def test_decode_through_c_abi(dev):
    """Same call through ctypes on the C ABI (the boundary a non-torch host binds)."""
    from gdn_18646_amd import abi
    d = synth.decode_inputs(4, 6, 128, 128, seed=5)
    g = {k: v.to(dev) for k, v in d.items()}
    B, H = 4, 6
    o = torch.empty(B, H, 128, device=dev)
    S_out = torch.empty_like(g["S"])
    stream = torch.cuda.current_stream().cuda_stream
    abi.call("gdn_decode_hip", g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(), g["a"].data_ptr(),
             g["b"].data_ptr(), g["A_log"].data_ptr(), g["dt_bias"].data_ptr(), g["S"].data_ptr(), 0.125,
             o.data_ptr(), S_out.data_ptr(), B, H, 128, 128, stream)
    torch.cuda.synchronize()
    o_ref, S_ref = _oracle(d, 0.125)
    assert torch.allclose(o.cpu(), o_ref, atol=1e-5, rtol=1e-4)
    assert torch.allclose(S_out.cpu(), S_ref, atol=1e-6, rtol=1e-5)


def test_decode_rejects_bad_shapes(exts, dev):
    d = synth.decode_inputs(2, 2, 128, 128, seed=1)
    g = {k: v.to(dev) for k, v in d.items()}
    o = torch.empty(2, 2, 48, device=dev)
    v48 = torch.zeros(2, 2, 48, device=dev, dtype=torch.bfloat16)
    S48 = torch.zeros(2, 2, 128, 48, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        exts["decode"].forward(g["q"], g["k"], v48, g["a"], g["b"], g["A_log"], g["dt_bias"], S48, 0.1, o, S48)
