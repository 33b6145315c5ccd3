"""CPU pins for the decode oracle (oracle/decode_ref.py <- reference/decode_ref.py:10-61).

Each check is independent of the oracle's own formula: a float64 per-token
brute force, the brief's closed form S <- g S (I - beta k k^T) + beta v k^T on
the transposed state, and invariants whose answers the mathematics fixes.
The mutation tests show that plausible mistakes fail these checks.
"""

import math

import numpy as np
import torch

from gdn_18646_amd import synth
from oracle import recurrence_f64 as rf
from oracle.decode_ref import ref_decode


def _call(d, scale):
    B, H, K = d["q"].shape
    return ref_decode(d["q"].reshape(B, 1, H, K), d["k"].reshape(B, 1, H, K), d["v"].reshape(B, 1, H, -1), d["S"],
                      d["A_log"], d["a"].reshape(B, 1, H), d["dt_bias"], d["b"].reshape(B, 1, H), scale)


def _f64(d, scale):
    B, H, K = d["q"].shape
    g, beta = rf.gates_f64(d["A_log"].numpy(), d["a"].float().numpy()[..., None], d["dt_bias"].numpy(),
                           d["b"].float().numpy()[..., None])
    o, S = rf.recurrence(d["q"].float().numpy()[:, :, None], d["k"].float().numpy()[:, :, None],
                         d["v"].float().numpy()[:, :, None], g, beta, np.ones((B, 1)), d["S"].numpy(), scale)
    return o[:, :, 0], S, g[..., 0], beta[..., 0]


def test_matches_float64_recurrence():
    d = synth.decode_inputs(3, 4, 128, 96, seed=0)
    o, S = _call(d, 0.125)
    o64, S64, _, _ = _f64(d, 0.125)
    np.testing.assert_allclose(o.numpy(), o64, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(S.numpy(), S64, rtol=1e-4, atol=1e-6)


def test_matches_brief_closed_form():
    """S_T <- g S_T (I - beta k k^T) + beta v k^T with S_T = S^T (the brief's convention)."""
    d = synth.decode_inputs(2, 3, 128, 128, seed=4)
    scale = 128 ** -0.5
    o, S = _call(d, scale)
    _, _, g, beta = _f64(d, scale)
    o_cf, S_cf = rf.decode_closed_form(d["q"].float().numpy(), d["k"].float().numpy(), d["v"].float().numpy(),
                                       d["S"].numpy(), g, beta, scale)
    np.testing.assert_allclose(o.numpy(), o_cf, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(S.numpy(), S_cf, rtol=1e-4, atol=1e-6)


def test_no_write_no_decay_leaves_state():
    """beta -> 0 (b = -60) and g -> 1 (A_log = -60): S unchanged, o = scale q^T S."""
    d = synth.decode_inputs(2, 2, 128, 64, seed=1)
    d["b"] = torch.full_like(d["b"], -60.0)
    d["A_log"] = torch.full_like(d["A_log"], -60.0)
    o, S = _call(d, 0.5)
    torch.testing.assert_close(S, d["S"], rtol=0, atol=1e-7)
    o_exp = 0.5 * torch.einsum("bhk,bhkv->bhv", d["q"].float(), d["S"])
    torch.testing.assert_close(o, o_exp, rtol=1e-5, atol=1e-7)


def test_delta_rule_retrieval():
    """g = 1, beta = 1, |k| = 1: after the write, k^T S = v exactly (delta rule)."""
    d = synth.decode_inputs(2, 3, 128, 32, seed=2)
    d["b"] = torch.full_like(d["b"], 60.0)
    d["A_log"] = torch.full_like(d["A_log"], -60.0)
    k = d["k"].double()
    k = (k / k.norm(dim=-1, keepdim=True))
    d["k"] = k.float().bfloat16()  # the oracle upcasts bf16 k to fp32
    kf = d["k"].double()
    kf_norm2 = (kf * kf).sum(-1, keepdim=True)
    _, S = _call(d, 1.0)
    retrieved = torch.einsum("bhk,bhkv->bhv", kf, S.double())
    # exact for |k| = 1; bf16 rounding of k leaves |k|^2 = 1 + O(2^-8), which enters linearly
    expected = d["v"].double() * kf_norm2 + (1 - kf_norm2) * torch.einsum("bhk,bhkv->bhv", kf, d["S"].double())
    torch.testing.assert_close(retrieved, expected, rtol=1e-5, atol=1e-5)


def test_zero_state_write():
    """S = 0: S'' = beta k v^T and o = scale beta (q.k) v."""
    d = synth.decode_inputs(2, 2, 128, 64, seed=3, state=False)
    o, S = _call(d, 0.3)
    beta = torch.sigmoid(d["b"].float())
    S_exp = beta[..., None, None] * d["k"].float()[..., :, None] * d["v"].float()[..., None, :]
    o_exp = 0.3 * beta[..., None] * (d["q"].float() * d["k"].float()).sum(-1, keepdim=True) * d["v"].float()
    torch.testing.assert_close(S, S_exp, rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(o, o_exp, rtol=1e-5, atol=1e-7)


def test_scale_none_is_rsqrt_k():
    d = synth.decode_inputs(1, 2, 128, 32, seed=5)
    o1, _ = _call(d, None)
    o2, _ = _call(d, 1 / math.sqrt(128))
    torch.testing.assert_close(o1, o2)


def _mutant_decode_no_decay_before_read(d, scale):
    """A plausible mistake: read r from the undecayed state."""
    B, H, K = d["q"].shape
    x = d["a"].float() + d["dt_bias"].float()
    g = torch.exp(-torch.exp(d["A_log"].float()) * torch.nn.functional.softplus(x))
    beta = torch.sigmoid(d["b"].float())
    S = d["S"].clone()
    r = torch.einsum("bhk,bhkv->bhv", d["k"].float(), S)  # bug: should use g * S
    S = g[..., None, None] * S + d["k"].float()[..., :, None] * (beta[..., None] * (d["v"].float() - r))[..., None, :]
    return scale * torch.einsum("bhk,bhkv->bhv", d["q"].float(), S), S


def test_checks_catch_a_planted_mistake():
    """The float64 brute force distinguishes a mutant oracle (so the pin has teeth)."""
    d = synth.decode_inputs(2, 2, 128, 32, seed=6)
    o_m, S_m = _mutant_decode_no_decay_before_read(d, 0.2)
    o64, S64, _, _ = _f64(d, 0.2)
    assert not np.allclose(S_m.numpy(), S64, rtol=1e-3, atol=1e-5)
