"""CPU pins for the chunked-prefill oracle (oracle/prefill_ref.py <- reference/prefill_ref.py:11-132).

Pins: equality with the float64 per-token recurrence (shares no code with the
chunked WY/UT algebra), chunk-size invariance, state composition, the
triangular solve against torch.linalg.solve_triangular, the mask and padding
semantics, special cases with known answers, and a planted-mistake check.
"""

import numpy as np
import pytest
import torch

from gdn_18646_amd import synth
from oracle import recurrence_f64 as rf
from oracle.prefill_ref import gates, ref_prefill, ref_prefill_varlen, ut_transform


def _oracle(d, C=64, mask=None, state=None, scale=0.0):
    m = d["mask"] if mask is None else mask
    return ref_prefill(d["q"], d["k"], d["v"], d["A_log"], d["a"], torch.tensor(d["dt_bias"]), d["b_logits"], m,
                       state_in=state, scale=scale, chunk_size=C)


def _f64(d, mask=None, state=None, scale=None):
    m = d["mask"] if mask is None else mask
    g, beta = rf.gates_f64(d["A_log"].numpy(), d["a"].float().numpy(), d["dt_bias"], d["b_logits"].float().numpy())
    return rf.recurrence(d["q"].float().numpy(), d["k"].float().numpy(), d["v"].float().numpy(), g, beta,
                         m.numpy(), None if state is None else state.numpy(), scale)


@pytest.mark.parametrize("T,C", [(1, 64), (63, 64), (64, 64), (65, 64), (200, 64), (200, 16), (130, 1), (100, None)])
def test_matches_float64_recurrence(T, C):
    d = synth.prefill_inputs(2, T, 3, 128, 48, seed=T, state=True)
    o, S = _oracle(d, C=C, state=d["state_in"])
    o64, S64 = _f64(d, state=d["state_in"])
    np.testing.assert_allclose(o.numpy(), o64, rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(S.numpy(), S64, rtol=1e-4, atol=2e-6)


def test_mask_quirk_masked_tokens_decay():
    """Masked tokens: no write, zero output, but the state still decays (reference/prefill_ref.py:64,79-80,130)."""
    d = synth.prefill_inputs(2, 150, 2, 128, 32, seed=8, state=True)
    mask = (torch.rand(2, 150, generator=torch.Generator().manual_seed(1)) > 0.4).float()
    o, S = _oracle(d, mask=mask, state=d["state_in"])
    o64, S64 = _f64(d, mask=mask, state=d["state_in"])
    np.testing.assert_allclose(o.numpy(), o64, rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(S.numpy(), S64, rtol=1e-4, atol=2e-6)
    assert (o[mask[:, None, :].expand(2, 2, 150) == 0] == 0).all()
    # all-masked sequence: the state is only decayed
    full = torch.zeros(2, 150)
    _, S0 = _oracle(d, mask=full, state=d["state_in"])
    g, _ = gates(d["A_log"], d["a"], d["dt_bias"], d["b_logits"])
    decay = g.double().prod(-1)
    torch.testing.assert_close(S0.double(), d["state_in"].double() * decay[..., None, None], rtol=1e-4, atol=1e-9)


def test_chunk_size_invariance():
    d = synth.prefill_inputs(1, 256, 2, 128, 32, seed=3, state=True)
    ref = _oracle(d, C=None, state=d["state_in"])
    for C in (1, 16, 64, 128):
        o, S = _oracle(d, C=C, state=d["state_in"])
        torch.testing.assert_close(o, ref[0], rtol=1e-4, atol=1e-6)
        torch.testing.assert_close(S, ref[1], rtol=1e-4, atol=1e-6)


def test_state_composition():
    d = synth.prefill_inputs(1, 300, 2, 128, 32, seed=4, state=True)
    o, S = _oracle(d, state=d["state_in"])
    t1 = 137

    def part(sl):
        return {k: (v[:, :, sl] if torch.is_tensor(v) and v.dim() >= 3 and k != "state_in" else v) for k, v in d.items()}

    d1, d2 = part(slice(0, t1)), part(slice(t1, None))
    o1, S1 = _oracle(d1, mask=torch.ones(1, t1), state=d["state_in"])
    o2, S2 = _oracle(d2, mask=torch.ones(1, 300 - t1), state=S1)
    torch.testing.assert_close(torch.cat([o1, o2], 2), o, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(S2, S, rtol=1e-4, atol=1e-6)


def test_ut_transform_is_the_inverse():
    """(I + A) T = I, and T equals a library triangular solve."""
    g = torch.Generator().manual_seed(0)
    C = 64
    k = torch.nn.functional.normalize(torch.randn(3, C, 128, generator=g), dim=-1)
    beta = torch.rand(3, C, generator=g)
    lg = -torch.rand(3, C, generator=g) * 0.3
    lgc = lg.cumsum(-1)
    G = (lgc[..., :, None] - lgc[..., None, :]).tril().exp().tril()
    kb = k * beta[..., None]
    T = ut_transform(kb, k, G)
    A = ((kb @ k.transpose(-1, -2)) * G).tril(-1)
    eye = torch.eye(C).expand(3, C, C)
    torch.testing.assert_close((eye + A) @ T, eye, rtol=0, atol=2e-5)
    T_lib = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
    torch.testing.assert_close(T, T_lib, rtol=1e-4, atol=2e-5)


def test_no_write_no_decay():
    """beta -> 0, g -> 1: state unchanged and o_t = scale q_t^T S0."""
    d = synth.prefill_inputs(1, 70, 2, 128, 16, seed=5, state=True)
    d["b_logits"] = torch.full_like(d["b_logits"], -60.0)
    d["A_log"] = torch.full_like(d["A_log"], -60.0)
    o, S = _oracle(d, state=d["state_in"], scale=0.25)
    torch.testing.assert_close(S, d["state_in"], rtol=0, atol=1e-7)
    torch.testing.assert_close(o, 0.25 * d["q"].float() @ d["state_in"], rtol=1e-5, atol=1e-7)


def test_varlen_equals_per_sequence_recurrence():
    lengths = [5, 0, 70, 64, 1]
    d = synth.varlen_inputs(lengths, 2, 128, 32, seed=6)
    o, S = ref_prefill_varlen(d["q"], d["k"], d["v"], d["A_log"], d["a"], 0.0, d["b_logits"], d["cu_seqlens"],
                              state_in=d["state_in"], chunk_size=64)
    cu = d["cu_seqlens"].tolist()
    g, beta = rf.gates_f64(d["A_log"].numpy(), d["a"].float().numpy(), 0.0, d["b_logits"].float().numpy())
    for i in range(len(lengths)):
        s, e = cu[i], cu[i + 1]
        o64, S64 = rf.recurrence(d["q"][:, :, s:e].float().numpy(), d["k"][:, :, s:e].float().numpy(),
                                 d["v"][:, :, s:e].float().numpy(), g[:, :, s:e], beta[:, :, s:e],
                                 np.ones((1, e - s)), d["state_in"][i:i + 1].numpy())
        np.testing.assert_allclose(o[:, :, s:e].numpy(), o64, rtol=1e-4, atol=2e-6)
        np.testing.assert_allclose(S[i:i + 1].numpy(), S64, rtol=1e-4, atol=2e-6)


def test_checks_catch_a_planted_mistake():
    """A mutant solve that drops the decay matrix G in A is caught by the float64 brute force."""
    d = synth.prefill_inputs(1, 64, 1, 128, 16, seed=9)
    import oracle.prefill_ref as pr

    orig = pr.ut_transform

    def mutant(k_beta, k, G):
        return orig(k_beta, k, torch.ones_like(G).tril())

    pr.ut_transform = mutant
    try:
        o_m, _ = _oracle(d)
    finally:
        pr.ut_transform = orig
    o64, _ = _f64(d)
    assert not np.allclose(o_m.numpy(), o64, rtol=1e-3, atol=1e-5)
