"""Shared tolerance checks (the brief's parity bar).

* outputs: |x - ref| <= atol + rtol |ref| elementwise with atol = rtol = 2e-2;
* final fp32 states: ||S - S_ref||_F / ||S_ref||_F <= 1e-2.
"""

import torch

OUT_ATOL = 2e-2
OUT_RTOL = 2e-2
STATE_REL = 1e-2


def assert_out_close(x, ref, atol=OUT_ATOL, rtol=OUT_RTOL, what="output"):
    x = x.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert x.shape == ref.shape, f"{what}: shape {tuple(x.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(x).all(), f"{what}: non-finite values"
    diff = (x - ref).abs()
    bad = diff > atol + rtol * ref.abs()
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.numel()} elements out of tolerance, "
                           f"max |diff| {diff.max().item():.3e}")
    return diff.max().item()


def rel_fro(x, ref):
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.norm().item()
    return (x - ref).norm().item() / (den if den > 0 else 1.0)


def assert_state_close(S, ref, tol=STATE_REL, what="state"):
    assert torch.isfinite(S.detach().float().cpu()).all(), f"{what}: non-finite values"
    r = rel_fro(S, ref)
    assert r <= tol, f"{what}: relative Frobenius error {r:.3e} > {tol}"
    return r
