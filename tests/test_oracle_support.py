"""CPU pins for the supporting-kernel oracles and the layer oracle.

* RMSNorm (oracle/rmsnorm_ref.py <- reference/rmsnorm_ref.py:8-28): the
  reference test's own ground truth, torch.nn.RMSNorm in fp32
  (tests/test_rmsnorm.py:31-40 of the reference), and a closed form.
* Projection + conv + SiLU (oracle/proj_ref.py): a brute-force loop, causality.
* Layer (oracle/layer_ref.py <- gdn_layer.py:108-200): decoding T tokens one at
  a time equals one prefill over them (the reference's own integration check,
  bench_gdn.py:200-219).
"""

import torch

from oracle.layer_ref import GDNLayerBaseline
from oracle.proj_ref import ref_proj_conv_silu, ref_proj_conv_silu_f32
from oracle.rmsnorm_ref import ref_rmsnorm


def test_rmsnorm_vs_torch_rmsnorm():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 2048, generator=g).bfloat16()
    gamma = (1 + 0.1 * torch.randn(2048, generator=g)).bfloat16()
    y = ref_rmsnorm(x, gamma, 1e-6)
    m = torch.nn.RMSNorm(2048, eps=1e-6, elementwise_affine=True, dtype=torch.float32)
    with torch.no_grad():
        m.weight.copy_(gamma.float())
        y32 = m(x.float())
    assert y.dtype == torch.bfloat16
    torch.testing.assert_close(y.float(), y32, rtol=2 ** -7, atol=1e-6)


def test_rmsnorm_closed_form_constant_row():
    x = torch.full((2, 512), 3.0).bfloat16()
    gamma = torch.full((512,), 2.0).bfloat16()
    y = ref_rmsnorm(x, gamma, 1e-6)
    torch.testing.assert_close(y.float(), torch.full((2, 512), 2.0 * 3.0 / (9.0 + 1e-6) ** 0.5), rtol=1e-2, atol=0)


def _brute_proj_conv_silu(x, W, cw):
    B, T, D = x.shape
    Do, Kc = cw.shape
    P = torch.zeros(B, T, Do, dtype=torch.float64)
    for t in range(T):
        P[:, t] = x[:, t].double() @ W.double().T
    out = torch.zeros_like(P)
    for t in range(T):
        for j in range(Kc):
            tt = t - (Kc - 1) + j
            if tt >= 0:
                out[:, t] += cw[:, j].double() * P[:, tt]
    return out * torch.sigmoid(out)


def test_proj_conv_silu_vs_brute_force():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 9, 64, generator=g).bfloat16()
    W = (torch.randn(48, 64, generator=g) * 64 ** -0.5).bfloat16()
    cw = (torch.randn(48, 4, generator=g) * 0.5).bfloat16()
    ref = _brute_proj_conv_silu(x, W, cw)
    torch.testing.assert_close(ref_proj_conv_silu_f32(x, W, cw).double(), ref, rtol=1e-2, atol=1e-2)
    # the reference's own bf16 rounding points stay within bf16 tolerance of the exact value
    torch.testing.assert_close(ref_proj_conv_silu(x, W, cw).double(), ref, rtol=5e-2, atol=5e-2)


def test_proj_conv_silu_is_causal():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, 12, 64, generator=g).bfloat16()
    W = (torch.randn(32, 64, generator=g) * 0.1).bfloat16()
    cw = torch.randn(32, 4, generator=g).bfloat16()
    y1 = ref_proj_conv_silu_f32(x, W, cw)
    x2 = x.clone()
    x2[:, 7:] = torch.randn(1, 5, 64, generator=g).bfloat16()
    y2 = ref_proj_conv_silu_f32(x2, W, cw)
    assert torch.equal(y1[:, :7], y2[:, :7]) and not torch.equal(y1[:, 7:], y2[:, 7:])


def _small_weights(D=64, H=2, DK=128, DV=32, CK=4, seed=0):
    g = torch.Generator().manual_seed(seed)

    def rnd(*s, scale=1.0):
        return (torch.randn(*s, generator=g) * s[-1] ** -0.5 * scale).bfloat16()

    return dict(norm_gamma=torch.ones(D).bfloat16(),
                W_q=rnd(H * DK, D, scale=DK ** -0.5), conv_q=(torch.randn(H * DK, CK, generator=g) * 0.5).bfloat16(),
                W_k=rnd(H * DK, D, scale=DK ** -0.5), conv_k=(torch.randn(H * DK, CK, generator=g) * 0.5).bfloat16(),
                W_v=rnd(H * DV, D, scale=DK ** -0.5), conv_v=(torch.randn(H * DV, CK, generator=g) * 0.5).bfloat16(),
                W_a=rnd(H, D), W_b=rnd(H, D), A_log=torch.zeros(H), dt_bias=torch.tensor(0.0),
                W_o=rnd(D, H * DV))


def test_layer_decode_matches_prefill():
    """Decoding tokens one by one through the baseline layer equals one prefill (bench_gdn.py:200-219)."""
    w = _small_weights()
    layer = GDNLayerBaseline(w, chunk_size=16)
    x = torch.randn(1, 20, 64, generator=torch.Generator().manual_seed(3)).bfloat16()
    y_pre = layer.forward(x)
    state = layer.init_decode_state(1)
    outs = []
    for t in range(20):
        y_t, state = layer.decode(x[:, t:t + 1], state)
        outs.append(y_t)
    y_dec = torch.cat(outs, 1)
    torch.testing.assert_close(y_dec.float(), y_pre.float(), rtol=5e-2, atol=2e-2)


def test_layer_fp32_proj_decode_matches_prefill():
    """The fp32-projection layer variant: T decode steps equal one prefill (outputs
    and the final recurrent state), as the reference's own layer check (bench_gdn.py:200-219)."""
    w = _small_weights(seed=4)
    layer = GDNLayerBaseline(w, chunk_size=16, fp32_proj=True)
    x = torch.randn(2, 37, 64, generator=torch.Generator().manual_seed(5)).bfloat16()
    y_pre, S_pre = layer.forward(x, return_state=True)
    state = layer.init_decode_state(2)
    outs = []
    for t in range(37):
        y_t, state = layer.decode(x[:, t:t + 1], state)
        outs.append(y_t)
    torch.testing.assert_close(torch.cat(outs, 1).float(), y_pre.float(), rtol=2e-2, atol=2e-2)
    rel = ((state["recurrent"] - S_pre).norm() / S_pre.norm()).item()
    assert rel < 1e-2, rel


def test_decode_conv_step_f32_vs_brute_force():
    """One decode conv step equals the last row of the fp64 brute-force projection + conv
    + SiLU over the cached window; the cache shifts in bf16(P)."""
    from oracle.layer_ref import decode_conv_step_f32
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 4, 64, generator=g).bfloat16()
    W = (torch.randn(40, 64, generator=g) * 64 ** -0.5).bfloat16()
    cw = (torch.randn(40, 4, generator=g) * 0.5).bfloat16()
    cache = (x[:, :3].float() @ W.float().T).bfloat16().transpose(1, 2).contiguous()  # [B, 40, 3]
    y, new_cache = decode_conv_step_f32(x[:, 3:4], W, cw, cache)
    P = torch.cat([cache.double(), (x[:, 3].double() @ W.double().T).unsqueeze(-1)], -1)
    conv = (P * cw.double().unsqueeze(0)).sum(-1)
    torch.testing.assert_close(y.double(), conv * torch.sigmoid(conv), rtol=1e-2, atol=1e-3)
    assert torch.equal(new_cache[:, :, :2], cache[:, :, 1:])
    assert torch.equal(new_cache[:, :, 2], (x[:, 3].float() @ W.float().T).bfloat16())


def _layer_f64(w, x, swap_ab=False):
    """The layer in float64, token by token, restated from the reference's text
    (gdn_layer.py:120-158, decode gdn_layer.py:161-200) and sharing no code with
    oracle/layer_ref.py: RMSNorm (eps 1e-6), q/k/v = SiLU(causal depthwise conv
    of xn W^T, taps w[c, j] on token t - (CK - 1) + j), a = xn W_a^T,
    b = xn W_b^T, the per-token recurrence (oracle/recurrence_f64.py), then
    y = o W_o^T.  ``swap_ab`` feeds W_b to the decay and W_a to beta: the
    wrong wiring, which the comparison must be able to tell apart."""
    from oracle.recurrence_f64 import gates_f64, recurrence
    B, T, D = x.shape
    H = w['A_log'].numel()
    DK, DV, CK = w['W_q'].shape[0] // H, w['W_v'].shape[0] // H, w['conv_q'].shape[1]
    x64 = x.double()
    xn = x64 * torch.rsqrt((x64 ** 2).mean(-1, keepdim=True) + 1e-6) * w['norm_gamma'].double()

    def pcs(W, cw):
        P = xn @ W.double().T
        Pp = torch.nn.functional.pad(P, (0, 0, CK - 1, 0))
        c = sum(Pp[:, j:j + T] * cw.double()[:, j] for j in range(CK))
        return c * torch.sigmoid(c)

    q = pcs(w['W_q'], w['conv_q']).reshape(B, T, H, DK).permute(0, 2, 1, 3)
    k = pcs(w['W_k'], w['conv_k']).reshape(B, T, H, DK).permute(0, 2, 1, 3)
    v = pcs(w['W_v'], w['conv_v']).reshape(B, T, H, DV).permute(0, 2, 1, 3)
    Wa, Wb = (w['W_b'], w['W_a']) if swap_ab else (w['W_a'], w['W_b'])
    a = (xn @ Wa.double().T).permute(0, 2, 1)
    b = (xn @ Wb.double().T).permute(0, 2, 1)
    g, beta = gates_f64(w['A_log'].numpy(), a.numpy(), float(w['dt_bias']), b.numpy())
    o, S = recurrence(q.numpy(), k.numpy(), v.numpy(), g, beta, torch.ones(B, T).numpy(), scale=DK ** -0.5)
    o = torch.from_numpy(o).permute(0, 2, 1, 3).reshape(B, T, H * DV)
    return o @ w['W_o'].double().T, torch.from_numpy(S)


def _rel_err(y, y_ref):
    y, y_ref = y.double(), y_ref.double()
    return ((y - y_ref).norm() / y_ref.norm()).item()


def test_layer_wiring_vs_f64_restatement():
    """The oracle layer (forward and token-by-token decode, fp32 projections)
    against the float64 restatement: output and final state within bf16
    rounding (1e-2 relative), while the same restatement with W_a and W_b
    swapped is far off -- so which weight feeds the decay, beta and the output
    projection is pinned by something other than the layer's own decode ==
    prefill check."""
    w = _small_weights(D=64, H=2, DK=16, DV=8, seed=21)
    w['A_log'] = torch.tensor([-0.5, 0.3])
    w['dt_bias'] = torch.tensor(0.2)
    w['norm_gamma'] = (1 + 0.2 * torch.randn(64, generator=torch.Generator().manual_seed(22))).bfloat16()
    x = torch.randn(2, 30, 64, generator=torch.Generator().manual_seed(23)).bfloat16()
    y64, S64 = _layer_f64(w, x)
    layer = GDNLayerBaseline(w, chunk_size=16, fp32_proj=True)
    y, S = layer.forward(x, return_state=True)
    assert _rel_err(y, y64) < 1e-2 and _rel_err(S, S64) < 1e-2
    state = layer.init_decode_state(2)
    outs = []
    for t in range(30):
        y_t, state = layer.decode(x[:, t:t + 1], state)
        outs.append(y_t)
    assert _rel_err(torch.cat(outs, 1), y64) < 1e-2 and _rel_err(state['recurrent'], S64) < 1e-2
    y_sw, S_sw = _layer_f64(w, x, swap_ab=True)
    assert _rel_err(y_sw, y64) > 0.1 and _rel_err(S_sw, S64) > 0.1
