"""CPU restatement of the reference's GDN decode step (test infrastructure).

Follows ``reference/decode_ref.py:10-61`` (``ref_decode``):

    g     = exp(-exp(A_log) * softplus(a + dt_bias))      (:39-40)
    beta  = sigmoid(b)                                    (:41)
    S'    = g * S                                         (:49)
    r     = k^T S'                                        (:52)
    delta = beta * (v - r)                                (:55)
    S''   = S' + k delta^T                                (:56)
    o     = scale * q^T S''                               (:59)

State layout is K-first, [B, H, K, V]; everything is float32.
"""

import math

import torch
import torch.nn.functional as F


@torch.no_grad()
def ref_decode(q, k, v, state, A_log, a_param, dt_bias, b_param, scale=None):
    """One decode step.

    q, k: [B, 1, H, K]; v: [B, 1, H, V]; state: [B, H, K, V] fp32;
    A_log, dt_bias: [H] fp32; a_param, b_param: [B, 1, H]; scale None means
    K**-0.5.  Returns (o [B, H, V] fp32, new_state [B, H, K, V] fp32).
    """
    B, T, H, K = q.shape
    assert T == 1, f"ref_decode expects one token, got T={T}"
    if scale is None:
        scale = 1.0 / math.sqrt(K)

    x = a_param.reshape(B, H).float() + dt_bias.float().reshape(1, -1)
    g = torch.exp(-torch.exp(A_log.float()).reshape(1, H) * F.softplus(x))
    beta = torch.sigmoid(b_param.reshape(B, H).float())

    qf = q.reshape(B, H, K).float()
    kf = k.reshape(B, H, K).float()
    vf = v.reshape(B, H, -1).float()

    S = state.float() * g[:, :, None, None]
    r = torch.einsum('bhk,bhkv->bhv', kf, S)
    delta = beta[:, :, None] * (vf - r)
    S = S + kf[..., :, None] * delta[..., None, :]
    o = scale * torch.einsum('bhk,bhkv->bhv', qf, S)
    return o, S
