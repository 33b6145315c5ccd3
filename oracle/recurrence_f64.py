"""Float64 per-token GDN recurrence in numpy (test infrastructure).

This is the brute-force definition both chunked forms must equal: the
per-token recurrence stated in the docstring of ``reference/prefill_ref.py``
(lines 18-23), and, for one token, ``reference/decode_ref.py:48-59``:

    S <- g_t S
    r  = k_t^T S
    S <- S + m_t beta_t k_t (v_t - r)^T
    o_t = m_t scale q_t^T S

It shares no code with the chunked oracle, so agreement pins the WY/UT
algebra (the triangular solve, the decay matrix, the chunk hand-off).
"""

import numpy as np


def gates_f64(A_log, a, dt_bias, b_logits):
    """g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b), in float64.

    A_log [H]; a, b_logits [B, H, T]; dt_bias scalar or [H].
    """
    A_log = np.asarray(A_log, np.float64)
    H = A_log.shape[0]
    dtb = np.asarray(dt_bias, np.float64)
    if dtb.size > 1:
        dtb = dtb.reshape(1, H, 1)
    x = np.asarray(a, np.float64) + dtb
    softplus = np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    g = np.exp(-np.exp(A_log).reshape(1, H, 1) * softplus)
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b_logits, np.float64)))
    return g, beta


def recurrence(q, k, v, g, beta, mask, state_in=None, scale=None):
    """Token-by-token GDN over [B, H, T, *] float64 arrays.

    q, k [B, H, T, K]; v [B, H, T, V]; g, beta [B, H, T]; mask [B, T];
    state_in [B, H, K, V] or None.  Returns (o [B, H, T, V], S [B, H, K, V]).
    """
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    B, H, T, K = q.shape
    V = v.shape[-1]
    if scale is None or scale == 0.0:
        scale = K ** -0.5
    S = np.zeros((B, H, K, V)) if state_in is None else np.array(state_in, np.float64)
    o = np.zeros((B, H, T, V))
    m = np.asarray(mask, np.float64)
    for t in range(T):
        S = S * g[:, :, t, None, None]
        r = np.einsum('bhk,bhkv->bhv', k[:, :, t], S)
        w = (m[:, t, None] * beta[:, :, t])[..., None]            # [B, H, 1]
        S = S + k[:, :, t, :, None] * (w * (v[:, :, t] - r))[..., None, :]
        o[:, :, t] = m[:, t, None, None] * scale * np.einsum('bhk,bhkv->bhv', q[:, :, t], S)
    return o, S


def decode_closed_form(q, k, v, S, g, beta, scale):
    """One decode step in the closed form S_T <- g S_T (I - beta k k^T) + beta v k^T.

    Works on the transposed state S_T = S^T ([.., V, K]), the value-first
    convention of that formula, and returns (o, S) back in the K-first layout.  Inputs are
    [B, H, *] float64 arrays, g/beta [B, H].
    """
    q, k, v, S = (np.asarray(x, np.float64) for x in (q, k, v, S))
    K = k.shape[-1]
    ST = np.swapaxes(S, -1, -2)                                       # [B, H, V, K]
    eye = np.eye(K)
    proj = eye - beta[..., None, None] * k[..., :, None] * k[..., None, :]
    ST = g[..., None, None] * ST @ proj + beta[..., None, None] * v[..., :, None] * k[..., None, :]
    o = scale * np.einsum('bhvk,bhk->bhv', ST, q)
    return o, np.swapaxes(ST, -1, -2)
