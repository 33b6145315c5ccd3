"""CPU restatement of the reference's chunked GDN prefill (test infrastructure).

Follows ``reference/prefill_ref.py:11-132`` (``ref_prefill``) step by step:

* gates (``:48-52``): ``g = exp(-exp(A_log) * softplus(a + dt_bias))``,
  ``beta = sigmoid(b_logits)``; the log-decay is taken as ``log(g)`` (``:64``);
* zero padding of T to a multiple of the chunk size (``:66-74``); padded tokens
  have beta = 0, log g = 0 and mask = 0, so they leave the state untouched;
* ``q *= scale``; ``k_beta = k*beta*m``; ``v_beta = v*beta*m`` (``:78-80``);
  the mask is NOT applied to the decay (masked tokens still decay) — the
  oracle's behaviour, which the product follows;
* in-chunk log-cumsum and the decay matrix ``G`` (``:90-93``);
* ``(I + A)^-1`` by forward substitution over rows (``:96-101``), with
  ``A = (k_beta k^T) * G`` strictly lower triangular;
* ``U = T v_beta``, ``W = T (k_beta * g_cum)`` (``:103-104``);
* the sequential chunk loop (``:113-126``) and the final masking (``:128-130``).

The arithmetic is float32 on CPU tensors, as in the reference.  The returned
``o`` is float32 (the reference casts its inputs to float32 at ``:57-60``).
"""

import math

import torch
import torch.nn.functional as F


def gates(A_log, a, dt_bias, b_logits):
    """Per-token decay g and write strength beta (reference/prefill_ref.py:48-52).

    A_log: [H] fp32; a, b_logits: [B, H, T]; dt_bias: python float or tensor
    (scalar, or [H] broadcast over heads).  Returns (g, beta) fp32 [B, H, T].
    """
    H = a.shape[1]
    dtb = torch.as_tensor(dt_bias, dtype=torch.float32)
    if dtb.numel() > 1:
        dtb = dtb.reshape(1, H, 1)
    x = a.float() + dtb
    g = torch.exp(-torch.exp(A_log.float().reshape(1, H, 1)) * F.softplus(x))
    beta = torch.sigmoid(b_logits.float())
    return g, beta


def ut_transform(k_beta, k, G):
    """(I + A)^-1 for A = strictly-lower (k_beta @ k^T) * G, per chunk.

    Forward substitution row by row, as in reference/prefill_ref.py:96-101:
    row i of L = -A gains sum_j L[i, j] * L[j, :i] over the already final rows
    j < i, then the identity is added.  Shapes [..., C, C].
    """
    C = G.shape[-1]
    strict_upper_or_diag = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=0)
    L = -((k_beta @ k.transpose(-1, -2)) * G).masked_fill(strict_upper_or_diag, 0.0)
    for i in range(1, C):
        row = L[..., i, :i].clone()
        row = row + (L[..., i, :i, None] * L[..., :i, :i]).sum(-2)
        L[..., i, :i] = row
    return L + torch.eye(C, dtype=L.dtype)


@torch.no_grad()
def ref_prefill(q, k, v, A_log, a, dt_bias, b_logits, mask,
                state_in=None, scale=0.0, chunk_size=None):
    """Chunked GDN prefill on CPU (reference/prefill_ref.py:11-132).

    q, k: [B, H, T, K]; v: [B, H, T, V]; A_log: [H]; a, b_logits: [B, H, T];
    dt_bias: scalar (float or tensor); mask: [B, T]; state_in: [B, H, K, V] or
    None; scale 0.0 means K**-0.5; chunk_size None means one chunk of length T.
    Returns (o [B, H, T, V] fp32, state [B, H, K, V] fp32).
    """
    B, H, T, K = q.shape
    V = v.shape[-1]
    C = chunk_size or T
    if scale == 0.0:
        scale = 1.0 / math.sqrt(K)

    g, beta = gates(A_log, a, dt_bias, b_logits)
    m = mask.float().reshape(B, 1, T, 1).expand(B, H, T, 1)
    qf, kf, vf = (x.contiguous().float() for x in (q, k, v))
    log_g = g.log()

    pad = (C - T % C) % C
    if pad:
        qf = F.pad(qf, (0, 0, 0, pad))
        kf = F.pad(kf, (0, 0, 0, pad))
        vf = F.pad(vf, (0, 0, 0, pad))
        beta = F.pad(beta, (0, pad))
        log_g = F.pad(log_g, (0, pad))
        m = F.pad(m, (0, 0, 0, pad))
    Tp = T + pad
    N = Tp // C

    qf = qf * scale
    k_beta = kf * beta[..., None] * m
    v_beta = vf * beta[..., None] * m

    def chunked(x):
        return x.reshape(B, H, N, C, x.shape[-1])

    qc, kc, kbc, vbc = chunked(qf), chunked(kf), chunked(k_beta), chunked(v_beta)
    lgc = log_g.reshape(B, H, N, C).cumsum(-1)                 # in-chunk log-cumsum
    gcum = lgc.exp()[..., None]                               # [B, H, N, C, 1]
    G = (lgc[..., :, None] - lgc[..., None, :]).tril().exp().tril()

    Tm = ut_transform(kbc, kc, G)
    U = Tm @ vbc                                               # new_v - old_v, intra part
    W = Tm @ (kbc * gcum)

    S = state_in.float().clone() if state_in is not None and state_in.numel() > 0 \
        else torch.zeros(B, H, K, V, dtype=torch.float32)
    causal_strict_upper = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=1)
    o = torch.zeros(B, H, N, C, V, dtype=torch.float32)
    for n in range(N):
        dv = U[:, :, n] - W[:, :, n] @ S
        o_cross = (qc[:, :, n] * gcum[:, :, n]) @ S
        attn = (qc[:, :, n] @ kc[:, :, n].transpose(-1, -2) * G[:, :, n]) \
            .masked_fill(causal_strict_upper, 0.0)
        o[:, :, n] = o_cross + attn @ dv
        decay_last = lgc[:, :, n, -1]
        k_tail = kc[:, :, n] * (decay_last[..., None] - lgc[:, :, n]).exp()[..., None]
        S = S * decay_last.exp()[..., None, None] + k_tail.transpose(-1, -2) @ dv

    o = o.reshape(B, H, Tp, V)[:, :, :T] * m[:, :, :T]
    return o, S


@torch.no_grad()
def ref_prefill_varlen(q, k, v, A_log, a, dt_bias, b_logits, cu_seqlens,
                       state_in=None, scale=0.0, chunk_size=64, mask=None):
    """Packed variable-length prefill: ``ref_prefill`` run per sequence.

    The reference has no varlen path; this is its per-sequence definition.
    q, k: [1, H, Ttot, K]; v: [1, H, Ttot, V]; a, b_logits: [1, H, Ttot];
    cu_seqlens: [N+1] int offsets into Ttot; state_in: [N, H, K, V] or None;
    mask: [1, Ttot] or None (all ones).  Returns (o [1, H, Ttot, V] fp32,
    state [N, H, K, V] fp32).
    """
    cu = [int(x) for x in torch.as_tensor(cu_seqlens).tolist()]
    nseq = len(cu) - 1
    H, K, V = q.shape[1], q.shape[-1], v.shape[-1]
    Ttot = q.shape[2]
    if mask is None:
        mask = torch.ones(1, Ttot, dtype=torch.float32)
    o = torch.zeros(1, H, Ttot, V, dtype=torch.float32)
    states = torch.zeros(nseq, H, K, V, dtype=torch.float32)
    for i in range(nseq):
        s, e = cu[i], cu[i + 1]
        if e == s:
            if state_in is not None:
                states[i] = state_in[i].float()
            continue
        si = state_in[i:i + 1] if state_in is not None else None
        oi, Si = ref_prefill(q[:, :, s:e], k[:, :, s:e], v[:, :, s:e], A_log,
                             a[:, :, s:e], dt_bias, b_logits[:, :, s:e], mask[:, s:e],
                             state_in=si, scale=scale, chunk_size=chunk_size)
        o[:, :, s:e] = oi
        states[i] = Si[0]
    return o, states
