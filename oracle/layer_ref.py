"""CPU restatement of the reference's baseline GDN layer (test infrastructure).

Follows ``gdn_layer.py:31-200`` of the reference (``_zero_decode_state``,
``_decode_conv_step``, ``_dt_bias_for_decode`` and ``GDNLayerBaseline``), with
the architecture read from the weight shapes instead of module constants so
that both the reference's shape (H=16, DK=128, DV=256) and the brief's layer
config (DV=128) run through the same code.
"""

import torch

from .decode_ref import ref_decode
from .prefill_ref import ref_prefill
from .proj_ref import ref_proj_conv_silu, ref_proj_conv_silu_f32
from .rmsnorm_ref import ref_rmsnorm


def dims(w):
    """(D, H, DK, DV, CONV_K) read from a weight dict (keys as gdn_layer.py:85-102)."""
    H = w['A_log'].numel()
    D = w['W_q'].shape[1]
    return D, H, w['W_q'].shape[0] // H, w['W_v'].shape[0] // H, w['conv_q'].shape[1]


def zero_decode_state(w, B, device=None):
    """Zeroed decode cache, as gdn_layer.py:31-40."""
    D, H, DK, DV, CK = dims(w)
    device = device or w['norm_gamma'].device
    bf = torch.bfloat16
    return dict(
        recurrent=torch.zeros(B, H, DK, DV, dtype=torch.float32, device=device),
        conv_q=torch.zeros(B, H * DK, CK - 1, dtype=bf, device=device),
        conv_k=torch.zeros(B, H * DK, CK - 1, dtype=bf, device=device),
        conv_v=torch.zeros(B, H * DV, CK - 1, dtype=bf, device=device),
        xn=torch.zeros(B, CK - 1, D, dtype=bf, device=device),
    )


def decode_conv_step(xn, W, conv_w, conv_state):
    """Projection + one-token causal conv + SiLU with a projected-token cache.

    gdn_layer.py:43-55: proj rounded to the activation dtype, window of the
    cached CONV_K-1 projections plus the new one, weighted sum in that dtype.
    """
    proj = (xn.squeeze(1) @ W.T).to(xn.dtype)
    window = torch.cat([conv_state, proj.unsqueeze(-1)], dim=-1)
    conv = (window * conv_w.unsqueeze(0)).sum(dim=-1)
    return torch.nn.functional.silu(conv).to(xn.dtype), window[:, :, 1:].contiguous()


def decode_conv_step_f32(xn, W, conv_w, conv_state):
    """decode_conv_step with the projection kept in float32 through the conv.

    These are the rounding points of the reference's CUDA projection kernel,
    which holds P in fp32 before the conv (kernels/fused_proj_conv_silu.cu:250-290):
    the window is the cached bf16 projections (widened) plus the new fp32
    one, the tap sum is fp32, and the cache receives bf16(P).
    """
    proj = xn.squeeze(1).float() @ W.float().T
    window = torch.cat([conv_state.float(), proj.unsqueeze(-1)], dim=-1)
    conv = (window * conv_w.float().unsqueeze(0)).sum(dim=-1)
    cache = torch.cat([conv_state, proj.to(xn.dtype).unsqueeze(-1)], dim=-1)[:, :, 1:]
    return torch.nn.functional.silu(conv).to(xn.dtype), cache.contiguous()


def dt_bias_per_head(dt_bias, H):
    """Scalar dt_bias expanded to [H] (gdn_layer.py:72-76)."""
    if dt_bias.numel() == 1:
        return dt_bias.reshape(1).expand(H).contiguous()
    return dt_bias.contiguous()


class GDNLayerBaseline:
    """Pure-PyTorch GDN layer (gdn_layer.py:108-200).

    ``fp32_proj=True`` keeps the q/k/v projections in float32 through the
    conv and SiLU (ref_proj_conv_silu_f32, decode_conv_step_f32): the
    rounding points of the reference's CUDA projection kernel and of this
    build's kernels; the default follows the reference's PyTorch baseline,
    which rounds the projection to bf16 before the conv.
    """

    def __init__(self, weights, chunk_size=None, fp32_proj=False):
        self.w = weights
        self.D, self.H, self.DK, self.DV, self.CK = dims(weights)
        self.scale = self.DK ** -0.5
        self.chunk_size = chunk_size
        self.fp32_proj = fp32_proj

    def init_decode_state(self, B, device=None):
        return zero_decode_state(self.w, B, device=device)

    @torch.no_grad()
    def forward(self, x, mask=None, return_state=False):
        """x [B, T, D] bf16 -> [B, T, D] bf16 (gdn_layer.py:120-158).

        ``return_state`` also returns the final recurrent state [B, H, DK, DV]
        (the reference discards it, gdn_layer.py:256).
        """
        B, T, _ = x.shape
        D, H, DK, DV = self.D, self.H, self.DK, self.DV
        w = self.w
        if mask is None:
            mask = x.new_ones(B, T, dtype=torch.float32)
        xn = ref_rmsnorm(x.reshape(B * T, D), w['norm_gamma']).reshape(B, T, D)

        pcs = ref_proj_conv_silu_f32 if self.fp32_proj else ref_proj_conv_silu

        def proj(W, cw, dh):
            return pcs(xn, W, cw).reshape(B, T, H, dh).transpose(1, 2).contiguous()

        q = proj(w['W_q'], w['conv_q'], DK)
        k = proj(w['W_k'], w['conv_k'], DK)
        v = proj(w['W_v'], w['conv_v'], DV)
        a = (xn @ w['W_a'].T).transpose(1, 2).contiguous()
        b = (xn @ w['W_b'].T).transpose(1, 2).contiguous()
        o, S = ref_prefill(q, k, v, w['A_log'], a, w['dt_bias'], b, mask,
                           state_in=None, scale=self.scale, chunk_size=self.chunk_size)
        y = o.to(x.dtype).transpose(1, 2).reshape(B, T, H * DV) @ w['W_o'].T
        return (y, S) if return_state else y

    @torch.no_grad()
    def decode(self, x, state=None):
        """One token: x [B, 1, D] -> (y [B, 1, D], new state dict) (gdn_layer.py:161-200)."""
        B, T, _ = x.shape
        assert T == 1, f"decode expects T=1, got T={T}"
        D, H, DK, DV = self.D, self.H, self.DK, self.DV
        w = self.w
        if state is None:
            state = self.init_decode_state(B, device=x.device)
        xn = ref_rmsnorm(x.reshape(B, D), w['norm_gamma']).reshape(B, 1, D)
        step = decode_conv_step_f32 if self.fp32_proj else decode_conv_step
        qp, conv_q = step(xn, w['W_q'], w['conv_q'], state['conv_q'])
        kp, conv_k = step(xn, w['W_k'], w['conv_k'], state['conv_k'])
        vp, conv_v = step(xn, w['W_v'], w['conv_v'], state['conv_v'])
        xn_state = torch.cat([state['xn'], xn], dim=1)[:, 1:, :].contiguous()
        q = qp.reshape(B, 1, H, DK)
        k = kp.reshape(B, 1, H, DK)
        v = vp.reshape(B, 1, H, DV)
        a = (xn @ w['W_a'].T).contiguous()
        b = (xn @ w['W_b'].T).contiguous()
        o, rec = ref_decode(q, k, v, state['recurrent'], w['A_log'], a,
                            dt_bias_per_head(w['dt_bias'], H), b, self.scale)
        y = o.to(x.dtype).reshape(B, 1, H * DV) @ w['W_o'].T
        return y, dict(recurrent=rec, conv_q=conv_q, conv_k=conv_k, conv_v=conv_v, xn=xn_state)
