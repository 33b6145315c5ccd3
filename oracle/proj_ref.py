"""CPU restatement of the reference projection + causal conv1d + SiLU.

Follows ``reference/fused_proj_conv_silu_ref.py:9-66``.  Note the rounding
points of the reference: despite the "upcast" comment at ``:48``, nothing is
upcast — ``x @ w.T`` runs in the input dtype (bf16 in, bf16 out), the
depthwise conv runs in that dtype too, and only the final ``.to(dtype)`` is a
no-op.  ``ref_proj_conv_silu_f32`` is the float32-throughout variant (the
reference CUDA kernel keeps the projection in fp32 before the conv,
``kernels/fused_proj_conv_silu.cu:250-290``), used as the tighter check for
the product kernel.
"""

import torch
import torch.nn.functional as F


@torch.no_grad()
def ref_proj(x, weight):
    """Linear projection x @ W^T (reference :9-11)."""
    return x @ weight.T


@torch.no_grad()
def ref_conv1d(x, conv_w):
    """Causal depthwise conv1d over time, left zero padding K-1 (reference :14-23).

    x: [B, T, D_out]; conv_w: [D_out, K].  Tap j of channel c multiplies
    x[t - (K-1) + j].
    """
    D_out, Kc = conv_w.shape
    xt = F.pad(x.transpose(1, 2), (Kc - 1, 0))
    return F.conv1d(xt, conv_w.unsqueeze(1), groups=D_out).transpose(1, 2)


@torch.no_grad()
def ref_silu(x):
    """SiLU (reference :26-28)."""
    return F.silu(x)


@torch.no_grad()
def ref_proj_conv_silu(x, weight, conv_w):
    """SiLU(causal_conv(x @ W^T)) with the reference's dtype behaviour (reference :32-66)."""
    dtype = x.dtype
    return ref_silu(ref_conv1d(ref_proj(x, weight), conv_w)).to(dtype)


@torch.no_grad()
def ref_proj_conv_silu_f32(x, weight, conv_w):
    """Same composition computed in float32 throughout, rounded to bf16 at the end."""
    y = ref_conv1d(ref_proj(x.float(), weight.float()), conv_w.float())
    return F.silu(y).to(torch.bfloat16)
