"""CPU restatement of the reference RMSNorm (test infrastructure).

Follows ``reference/rmsnorm_ref.py:8-28``: the mean of squares and the scaling
are float32; the result is rounded to bfloat16 once at the end.
"""

import torch


@torch.no_grad()
def ref_rmsnorm(x, gamma, eps=1e-6):
    """y = bf16(x * rsqrt(mean(x^2) + eps) * gamma); x [R, D] bf16, gamma [D] bf16."""
    xf = x.float()
    inv_rms = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * inv_rms * gamma.float()).to(torch.bfloat16)
