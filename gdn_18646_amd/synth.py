"""Seeded synthetic inputs for the GDN hot paths (the brief's configs).

Draws come from a CPU ``torch.Generator`` in the fixed order q, k, v, a, b,
S0, so a CPU checker and the GPU kernels see bit-identical inputs:

* q, k ~ N(0, 1) fp32, L2-normalised per head along K in fp32, cast to bf16;
* v ~ N(0, 1) -> bf16;
* b_logits ~ N(0, 1) -> bf16, so beta = sigmoid(N(0, 1));
* a ~ N(0, 1) -> bf16 with A_log = ln 0.5 and dt_bias = 0, so
  log g = -0.5 softplus(a) (the kernels' gate formula with those constants);
* S0 ~ N(0, 0.02) fp32 (std 0.02).

Layouts follow the reference contracts: prefill q/k/v [B, H, T, d], a/b
[B, H, T]; decode q/k [B, H, K], v [B, H, V], a/b [B, H].
"""

import math

import torch

LN_HALF = math.log(0.5)


def _gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _unit_rows(x):
    return (x / x.norm(dim=-1, keepdim=True)).to(torch.bfloat16)


def prefill_inputs(B, T, H, K=128, V=128, seed=1, state=False, device="cpu"):
    """Inputs of the chunked prefill contract; ``state`` adds S0 ~ N(0, 0.02)."""
    g = _gen(seed)
    q = _unit_rows(torch.randn(B, H, T, K, generator=g))
    k = _unit_rows(torch.randn(B, H, T, K, generator=g))
    v = torch.randn(B, H, T, V, generator=g).to(torch.bfloat16)
    a = torch.randn(B, H, T, generator=g).to(torch.bfloat16)
    b = torch.randn(B, H, T, generator=g).to(torch.bfloat16)
    S0 = torch.randn(B, H, K, V, generator=g) * 0.02 if state else None
    d = dict(q=q, k=k, v=v, a=a, b_logits=b,
             A_log=torch.full((H,), LN_HALF, dtype=torch.float32),
             dt_bias=0.0, mask=torch.ones(B, T, dtype=torch.float32), state_in=S0)
    return {key: (val.to(device) if torch.is_tensor(val) else val) for key, val in d.items()}


def prefill_inputs_on_device(B, T, H, K=128, V=128, seed=1, device="cuda"):
    """prefill_inputs' distributions drawn on the device (a generator there):
    for sizes whose fp32 CPU draws would take gigabytes of host memory.  The
    values differ from prefill_inputs' at the same seed."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def unit_rows(shape):
        x = torch.randn(shape, generator=g, device=device)
        x /= x.norm(dim=-1, keepdim=True)
        return x.to(torch.bfloat16)

    q = unit_rows((B, H, T, K))
    k = unit_rows((B, H, T, K))
    bf = dict(generator=g, device=device)
    return dict(q=q, k=k, v=torch.randn(B, H, T, V, **bf).to(torch.bfloat16),
                a=torch.randn(B, H, T, **bf).to(torch.bfloat16), b_logits=torch.randn(B, H, T, **bf).to(torch.bfloat16),
                A_log=torch.full((H,), LN_HALF, dtype=torch.float32, device=device), dt_bias=0.0,
                mask=torch.ones(B, T, dtype=torch.float32, device=device), state_in=None)


def decode_inputs(B, H, K=128, V=128, seed=0, state=True, device="cpu"):
    """Inputs of the decode kernel contract (q, k [B,H,K]; v [B,H,V]; a, b [B,H])."""
    g = _gen(seed)
    q = _unit_rows(torch.randn(B, H, K, generator=g))
    k = _unit_rows(torch.randn(B, H, K, generator=g))
    v = torch.randn(B, H, V, generator=g).to(torch.bfloat16)
    a = torch.randn(B, H, generator=g).to(torch.bfloat16)
    b = torch.randn(B, H, generator=g).to(torch.bfloat16)
    S0 = torch.randn(B, H, K, V, generator=g) * 0.02 if state else torch.zeros(B, H, K, V)
    d = dict(q=q, k=k, v=v, a=a, b=b,
             A_log=torch.full((H,), LN_HALF, dtype=torch.float32),
             dt_bias=torch.zeros(H, dtype=torch.float32), S=S0)
    return {key: val.to(device) for key, val in d.items()}


def decode_step_stream(steps, B, H, K=128, V=128, seed=2):
    """``steps`` fresh (q, k, v, a, b) sets for a multi-step decode run (CPU tensors)."""
    g = _gen(seed)
    out = []
    for _ in range(steps):
        q = _unit_rows(torch.randn(B, H, K, generator=g))
        k = _unit_rows(torch.randn(B, H, K, generator=g))
        v = torch.randn(B, H, V, generator=g).to(torch.bfloat16)
        a = torch.randn(B, H, generator=g).to(torch.bfloat16)
        b = torch.randn(B, H, generator=g).to(torch.bfloat16)
        out.append(dict(q=q, k=k, v=v, a=a, b=b))
    return out


def varlen_lengths(nseq=8, lo=512, hi=8192, seed=3):
    """Sequence lengths drawn uniformly from [lo, hi] (inclusive)."""
    g = _gen(seed)
    return torch.randint(lo, hi + 1, (nseq,), generator=g).tolist()


def varlen_inputs(lengths, H, K=128, V=128, seed=3, device="cpu"):
    """Packed inputs [1, H, sum(lengths), d] with cu_seqlens and per-sequence S0."""
    g = _gen(seed + 1000)
    Ttot = int(sum(lengths))
    q = _unit_rows(torch.randn(1, H, Ttot, K, generator=g))
    k = _unit_rows(torch.randn(1, H, Ttot, K, generator=g))
    v = torch.randn(1, H, Ttot, V, generator=g).to(torch.bfloat16)
    a = torch.randn(1, H, Ttot, generator=g).to(torch.bfloat16)
    b = torch.randn(1, H, Ttot, generator=g).to(torch.bfloat16)
    S0 = torch.randn(len(lengths), H, K, V, generator=g) * 0.02
    cu = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(lengths, dtype=torch.int32).cumsum(0)
    d = dict(q=q, k=k, v=v, a=a, b_logits=b, cu_seqlens=cu, state_in=S0,
             A_log=torch.full((H,), LN_HALF, dtype=torch.float32), dt_bias=0.0)
    return {key: (val.to(device) if torch.is_tensor(val) else val) for key, val in d.items()}
