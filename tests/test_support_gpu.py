"""GPU parity of the supporting kernels: RMSNorm and projection + conv + SiLU.

RMSNorm is checked against the CPU oracle (reference/rmsnorm_ref.py restated)
and, like the reference's test (tests/test_rmsnorm.py:31-48), against fp32
torch.nn.RMSNorm.  The projection kernel keeps P in fp32 before the conv (as the
reference kernel does), so it is held to the fp32 composition within bf16
output tolerance, and to the reference's bf16-rounded oracle with the
reference test's max-error bound (tests/test_fused_proj_conv_silu.py:55-59)
plus a relative term.  The decode-step projections (one token, B <= 16) are
held to the same fp32 compositions, with x_n bit-equal to the RMSNorm kernel's.
"""

import pytest
import torch

from oracle.proj_ref import ref_proj_conv_silu, ref_proj_conv_silu_f32
from oracle.rmsnorm_ref import ref_rmsnorm
from tests.helpers import assert_out_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T", [(1, 1), (1, 2048), (8, 1), (8, 2048), (32, 1), (4, 4096)])
def test_rmsnorm_reference_shapes(exts, dev, B, T):
    D = 2048
    g = torch.Generator().manual_seed(B * 7 + T)
    x = torch.randn(B * T, D, generator=g).bfloat16()
    gamma = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    y = exts["rmsnorm"].forward(x.to(dev), gamma.to(dev), 1e-6, 256, 2).cpu()
    y_ref = ref_rmsnorm(x, gamma, 1e-6)
    # same fp32 math and one final rounding: at most one bf16 ulp apart
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=2 ** -7, atol=1e-6)
    m = torch.nn.RMSNorm(D, eps=1e-6, dtype=torch.float32)
    with torch.no_grad():
        m.weight.copy_(gamma.float())
        y32 = m(x.float())
    diff = (y.float() - y32).abs()
    assert diff.max().item() < 5e-2 and (diff / (y32.abs() + 1e-8)).max().item() < 0.02


@pytest.mark.parametrize("B,T", [(8, 4096), (32, 2048), (32, 4096)])
def test_rmsnorm_reference_largest_shapes(exts, dev, B, T):
    """The reference test's largest shapes (B up to 32, T up to 4096, D=2048,
    tests/test_rmsnorm.py:63-65), inputs drawn on the GPU; the same
    float32 formula evaluated by torch on the GPU as the reference: at most one
    bf16 ulp apart, and the reference test's own bar against nn.RMSNorm."""
    D = 2048
    g = torch.Generator(device=dev).manual_seed(B * 13 + T)
    x = torch.randn(B * T, D, generator=g, device=dev).bfloat16()
    gamma = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).bfloat16()
    y = exts["rmsnorm"].forward(x, gamma, 1e-6, 256, 2)
    xf = x.float()
    y32 = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + 1e-6) * gamma.float()
    torch.testing.assert_close(y.float(), y32.bfloat16().float(), rtol=2 ** -7, atol=1e-6)
    diff = (y.float() - y32).abs()
    assert diff.max().item() < 5e-2 and (diff / (y32.abs() + 1e-8)).max().item() < 0.02


@pytest.mark.parametrize("D", [8, 64, 1000 - 1000 % 8, 4096, 16384])
def test_rmsnorm_generic_D(exts, dev, D):
    g = torch.Generator().manual_seed(D)
    x = (3 * torch.randn(37, D, generator=g)).bfloat16()
    gamma = torch.randn(D, generator=g).bfloat16()
    y = exts["rmsnorm"].forward(x.to(dev), gamma.to(dev), 1e-5, 64, 1).cpu()
    torch.testing.assert_close(y.float(), ref_rmsnorm(x, gamma, 1e-5).float(), rtol=2 ** -7, atol=1e-6)


def test_rmsnorm_rejects_bad_D(exts, dev):
    x = torch.zeros(2, 12, device=dev, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        exts["rmsnorm"].forward(x, torch.ones(12, device=dev, dtype=torch.bfloat16), 1e-6, 256, 2)


def _proj_case(B, T, D, Dout, ck=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g).bfloat16()
    W = (torch.randn(Dout, D, generator=g) * D ** -0.5).bfloat16()
    cw = (torch.randn(Dout, ck, generator=g) * 0.5).bfloat16()
    return x, W, cw


@pytest.mark.parametrize("B,T,Dout", [(1, 1, 2048), (1, 64, 2048), (4, 128, 2048), (4, 256, 2048),
                                      (1, 1, 4096), (4, 64, 4096), (4, 128, 4096)])
def test_proj_reference_shapes(exts, dev, B, T, Dout):
    x, W, cw = _proj_case(B, T, 2048, Dout, seed=B * 1000 + T + Dout)
    y = exts["proj"].forward(x.to(dev), W.to(dev), cw.to(dev)).cpu()
    assert y.shape == (B, T, Dout) and y.dtype == torch.bfloat16
    assert_out_close(y, ref_proj_conv_silu_f32(x, W, cw))
    # The reference's bf16-rounded oracle differs from the fp32 composition by up to a
    # bf16 ulp of |y| (0.0625 at |y| ~ 8), so its absolute 5e-2 bound gets a relative term.
    assert_out_close(y, ref_proj_conv_silu(x, W, cw), atol=5e-2, rtol=2e-2)


@pytest.mark.parametrize("T", [2, 3, 124, 125, 126, 250, 251, 1000])
def test_proj_tile_boundaries(exts, dev, T):
    """125-token tiles with a 3-token halo: outputs across tile edges must see the previous tile's tokens."""
    x, W, cw = _proj_case(2, T, 256, 128, seed=T)
    y = exts["proj"].forward(x.to(dev), W.to(dev), cw.to(dev)).cpu()
    assert_out_close(y, ref_proj_conv_silu_f32(x, W, cw))


@pytest.mark.parametrize("ck", [1, 2, 3, 4])
@pytest.mark.parametrize("Dout", [48, 2080])
def test_proj_conv_taps_and_ragged_Dout(exts, dev, ck, Dout):
    x, W, cw = _proj_case(3, 140, 192, Dout, ck=ck, seed=ck + Dout)
    y = exts["proj"].forward(x.to(dev), W.to(dev), cw.to(dev)).cpu()
    assert_out_close(y, ref_proj_conv_silu_f32(x, W, cw))


@pytest.mark.parametrize("B,T", [(1, 253), (1, 254), (2, 253), (1, 509), (3, 300), (5, 131), (64, 1), (40, 2),
                                 (30, 3), (9, 57)])
def test_proj_flattened_token_tiles(exts, dev, B, T):
    """The MFMA kernel tiles the flattened B*T token axis in 256-row tiles with 253
    outputs: tile edges at multiples of 253, sequence starts inside a tile (their
    taps must not reach into the previous sequence) and the hand-over between the
    two 128-token waves of a tile (local tokens 128..130)."""
    x, W, cw = _proj_case(B, T, 128, 160, seed=B * 7 + T)
    y = exts["proj"].forward(x.to(dev), W.to(dev), cw.to(dev)).cpu()
    assert_out_close(y, ref_proj_conv_silu_f32(x, W, cw))


def _in_proj_expected(x, W, cw, H, dk, dv, caches):
    """fp32 composition of the fused in-projection with conv caches: the conv runs
    over cache ++ P (cache = projections of the 3 tokens before t = 0)."""
    from oracle.proj_ref import ref_conv1d
    B, T, _ = x.shape
    nc = cw.shape[1] - 1
    Hk, Hv = H * dk, H * dv
    P = x.float() @ W.float().T
    C = 2 * Hk + Hv
    prefix = torch.cat(caches, 1).float().transpose(1, 2) if caches is not None else torch.zeros(B, nc, C)
    ext = torch.cat([prefix, P[..., :C]], 1)
    y = torch.nn.functional.silu(ref_conv1d(ext, cw.float())[:, nc:]).bfloat16()
    hm = lambda t, d: t.reshape(B, T, H, d).transpose(1, 2)
    outs = [hm(y[..., :Hk], dk), hm(y[..., Hk:2 * Hk], dk), hm(y[..., 2 * Hk:C], dv),
            P[..., C:C + H].bfloat16().transpose(1, 2), P[..., C + H:].bfloat16().transpose(1, 2)]
    tail = ext[:, -nc:].bfloat16().transpose(1, 2)  # [B, C, nc]
    return outs, [tail[:, :Hk], tail[:, Hk:2 * Hk], tail[:, 2 * Hk:]]


# H = 2 leaves the b group at column 2 H dk + H dv + H = 162 (not on a 4-column
# boundary): the tiled kernel runs; H = 4 puts every group on one: the MFMA kernel.
@pytest.mark.parametrize("H", [2, 4])
@pytest.mark.parametrize("B,T", [(3, 1), (2, 3), (2, 5), (5, 70), (2, 300)])
@pytest.mark.parametrize("with_cache", [False, True])
def test_in_proj_matches_fp32_composition(dev, H, B, T, with_cache):
    from gdn_18646_amd import native_extension
    lay = native_extension().layer
    dk, dv, D, ck = 32, 16, 128, 4
    g = torch.Generator().manual_seed(H * 100 + B * 10 + T + int(with_cache))
    Dout = 2 * H * dk + H * dv + 2 * H
    x = torch.randn(B, T, D, generator=g).bfloat16()
    W = (torch.randn(Dout, D, generator=g) * D ** -0.5).bfloat16()
    cw = (torch.randn(Dout - 2 * H, ck, generator=g) * 0.5).bfloat16()
    caches = None
    if with_cache:
        caches = [torch.randn(B, H * d, ck - 1, generator=g).bfloat16() for d in (dk, dk, dv)]
    want = _in_proj_expected(x, W, cw, H, dk, dv, caches)
    cd = [c.to(dev) for c in caches] if caches is not None else [None] * 3
    got = lay.in_proj(x.to(dev), W.to(dev), cw.to(dev), H, dk, dv, *cd, True)
    for name, y, r in zip("qkvab", got[:5], want[0]):
        assert_out_close(y.cpu(), r, what=name)
    for name, y, r in zip(("cache_q", "cache_k", "cache_v"), got[5:], want[1]):
        assert_out_close(y.cpu(), r, atol=1e-2, rtol=1e-2, what=name)


# Decode-step projections (B <= 16).  D = 96 leaves five of the eight waves
# without K steps; D = 2048 / H = 16 is the layer's shape; D = 4096 runs the
# 16-step variant (x for 16 rows fills 128 KiB of LDS); conv width 1 has no
# cache and no x_n history.
@pytest.mark.parametrize("B", [1, 4, 16])
@pytest.mark.parametrize("H,dk,dv,D,ck", [(2, 32, 16, 128, 4), (4, 32, 16, 96, 3), (2, 32, 16, 256, 2),
                                          (16, 128, 128, 2048, 4), (2, 32, 16, 4096, 4), (2, 32, 16, 128, 1)])
def test_decode_in_proj_matches_composition(exts, dev, B, H, dk, dv, D, ck):
    from gdn_18646_amd import native_extension
    lay = native_extension().layer
    g = torch.Generator().manual_seed(B * 1000 + D + ck)
    Dout = 2 * H * dk + H * dv + 2 * H
    x = torch.randn(B, D, generator=g).bfloat16()
    gamma = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    W = (torch.randn(Dout, D, generator=g) * D ** -0.5).bfloat16()
    cw = (torch.randn(Dout - 2 * H, ck, generator=g) * 0.5).bfloat16()
    caches = [torch.randn(B, H * d, ck - 1, generator=g).bfloat16() for d in (dk, dk, dv)]
    hist = torch.randn(B, ck - 1, D, generator=g).bfloat16()
    # x_n is the RMSNorm kernel's output bit for bit
    xn = exts["rmsnorm"].forward(x.to(dev), gamma.to(dev), 1e-6, 256, 2).cpu()
    assert_out_close(xn, ref_rmsnorm(x, gamma), what="rmsnorm")
    want, want_cache = _in_proj_expected(xn.reshape(B, 1, D), W, cw, H, dk, dv, caches)
    cd, hd = [c.to(dev) for c in caches], hist.to(dev)
    got = lay.decode_in_proj(x.to(dev), gamma.to(dev), 1e-6, W.to(dev), cw.to(dev), *cd, hd, H, dk, dv)
    for name, y, r in zip("qkvab", got, want):
        assert_out_close(y.cpu(), r.reshape(y.shape), what=name)
    if ck == 1:
        return
    for name, y, r in zip(("cache_q", "cache_k", "cache_v"), cd, want_cache):
        assert_out_close(y.cpu(), r, atol=1e-2, rtol=1e-2, what=name)
    assert torch.equal(hd.cpu(), torch.cat([hist[:, 1:], xn[:, None]], 1)), "x_n history"


@pytest.mark.parametrize("B,K,N", [(1, 2048, 2048), (4, 2048, 2048), (16, 128, 256), (3, 96, 40), (7, 4096, 100)])
def test_decode_out_proj_matches_composition(dev, B, K, N):
    from gdn_18646_amd import native_extension
    lay = native_extension().layer
    g = torch.Generator().manual_seed(B + K + N)
    o = torch.randn(B, K, generator=g)
    W = (torch.randn(N, K, generator=g) * K ** -0.5).bfloat16()
    want = (o.bfloat16().float() @ W.float().T).bfloat16()
    assert_out_close(lay.decode_out_proj(o.to(dev), W.to(dev)).cpu(), want, what="out proj")
    with pytest.raises(RuntimeError, match="B=17"):
        lay.decode_out_proj(torch.zeros(17, K, device=dev), W.to(dev))



# Packed in-projection (gdn_in_proj_varlen_hip): one launch of the MFMA kernel
# per run of up to 256 sequences, whose row space holds every sequence's 3
# cache rows and tokens back to back.  Each output row is the same dot product
# as in a launch of that sequence alone, so the result must equal, bit for bit,
# the batch entry point run on every sequence by itself (its own cache in, its
# cache out).  Cases: config 4's lengths at config 5's dims; empty and 1..3
# token sequences (shorter than the conv window, so the new cache takes cache
# rows); conv width 2 without caches in; 300 sequences (two launches).
@pytest.mark.parametrize("lengths,H,dk,dv,D,ck,with_cache", [
    ([3670, 1053, 3636, 3547, 4688, 709, 2874, 4497], 16, 128, 128, 2048, 4, True),
    ([0, 1, 2, 5, 0, 300, 64, 3, 0], 4, 32, 16, 128, 4, True),
    ([1, 2, 3, 250, 0, 17], 4, 32, 16, 128, 2, False),
    ([7] * 150 + [0, 1] * 75, 4, 32, 16, 128, 4, True),
])
def test_in_proj_packed_one_launch_matches_per_sequence(dev, lengths, H, dk, dv, D, ck, with_cache):
    from gdn_18646_amd import native_extension
    lay = native_extension().layer
    N = len(lengths)
    print(f"packed in_proj case N={N} T_total={sum(lengths)} H={H} D={D} conv {ck}", flush=True)
    g = torch.Generator().manual_seed(N * 7 + D + ck)
    Dout = 2 * H * dk + H * dv + 2 * H
    Tt = sum(lengths)
    cu = torch.tensor([0] + lengths).cumsum(0).to(torch.int32)
    x = torch.randn(Tt, D, generator=g).bfloat16().to(dev)
    W = (torch.randn(Dout, D, generator=g) * D ** -0.5).bfloat16().to(dev)
    cw = (torch.randn(Dout - 2 * H, ck, generator=g) * 0.5).bfloat16().to(dev)
    caches = [None] * 3
    if with_cache:
        caches = [torch.randn(N, H * d, ck - 1, generator=g).bfloat16().to(dev) for d in (dk, dk, dv)]
    got = lay.in_proj_varlen(x, W, cw, H, dk, dv, cu, *caches, True)
    torch.cuda.synchronize()
    for i in range(N):
        t0, t1 = int(cu[i]), int(cu[i + 1])
        cin = [c[i:i + 1] if c is not None else None for c in caches]
        if t1 == t0:  # an empty sequence keeps its cache (zeros without one)
            for name, y, c in zip(("cache_q", "cache_k", "cache_v"), got[5:], cin):
                want = c[0] if c is not None else torch.zeros_like(y[i])
                assert torch.equal(y[i], want), f"sequence {i} (empty): {name}"
            continue
        ref = lay.in_proj(x[t0:t1].unsqueeze(0), W, cw, H, dk, dv, *cin, True)
        for name, y, r in zip("qkvab", got[:5], ref[:5]):
            assert torch.equal(y[:, :, t0:t1], r), f"sequence {i} (length {t1 - t0}): {name}"
        for name, y, r in zip(("cache_q", "cache_k", "cache_v"), got[5:], ref[5:]):
            assert torch.equal(y[i], r[0]), f"sequence {i} (length {t1 - t0}): {name}"
