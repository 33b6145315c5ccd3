// Layer-level entry points around the GDN hot path.
//
// gdn_in_proj_hip — one GEMM for the q/k/v/a/b in-projection of a prefill
// (x_n W^T with W = [W_q; W_k; W_v; W_a; W_b]), conv + SiLU applied to the
// q/k/v columns only, outputs written head-major ([B, H, T, d] and [B, H, T])
// as the prefill kernel reads them, and the causal-conv cache handed to decode.
// The reference runs three projection launches, two torch GEMMs and five
// transpose copies for this (gdn_layer.py:240-252).
//
// gdn_decode_conv_step_hip — the one-token conv step of decode over a cache of
// the last conv_k-1 projected tokens (the reference baseline's semantics,
// gdn_layer.py:43-55), fused with SiLU and the split into the decode kernel's
// q/k/v/a/b layouts.  The reference's custom layer instead re-ran the fused
// projection over a 4-token window of cached inputs (gdn_layer.py:58-69).
#include "gdn_common.hpp"
#include "proj.hpp"

namespace {

using namespace gdn;

struct ConvStepParams {
    const uint16_t* P;       // [B, Dp] projections of the new token
    const uint16_t* conv_w;  // [2 H dk + H dv, conv_k]
    uint16_t* cache[3];      // q, k, v: [B, width, conv_k - 1], updated in place
    uint16_t* dst[5];        // q, k [B, H dk]; v [B, H dv]; a, b [B, H]
    int col0[5];
    int width[5];
    int B, Dp, conv_k;
};

__global__ __launch_bounds__(256) void gdn_decode_conv_step_kernel(ConvStepParams p) {
    const long long idx = blockIdx.x * 256ll + threadIdx.x;
    if (idx >= static_cast<long long>(p.B) * p.Dp) return;
    const int b = static_cast<int>(idx / p.Dp);
    const int c = static_cast<int>(idx % p.Dp);
    int gi = 0;
#pragma unroll
    for (int q = 1; q < 5; ++q)
        if (c >= p.col0[q]) gi = q;
    const int cc = c - p.col0[gi];
    const float pn = bf2f(p.P[idx]);
    float y;
    if (gi < 3) {
        const int nc = p.conv_k - 1;
        uint16_t* cache = p.cache[gi] + (static_cast<size_t>(b) * p.width[gi] + cc) * nc;
        const uint16_t* w = p.conv_w + static_cast<size_t>(c) * p.conv_k;
        float s = bf2f(w[nc]) * pn;
        float win[3];
        for (int j = 0; j < nc; ++j) {
            win[j] = bf2f(cache[j]);
            s += bf2f(w[j]) * win[j];
        }
        for (int j = 0; j + 1 < nc; ++j) cache[j] = f2bf_bits(win[j + 1]);
        if (nc > 0) cache[nc - 1] = p.P[idx];
        y = s / (1.f + expf(-s));
    } else {
        y = pn;
    }
    p.dst[gi][static_cast<size_t>(b) * p.width[gi] + cc] = f2bf_bits(y);
}

}  // namespace

extern "C" int gdn_in_proj_hip(const gdn_bf16_t* xn, const gdn_bf16_t* W_qkvab, const gdn_bf16_t* conv_w_qkv,
                               const gdn_bf16_t* cache_q_in, const gdn_bf16_t* cache_k_in,
                               const gdn_bf16_t* cache_v_in, gdn_bf16_t* cache_q_out, gdn_bf16_t* cache_k_out,
                               gdn_bf16_t* cache_v_out, gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a,
                               gdn_bf16_t* b, int B, int T, int D, int H, int dk, int dv, int conv_k,
                               void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (B < 0 || T < 0 || D <= 0 || H <= 0 || dk <= 0 || dv <= 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj: B=%d T=%d D=%d H=%d dk=%d dv=%d", B, T, D, H, dk, dv);
    if (D % 64 != 0) return fail(GDN_ERR_UNSUPPORTED, "in_proj: D=%d must be a multiple of 64", D);
    if (conv_k < 1 || conv_k > 4) return fail(GDN_ERR_UNSUPPORTED, "in_proj: conv_k=%d must be in 1..4", conv_k);
    if (B == 0 || T == 0) return GDN_OK;
    if (!xn || !W_qkvab || !conv_w_qkv || !q || !k || !v || !a || !b)
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj: null pointer argument");
    if (!aligned(xn, 16) || !aligned(W_qkvab, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj: xn/W need 16-byte alignment");
    if ((cache_q_out && (cache_q_out == cache_q_in)) || (cache_k_out && (cache_k_out == cache_k_in)) ||
        (cache_v_out && (cache_v_out == cache_v_in)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj: conv caches in and out must not alias");
    gdn_proj::ProjParams p = {};
    p.x = xn;
    p.W = W_qkvab;
    p.conv_w = conv_w_qkv;
    p.B = B;
    p.T = T;
    p.D = D;
    const int Hk = H * dk, Hv = H * dv;
    p.D_out = 2 * Hk + Hv + 2 * H;
    p.conv_k = conv_k;
    p.ngroups = 5;
    p.groups[0] = gdn_proj::ProjGroup{0, Hk, dk, 1, 0, q, cache_q_in, cache_q_out};
    p.groups[1] = gdn_proj::ProjGroup{Hk, Hk, dk, 1, Hk, k, cache_k_in, cache_k_out};
    p.groups[2] = gdn_proj::ProjGroup{2 * Hk, Hv, dv, 1, 2 * Hk, v, cache_v_in, cache_v_out};
    p.groups[3] = gdn_proj::ProjGroup{2 * Hk + Hv, H, 1, 0, 0, a, nullptr, nullptr};
    p.groups[4] = gdn_proj::ProjGroup{2 * Hk + Hv + H, H, 1, 0, 0, b, nullptr, nullptr};
    return gdn_proj::launch_proj(p, static_cast<hipStream_t>(stream));
}

extern "C" int gdn_decode_conv_step_hip(const gdn_bf16_t* P, const gdn_bf16_t* conv_w_qkv, gdn_bf16_t* cache_q,
                                        gdn_bf16_t* cache_k, gdn_bf16_t* cache_v, gdn_bf16_t* q, gdn_bf16_t* k,
                                        gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b, int B, int H, int dk, int dv,
                                        int conv_k, void* stream) {
    using gdn_host::fail;
    if (B < 0 || H <= 0 || dk <= 0 || dv <= 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_conv_step: B=%d H=%d dk=%d dv=%d", B, H, dk, dv);
    if (conv_k < 1 || conv_k > 4)
        return fail(GDN_ERR_UNSUPPORTED, "decode_conv_step: conv_k=%d must be in 1..4", conv_k);
    if (B == 0) return GDN_OK;
    if (!P || !conv_w_qkv || !q || !k || !v || !a || !b || (conv_k > 1 && (!cache_q || !cache_k || !cache_v)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_conv_step: null pointer argument");
    ConvStepParams p = {};
    p.P = P;
    p.conv_w = conv_w_qkv;
    p.cache[0] = cache_q;
    p.cache[1] = cache_k;
    p.cache[2] = cache_v;
    p.dst[0] = q;
    p.dst[1] = k;
    p.dst[2] = v;
    p.dst[3] = a;
    p.dst[4] = b;
    const int Hk = H * dk, Hv = H * dv;
    const int col0[5] = {0, Hk, 2 * Hk, 2 * Hk + Hv, 2 * Hk + Hv + H};
    const int width[5] = {Hk, Hk, Hv, H, H};
    for (int i = 0; i < 5; ++i) {
        p.col0[i] = col0[i];
        p.width[i] = width[i];
    }
    p.B = B;
    p.Dp = 2 * Hk + Hv + 2 * H;
    p.conv_k = conv_k;
    const long long n = static_cast<long long>(B) * p.Dp;
    hipLaunchKernelGGL(gdn_decode_conv_step_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p);
    return gdn_host::check_launch("gdn_decode_conv_step_kernel");
}
