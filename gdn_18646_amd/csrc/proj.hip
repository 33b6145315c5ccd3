// Projection GEMM + causal depthwise conv (<= 4 taps) + SiLU, bf16 MFMA.
//
// Reference: kernels/fused_proj_conv_silu.cu:105-295 (WMMA, 125-token tile +
// 3-token halo, cp.async pipeline) and reference/fused_proj_conv_silu_ref.py
// for the math.  P = x W^T is accumulated in fp32 and never rounded before the
// conv (as the reference kernel does; the PyTorch reference rounds P to bf16).
//
// Tiling: a workgroup computes a 128 x 128 tile of P whose 128 GEMM rows are
// the tokens t0-3 .. t0+124 of one sequence; the first 3 rows are the causal
// halo, recomputed instead of exchanged, and 125 outputs are produced.
// 4 waves in a 2 x 2 grid, each 64 x 64 = 4 x 4 MFMA 16x16x32 tiles; K steps
// of 64 staged through LDS with the next step prefetched into registers.
// The epilogue parks P in LDS (fp32) and applies conv + SiLU per column.
//
// Output routing: up to 5 column groups, each written either token-major
// [B, T, width] or head-major [B, width/hd, T, hd], with or without the
// conv + SiLU (a plain projection takes the current token's row of P).
#include "gdn_common.hpp"
#include "proj.hpp"

namespace {

using namespace gdn;

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kHalo = 3;
constexpr int kOutT = kBM - kHalo;  // 125 outputs per tile
constexpr int kLD = kBK + 8;        // padded LDS row, bf16
constexpr int kPLD = kBN + 4;       // padded LDS row, fp32 epilogue

__device__ __forceinline__ int group_of(const gdn_proj::ProjParams& p, int c) {
    int gi = 0;
#pragma unroll
    for (int q = 1; q < gdn_proj::kMaxGroups; ++q)
        if (q < p.ngroups && c >= p.groups[q].col0) gi = q;
    return gi;
}

__global__ __launch_bounds__(256, 2) void gdn_proj_conv_kernel(gdn_proj::ProjParams p) {
    const int tile_t = blockIdx.x, tile_c = blockIdx.y, b = blockIdx.z;
    const int t0 = tile_t * kOutT;
    const int c0 = tile_c * kBN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int m16 = lane & 15, g4 = lane >> 4;

    // Union: two K stages of A/B tiles, or the fp32 P tile in the epilogue.
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * 2 * kBM * kLD * 2 > kBM * kPLD * 4
                                                                 ? 2 * 2 * kBM * kLD * 2
                                                                 : kBM * kPLD * 4];
    bf16(*As)[kBM][kLD] = reinterpret_cast<bf16(*)[kBM][kLD]>(smem);
    bf16(*Bs)[kBM][kLD] = reinterpret_cast<bf16(*)[kBM][kLD]>(smem + 2 * kBM * kLD * 2);
    float(*Pt)[kPLD] = reinterpret_cast<float(*)[kPLD]>(smem);

    // Each thread moves 4 A chunks and 4 B chunks (16 B) per K step.
    u32x4 ra[4], rb[4];
    auto gload = [&](int k0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = tid + 256 * u;
            const int row = idx >> 3, c8 = (idx & 7) * 8;
            const int tok = t0 - kHalo + row;
            ra[u] = (tok >= 0 && tok < p.T)
                        ? *reinterpret_cast<const u32x4*>(p.x + (static_cast<size_t>(b) * p.T + tok) * p.D + k0 + c8)
                        : u32x4{0u, 0u, 0u, 0u};
            const int col = c0 + row;
            rb[u] = col < p.D_out ? *reinterpret_cast<const u32x4*>(p.W + static_cast<size_t>(col) * p.D + k0 + c8)
                                  : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = tid + 256 * u;
            const int row = idx >> 3, c8 = (idx & 7) * 8;
            *reinterpret_cast<u32x4*>(&As[st][row][c8]) = ra[u];
            *reinterpret_cast<u32x4*>(&Bs[st][row][c8]) = rb[u];
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = p.D / kBK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int st = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            bf16x8 af[4], bfr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(&As[st][64 * wm + 16 * i + m16][32 * s + 8 * g4]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[st][64 * wn + 16 * j + m16][32 * s + 8 * g4]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
        }
        if (kt + 1 < nk) lstore(st ^ 1);
        __syncthreads();
    }

    // Epilogue: P tile to LDS (the staging buffers are dead after the last barrier).
    // In the first tile, halo rows of tokens < 0 take the group's cached
    // projections when it has a cache (x rows there are zero, so P is 0).
    const int ncache = p.conv_k - 1;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = 64 * wm + 16 * i + 4 * g4 + e, col = 64 * wn + 16 * j + m16;
                float val = acc[i][j][e];
                if (t0 == 0 && row < kHalo && row >= kHalo - ncache && c0 + col < p.D_out) {
                    const gdn_proj::ProjGroup& gq = p.groups[group_of(p, c0 + col)];
                    if (gq.conv && gq.cache_in)
                        val = bf2f(gq.cache_in[(static_cast<size_t>(b) * gq.width + (c0 + col - gq.col0)) * ncache +
                                               (row - (kHalo - ncache))]);
                }
                Pt[row][col] = val;
            }
    __syncthreads();

    const int cl = tid & (kBN - 1);
    const int c = c0 + cl;
    if (c >= p.D_out) return;
    const gdn_proj::ProjGroup grp = p.groups[group_of(p, c)];
    const int cc = c - grp.col0;
    // The workgroup holding the last token refreshes the cache: bf16(P) of
    // tokens T-ncache .. T-1 (rows of negative tokens hold the old cache).
    if (grp.conv && grp.cache_out && tid < kBN && t0 + kOutT >= p.T) {
        for (int j = 0; j < ncache; ++j) {
            const int tok = p.T - ncache + j;
            grp.cache_out[(static_cast<size_t>(b) * grp.width + cc) * ncache + j] = f2bf_bits(Pt[tok - t0 + kHalo][cl]);
        }
    }
    float w[4] = {0.f, 0.f, 0.f, 0.f};
    if (grp.conv) {
        // Taps aligned to the right: tap conv_k-1 multiplies the current token.
        for (int j = 0; j < p.conv_k; ++j) w[4 - p.conv_k + j] = bf2f(p.conv_w[static_cast<size_t>(grp.cw_row0 + cc) * p.conv_k + j]);
    }
    for (int tl = tid >> 7; tl < kOutT; tl += 2) {
        const int t = t0 + tl;
        if (t >= p.T) break;
        float y;
        if (grp.conv) {
            const float s = w[0] * Pt[tl][cl] + w[1] * Pt[tl + 1][cl] + w[2] * Pt[tl + 2][cl] + w[3] * Pt[tl + 3][cl];
            y = s / (1.f + expf(-s));
        } else {
            y = Pt[tl + kHalo][cl];
        }
        size_t idx;
        if (grp.head_dim > 0) {
            const int hh = cc / grp.head_dim, dd = cc % grp.head_dim;
            idx = ((static_cast<size_t>(b) * (grp.width / grp.head_dim) + hh) * p.T + t) * grp.head_dim + dd;
        } else {
            idx = (static_cast<size_t>(b) * p.T + t) * grp.width + cc;
        }
        grp.dst[idx] = f2bf_bits(y);
    }
}

}  // namespace

namespace gdn_proj {

int launch_proj(const ProjParams& p, hipStream_t stream) {
    if (p.B == 0 || p.T == 0 || p.D_out == 0) return GDN_OK;
    const dim3 grid((p.T + kOutT - 1) / kOutT, (p.D_out + kBN - 1) / kBN, p.B);
    hipLaunchKernelGGL(gdn_proj_conv_kernel, grid, dim3(256), 0, stream, p);
    return gdn_host::check_launch("gdn_proj_conv_kernel");
}

}  // namespace gdn_proj

extern "C" int gdn_proj_conv_silu_hip(const gdn_bf16_t* x, const gdn_bf16_t* W, const gdn_bf16_t* conv_w,
                                      gdn_bf16_t* out, int B, int T, int D, int D_out, int conv_k, void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (B < 0 || T < 0 || D <= 0 || D_out <= 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "proj: B=%d T=%d D=%d D_out=%d", B, T, D, D_out);
    if (D % 64 != 0) return fail(GDN_ERR_UNSUPPORTED, "proj: D=%d must be a multiple of 64", D);
    if (D_out % 16 != 0) return fail(GDN_ERR_UNSUPPORTED, "proj: D_out=%d must be a multiple of 16", D_out);
    if (conv_k < 1 || conv_k > 4) return fail(GDN_ERR_UNSUPPORTED, "proj: conv_k=%d must be in 1..4", conv_k);
    if (B == 0 || T == 0) return GDN_OK;
    if (!x || !W || !conv_w || !out) return fail(GDN_ERR_INVALID_ARGUMENT, "proj: null pointer argument");
    if (!aligned(x, 16) || !aligned(W, 16)) return fail(GDN_ERR_INVALID_ARGUMENT, "proj: x/W need 16-byte alignment");
    gdn_proj::ProjParams p = {};
    p.x = x;
    p.W = W;
    p.conv_w = conv_w;
    p.B = B;
    p.T = T;
    p.D = D;
    p.D_out = D_out;
    p.conv_k = conv_k;
    p.ngroups = 1;
    p.groups[0] = gdn_proj::ProjGroup{0, D_out, 0, 1, 0, out, nullptr, nullptr};
    return gdn_proj::launch_proj(p, static_cast<hipStream_t>(stream));
}
