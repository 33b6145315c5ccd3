// RMSNorm for bf16 rows of any D % 8 == 0 (D <= 16384).
//
// Reference: kernels/rmsnorm.cu:17-103 (one 32-lane warp per row, D = 2048
// fixed, scalar 2-byte loads) and reference/rmsnorm_ref.py:8-28 for the math:
//   y = bf16((x * rsqrt(mean(x^2) + eps)) * gamma), all in fp32.
// Here one wave64 owns a row; each lane moves 16-byte chunks (8 bf16), the
// row stays in VGPRs between the sum of squares and the scaling, so x is read
// once and y written once.  One row per 64-thread workgroup up to 1024 rows,
// else four rows per 256-thread workgroup.
//
// The decode step's launch (gdn_host::rmsnorm_launch with a history) also
// moves the row's x_n history [R, nc, D] one token older and appends y: each
// lane shifts the chunks it owns, so the update is in place.
#include "gdn_common.hpp"

namespace {

using namespace gdn;


template <int CHUNKS>  // 16-byte chunks per lane
__global__ __launch_bounds__(256) void gdn_rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ gamma,
                                                          uint16_t* __restrict__ y, int R, int D, float eps,
                                                          uint16_t* __restrict__ hist, int nc) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= R) return;
    const int nch = D >> 3;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + static_cast<size_t>(row) * D);
    u32x4* const hrow = hist ? reinterpret_cast<u32x4*>(hist + static_cast<size_t>(row) * nc * D) : nullptr;
    // History entries 1 .. nc - 1 (nc <= 3) of the lane's chunks load with x,
    // so the shift below does not wait for a load per store.
    constexpr bool kHoldHist = CHUNKS <= 8;
    u32x4 hv[kHoldHist ? CHUNKS : 1][2];
    if (kHoldHist && hrow) {
#pragma unroll
        for (int u = 0; u < (kHoldHist ? CHUNKS : 1); ++u) {
            const int c = lane + 64 * u;
#pragma unroll
            for (int j = 1; j < 3; ++j)
                if (j < nc && c < nch) hv[u][j - 1] = hrow[j * nch + c];
        }
    }
    u32x4 xv[CHUNKS];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < CHUNKS; ++u) {
        const int c = lane + 64 * u;
        xv[u] = c < nch ? xr[c] : u32x4{0u, 0u, 0u, 0u};
        float f[8];
        unpack8(xv[u], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
    }
    const float inv = 1.f / sqrtf(wave_sum_dpp(ss) / static_cast<float>(D) + eps);
    const u32x4* gr = reinterpret_cast<const u32x4*>(gamma);
    u32x4* yr = reinterpret_cast<u32x4*>(y + static_cast<size_t>(row) * D);
#pragma unroll
    for (int u = 0; u < CHUNKS; ++u) {
        const int c = lane + 64 * u;
        if (c < nch) {
            float f[8], gm[8];
            unpack8(xv[u], f);
            unpack8(gr[c], gm);
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o[e] = pack2_bf16((f[2 * e] * inv) * gm[2 * e], (f[2 * e + 1] * inv) * gm[2 * e + 1]);
            }
            yr[c] = o;
            if (hrow) {
                u32x4* const h = hrow + c;
                if constexpr (kHoldHist) {
                    if (nc > 1) h[0] = hv[u][0];
                    if (nc > 2) h[nch] = hv[u][1];
                } else {
                    for (int j = 0; j + 1 < nc; ++j) h[j * nch] = h[(j + 1) * nch];
                }
                h[(nc - 1) * nch] = o;
            }
        }
    }
}

}  // namespace

int gdn_host::rmsnorm_launch(const void* x, const void* gamma, void* y, void* hist, int nc, int R, int D, float eps,
                             hipStream_t s) {
    if (nc < 0 || nc > 3) return gdn_host::fail(GDN_ERR_UNSUPPORTED, "rmsnorm: history of %d tokens, at most 3", nc);
    // Up to a few hundred rows (a decode step's batch), one row per
    // workgroup spreads them over more CUs; else four rows a workgroup.
    const int rows_per_wg = R <= 1024 ? 1 : 4;
    const dim3 grid((R + rows_per_wg - 1) / rows_per_wg), block(64 * rows_per_wg);
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* gp = static_cast<const uint16_t*>(gamma);
    auto* yp = static_cast<uint16_t*>(y);
    auto* hp = nc > 0 ? static_cast<uint16_t*>(hist) : nullptr;
    const int nch = D / 8;
    if (nch <= 64 * 4)
        hipLaunchKernelGGL(gdn_rmsnorm_kernel<4>, grid, block, 0, s, xp, gp, yp, R, D, eps, hp, nc);
    else if (nch <= 64 * 8)
        hipLaunchKernelGGL(gdn_rmsnorm_kernel<8>, grid, block, 0, s, xp, gp, yp, R, D, eps, hp, nc);
    else if (nch <= 64 * 16)
        hipLaunchKernelGGL(gdn_rmsnorm_kernel<16>, grid, block, 0, s, xp, gp, yp, R, D, eps, hp, nc);
    else
        hipLaunchKernelGGL(gdn_rmsnorm_kernel<32>, grid, block, 0, s, xp, gp, yp, R, D, eps, hp, nc);
    return gdn_host::check_launch("gdn_rmsnorm_kernel");
}

extern "C" int gdn_rmsnorm_hip(const gdn_bf16_t* x, const gdn_bf16_t* gamma, gdn_bf16_t* y, int R, int D,
                               float eps, void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (R < 0 || D <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "rmsnorm: R=%d D=%d", R, D);
    if (D % 8 != 0 || D > 16384) return fail(GDN_ERR_UNSUPPORTED, "rmsnorm: D=%d must be a multiple of 8, <= 16384", D);
    if (R == 0) return GDN_OK;
    if (!x || !gamma || !y) return fail(GDN_ERR_INVALID_ARGUMENT, "rmsnorm: null pointer argument");
    if (!aligned(x, 16) || !aligned(gamma, 16) || !aligned(y, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "rmsnorm: buffers need 16-byte alignment");
    return gdn_host::rmsnorm_launch(x, gamma, y, nullptr, 0, R, D, eps, static_cast<hipStream_t>(stream));
}
