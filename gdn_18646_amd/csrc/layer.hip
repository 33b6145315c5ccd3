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
//
// gdn_decode_in_proj_hip / gdn_decode_out_proj_hip — a decode step's two
// projections for up to 16 sequences, where the step is bound by streaming
// the weights (25 MB and 8 MB at the layer's shape) and a library GEMM with
// 4 rows reaches a fraction of HBM bandwidth.  Each workgroup owns 16 weight
// rows and splits K over 8 waves, every lane loading its 16-byte B fragments
// straight from memory; the rows of x (or o) are the MFMA A operand padded to
// 16.  The in-projection also recomputes RMSNorm of x (same order of
// operations as gdn_rmsnorm_kernel), keeps x_n W^T in fp32 for the conv step
// + SiLU (as the prefill in-projection does), updates the conv caches and
// the x_n history in place, and writes q/k/v/a/b in the decode kernel's
// layouts; the out-projection rounds o to bf16 as it loads it.
#include <algorithm>

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
    const uint16_t* xn;      // [B, D] (with xn_hist): the new token's x_n
    uint16_t* xn_hist;       // [B, conv_k - 1, D] (nullable): shifted by one token, x_n appended
    int D;
};

// Grid: x over Dp + D columns (D only with a history), y = sequence.  Column
// c < Dp: conv step + SiLU of P's column c (q/k/v) or the plain value (a/b);
// column Dp + d: the x_n history of feature d moves one token older and takes
// x_n[d] as the newest (each thread shifts one feature, so in place is safe).
__global__ __launch_bounds__(256) void gdn_decode_conv_step_kernel(ConvStepParams p) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    const int nc = p.conv_k - 1;
    if (c >= p.Dp) {
        const int d = c - p.Dp;
        if (!p.xn_hist || d >= p.D || nc == 0) return;
        uint16_t* h = p.xn_hist + static_cast<size_t>(b) * nc * p.D + d;
        for (int j = 0; j + 1 < nc; ++j) h[static_cast<size_t>(j) * p.D] = h[static_cast<size_t>(j + 1) * p.D];
        h[static_cast<size_t>(nc - 1) * p.D] = p.xn[static_cast<size_t>(b) * p.D + d];
        return;
    }
    int gi = 0;
#pragma unroll
    for (int q = 1; q < 5; ++q)
        if (c >= p.col0[q]) gi = q;
    const int cc = c - p.col0[gi];
    const size_t idx = static_cast<size_t>(b) * p.Dp + c;
    const float pn = bf2f(p.P[idx]);
    float y;
    if (gi < 3) {
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


// ---------------------------------------------------------------------------
// Decode-step projections for B <= 16 (one token per sequence).
//
// A step streams the whole weight matrix once, so the kernel is built to keep
// HBM busy: each lane's weight loads for all its K steps are issued at the
// start and are the only data held in VGPRs while they fly (at most 128
// VGPRs with MAXSTEPS <= 8, two 8-wave workgroups per CU: the in-projection's
// ~390 workgroups are resident at once).  The in-projection's x and gamma go
// to LDS by DMA before the weight loads, so RMSNorm runs while the weights
// are still in flight.
// ---------------------------------------------------------------------------
constexpr int kSkM = 16;     // A-operand rows: sequences (rows past B repeat row B - 1, outputs discarded)
constexpr int kSkWaves = 8;  // K split over the waves of a workgroup
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkMaxCols = 16;  // weight rows (output columns) per workgroup: 16, or 8 to spread small N
constexpr int kSkStride = 32 * kSkWaves;  // K elements between a wave's consecutive steps
constexpr int kSkCUs = 256;
constexpr int kStepMaxB = 64;  // gdn_layer_decode_step_hip: sequences, as groups of kSkM

struct SkinnyParams {
    const uint16_t* W;  // [N, K]
    int B, K, N, cols;
    const uint16_t* x;  // in-projection: x [B, K], normalised here
    const uint16_t* gamma;
    float eps;
    const float* o;     // out-projection: o [B, K] fp32
    uint16_t* y;        // out-projection: y [B, N]
    const uint16_t* conv_w;  // in-projection epilogue: conv over the caches for groups 0..2
    int conv_k;
    uint16_t* cache[3];      // [B, width, conv_k - 1], oldest first, updated in place
    uint16_t* dst[5];        // [B, width]
    int col0[5];
    int width[5];
    uint16_t* xn_hist;       // [B, conv_k - 1, K] (nullable): shifted, x_n appended
};

// In-projection LDS (dynamic): x [B, K] bf16 rounded up to 1 KB plus a 1 KB
// tail, then gamma (MAXSTEPS * 512 bytes).
__host__ __device__ inline size_t skinny_x_bytes(int B, int K) { return (static_cast<size_t>(B) * K * 2 + 1023) / 1024 * 1024; }

// The output group (q, k, v, a, b) of the workgroup's columns, as a uniform
// value.  The host guarantees that the q, k and v widths are multiples of the
// workgroup's column count, so only the a and b columns can share a
// workgroup; those take group 3 here and pick a or b per lane.  Selecting
// group descriptors with a uniform index keeps them in scalar registers
// (a per-lane select between kernel arguments becomes a vector load from the
// argument block, and its wait also waits for every weight load in flight).
__device__ __forceinline__ int skinny_wg_group(const SkinnyParams& p, int n0) {
    return n0 >= p.col0[3] ? 3 : n0 >= p.col0[2] ? 2 : n0 >= p.col0[1] ? 1 : 0;
}

// MODE 0: in-projection, MODE 1: out-projection.  Wave w takes the 32-wide
// K steps w, w + 8, w + 16, ...: nsteps of them.  All MAXSTEPS step slots run;
// a slot past the wave's last step multiplies finite values by zero weights.
template <int MODE, int MAXSTEPS>
__global__ __launch_bounds__(kSkThreads)
__attribute__((amdgpu_waves_per_eu(MAXSTEPS <= 8 ? 4 : 2, MAXSTEPS <= 8 ? 4 : 2)))
void gdn_decode_skinny_kernel(SkinnyParams p) {
    extern __shared__ __attribute__((aligned(1024))) unsigned char s_dyn[];
    __shared__ float s_inv[kSkM];
    __shared__ float s_red[kSkWaves][64][4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g4 = lane >> 4;
    const int n0 = blockIdx.x * p.cols;
    const int ksteps = p.K / 32;
    const int nsteps = (ksteps - wave + kSkWaves - 1) / kSkWaves;
    const int kl = 32 * wave + 8 * g4;  // this lane's first K element
    const bool arow = r16 < p.B;
    // Lanes past B (A rows) or past the workgroup's columns (B columns) read a
    // valid row, or zeros: they feed only MFMA output rows / columns that the
    // epilogue discards.
    const int arow_ld = min(r16, p.B - 1);
    // Lane offset past any buffer: the range check (which always covers the
    // lane offset) turns the load into zeros.
    constexpr uint32_t kPast = 0x80000000u;

    lds_u8* const s_x = (lds_u8*)&s_dyn[0];
    const uint32_t xbytes = static_cast<uint32_t>(p.B) * p.K * 2;
    const uint32_t xregion = static_cast<uint32_t>(skinny_x_bytes(p.B, p.K));
    lds_u8* const s_gamma = s_x + xregion + 1024;
    if constexpr (MODE == 0) {
        // x and gamma -> LDS by DMA, 1 KB per wave instruction (lanes past the
        // end re-read the last 16 bytes); the 1 KB after x and the gamma slots
        // past 2 K are zero-filled, so padded step slots read finite values.
        for (uint32_t c = wave; c * 1024 < xregion; c += kSkWaves)
            dma16(p.x, min(c * 1024 + 16 * lane, xbytes - 16), s_x + c * 1024);
        if (wave == kSkWaves - 1) *reinterpret_cast<lds_u32x4*>(s_x + xregion + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
        const int gbytes = 2 * p.K;
        if (wave < MAXSTEPS / 2) {
            if (wave * 1024 < gbytes)
                dma16(p.gamma, static_cast<uint32_t>(min(wave * 1024 + 16 * lane, gbytes - 16)), s_gamma + wave * 1024);
            else
                *reinterpret_cast<lds_u32x4*>(s_gamma + wave * 1024 + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
        }
    }

    bf16x8 af[MAXSTEPS];
    const int er = tid >> 4, ec = tid & 15, en = n0 + ec;
    const bool eown = tid < kSkM * kSkMaxCols && er < p.B && ec < p.cols && en < p.N;
    int egi = 0;
    uint16_t* ecache = nullptr;
    const int nc = p.conv_k - 1, sh = 4 - p.conv_k;
    // in-projection epilogue inputs, raw bf16 (converted where used, after
    // the products, so no wait for them lands before the weight loads issue):
    // kEpiLoads loads, all unconditional
    constexpr int kEpiLoads = 9;
    uint16_t rt0 = 0, rt1 = 0, rt2 = 0, rt3 = 0, ru0 = 0, ru1 = 0, ru2 = 0;
    u32x4 hold1 = {0u, 0u, 0u, 0u}, hold2 = {0u, 0u, 0u, 0u};
    const int hstep = blockIdx.x;
    const bool hown = MODE == 0 && p.xn_hist && nc > 0 && hstep < ksteps && wave == hstep % kSkWaves;
    uint16_t* const hrow = p.xn_hist + static_cast<size_t>(arow_ld) * nc * p.K + 32 * hstep + 8 * g4;
    if constexpr (MODE == 0) {
        // Epilogue ownership: thread t < 256 computes output (row t / 16,
        // column n0 + t % 16).  Its conv taps and cache window load first
        // (from clamped, valid positions; small loads issued behind the
        // weight loads would wait for a queue full of them), right-aligned in
        // four slots: slot 3 = the new token, slots 0..2 = the cached tokens,
        // oldest first; slots before 4 - conv_k hold zero weight and input.
        const int er_ld = min(er, p.B - 1), en_ld = min(en, p.N - 1);
        const int wgi = __builtin_amdgcn_readfirstlane(skinny_wg_group(p, n0));
        egi = wgi < 3 ? wgi : (en_ld >= p.col0[4] ? 4 : 3);
        const int cgi = wgi < 3 ? wgi : 0;  // a/b columns read column 0's entries, unused
        const int ccol = wgi < 3 ? en_ld : 0;
        const uint16_t* wrow = p.conv_w + static_cast<size_t>(ccol) * p.conv_k;
        uint16_t* const cbase = cgi == 0 ? p.cache[0] : cgi == 1 ? p.cache[1] : p.cache[2];
        const int cwidth = cgi == 0 ? p.width[0] : cgi == 1 ? p.width[1] : p.width[2];
        const int ccol0 = cgi == 0 ? p.col0[0] : cgi == 1 ? p.col0[1] : p.col0[2];
        ecache = cbase + (static_cast<size_t>(er_ld) * cwidth + (ccol - ccol0)) * nc;
        const uint16_t* cread = nc > 0 ? ecache : wrow;  // conv_k == 1: no cache
        rt0 = wrow[max(0 - sh, 0)];
        rt1 = wrow[max(1 - sh, 0)];
        rt2 = wrow[max(2 - sh, 0)];
        rt3 = wrow[3 - sh];
        ru0 = cread[max(0 - sh, 0)];
        ru1 = cread[max(1 - sh, 0)];
        ru2 = cread[max(2 - sh, 0)];
        // x_n history: workgroup b shifts and appends K step b (wave b % 8,
        // slot b / 8); the grid has at least K / 32 workgroups (extra ones own
        // no columns).  The entries it moves load now (unconditionally, from
        // x where there is nothing to move: a conditional load would merge
        // registers across a branch and wait).
        hold1 = *reinterpret_cast<const u32x4*>(hown && nc > 1 ? hrow + p.K : p.x);
        hold2 = *reinterpret_cast<const u32x4*>(hown && nc > 2 ? hrow + 2 * p.K : p.x);
    }

    // Weight rows n0 + lane % 16 (B operand): one buffer load per step slot
    // (rows past N and slots past the last step read zeros).
    const auto wrs = buffer_rsrc(p.W + static_cast<size_t>(min(n0, p.N)) * p.K,
                                 static_cast<uint32_t>(max(0, min(p.cols, p.N - n0))) * p.K * 2);
    const uint32_t wvoff = static_cast<uint32_t>(min(r16, p.cols - 1) * p.K + kl) * 2;
    u32x4 bw[MAXSTEPS];
#pragma unroll
    for (int s = 0; s < MAXSTEPS; ++s) bw[s] = buffer_load16(wrs, s < nsteps ? wvoff : kPast, 2 * kSkStride * s);

    if constexpr (MODE == 0) {
        // The DMA has landed (the kEpiLoads epilogue loads and the MAXSTEPS
        // weight loads issued after it may still be in flight).  Barriers
        // here order LDS only: a full __syncthreads() fence would also wait
        // for the loads.
        wait_vm<MAXSTEPS + kEpiLoads>();
        lds_barrier();
        // RMSNorm statistics in gdn_rmsnorm_kernel's order (a lane sums its
        // 16-byte chunks lane + 64 u, then wave_sum_dpp), so x_n equals that
        // kernel's output bit for bit.
        for (int m = wave; m < p.B; m += kSkWaves) {
            float ss = 0.f;
            for (int c = lane; c < p.K / 8; c += 64) {
                float f[8];
                unpack8(*reinterpret_cast<const lds_u32x4*>(s_x + (m * p.K + 8 * c) * 2), f);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
            }
            ss = wave_sum_dpp(ss);
            if (lane == 0) s_inv[m] = 1.f / sqrtf(ss / static_cast<float>(p.K) + p.eps);
        }
        lds_barrier();

        // A operand x_n = bf16((x * inv) * gamma), as gdn_rmsnorm_kernel.
        const float inv = s_inv[arow_ld];
        const lds_u8* xrow = s_x + (arow_ld * p.K + kl) * 2;
#pragma unroll
        for (int s = 0; s < MAXSTEPS; ++s) {
            float f[8], gm[8];
            unpack8(*reinterpret_cast<const lds_u32x4*>(xrow + 2 * kSkStride * s), f);
            unpack8(*reinterpret_cast<const lds_u32x4*>(s_gamma + 2 * (kl + kSkStride * s)), gm);
            af[s] = as_bf16x8(u32x4{pack2_bf16((f[0] * inv) * gm[0], (f[1] * inv) * gm[1]),
                                    pack2_bf16((f[2] * inv) * gm[2], (f[3] * inv) * gm[3]),
                                    pack2_bf16((f[4] * inv) * gm[4], (f[5] * inv) * gm[5]),
                                    pack2_bf16((f[6] * inv) * gm[6], (f[7] * inv) * gm[7])});
        }
        if (hown && arow) {
            const int hs = hstep / kSkWaves;
            u32x4 xn = as_u32x4(af[0]);
#pragma unroll
            for (int s = 1; s < MAXSTEPS; ++s)
                if (s == hs) xn = as_u32x4(af[s]);
            if (nc > 1) *reinterpret_cast<u32x4*>(hrow) = hold1;
            if (nc > 2) *reinterpret_cast<u32x4*>(hrow + static_cast<size_t>(p.K)) = hold2;
            *reinterpret_cast<u32x4*>(hrow + static_cast<size_t>(nc - 1) * p.K) = xn;
        }
    } else {
        const auto ors = buffer_rsrc(p.o, static_cast<uint32_t>(p.B) * p.K * 4);
        const uint32_t ovoff = static_cast<uint32_t>(arow_ld * p.K + kl) * 4;
#pragma unroll
        for (int s = 0; s < MAXSTEPS; ++s) {
            const uint32_t vo = s < nsteps ? ovoff : kPast;
            af[s] = pack8(__builtin_bit_cast(f32x4, buffer_load16(ors, vo, 4 * kSkStride * s)),
                          __builtin_bit_cast(f32x4, buffer_load16(ors, vo + 16, 4 * kSkStride * s)));
        }
    }

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < MAXSTEPS; ++s) acc = mfma16x16x32(af[s], as_bf16x8(bw[s]), acc);
    // acc: column n0 + lane % 16, rows 4 (lane / 16) + i.
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[wave][lane][i] = acc[i];
    lds_barrier();
    if (!eown) return;
    float P = 0.f;
#pragma unroll
    for (int w = 0; w < kSkWaves; ++w) P += s_red[w][(er >> 2) * 16 + ec][er & 3];
    if constexpr (MODE == 1) {
        p.y[static_cast<size_t>(er) * p.N + en] = f2bf_bits(P);
    } else {
        float y = P;
        if (egi < 3) {
            const float ws0 = sh <= 0 ? bf2f(rt0) : 0.f, ws1 = sh <= 1 ? bf2f(rt1) : 0.f;
            const float ws2 = sh <= 2 ? bf2f(rt2) : 0.f, ws3 = bf2f(rt3);
            const float cs0 = sh <= 0 ? bf2f(ru0) : 0.f, cs1 = sh <= 1 ? bf2f(ru1) : 0.f;
            const float cs2 = sh <= 2 ? bf2f(ru2) : 0.f;
            float sc = ws3 * P;
            sc += ws0 * cs0;
            sc += ws1 * cs1;
            sc += ws2 * cs2;
            // shift: entry e takes slot sh + e + 1, the last entry the new token
            if (nc == 3) {
                ecache[0] = f2bf_bits(cs1);
                ecache[1] = f2bf_bits(cs2);
            } else if (nc == 2) {
                ecache[0] = f2bf_bits(cs2);
            }
            if (nc > 0) ecache[nc - 1] = f2bf_bits(P);
            y = silu_f(sc);
        }
        // uniform selects, then the per-lane a / b choice between two scalars
        const int wgi = __builtin_amdgcn_readfirstlane(skinny_wg_group(p, n0));
        uint16_t* dbase = wgi == 0 ? p.dst[0] : wgi == 1 ? p.dst[1] : wgi == 2 ? p.dst[2] : p.dst[3];
        int dw = wgi == 0 ? p.width[0] : wgi == 1 ? p.width[1] : wgi == 2 ? p.width[2] : p.width[3];
        int dc = wgi == 0 ? p.col0[0] : wgi == 1 ? p.col0[1] : wgi == 2 ? p.col0[2] : p.col0[3];
        if (egi == 4) {
            dbase = p.dst[4];
            dw = p.width[4];
            dc = p.col0[4];
        }
        dbase[static_cast<size_t>(er) * dw + (en - dc)] = f2bf_bits(y);
    }
}

// Weight rows per workgroup: 16, or 8 when 16 would leave CUs idle.
inline int skinny_cols(int N) { return (N + 15) / 16 >= kSkCUs ? 16 : 8; }

template <int MODE>
int launch_skinny(SkinnyParams& p, hipStream_t st, const char* who) {
    p.cols = skinny_cols(p.N);
    // the in-projection's grid also covers the K / 32 slices of the x_n history
    const dim3 grid(max((p.N + p.cols - 1) / p.cols, MODE == 0 ? p.K / 32 : 0));
    const bool small = p.K <= kSkStride * 8;
    const size_t lds = MODE == 0 ? skinny_x_bytes(p.B, p.K) + 1024 + kSkStride * (small ? 8 : 16) * 2 : 0;
    if (small)
        hipLaunchKernelGGL((gdn_decode_skinny_kernel<MODE, 8>), grid, dim3(kSkThreads), lds, st, p);
    else
        hipLaunchKernelGGL((gdn_decode_skinny_kernel<MODE, 16>), grid, dim3(kSkThreads), lds, st, p);
    return gdn_host::check_launch(who);
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

namespace {
__global__ void gdn_zero_u16_kernel(uint16_t* __restrict__ p, size_t n) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[i] = 0;
}
}  // namespace

extern "C" int gdn_in_proj_varlen_hip(const gdn_bf16_t* xn, const gdn_bf16_t* W_qkvab, const gdn_bf16_t* conv_w_qkv,
                                      const int32_t* cu_seqlens, int num_seqs, const gdn_bf16_t* cache_q_in,
                                      const gdn_bf16_t* cache_k_in, const gdn_bf16_t* cache_v_in,
                                      gdn_bf16_t* cache_q_out, gdn_bf16_t* cache_k_out, gdn_bf16_t* cache_v_out,
                                      gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b,
                                      int T_total, int D, int H, int dk, int dv, int conv_k, void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (num_seqs < 0 || T_total < 0 || D <= 0 || H <= 0 || dk <= 0 || dv <= 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: num_seqs=%d T_total=%d D=%d H=%d dk=%d dv=%d", num_seqs,
                    T_total, D, H, dk, dv);
    if (D % 64 != 0) return fail(GDN_ERR_UNSUPPORTED, "in_proj_varlen: D=%d must be a multiple of 64", D);
    if (conv_k < 1 || conv_k > 4)
        return fail(GDN_ERR_UNSUPPORTED, "in_proj_varlen: conv_k=%d must be in 1..4", conv_k);
    if (num_seqs == 0) return GDN_OK;
    if (!cu_seqlens) return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: null cu_seqlens");
    if (cu_seqlens[0] != 0 || cu_seqlens[num_seqs] != T_total)
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: cu_seqlens must run from 0 to T_total=%d", T_total);
    for (int i = 0; i < num_seqs; ++i)
        if (cu_seqlens[i + 1] < cu_seqlens[i])
            return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: cu_seqlens must be non-decreasing (at %d)", i);
    if (T_total > 0 && (!xn || !W_qkvab || !conv_w_qkv || !q || !k || !v || !a || !b))
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: null pointer argument");
    if ((cache_q_out && (cache_q_out == cache_q_in)) || (cache_k_out && (cache_k_out == cache_k_in)) ||
        (cache_v_out && (cache_v_out == cache_v_in)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: conv caches in and out must not alias");
    const int Hk = H * dk, Hv = H * dv, nc = conv_k - 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto cin = [&](const gdn_bf16_t* c, int i, int width) {
        return c ? c + static_cast<size_t>(i) * width * nc : nullptr;
    };
    auto cout = [&](gdn_bf16_t* c, int i, int width) { return c ? c + static_cast<size_t>(i) * width * nc : nullptr; };
    // Parameters for sequences [i, i + 1) ... starting at packed token t0.
    auto params = [&](int i, int t0) {
        gdn_proj::ProjParams p = {};
        p.x = xn + static_cast<size_t>(t0) * D;
        p.W = W_qkvab;
        p.conv_w = conv_w_qkv;
        p.T_out = T_total;
        p.D = D;
        p.D_out = 2 * Hk + Hv + 2 * H;
        p.conv_k = conv_k;
        p.ngroups = 5;
        p.groups[0] = gdn_proj::ProjGroup{0, Hk, dk, 1, 0, q + static_cast<size_t>(t0) * dk, cin(cache_q_in, i, Hk),
                                          cout(cache_q_out, i, Hk)};
        p.groups[1] = gdn_proj::ProjGroup{Hk, Hk, dk, 1, Hk, k + static_cast<size_t>(t0) * dk, cin(cache_k_in, i, Hk),
                                          cout(cache_k_out, i, Hk)};
        p.groups[2] = gdn_proj::ProjGroup{2 * Hk, Hv, dv, 1, 2 * Hk, v + static_cast<size_t>(t0) * dv,
                                          cin(cache_v_in, i, Hv), cout(cache_v_out, i, Hv)};
        p.groups[3] = gdn_proj::ProjGroup{2 * Hk + Hv, H, 1, 0, 0, a + t0, nullptr, nullptr};
        p.groups[4] = gdn_proj::ProjGroup{2 * Hk + Hv + H, H, 1, 0, 0, b + t0, nullptr, nullptr};
        return p;
    };
    // Sequence i on its own (a launch of its tokens, or the cache hand-over of
    // an empty sequence).
    auto one_seq = [&](int i) -> int {
        const int t0 = cu_seqlens[i], len = cu_seqlens[i + 1] - t0;
        if (len == 0) {
            // An empty sequence keeps its conv history (zeros without one).
            const struct { const gdn_bf16_t* in; gdn_bf16_t* out; int width; } caches[3] = {
                {cin(cache_q_in, i, Hk), cout(cache_q_out, i, Hk), Hk},
                {cin(cache_k_in, i, Hk), cout(cache_k_out, i, Hk), Hk},
                {cin(cache_v_in, i, Hv), cout(cache_v_out, i, Hv), Hv}};
            for (const auto& c : caches) {
                if (!c.out || nc == 0) continue;
                const size_t bytes = static_cast<size_t>(c.width) * nc * 2;
                if (c.in) {
                    if (hipMemcpyAsync(c.out, c.in, bytes, hipMemcpyDeviceToDevice, st) != hipSuccess)
                        return fail(GDN_ERR_HIP, "in_proj_varlen: cache copy failed");
                } else {
                    // a fill kernel, not a memset node, so the call stays safe to capture
                    hipLaunchKernelGGL(gdn_zero_u16_kernel, dim3(64), dim3(256), 0, st, c.out, bytes / 2);
                    const int rc = gdn_host::check_launch("gdn_zero_u16_kernel");
                    if (rc != GDN_OK) return rc;
                }
            }
            return GDN_OK;
        }
        gdn_proj::ProjParams p = params(i, t0);
        if (!aligned(p.x, 16) || !aligned(W_qkvab, 16))
            return fail(GDN_ERR_INVALID_ARGUMENT, "in_proj_varlen: xn/W need 16-byte alignment");
        p.B = 1;
        p.T = len;
        return gdn_proj::launch_proj(p, st);
    };
    // One launch of the MFMA kernel per run of up to kPackMax sequences: its
    // row space holds every sequence's 3 cache rows and tokens back to back,
    // so short sequences share tiles and no launch waits for another.  A run
    // with no tokens (only empty sequences), or a shape the MFMA kernel does
    // not take, goes sequence by sequence.
    for (int i = 0; i < num_seqs;) {
        const int j = std::min(num_seqs, i + gdn_proj::kPackMax);
        const int t0 = cu_seqlens[i], t1 = cu_seqlens[j];
        gdn_proj::ProjParams p = params(i, t0);
        p.B = 1;
        p.T = t1 - t0;
        p.packed = j - i;
        for (int s = 0; s <= j - i; ++s) p.row_off[s] = cu_seqlens[i + s] - t0 + gdn_proj::kCacheRows * s;
        if (t1 > t0 && aligned(p.x, 16) && gdn_proj::mfma_path_ok(p)) {
            const int rc = gdn_proj::launch_proj(p, st);
            if (rc != GDN_OK) return rc;
        } else {
            for (int s = i; s < j; ++s) {
                const int rc = one_seq(s);
                if (rc != GDN_OK) return rc;
            }
        }
        i = j;
    }
    return GDN_OK;
}

extern "C" int gdn_decode_conv_step_hip(const gdn_bf16_t* P, const gdn_bf16_t* conv_w_qkv, gdn_bf16_t* cache_q,
                                        gdn_bf16_t* cache_k, gdn_bf16_t* cache_v, const gdn_bf16_t* xn,
                                        gdn_bf16_t* xn_hist, gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v,
                                        gdn_bf16_t* a, gdn_bf16_t* b, int B, int D, int H, int dk, int dv, int conv_k,
                                        void* stream) {
    using gdn_host::fail;
    if (B < 0 || H <= 0 || dk <= 0 || dv <= 0 || (xn_hist && D <= 0))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_conv_step: B=%d H=%d dk=%d dv=%d D=%d", B, H, dk, dv, D);
    if (conv_k < 1 || conv_k > 4)
        return fail(GDN_ERR_UNSUPPORTED, "decode_conv_step: conv_k=%d must be in 1..4", conv_k);
    if (B > 65535) return fail(GDN_ERR_UNSUPPORTED, "decode_conv_step: B=%d, at most 65535 sequences", B);
    if (B == 0) return GDN_OK;
    if (!P || !conv_w_qkv || !q || !k || !v || !a || !b || (conv_k > 1 && (!cache_q || !cache_k || !cache_v)) ||
        (xn_hist && conv_k > 1 && !xn))
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
    p.xn = xn;
    p.xn_hist = conv_k > 1 ? xn_hist : nullptr;
    p.D = xn_hist ? D : 0;
    const int ncols = p.Dp + p.D;
    hipLaunchKernelGGL(gdn_decode_conv_step_kernel, dim3((ncols + 255) / 256, B), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p);
    return gdn_host::check_launch("gdn_decode_conv_step_kernel");
}

namespace {

// Argument checks of the decode-step projections: GDN_OK when the call would
// launch (or, for B == 0, do nothing), else the error status.
int in_proj_check(const void* x, const void* gamma, const void* W_qkvab, const void* conv_w_qkv, const void* cache_q,
                  const void* cache_k, const void* cache_v, const void* q, const void* k, const void* v, const void* a,
                  const void* b, int B, int D, int H, int dk, int dv, int conv_k) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (B < 0 || D <= 0 || H <= 0 || dk <= 0 || dv <= 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_in_proj: B=%d D=%d H=%d dk=%d dv=%d", B, D, H, dk, dv);
    if (B > kSkM) return fail(GDN_ERR_UNSUPPORTED, "decode_in_proj: B=%d, at most %d sequences", B, kSkM);
    if (D % 32 != 0 || D > kSkStride * 16)
        return fail(GDN_ERR_UNSUPPORTED, "decode_in_proj: D=%d must be a multiple of 32, at most %d", D,
                    kSkStride * 16);
    if (conv_k < 1 || conv_k > 4) return fail(GDN_ERR_UNSUPPORTED, "decode_in_proj: conv_k=%d must be in 1..4", conv_k);
    if ((H * dk) % 16 != 0 || (H * dv) % 16 != 0)
        return fail(GDN_ERR_UNSUPPORTED, "decode_in_proj: H dk=%d and H dv=%d must be multiples of 16", H * dk, H * dv);
    if (B == 0) return GDN_OK;
    if (!x || !gamma || !W_qkvab || !conv_w_qkv || !q || !k || !v || !a || !b ||
        (conv_k > 1 && (!cache_q || !cache_k || !cache_v)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_in_proj: null pointer argument");
    if (!aligned(x, 16) || !aligned(gamma, 16) || !aligned(W_qkvab, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_in_proj: x/gamma/W need 16-byte alignment");
    return GDN_OK;
}

int out_proj_check(const void* o, const void* W_o, const void* y, int B, int K, int N) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (B < 0 || K <= 0 || N <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "decode_out_proj: B=%d K=%d N=%d", B, K, N);
    if (B > kSkM) return fail(GDN_ERR_UNSUPPORTED, "decode_out_proj: B=%d, at most %d sequences", B, kSkM);
    if (K % 32 != 0 || K > kSkStride * 16)
        return fail(GDN_ERR_UNSUPPORTED, "decode_out_proj: K=%d must be a multiple of 32, at most %d", K,
                    kSkStride * 16);
    if (B == 0) return GDN_OK;
    if (!o || !W_o || !y) return fail(GDN_ERR_INVALID_ARGUMENT, "decode_out_proj: null pointer argument");
    if (!aligned(o, 16) || !aligned(W_o, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_out_proj: o/W need 16-byte alignment");
    return GDN_OK;
}

}  // namespace

extern "C" int gdn_decode_in_proj_hip(const gdn_bf16_t* x, const gdn_bf16_t* gamma, float eps,
                                      const gdn_bf16_t* W_qkvab, const gdn_bf16_t* conv_w_qkv, gdn_bf16_t* cache_q,
                                      gdn_bf16_t* cache_k, gdn_bf16_t* cache_v, gdn_bf16_t* xn_hist, gdn_bf16_t* q,
                                      gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b, int B, int D, int H,
                                      int dk, int dv, int conv_k, void* stream) {
    const int chk = in_proj_check(x, gamma, W_qkvab, conv_w_qkv, cache_q, cache_k, cache_v, q, k, v, a, b, B, D, H,
                                  dk, dv, conv_k);
    if (chk != GDN_OK || B == 0) return chk;
    SkinnyParams p = {};
    p.W = W_qkvab;
    p.B = B;
    p.K = D;
    const int Hk = H * dk, Hv = H * dv;
    p.N = 2 * Hk + Hv + 2 * H;
    p.x = x;
    p.gamma = gamma;
    p.eps = eps;
    p.conv_w = conv_w_qkv;
    p.conv_k = conv_k;
    p.cache[0] = cache_q;
    p.cache[1] = cache_k;
    p.cache[2] = cache_v;
    uint16_t* dst[5] = {q, k, v, a, b};
    const int col0[5] = {0, Hk, 2 * Hk, 2 * Hk + Hv, 2 * Hk + Hv + H};
    const int width[5] = {Hk, Hk, Hv, H, H};
    for (int i = 0; i < 5; ++i) {
        p.dst[i] = dst[i];
        p.col0[i] = col0[i];
        p.width[i] = width[i];
    }
    p.xn_hist = xn_hist;
    return launch_skinny<0>(p, static_cast<hipStream_t>(stream), "gdn_decode_skinny_kernel<in>");
}

extern "C" int gdn_decode_out_proj_hip(const float* o, const gdn_bf16_t* W_o, gdn_bf16_t* y, int B, int K, int N,
                                       void* stream) {
    const int chk = out_proj_check(o, W_o, y, B, K, N);
    if (chk != GDN_OK || B == 0) return chk;
    SkinnyParams p = {};
    p.W = W_o;
    p.B = B;
    p.K = K;
    p.N = N;
    p.o = o;
    p.y = y;
    return launch_skinny<1>(p, static_cast<hipStream_t>(stream), "gdn_decode_skinny_kernel<out>");
}

extern "C" int gdn_layer_decode_step_hip(const gdn_bf16_t* x, const gdn_bf16_t* gamma, float eps,
                                         const gdn_bf16_t* W_qkvab, const gdn_bf16_t* conv_w_qkv, gdn_bf16_t* cache_q,
                                         gdn_bf16_t* cache_k, gdn_bf16_t* cache_v, gdn_bf16_t* xn_hist,
                                         const float* A_log, const float* dt_bias, const float* S_in, float* S_out,
                                         float scale, const gdn_bf16_t* W_o, gdn_bf16_t* q, gdn_bf16_t* k,
                                         gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b, float* o, gdn_bf16_t* y, int B,
                                         int D, int H, int dk, int dv, int conv_k, void* stream) {
    // Every stage's arguments are checked before the first launch: the
    // in-projection updates the conv caches and x_n history in place, so a
    // later stage refusing its arguments would leave the state half-advanced.
    // Up to kStepMaxB sequences run as groups of kSkM: one in- and one
    // out-projection launch per group (each streams the weights once more),
    // one recurrence launch for all; the groups' row offsets keep every
    // pointer's alignment, so checking the first group covers them all.
    if (B < 0 || B > kStepMaxB)
        return gdn_host::fail(B < 0 ? GDN_ERR_INVALID_ARGUMENT : GDN_ERR_UNSUPPORTED,
                              "decode_step: B=%d, at most %d sequences", B, kStepMaxB);
    const int B0 = std::min(B, kSkM);
    int st = in_proj_check(x, gamma, W_qkvab, conv_w_qkv, cache_q, cache_k, cache_v, q, k, v, a, b, B0, D, H, dk, dv,
                           conv_k);
    if (st == GDN_OK) st = gdn_host::decode_check(q, k, v, a, b, A_log, dt_bias, S_in, o, S_out, B, H, dk, dv);
    if (st == GDN_OK) st = out_proj_check(o, W_o, y, B0, H * dv, D);
    if (st != GDN_OK || B == 0) return st;
    const int nc = conv_k - 1;
    const size_t Hk = static_cast<size_t>(H) * dk, Hv = static_cast<size_t>(H) * dv;
    auto off = [](auto* ptr, size_t n) { return ptr ? ptr + n : ptr; };
    for (int r0 = 0; r0 < B; r0 += kSkM) {
        const int Bg = std::min(kSkM, B - r0);
        const size_t r = static_cast<size_t>(r0);
        st = gdn_decode_in_proj_hip(x + r * D, gamma, eps, W_qkvab, conv_w_qkv, off(cache_q, r * Hk * nc),
                                    off(cache_k, r * Hk * nc), off(cache_v, r * Hv * nc),
                                    off(xn_hist, r * nc * D), q + r * Hk, k + r * Hk, v + r * Hv, a + r * H,
                                    b + r * H, Bg, D, H, dk, dv, conv_k, stream);
        if (st != GDN_OK) return st;
    }
    st = gdn_decode_hip(q, k, v, a, b, A_log, dt_bias, S_in, scale, o, S_out, B, H, dk, dv, stream);
    if (st != GDN_OK) return st;
    for (int r0 = 0; r0 < B; r0 += kSkM) {
        const int Bg = std::min(kSkM, B - r0);
        const size_t r = static_cast<size_t>(r0);
        st = gdn_decode_out_proj_hip(o + r * Hv, W_o, y + r * D, Bg, static_cast<int>(Hv), D, stream);
        if (st != GDN_OK) return st;
    }
    return GDN_OK;
}
