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
constexpr int kStepMaxB = 65535;     // gdn_layer_decode_step_hip: sequences

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

// ---------------------------------------------------------------------------
// Decode-step projections for larger batches: output tiles of 64 sequences x
// 32 or 64 weight rows on MFMA.  The out-projection (a 4x smaller weight
// matrix) always takes 32-wide tiles, the in-projection while the batch fits
// one row tile; both give twice the workgroups of 64-wide tiles (1.2-1.6 us
// less a decode step at config 5, B = 17..64) with bit-identical results.
//
// The skinny kernel streams the weights once per group of 16 sequences; here
// the row tiles of one weight tile are dispatched to the same XCD, so the
// weights cross HBM about once and the row tiles share them through that
// XCD's L2.  K moves through LDS in 64-wide slices, DMA'd into a ring of
// stages.  Eight waves: waves 0-3 take the first 32 K of every slice, waves
// 4-7 the second, each wave a 32 x TN/2 block of the tile; the two halves'
// sums meet in LDS at the end.  (A workgroup's load rate grows with its wave
// count -- measured from L2, 4 waves pull ~90 GB/s, 8 waves ~130 -- and the
// K split keeps LDS reads at one pass over each slice.)  In LDS, tile rows
// sit in 1 KB blocks with their 16-byte chunks XOR-swizzled, so the 16 lanes
// of an operand read (16 rows, one chunk) hit 16 different bank groups.
//
// The loop keeps the ring full: slice i's MFMAs run on fragments read from
// LDS during the previous iteration, while slice i + 1's fragments are read,
// and slice i's slot is refilled as soon as its fragments are in registers.
//
// MODE 0, the in-projection: A = x_n [B, K] bf16, W = [W_q; W_k; W_v; W_a;
// W_b].  P = x_n W^T stays fp32 for the conv step (as in the skinny kernel):
// q/k/v take SiLU(conv over the cached tokens and P), their caches shift one
// token in place, a and b take P.  MODE 1, the out-projection: A = o [B, K]
// as bf16 (the recurrence writes it rounded to nearest even, the rounding of
// the reference's o.to(bf16)); y = bf16(o W_o^T).
// ---------------------------------------------------------------------------
constexpr int kTlM = 64;    // sequences per tile
constexpr int kTlN = 64;    // weight rows (output columns) per in-projection tile (above kTlNarrowB sequences)
constexpr int kTlNarrowB = 64;  // up to this many sequences (one row tile) the in-projection takes 32-wide tiles
constexpr int kTlNOut = 32;  // ... per out-projection tile (twice the workgroups: W_o is a quarter of the weights)
constexpr int kTlK = 64;    // K per LDS stage
constexpr int kTlWaves = 8;
constexpr int kTlThreads = 64 * kTlWaves;

struct TileParams {
    const uint16_t* W;       // [N, K]
    int B, K, N;
    int mtiles, ntiles;
    const uint16_t* A;       // [B, K] bf16: x_n (MODE 0) or o (MODE 1)
    uint16_t* y;             // MODE 1: y [B, N] bf16
    const uint16_t* conv_w;  // MODE 0: [2 H dk + H dv, conv_k]
    int conv_k;
    uint16_t* cache[3];      // q, k, v: [B, width, conv_k - 1] bf16, oldest first, updated in place
    uint16_t* dst[5];        // q, k [B, H dk]; v [B, H dv]; a, b [B, H]
    int col0[5];
    int width[5];
};

// TN weight rows per tile: 64 (in-projection) or 32 (out-projection).
template <int MODE, int TN>
struct TileCfg {
    static constexpr int kABytes = kTlM * kTlK * 2;  // A slice of one stage
    static constexpr int kBBytes = TN * kTlK * 2;
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int kStages = 4;
    // A W slice of 32 rows is 4 KB: each wave copies 512 bytes with its
    // lanes 0..31, so every wave still issues one copy per slice and the
    // vmcnt waits stay the same on all waves.
    static constexpr int kBLanes = TN >= 64 ? 64 : 32;
    static constexpr int kADma = kABytes / (1024 * kTlWaves);  // 1 KB DMA instructions per wave per stage
    static constexpr int kBDma = kBBytes / (16 * kBLanes * kTlWaves);
    static constexpr int kDma = kADma + kBDma;
    static constexpr int kRingBytes = kStages * kStageBytes;
    static constexpr int kTapOff = kRingBytes;  // MODE 0: conv taps [TN][4] bf16, right-aligned
    static constexpr int kLdsBytes = kRingBytes + (MODE == 0 ? TN * 8 : 0);
    static constexpr int kNI = TN / 32;                     // 16-column fragments per wave
    static constexpr int kEC = kTlM * TN / kTlThreads;      // epilogue columns per thread (8 or 4)
    static constexpr int kPitch = TN + 4;                   // fp32 words per row of the epilogue's P tile
    static_assert(kTlM * kPitch * 4 <= kRingBytes, "the epilogue's P tile reuses the ring");
    static_assert(kADma >= 1 && kBDma >= 1, "every wave issues whole copies");
    static_assert(kBBytes % (16 * kBLanes * kTlWaves) == 0 && TN % 32 == 0, "W slice split over the waves");
    static_assert(kEC * 8 == TN, "epilogue: 8 threads a row");
};

// Byte offset in a stage of (row r, 16-byte chunk c) of a slice: 8 chunks a
// row, 8 rows a KB.
__device__ __forceinline__ uint32_t tl_off(int r, int c) {
    return (r >> 3) * 1024 + (r & 7) * 128 + ((c ^ ((r >> 1) & 7)) << 4);
}

template <int N>
struct U16Arr { uint16_t v[N]; };
template <int N>
struct U4Arr { u32x4 v[N]; };
template <typename T, int N>
struct VArr { T v[N]; };

// NC = conv_k - 1 (MODE 0; 0 for MODE 1); TN weight rows per tile.
template <int MODE, int NC, int TN>
__global__ __launch_bounds__(kTlThreads) void gdn_decode_tile_kernel(TileParams p) {
    using Cfg = TileCfg<MODE, TN>;
    constexpr int EC = Cfg::kEC, PITCH = Cfg::kPitch, NI = Cfg::kNI;
    __shared__ __attribute__((aligned(1024))) unsigned char s_tile[Cfg::kLdsBytes];
    lds_u8* const ring = (lds_u8*)&s_tile[0];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Tile of this workgroup: workgroup id i runs on XCD i % 8; the row tiles
    // of column tile nt are ids with the same i % 8, so they share one L2.
    const int id = blockIdx.x, xcd = id & 7, j8 = id >> 3;
    const int mt = j8 % p.mtiles, nt = xcd + 8 * (j8 / p.mtiles);
    if (nt >= p.ntiles) return;
    const int m0 = mt * kTlM, n0 = nt * TN;
    const int nk = p.K / kTlK;
    // K slice order: the tile starts at slice (n0 / 64) % nk, so the
    // workgroups are spread over the slices (and the memory channels that
    // hold them) rather than all on the same one; row tiles of one column
    // tile keep the same order and share its weight slices through L2.
    // Counted in 64-column blocks whatever the tile width, so every output
    // sums its K slices in the same order with 32- and 64-wide tiles and
    // both give bit-identical results.
    const int kstart = (n0 / 64) % nk;

    // Output group of the tile (uniform): q/k/v tiles never straddle groups
    // (their widths are multiples of TN); a and b share the tiles after v.
    const int g = MODE == 0 ? (n0 >= p.col0[3] ? 3 : n0 >= p.col0[2] ? 2 : n0 >= p.col0[1] ? 1 : 0) : 0;
    const bool conv_tile = MODE == 0 && g < 3;

    // Epilogue ownership: thread t takes row t / 8 of the tile, columns
    // EC (t % 8) .. + EC - 1.
    const int er = tid >> 3, ec0 = EC * (tid & 7);
    const int eb = m0 + er;
    const int eb_ld = min(eb, p.B - 1);

    // Conv-tile inputs load first and are held through the K loop: the
    // thread's cached tokens (EC NC bf16, contiguous) and, for threads
    // t < TN, the conv taps of column n0 + t.
    using CVec = std::conditional_t<EC == 8, u32x4, u32x2>;  // EC bf16
    CVec hold[NC > 0 ? NC : 1];
    uint16_t tap[4] = {0, 0, 0, 0};
    int cwidth = 0, ccol = 0;
    uint16_t* cbase = nullptr;
    if constexpr (MODE == 0) {
        if (conv_tile) {
            cbase = g == 0 ? p.cache[0] : g == 1 ? p.cache[1] : p.cache[2];
            cwidth = g == 0 ? p.width[0] : g == 1 ? p.width[1] : p.width[2];
            const int gc0 = g == 0 ? p.col0[0] : g == 1 ? p.col0[1] : p.col0[2];
            ccol = n0 - gc0 + ec0;
            if constexpr (NC > 0) {
                const auto crs = buffer_rsrc(cbase, static_cast<uint32_t>(p.B) * cwidth * NC * 2);
                const uint32_t voff = static_cast<uint32_t>((eb_ld * cwidth + ccol) * NC) * 2;
#pragma unroll
                for (int u = 0; u < NC; ++u) {
                    if constexpr (EC == 8)
                        hold[u] = buffer_load16(crs, voff, 16 * u);
                    else
                        hold[u] = __builtin_amdgcn_raw_buffer_load_b64(crs, voff, 8 * u, 0);
                }
            }
            if (tid < TN) {
                const uint16_t* wr = p.conv_w + static_cast<size_t>(n0 + tid) * (NC + 1);
#pragma unroll
                for (int e = 0; e <= NC; ++e) tap[3 - NC + e] = wr[e];
            }
        }
    }

    // DMA source offsets (bytes from the slice's first K column) of this
    // lane's chunk in its 1 KB blocks of A and of W.
    const uint16_t* const Wt = p.W + static_cast<size_t>(n0) * p.K;
    uint32_t aoff[Cfg::kADma], boff[Cfg::kBDma];
#pragma unroll
    for (int u = 0; u < Cfg::kBDma; ++u) {
        const int r = Cfg::kBLanes / 8 * (wave + kTlWaves * u) + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        boff[u] = static_cast<uint32_t>(min(r, p.N - 1 - n0) * p.K + 8 * c) * 2;
    }
#pragma unroll
    for (int u = 0; u < Cfg::kADma; ++u) {
        const int r = 8 * (wave + kTlWaves * u) + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        aoff[u] = static_cast<uint32_t>(min(m0 + r, p.B - 1) * p.K + 8 * c) * 2;
    }
    auto issue = [&](int ks, int slot) {
        lds_u8* const st = ring + slot * Cfg::kStageBytes;
        const int k0 = (ks + kstart < nk ? ks + kstart : ks + kstart - nk) * kTlK;
#pragma unroll
        for (int u = 0; u < Cfg::kADma; ++u) dma16(p.A + k0, aoff[u], st + (wave + kTlWaves * u) * 1024);
#pragma unroll
        for (int u = 0; u < Cfg::kBDma; ++u)
            if (Cfg::kBLanes == 64 || lane < Cfg::kBLanes)
                dma16(Wt + k0, boff[u], st + Cfg::kABytes + (wave + kTlWaves * u) * (16 * Cfg::kBLanes));
    };

    // wave = 4 kh + 2 wm + wn: K half kh of every slice, rows 32 wm, columns
    // TN / 2 wn (NI 16-column fragments)
    const int kh = wave >> 2, wm = (wave >> 1) & 1, wn = wave & 1;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int kc = 4 * kh + g4;  // the lane's 16-byte chunk of every slice row
    f32x4 acc[2][NI];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};
    // The wave's A and W fragments of the slice in `slot`.
    auto read_frags = [&](int slot, bf16x8* af, bf16x8* bw) {
        const lds_u8* const sa = ring + slot * Cfg::kStageBytes;
        const lds_u8* const sb = sa + Cfg::kABytes;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
            af[mi] = *reinterpret_cast<const lds_bf16x8*>(sa + tl_off(32 * wm + 16 * mi + r16, kc));
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
            bw[ni] = *reinterpret_cast<const lds_bf16x8*>(sb + tl_off(TN / 2 * wn + 16 * ni + r16, kc));
    };

    // Slices s go to slot s % S.  All S slots fill first; at iteration i
    // slice i + 1 is waited for (the slices issued after it may fly), slice
    // i's slot -- its fragments already in registers -- takes slice i + S,
    // and slice i + 1's fragments are read while slice i's MFMAs run.
    constexpr int S = Cfg::kStages;
#pragma unroll
    for (int s = 0; s < S; ++s)
        if (s < nk) issue(s, s);
    if (S <= nk)
        wait_vm<(S - 1) * Cfg::kDma>();
    else
        wait_vm<0>();
    lds_barrier();
    bf16x8 af[2], bw[NI];
    read_frags(0, af, bw);
    for (int i = 0; i < nk; ++i) {
        // Slice i + 1 has landed when at most the S - 2 slices issued after
        // it are in flight (fewer are issued near the end: wait for all).
        if (i + S - 1 < nk)
            wait_vm<(S - 2) * Cfg::kDma>();
        else
            wait_vm<0>();
        // Every wave's part of slice i + 1 is in LDS, and every wave has
        // slice i's fragments in registers (the barrier waits for its LDS
        // reads), so slice i's slot is free.
        lds_barrier();
        if (i + S < nk) issue(i + S, i % S);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma16x16x32(af[mi], bw[ni], acc[mi][ni]);
        // slice i + 1's fragments (past the last slice: a valid slot, unused)
        read_frags((i + 1) % S, af, bw);
    }

    // P tile [kTlM][PITCH] fp32 over the ring (every wave is past its
    // last read of it after the first barrier): the second K half's sums,
    // then the first half's added.
    lds_barrier();
    lds_f32* const ps = (lds_f32*)ring;
    auto ps_at = [&](int mi, int ni, int e) {
        return (32 * wm + 16 * mi + 4 * g4 + e) * PITCH + TN / 2 * wn + 16 * ni + r16;
    };
    if (kh == 1) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                for (int e = 0; e < 4; ++e) ps[ps_at(mi, ni, e)] = acc[mi][ni][e];
    }
    if constexpr (MODE == 0) {
        if (conv_tile && tid < TN)
            *reinterpret_cast<lds_u32x2*>(ring + Cfg::kTapOff + 8 * tid) =
                u32x2{static_cast<uint32_t>(tap[0]) | (static_cast<uint32_t>(tap[1]) << 16),
                      static_cast<uint32_t>(tap[2]) | (static_cast<uint32_t>(tap[3]) << 16)};
    }
    lds_barrier();
    if (kh == 0) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                for (int e = 0; e < 4; ++e) ps[ps_at(mi, ni, e)] = acc[mi][ni][e] + ps[ps_at(mi, ni, e)];
    }
    lds_barrier();
    if (eb >= p.B) return;
    float P[EC];
#pragma unroll
    for (int u = 0; u < EC / 4; ++u) {
        const f32x4 v = *reinterpret_cast<const lds_f32x4*>(ring + 4 * (er * PITCH + ec0 + 4 * u));
#pragma unroll
        for (int e = 0; e < 4; ++e) P[4 * u + e] = v[e];
    }
    if constexpr (MODE == 1) {
        if (n0 + ec0 >= p.N) return;
        uint16_t* const yo = p.y + static_cast<size_t>(eb) * p.N + n0 + ec0;
        if constexpr (EC == 8)
            *reinterpret_cast<u32x4*>(yo) = u32x4{pack2_bf16(P[0], P[1]), pack2_bf16(P[2], P[3]),
                                                  pack2_bf16(P[4], P[5]), pack2_bf16(P[6], P[7])};
        else
            *reinterpret_cast<u32x2*>(yo) = u32x2{pack2_bf16(P[0], P[1]), pack2_bf16(P[2], P[3])};
    } else if (!conv_tile) {
        // a / b columns: per column (the a | b boundary may fall inside the
        // thread's 8).
#pragma unroll
        for (int j = 0; j < EC; ++j) {
            const int n = n0 + ec0 + j;
            if (n < p.N) {
                const int gi = n >= p.col0[4] ? 4 : 3;
                uint16_t* const d = gi == 4 ? p.dst[4] : p.dst[3];
                const int w = gi == 4 ? p.width[4] : p.width[3];
                d[static_cast<size_t>(eb) * w + (n - (gi == 4 ? p.col0[4] : p.col0[3]))] = f2bf_bits(P[j]);
            }
        }
    } else {
        // Conv taps of the EC columns (4 bf16 each, right-aligned: slot 3
        // multiplies the new token, slots 3 - NC .. 2 the cached tokens,
        // oldest first).
        U16Arr<4 * EC> tp;
        {
            U4Arr<EC / 2> t4;
#pragma unroll
            for (int u = 0; u < EC / 2; ++u)
                t4.v[u] = *reinterpret_cast<const lds_u32x4*>(ring + Cfg::kTapOff + 8 * ec0 + 16 * u);
            tp = __builtin_bit_cast(U16Arr<4 * EC>, t4);
        }
        float yv[EC];
        U16Arr<(NC > 0 ? EC * NC : 1)> nwc;
        U16Arr<(NC > 0 ? EC * NC : 1)> old;
        if constexpr (NC > 0) {
            VArr<CVec, NC> h;
#pragma unroll
            for (int u = 0; u < NC; ++u) h.v[u] = hold[u];
            old = __builtin_bit_cast(U16Arr<EC * NC>, h);
        }
#pragma unroll
        for (int j = 0; j < EC; ++j) {
            float s = bf2f(tp.v[4 * j + 3]) * P[j];
#pragma unroll
            for (int e = 0; e < NC; ++e) s += bf2f(tp.v[4 * j + 3 - NC + e]) * bf2f(old.v[NC * j + e]);
#pragma unroll
            for (int e = 0; e + 1 < NC; ++e) nwc.v[NC * j + e] = old.v[NC * j + e + 1];
            if constexpr (NC > 0) nwc.v[NC * j + NC - 1] = f2bf_bits(P[j]);
            yv[j] = silu_f(s);
        }
        uint16_t* const d = g == 0 ? p.dst[0] : g == 1 ? p.dst[1] : p.dst[2];
        uint16_t* const dq = d + static_cast<size_t>(eb) * cwidth + ccol;
        if constexpr (EC == 8)
            *reinterpret_cast<u32x4*>(dq) = u32x4{pack2_bf16(yv[0], yv[1]), pack2_bf16(yv[2], yv[3]),
                                                  pack2_bf16(yv[4], yv[5]), pack2_bf16(yv[6], yv[7])};
        else
            *reinterpret_cast<u32x2*>(dq) = u32x2{pack2_bf16(yv[0], yv[1]), pack2_bf16(yv[2], yv[3])};
        if constexpr (NC > 0) {
            const VArr<CVec, NC> nw = __builtin_bit_cast(VArr<CVec, NC>, nwc);
            CVec* cq = reinterpret_cast<CVec*>(cbase + (static_cast<size_t>(eb) * cwidth + ccol) * NC);
#pragma unroll
            for (int u = 0; u < NC; ++u) cq[u] = nw.v[u];
        }
    }
}

template <int MODE, int TN>
void launch_tile_tn(TileParams& p, hipStream_t st) {
    p.mtiles = (p.B + kTlM - 1) / kTlM;
    p.ntiles = (p.N + TN - 1) / TN;
    const dim3 grid(p.mtiles * ((p.ntiles + 7) / 8) * 8);
    if constexpr (MODE == 1) {
        hipLaunchKernelGGL((gdn_decode_tile_kernel<1, 0, TN>), grid, dim3(kTlThreads), 0, st, p);
    } else {
        switch (p.conv_k - 1) {
            case 0: hipLaunchKernelGGL((gdn_decode_tile_kernel<0, 0, TN>), grid, dim3(kTlThreads), 0, st, p); break;
            case 1: hipLaunchKernelGGL((gdn_decode_tile_kernel<0, 1, TN>), grid, dim3(kTlThreads), 0, st, p); break;
            case 2: hipLaunchKernelGGL((gdn_decode_tile_kernel<0, 2, TN>), grid, dim3(kTlThreads), 0, st, p); break;
            default: hipLaunchKernelGGL((gdn_decode_tile_kernel<0, 3, TN>), grid, dim3(kTlThreads), 0, st, p); break;
        }
    }
}

// The out-projection always takes 32-wide tiles; the in-projection up to
// kTlNarrowB sequences (one row tile: 32-wide tiles double its workgroups,
// which still fit the CUs), 64-wide tiles above (with two row tiles, 32-wide
// tiles put two workgroups on most CUs and measured ~3 us slower a step at
// B = 65..128).
template <int MODE>
int launch_tile(TileParams& p, hipStream_t st, const char* who) {
    if constexpr (MODE == 1)
        launch_tile_tn<1, kTlNOut>(p, st);
    else if (p.B <= kTlNarrowB)
        launch_tile_tn<0, kTlNOut>(p, st);
    else
        launch_tile_tn<0, kTlN>(p, st);
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

// Argument checks of the tiled decode step (B > kSkM).
int tile_step_check(const void* x, const void* gamma, const void* W_qkvab, const void* conv_w_qkv,
                    const void* cache_q, const void* cache_k, const void* cache_v, const void* xn_hist,
                    const void* q, const void* k, const void* v, const void* a, const void* b, const void* o,
                    const void* W_o, const void* y, int B, int D, int H, int dk, int dv, int conv_k) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (D <= 0 || H <= 0 || dk <= 0 || dv <= 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_step: D=%d H=%d dk=%d dv=%d", D, H, dk, dv);
    if (D % kTlK != 0 || D > 16384)
        return fail(GDN_ERR_UNSUPPORTED, "decode_step: D=%d must be a multiple of %d, at most 16384", D, kTlK);
    if ((H * dk) % kTlN != 0 || (H * dv) % kTlN != 0)
        return fail(GDN_ERR_UNSUPPORTED, "decode_step: H dk=%d and H dv=%d must be multiples of %d for B > %d",
                    H * dk, H * dv, kTlN, kSkM);
    if (conv_k < 1 || conv_k > 4) return fail(GDN_ERR_UNSUPPORTED, "decode_step: conv_k=%d must be in 1..4", conv_k);
    // 32-bit byte offsets into x_n (bf16) and o (fp32)
    if (static_cast<size_t>(B) * std::max(D, H * dv) * 4 > 0xFFFFFFFFull)
        return fail(GDN_ERR_UNSUPPORTED, "decode_step: B=%d rows of D=%d / H dv=%d exceed 4 GiB", B, D, H * dv);
    if (B == 0) return GDN_OK;
    if (!x || !gamma || !W_qkvab || !conv_w_qkv || !q || !k || !v || !a || !b || !o || !W_o || !y ||
        (conv_k > 1 && (!cache_q || !cache_k || !cache_v)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_step: null pointer argument");
    if (!aligned(x, 16) || !aligned(gamma, 16) || !aligned(W_qkvab, 16) || !aligned(W_o, 16) || !aligned(y, 16) ||
        !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 16) || !aligned(xn_hist, 16) ||
        !aligned(cache_q, 16) || !aligned(cache_k, 16) || !aligned(cache_v, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode_step: x/gamma/W/W_o/y/q/k/v/o/caches/xn_hist need 16-byte alignment");
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
    // Up to kSkM sequences run the skinny projections around the recurrence;
    // larger batches run RMSNorm (x_n into y, the x_n history shifted), the
    // tiled in-projection, the recurrence and the tiled out-projection
    // (measured at config 5: 33 against 38 us at B=17, 44 against 70 at
    // B=48 for the skinny kernels in groups of 16).
    if (B < 0 || B > kStepMaxB)
        return gdn_host::fail(B < 0 ? GDN_ERR_INVALID_ARGUMENT : GDN_ERR_UNSUPPORTED,
                              "decode_step: B=%d, at most %d sequences", B, kStepMaxB);
    const bool tiled = B > kSkM;
    int st = tiled ? tile_step_check(x, gamma, W_qkvab, conv_w_qkv, cache_q, cache_k, cache_v, xn_hist, q, k, v, a,
                                     b, o, W_o, y, B, D, H, dk, dv, conv_k)
                   : in_proj_check(x, gamma, W_qkvab, conv_w_qkv, cache_q, cache_k, cache_v, q, k, v, a, b, B, D, H,
                                   dk, dv, conv_k);
    if (st == GDN_OK) st = gdn_host::decode_check(q, k, v, a, b, A_log, dt_bias, S_in, o, S_out, B, H, dk, dv);
    if (st == GDN_OK && !tiled) st = out_proj_check(o, W_o, y, B, H * dv, D);
    if (st != GDN_OK || B == 0) return st;
    if (tiled) {
        hipStream_t hs = static_cast<hipStream_t>(stream);
        st = gdn_host::rmsnorm_launch(x, gamma, y, xn_hist, xn_hist ? conv_k - 1 : 0, B, D, eps, hs);
        if (st != GDN_OK) return st;
        const int Hk = H * dk, Hv = H * dv;
        TileParams p = {};
        p.W = W_qkvab;
        p.B = B;
        p.K = D;
        p.N = 2 * Hk + Hv + 2 * H;
        p.A = y;
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
        st = launch_tile<0>(p, hs, "gdn_decode_tile_kernel<in>");
        if (st != GDN_OK) return st;
        // o as bf16 in the first half of the caller's fp32 o buffer
        st = gdn_host::decode_launch(q, k, v, a, b, A_log, dt_bias, S_in, scale, o, true, S_out, B, H, dv, hs);
        if (st != GDN_OK) return st;
        TileParams po = {};
        po.W = W_o;
        po.B = B;
        po.K = Hv;
        po.N = D;
        po.A = reinterpret_cast<const uint16_t*>(o);
        po.y = y;
        return launch_tile<1>(po, hs, "gdn_decode_tile_kernel<out>");
    }
    st = gdn_decode_in_proj_hip(x, gamma, eps, W_qkvab, conv_w_qkv, cache_q, cache_k, cache_v, xn_hist, q, k, v, a, b,
                                B, D, H, dk, dv, conv_k, stream);
    if (st != GDN_OK) return st;
    st = gdn_decode_hip(q, k, v, a, b, A_log, dt_bias, S_in, scale, o, S_out, B, H, dk, dv, stream);
    if (st != GDN_OK) return st;
    return gdn_decode_out_proj_hip(o, W_o, y, B, H * dv, D, stream);
}
