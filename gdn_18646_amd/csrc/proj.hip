// Projection GEMM + causal depthwise conv (<= 4 taps) + SiLU, bf16 MFMA.
//
// Reference: kernels/fused_proj_conv_silu.cu:105-295 (WMMA, 125-token tile +
// 3-token halo, cp.async pipeline) and reference/fused_proj_conv_silu_ref.py
// for the math.  P = x W^T is accumulated in fp32 and never rounded before the
// conv (as the reference kernel does; the PyTorch reference rounds P to bf16).
//
// Two kernels:
//
// gdn_proj_conv_mfma_kernel (the fast path) computes the transposed product
// P^T = W x^T in 256-column x 256-token tiles, one workgroup of 8 waves per
// CU.  Rows run over a flattened token axis where each sequence is 3 cache
// rows followed by its T tokens; a tile's first 3 rows are the causal halo
// (recomputed), so 253 rows are written per tile, and cache rows take the
// conv cache (or zero) so no tap reaches into another sequence.  Operands
// reach LDS by DMA (global_load_lds) in two 64-wide K stages: every 8 lanes
// of a copy read one whole 128-byte line (a row's K slice), placed with an
// XOR swizzle that keeps the MFMA fragment reads at linear-read speed.
// Waves form a 4 x 2 grid of 64 columns x 128 tokens = 4 x 8 MFMA 16x16x32
// tiles.  In the transposed C layout a lane holds 4 adjacent columns of one
// token, 16 tokens a tile: the conv taps are reads of a per-wave LDS window
// shifted by whole tokens.  The bf16 results go into an output tile in LDS
// (the two stages) and leave as whole rows, 16 bytes per lane.
//
// gdn_proj_conv_kernel (general shapes: group boundaries not on 4 columns,
// unaligned outputs, K not a multiple of 64) computes 128 x 128 tiles of P whose rows are
// tokens t0-3 .. t0+124 of one sequence and parks P in LDS for the conv.
//
// Output routing: up to 5 column groups, each written either token-major
// [B, T, width] or head-major [B, width/hd, T, hd], with or without the
// conv + SiLU (a plain projection takes the current token's row of P).
#include <cstddef>
#include <type_traits>

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
            idx = ((static_cast<size_t>(b) * (grp.width / grp.head_dim) + hh) * p.T_out + t) * grp.head_dim + dd;
        } else {
            idx = (static_cast<size_t>(b) * p.T_out + t) * grp.width + cc;
        }
        grp.dst[idx] = f2bf_bits(y);
    }
}


// ---------------------------------------------------------------------------
// Fast path: transposed MFMA tiles, DMA staging, register epilogue.
// ---------------------------------------------------------------------------
constexpr int kMCols = 256;                   // output columns (W rows) per workgroup
constexpr int kMToks = 256;                   // token rows per workgroup
constexpr int kMOut = kMToks - kHalo;         // 253 tokens written per workgroup
constexpr int kMK = 64;                       // K per stage: one 128-byte line per row
constexpr int kMStages = 2;
constexpr int kWMT = 4;                       // 16-column MFMA tiles per wave
constexpr int kWNT = 8;                       // 16-token MFMA tiles per wave (128 tokens: 2 token waves)
constexpr int kMWaves = (kMCols / (16 * kWMT)) * (kMToks / (16 * kWNT));
constexpr int kMRowB = kMK * 2;               // 128 bytes per staged row
constexpr int kMStageB = (kMCols + kMToks) * kMRowB;  // 64 KiB: W rows, then x rows
constexpr int kMDma = (kMCols + kMToks) / 8 / kMWaves;  // 1 KiB copies (8 rows) per wave per stage
static_assert((kMCols + kMToks) % (8 * kMWaves) == 0 && kMCols % (8 * kMWaves) == 0, "copies split evenly");
static_assert(kMToks == 2 * 16 * kWNT, "two token waves");
constexpr int kMHandB = (kMCols / (16 * kWMT)) * kWMT * 1024;  // hand-over area: one 16-token fp32 tile per column wave and MFMA tile
static_assert(kMStages * kMStageB == kMToks * kMCols * 2, "the stages hold the bf16 output tile");
// Conv window per wave: for each column quad a strip of 32 16-byte slots
// (slots 0..2: the previous 16-token tile's last 3 tokens, 3..18: the current
// tile's tokens, fp32 x 4 columns), so a tap is a plain b128 read shifted by
// whole slots, conflict free like a linear read.
constexpr int kMConvB = kMWaves * 4 * 32 * 16;
static_assert(kMStages * kMStageB + kMHandB + kMConvB <= 160 * 1024, "LDS");

// Staged row r holds its 8 16-byte chunks (k 8c .. 8c+7) at slot c ^ (r & 7):
// a fragment read (16 rows, one chunk each) then spreads every 8 consecutive
// rows over the 8 slots of a 128-byte line, which reads at the rate of a
// linear ds_read_b128 on gfx950 (measured; (r ^ (r >> 3)) & 7 lost a third).
__device__ __forceinline__ int swz(int r) { return r & 7; }

// Packed row table of the launch (ProjParams::row_off), read from the
// kernel's argument block (the ProjParams argument sits at its start):
// indexing the by-value parameter with a runtime index would copy it to
// private memory.
using kconst_i32 = __attribute__((address_space(4))) const int32_t;
__device__ __forceinline__ const kconst_i32* packed_rows() {
    const __attribute__((address_space(4))) char* base =
        (const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr();
    return reinterpret_cast<const kconst_i32*>(base + offsetof(gdn_proj::ProjParams, row_off));
}

// Groups whose output goes out through the LDS output tile in 16-byte
// chunks: 8-column aligned, 8-column head_dim (or token-major), 16-byte
// aligned destination.
__device__ __forceinline__ bool staged_group(const gdn_proj::ProjGroup& g) {
    return ((g.col0 | g.width | g.head_dim) & 7) == 0 && (reinterpret_cast<uintptr_t>(g.dst) & 15) == 0;
}

// The group holding column c, by compare-and-select over constant indices
// (indexing the parameter block with a runtime index would copy it to
// private memory).
__device__ __forceinline__ gdn_proj::ProjGroup select_group(const gdn_proj::ProjParams& p, int c) {
    gdn_proj::ProjGroup g = p.groups[0];
#pragma unroll
    for (int q = 1; q < gdn_proj::kMaxGroups; ++q)
        if (q < p.ngroups && c >= p.groups[q].col0) g = p.groups[q];
    return g;
}

// PACKED: sequences of unequal lengths (ProjParams::packed > 0), rows mapped
// through the row table; a separate instantiation, so the equal-length kernel
// carries none of that code.
template <bool PACKED>
__global__ __launch_bounds__(kMWaves * 64) __attribute__((amdgpu_waves_per_eu(kMWaves / 4, kMWaves / 4))) void gdn_proj_conv_mfma_kernel(
    gdn_proj::ProjParams p, int n_tok, int n_col) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem_raw[kMStages * kMStageB + kMHandB + kMConvB];
    lds_u8* const smem = (lds_u8*)&smem_raw[0];

    // Workgroup -> tile.  Dispatch deals workgroups to the 8 XCDs round-robin;
    // give each XCD a contiguous range of tiles, ordered in bands of 4 column
    // tiles with the token tile slowest, so the workgroups resident on one
    // XCD share W and x tiles in its L2.
    const int ntiles = n_tok * n_col;
    int lin;
    {
        const int id = blockIdx.x, xcd = id & 7, j = id >> 3, q = ntiles >> 3, r = ntiles & 7;
        lin = xcd < r ? xcd * (q + 1) + j : r * (q + 1) + (xcd - r) * q + j;
        const int band = lin / (4 * n_tok), base = 4 * band, gs = min(n_col - base, 4);
        const int within = lin - band * 4 * n_tok;
        lin = (within / gs) * n_col + base + within % gs;
    }
    const int tile_t = lin / n_col, tile_c = lin % n_col;
    // Row space: each sequence is kHalo cache rows (t = -3 .. -1) followed by
    // its tokens, so row r is (b, t) = (r / T3, r % T3 - 3) for equal lengths
    // T, or, for packed sequences, b the last with row_off[b] <= r and
    // t = r - row_off[b] - 3.  Cache rows take the cached projections (or
    // zero) after the product, so conv taps never reach into another
    // sequence.
    const int T3 = p.T + kHalo;
    constexpr bool packed = PACKED;
    const kconst_i32* prow = packed_rows();
    const int nseq = packed ? p.packed : p.B;
    const int F3 = packed ? prow[p.packed] : p.B * T3;
    const int f0 = tile_t * kMOut - kHalo;  // row of tile row 0 (>= -3; rows < 0 are never used)
    // Packed: the sequence of the tile's first row (uniform), the start of
    // every per-row search below.
    int pb0 = 0;
    if (packed) {
        int lo = 0, hi = p.packed;  // prow[lo] <= max(f0, 0) < prow[hi]
        const int r = max(f0, 0);
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (prow[mid] <= r) lo = mid; else hi = mid;
        }
        pb0 = lo;
    }
    auto len3 = [&](int b) { return packed ? prow[b + 1] - prow[b] : T3; };     // rows of sequence b
    auto tok0 = [&](int b) { return packed ? prow[b] - kHalo * b : b * p.T; };  // x row of its first token
    // (b, t3 = t + 3) of row r >= 0 (packed rows past the last sequence stay in it).
    auto locate = [&](int r, int& b, int& t3) {
        if (packed) {
            int bb = pb0;
            while (bb + 1 < p.packed && prow[bb + 1] <= r) ++bb;
            b = bb;
            t3 = r - prow[bb];
        } else {
            b = r / T3;
            t3 = r - b * T3;
        }
    };
    const int c0 = tile_c * kMCols;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: DMA bases stay scalar
    const int wm = wave >> 1, wn = wave & 1;                      // column slice, 128-token half
    const int r16 = lane & 15, g4 = lane >> 4;

    // x row feeding row r: the token itself, the sequence's first token for
    // cache rows, clamped at both ends (those products are never used).
    auto xrow_of = [&](int r) {
        if constexpr (PACKED) {
            const int ntok = F3 - kHalo * p.packed;  // x rows
            if (r < 0) return 0;
            if (r >= F3) return ntok - 1;
            int b, t3;
            locate(r, b, t3);
            return min(tok0(b) + max(t3 - kHalo, 0), ntok - 1);  // an empty last sequence has no token of its own
        } else {
            if (r < 0) return 0;
            if (r >= F3) return p.B * p.T - 1;
            const int b = r / T3, t = r - b * T3 - kHalo;
            return b * p.T + max(t, 0);
        }
    };

    // DMA sources.  Copy j of a wave moves staged rows 8 q .. 8 q + 7 with
    // q = wave + 8 j (q < 32: W rows, else x rows); lane l takes row 8 q + l / 8
    // and fills slot l % 8 with chunk (l % 8) ^ swz(row): every 8 lanes read
    // one whole 128-byte line.  Columns >= D_out are clamped to a valid row;
    // their products are never stored.
    const int xrow0 = xrow_of(f0);
    const unsigned char* wsrc = reinterpret_cast<const unsigned char*>(p.W + static_cast<size_t>(c0) * p.D);
    const unsigned char* xsrc = reinterpret_cast<const unsigned char*>(p.x + static_cast<size_t>(xrow0) * p.D);
    uint32_t voff[kMDma];
#pragma unroll
    for (int j = 0; j < kMDma; ++j) {
        const int q = wave + kMWaves * j;
        const int srow = 8 * q + (lane >> 3);  // staged row
        int row;
        if (srow < kMCols) {
            row = min(c0 + srow, p.D_out - 1) - c0;
        } else {
            row = xrow_of(f0 + srow - kMCols) - xrow0;
        }
        const int chunk = (lane & 7) ^ swz(srow);
        voff[j] = static_cast<uint32_t>(row) * static_cast<uint32_t>(p.D) * 2u + 16u * chunk;
    }
    auto issue_copy = [&](int stage, int kk, int j) {
        const int q = wave + kMWaves * j;
        const unsigned char* src = (8 * q < kMCols ? wsrc : xsrc) + kk * kMRowB;
        dma16(src, voff[j], smem + stage * kMStageB + q * 1024);
    };
    auto issue = [&](int stage, int kk) {
#pragma unroll
        for (int j = 0; j < kMDma; ++j) issue_copy(stage, kk, j);
    };
    // Half `half` of a stage's copies.
    auto issue_part = [&](int stage, int kk, int half) {
#pragma unroll
        for (int j = 0; j < kMDma / 2; ++j) issue_copy(stage, kk, half * kMDma / 2 + j);
    };

    // Fragment reads: lane l takes row 16 f + l % 16, chunk 4 h + l / 16 of
    // the staged rows (h: which 32-wide half of the stage's K); rd[h] is the
    // lane's byte offset within the fragment.
    uint32_t rd[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) rd[h] = r16 * kMRowB + 16u * ((4 * h + g4) ^ swz(r16));

    // Conv weights of this lane's columns, fetched now so their latency hides
    // under the main loop: for conv_k == 4 the 4 columns' taps are 16
    // adjacent bf16 (32-byte aligned: groups start on 4 columns).
    u32x4 wraw[kWMT][2];
#pragma unroll
    for (int mt = 0; mt < kWMT; ++mt) {
        wraw[mt][0] = wraw[mt][1] = u32x4{0u, 0u, 0u, 0u};
        const int cb = c0 + 16 * kWMT * wm + 16 * mt + 4 * g4;
        if (cb < p.D_out && p.conv_k == 4) {
            const gdn_proj::ProjGroup gq = select_group(p, cb);
            if (gq.conv) {
                const u32x4* src = reinterpret_cast<const u32x4*>(p.conv_w + static_cast<size_t>(gq.cw_row0 + cb - gq.col0) * 4);
                wraw[mt][0] = src[0];
                wraw[mt][1] = src[1];
            }
        }
    }

    f32x4 acc[kWMT][kWNT];
#pragma unroll
    for (int mt = 0; mt < kWMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kWNT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = p.D / kMK;
    issue(0, 0);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vm<0>();
        lds_barrier();  // stage kt landed for every wave; the other stage fully read
        // The next stage's copies go out in two halves, one before each K
        // half's MFMAs: a wave that issues all of them at once stalls on
        // the copy queue before its first MFMA.
        const bool next = kt + 1 < nk;
        const lds_u8* st = smem + (kt & 1) * kMStageB;
        static_for<0, 2>([&](auto H) {
            constexpr int h = decltype(H)::value;
            if (next) issue_part((kt + 1) & 1, kt + 1, h);
            bf16x8 a[kWMT], bx[kWNT];
            static_for<0, kWMT>([&](auto MT) {
                constexpr int mt = decltype(MT)::value;
                a[mt] = *reinterpret_cast<const lds_bf16x8*>(st + (16 * kWMT * wm + 16 * mt) * kMRowB + rd[h]);
            });
            static_for<0, kWNT>([&](auto NT) {
                constexpr int nt = decltype(NT)::value;
                bx[nt] = *reinterpret_cast<const lds_bf16x8*>(st + (kMCols + 16 * kWNT * wn + 16 * nt) * kMRowB + rd[h]);
            });
#pragma unroll
            for (int nt = 0; nt < kWNT; ++nt)
#pragma unroll
                for (int mt = 0; mt < kWMT; ++mt) acc[mt][nt] = mfma16x16x32(a[mt], bx[nt], acc[mt][nt]);
        });
    }

    // The token waves meet at token 128: the wn = 1 wave's first tile takes
    // its conv taps from the wn = 0 wave's last tile, handed over through an
    // LDS area of its own (the stages become the output tile below).
    const lds_u8* xs = smem + kMStages * kMStageB + wm * kWMT * 1024 + lane * 16;
    if (wn == 0) {
#pragma unroll
        for (int mt = 0; mt < kWMT; ++mt)
            *reinterpret_cast<lds_f32x4*>(const_cast<lds_u8*>(xs) + mt * 1024) = acc[mt][kWNT - 1];
    }
    lds_barrier();  // hand-over written; every wave is past its last stage read

    // This lane's row in token tile 0 of the wave, as (b, t3 = t + 3); tile
    // nt adds 16 rows.  Rows before local row kHalo are the tile's halo.
    const int nloc0 = 16 * kWNT * wn + r16;
    auto split = [&](int r, int& b, int& t3) {
        if (r < 0) {
            b = 0;
            t3 = r;
        } else {
            locate(r, b, t3);
        }
    };
    int b0, t30;
    split(f0 + nloc0, b0, t30);
    int bx, t3x;  // row of the handed-over tile (16 rows before tile 0)
    split(f0 + nloc0 - 16, bx, t3x);
    const int ncache = p.conv_k - 1;
    // Lean epilogue when the wave's 16 kWNT rows are all tokens of one
    // sequence (no cache rows, no sequence start) and none of them is in the
    // conv cache refresh window (the last ncache tokens).
    bool lean;
    {
        const int R0 = f0 + 16 * kWNT * wn;
        int bR, t3R;
        split(R0, bR, t3R);
        lean = R0 >= 0 && R0 + 16 * kWNT <= F3 && t3R >= kHalo && t3R + 16 * kWNT <= len3(bR) - ncache;
    }

    // Output tile in LDS (the two stages): row = token of the tile (512
    // bytes, 256 columns bf16), 32-byte unit u of a row stored at unit
    // u ^ (row & 15), so the 16 tokens of a fragment write spread over the
    // banks and a row reads back whole.
    lds_u8* const otile = smem;
    auto ounit = [](int row, int u) { return row * 512 + ((u ^ (row & 15)) << 5); };

    static_for<0, kWMT>([&](auto MT) {
        constexpr int mt = decltype(MT)::value;
        const int cb = c0 + 16 * kWMT * wm + 16 * mt + 4 * g4;  // this lane's 4 columns (same for the tile's 16 tokens)
        if (cb >= p.D_out) return;
        const gdn_proj::ProjGroup gq = select_group(p, cb);
        const int cc = cb - gq.col0, width = gq.width, hd = gq.head_dim;
        const bool conv = gq.conv != 0;
        const bool staged = staged_group(gq);
        float w[4][4];  // [column][tap], taps right-aligned: tap 3 multiplies the current token
        if (p.conv_k == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 q = wraw[mt][i >> 1];
                const uint32_t lo = q[2 * (i & 1)], hi = q[2 * (i & 1) + 1];
                w[i][0] = __uint_as_float(lo << 16);
                w[i][1] = __uint_as_float(lo & 0xffff0000u);
                w[i][2] = __uint_as_float(hi << 16);
                w[i][3] = __uint_as_float(hi & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int jw = j - (4 - p.conv_k);  // weight index of tap j
                    w[i][j] = conv && jw >= 0
                                  ? bf2f(p.conv_w[static_cast<size_t>(gq.cw_row0 + cc + i) * p.conv_k + jw])
                                  : 0.f;
                }
        }
        // Cache row (t < 0) of a conv group: the cached projection of token t
        // (cache index t + ncache, oldest first), zero before the cache or
        // without one.
        auto cache_row = [&](f32x4 v, int b, int t3) {
            const int q = t3 - kHalo + ncache;
            if (conv && t3 < kHalo) {
                const uint16_t* cin = gq.cache_in;
                const bool has = cin != nullptr && q >= 0;
                // rows past the last sequence (in the last tile; never stored)
                // read the last sequence's entries, not past the buffer
                const uint16_t* src =
                    has ? cin + (static_cast<size_t>(min(b, nseq - 1)) * width + cc) * ncache + q : nullptr;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = has ? bf2f(src[i * ncache]) : 0.f;
            }
            return v;
        };
        f32x4 pv = f32x4{0.f, 0.f, 0.f, 0.f};
        if (wn == 1) pv = cache_row(*reinterpret_cast<const lds_f32x4*>(xs + mt * 1024), bx, t3x);
        // This lane's conv window strip; the previous tile's last 3 tokens
        // (lanes 13..15) go to slots 0..2.
        lds_u8* const cw = smem + kMStages * kMStageB + kMHandB + (wave * 4 + g4) * 512;
        if (conv && r16 >= 13) *reinterpret_cast<lds_f32x4*>(cw + (r16 - 13) * 16) = pv;
        // The window is shared by the wave's lanes, which the compiler's
        // per-lane view does not see: these fences keep its accesses in
        // program order (the hardware then runs them in order).
        asm volatile("" ::: "memory");
        // Unstaged groups (head_dim 1..3 or 4-column aligned only) store from
        // registers.  Element index of (b, t, column cc + i): b width T + t
        // tstride + coff[i] (token-major: tstride = width, coff = cc + i;
        // head-major [B, width/hd, T, hd]: tstride = hd, coff = ((cc + i) /
        // hd) T hd + (cc + i) % hd).
        const size_t seq = static_cast<size_t>(width) * p.T_out;
        const int tstride = hd ? hd : width;
        // token t of sequence b: b width T_out + t tstride, or, packed, its
        // token offset in the packed outputs times tstride
        auto orow = [&](int b, int t) {
            return packed ? static_cast<size_t>(tok0(b) + t) * tstride
                          : static_cast<size_t>(b) * seq + static_cast<size_t>(t) * tstride;
        };
        const bool vec = hd == 0 || (hd & 3) == 0;  // the 4 columns are adjacent in memory
        size_t coff[4] = {0, 0, 0, 0};
        if (!staged) {
            int h = hd ? cc / hd : 0, d = hd ? cc - h * hd : cc;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                coff[i] = hd ? static_cast<size_t>(h) * p.T_out * hd + d : static_cast<size_t>(cc + i);
                if (hd && ++d == hd) {
                    d = 0;
                    ++h;
                }
            }
        }
        auto store = [&](uint16_t* row, const float (&y)[4]) {
            if (vec) {
                *reinterpret_cast<u32x2*>(row + coff[0]) = u32x2{pack2_bf16(y[0], y[1]), pack2_bf16(y[2], y[3])};
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) row[coff[i]] = f2bf_bits(y[i]);
            }
        };
        const int unit = 4 * wm + mt;  // 32-byte unit of the output row holding this fragment's columns
        int b = b0, t3 = t30;
        static_for<0, kWNT>([&](auto NT) {
            constexpr int nt = decltype(NT)::value;
            if (nt > 0 && !lean) {
                t3 += 16;
                if (packed) {
                    while (b + 1 < p.packed && t3 >= len3(b)) {
                        t3 -= len3(b);
                        ++b;
                    }
                } else if (t3 >= T3) {
                    b += t3 / T3;
                    t3 %= T3;
                }
            }
            const int nloc = nloc0 + 16 * nt;
            f32x4 cur = acc[mt][nt];
            if (!lean) cur = cache_row(cur, b, t3);
            // conv + SiLU (plain groups: the current row)
            float y[4];
            if (conv) {
                // Taps through the window: tokens n - 1, n - 2, n - 3 are
                // slots n + 2, n + 1, n (one wave: its LDS accesses run in
                // order, so the reads see this tile's writes and the slide of
                // the last 3 tokens to slots 0..2 comes after every read).
                *reinterpret_cast<lds_f32x4*>(cw + (3 + r16) * 16) = cur;
                asm volatile("" ::: "memory");
                const f32x4 t1 = *reinterpret_cast<const lds_f32x4*>(cw + (2 + r16) * 16);
                const f32x4 t2 = *reinterpret_cast<const lds_f32x4*>(cw + (1 + r16) * 16);
                const f32x4 t3v = *reinterpret_cast<const lds_f32x4*>(cw + r16 * 16);
                asm volatile("" ::: "memory");
                if (r16 >= 13) *reinterpret_cast<lds_f32x4*>(cw + (r16 - 13) * 16) = cur;
                asm volatile("" ::: "memory");
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float s = w[i][3] * cur[i] + w[i][2] * t1[i] + w[i][1] * t2[i] + w[i][0] * t3v[i];
                    y[i] = silu_f(s);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = cur[i];
            }
            if (staged) {
                *reinterpret_cast<lds_u32x2*>(otile + ounit(nloc, unit) + 8 * g4) =
                    u32x2{pack2_bf16(y[0], y[1]), pack2_bf16(y[2], y[3])};
            } else if (lean) {
                if (!(nt == 0 && nloc0 < kHalo))  // the tile's halo rows
                    store(gq.dst + orow(b0, t30 - kHalo + 16 * nt), y);
            } else if (nloc >= kHalo && f0 + nloc < F3 && t3 >= kHalo) {
                store(gq.dst + orow(b, t3 - kHalo), y);
            }
            // New cache: rows t = T - ncache .. T - 1 of the extended sequence
            // (cache rows included when T < ncache).
            const int Tb = len3(b) - kHalo;
            if (!lean && conv && gq.cache_out && nloc >= kHalo && f0 + nloc < F3 && t3 - kHalo >= Tb - ncache) {
                const int t = t3 - kHalo;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    gq.cache_out[(static_cast<size_t>(b) * width + cc + i) * ncache + (t - (Tb - ncache))] =
                        f2bf_bits(cur[i]);
            }
        });
    });
    lds_barrier();  // output tile complete

    // Store the tile's staged columns row by row: thread tid takes 16-byte
    // chunk j = tid % 32 (8 columns) of tile rows tid / 32 + 16 i, so a wave
    // writes two whole 512-byte rows per instruction (for head-major groups,
    // two 256-byte token rows of each head).
    {
        const int j = tid & 31;
        const int c = c0 + 8 * j;
        if (c >= p.D_out) return;
        const gdn_proj::ProjGroup gq = select_group(p, c);
        if (!staged_group(gq)) return;
        const int cc = c - gq.col0, hd = gq.head_dim;
        const size_t seq = static_cast<size_t>(gq.width) * p.T_out;
        const size_t tstride = hd ? hd : gq.width;
        uint16_t* const colp = gq.dst + (hd ? static_cast<size_t>(cc / hd) * p.T_out * hd + cc % hd : static_cast<size_t>(cc));
        const int row0 = tid >> 5;
        int b, t3;
        split(f0 + row0, b, t3);
#pragma unroll 4
        for (int i = 0; i < kMToks / 16; ++i) {
            const int row = row0 + 16 * i;
            if (i > 0) {
                t3 += 16;
                while ((!packed || b + 1 < p.packed) && t3 >= len3(b)) {
                    t3 -= len3(b);
                    ++b;
                }
            }
            if (row >= kHalo && f0 + row < F3 && t3 >= kHalo) {
                const u32x4 v = *reinterpret_cast<const lds_u32x4*>(otile + ounit(row, j >> 1) + 16 * (j & 1));
                const size_t o = packed ? static_cast<size_t>(tok0(b) + t3 - kHalo) * tstride
                                        : static_cast<size_t>(b) * seq + static_cast<size_t>(t3 - kHalo) * tstride;
                *reinterpret_cast<u32x4*>(colp + o) = v;
            }
        }
    }
}

}  // namespace

namespace gdn_proj {

// The fast kernel needs every group to start on a 4-column boundary (a lane's
// 4 columns share a group), 8-byte aligned outputs for its vector stores,
// 16-byte aligned conv weights (read 4 columns x 4 taps at a time) and 32-bit
// DMA offsets.
static_assert(kCacheRows == kHalo, "row space");

bool mfma_path_ok(const ProjParams& p) {
    if (p.D % kMK != 0 || p.D_out % 4 != 0) return false;
    if (!gdn_host::aligned(p.conv_w, 16)) return false;
    if (static_cast<long long>(p.D_out) * p.D * 2 >= (1ll << 31)) return false;
    if (static_cast<long long>(kMToks) * p.D * 2 >= (1ll << 31)) return false;
    if (static_cast<long long>(p.B) * (p.T + kHalo) >= (1ll << 30)) return false;
    if (p.packed < 0 || p.packed > kPackMax) return false;
    for (int g = 0; g < p.ngroups; ++g) {
        const ProjGroup& q = p.groups[g];
        if (q.col0 % 4 != 0 || q.width % 4 != 0 || q.cw_row0 % 4 != 0) return false;
        // 8-byte stores where a lane's 4 columns are adjacent in memory;
        // head_dim 1..3 (the layer's a/b) stores element by element.
        const bool vec = q.head_dim == 0 || q.head_dim % 4 == 0;
        if (!gdn_host::aligned(q.dst, vec ? 8 : 2)) return false;
    }
    return true;
}

int launch_proj(const ProjParams& pin, hipStream_t stream) {
    ProjParams p = pin;
    if (p.T_out < p.T) p.T_out = p.T;
    if (p.packed > 0) {
        // Packed sequences: the MFMA kernel only (callers check mfma_path_ok
        // first); rows: kHalo cache rows + the tokens of every sequence.
        if (!mfma_path_ok(p)) return gdn_host::fail(GDN_ERR_UNSUPPORTED, "proj: packed launch off the MFMA path");
        const int F3 = p.row_off[p.packed];
        const int n_tok = (F3 + kMOut - 1) / kMOut, n_col = (p.D_out + kMCols - 1) / kMCols;
        hipLaunchKernelGGL(gdn_proj_conv_mfma_kernel<true>, dim3(n_tok * n_col), dim3(kMWaves * 64), 0, stream, p, n_tok,
                           n_col);
        return gdn_host::check_launch("gdn_proj_conv_mfma_kernel");
    }
    if (p.B == 0 || p.T == 0 || p.D_out == 0) return GDN_OK;
    if (mfma_path_ok(p)) {
        const int F3 = p.B * (p.T + kHalo);  // rows: kHalo cache rows + T tokens per sequence
        const int n_tok = (F3 + kMOut - 1) / kMOut, n_col = (p.D_out + kMCols - 1) / kMCols;
        hipLaunchKernelGGL(gdn_proj_conv_mfma_kernel<false>, dim3(n_tok * n_col), dim3(kMWaves * 64), 0, stream, p, n_tok,
                           n_col);
        return gdn_host::check_launch("gdn_proj_conv_mfma_kernel");
    }
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
