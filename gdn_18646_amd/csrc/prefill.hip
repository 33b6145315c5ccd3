// GDN chunked prefill (chunk C = 64, dk = 128).
//
// Reference: kernels/prefill_chunked.cu:41-417 (one fused block per (b,h),
// WMMA for two products, the rest scalar) with the semantics of
// reference/prefill_ref.py:11-132.  Per chunk (Appendix-A notation):
//   gamma_t = exp(sum_{s<=t} log g_s)            Gamma_ts = gamma_t / gamma_s
//   A_ts    = beta_t m_t (k_t.k_s) Gamma_ts, t>s T = (I + A)^-1
//   dV      = T diag(beta m) (V - diag(gamma) K S)
//   O       = m (scale gamma (Q S) + scale (Q K^T o Gamma)_causal dV)
//   S      <- gamma_C S + (K o gamma_C/gamma)^T dV
//
// Kernel 1, gdn_prefill_intra_kernel — one 256-thread workgroup per
// (chunk, head, sequence); every chunk in parallel.  Builds K K^T and Q K^T on
// bf16 MFMA, the decay matrix, the fp32 forward substitution for T, and writes
// per chunk (bf16 unless noted), already in the register order the state
// kernels' MFMA operands need (one 16-byte load per lane per fragment):
//   Tp  = T diag(beta m)                       8 fragments  (8 KiB)
//   Aq  = m scale (Q K^T o Gamma), t >= s      the 6 nonzero fragments (6 KiB)
//   G   = [gamma_t, m_t scale gamma_t, gamma_C / gamma_t, -]   256 fp32
// The state update's K^T operand is not stored: the state kernels build it
// from the K tile they stage anyway, with transposing LDS reads, and apply
// gamma_C / gamma_t to the rows of dV instead.
// Kernel 2, gdn_prefill_state_kernel — each wave owns 16*NT state columns of
// one (sequence, head) and walks chunks in order.  The fp32 state tile lives
// in MFMA accumulator registers the whole time; its bf16 copy feeds the next
// chunk's products directly (no LDS), because the k order inside an MFMA
// operand is free: the state rows are assigned to accumulator slots so that
// the accumulator of the state update IS the B operand of K S and Q S.
// When (sequence, head) pairs alone cannot fill the chip, each sequence is cut
// into G chunk groups (S maps affinely across a group: S_out = phi S_in + psi):
//   map pass   (kernel 2, map mode)  psi and phi of every group but the last,
//   scan       (gdn_prefill_scan_kernel)  S_in of every group, in order,
//   output pass (kernel 2, output mode) every group from its S_in, in parallel.
//
// Fragment k-order conventions (lane l: m = l%16 row/column, g = l/16 group):
//   pi(g, j)   = j < 4 ? 4g + j : 16 + 4g + (j-4)   chunk position inside a
//                32-wide k-step, the order produced by two stacked accumulators
//   rho(r,g,i) = 32(r/2) + 8g + 4(r%2) + i          state row held in
//                accumulator tile r, slot i, of lane group g
#include <algorithm>
#include <mutex>

#include "gdn_common.hpp"

namespace {

using namespace gdn;

constexpr int kC = 64;    // chunk length
constexpr int kDK = 128;  // key / query dim

// Workspace record of one (chunk, head), written by the intra kernel and read
// by the state kernels, in 1 KiB MFMA fragments (lane l's 16 bytes at 16 l).
// For the 16-column state kernel: the six nonzero fragments of Tp, the six of
// Aq, the gate block.  The 32-column state kernel forms Aq itself and reads
// the six of Tp, the gate block and the token block (log2 of the in-chunk
// decay, m scale).  Gate block: gamma, m scale gamma, gamma_C / gamma.
constexpr int kRecTp = 0;
constexpr int kRecAq = 6;
constexpr int kRecFull = 13;   // Tp, Aq, gates
constexpr int kRecShort = 8;   // Tp, gates, tokens
constexpr int kRecGShort = 6;  // gate block of the short record
constexpr int kRecH = 7;       // token block of the short record

struct PrefillParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* a;
    const uint16_t* b;
    const float* A_log;
    const float* mask;      // nullable: all ones
    const float* state_in;  // nullable: zero state
    uint16_t* out;
    float* state_out;
    const int32_t* cu;  // varlen offsets (nullable: batch mode)
    u32x4* wsR;          // per (chunk, head) workspace records (rec_frags 1 KiB fragments each)
    int intra_aq;        // the intra kernel forms Aq (kRecFull records, for the 16-column state kernel)
    float dt_bias;
    float scale;
    int H;
    int dv;
    int T_stride;        // tokens per (b, h) row block of q/k/v/a/b/out
    int T_len;           // batch mode: sequence length
    int chunks_per_seq;  // batch mode: ceil(T_len / 64)
    int xcd_heads;       // (sequence, head) pairs are a multiple of 8: head-aligned XCD mapping
    int out_tm;          // out is token-major ([B, T, H, dv] / [T_total, H, dv]) instead of head-major
    int nchunk_grid;     // intra kernel: chunks per (sequence, head) in the grid
    int intra_units;     // intra kernel: (sequence, head) pairs x nchunk_grid
};

struct SeqInfo {
    int b, tok0, len, slot0;
};

__device__ __forceinline__ SeqInfo seq_info(const PrefillParams& p, int sidx) {
    SeqInfo s;
    if (p.cu) {
        s.b = 0;
        s.tok0 = p.cu[sidx];
        s.len = p.cu[sidx + 1] - s.tok0;
        // Chunk slots floor(tok0/64) + sidx never overlap between sequences
        // and total at most T_total/64 + num_seqs.
        s.slot0 = s.tok0 / kC + sidx;
    } else {
        s.b = sidx;
        s.tok0 = 0;
        s.len = p.T_len;
        s.slot0 = sidx * p.chunks_per_seq;
    }
    return s;
}

__device__ __forceinline__ int pi_pos(int g, int j) { return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4); }
__device__ __forceinline__ int rho_row(int r, int g, int i) { return 32 * (r >> 1) + 8 * g + 4 * (r & 1) + i; }

// Workgroups are dealt to the 8 XCDs round robin by linear id, and each XCD
// has its own L2.  With a multiple of 8 (sequence, head) pairs every prefill
// kernel puts head `hd` on XCD hd % 8, so what one kernel writes for a head
// is read from the same L2 by the next: linear id L -> head (L % 8) + 8 q,
// item r of that head, where L / 8 = q * per_head + r.
struct HeadItem {
    int head, item;
};
__device__ __forceinline__ HeadItem head_major_xcd(int L, int per_head) {
    const int q = (L >> 3) / per_head;
    return {(L & 7) + 8 * q, (L >> 3) - q * per_head};
}

// The nonzero fragments (mt, s) of the causal Aq, in workspace order:
// (0,0),(1,0),(2,0),(2,1),(3,0),(3,1) as f = 2 mt + s.
__device__ __forceinline__ constexpr int aq_slot(int i) { return i < 2 ? 2 * i : i + 2; }
// Inverse: slot of the nonzero fragment (mt, s) (s = 1 needs mt >= 2).
__device__ __forceinline__ constexpr int aq_index(int mt, int s) { return mt < 2 ? mt : 2 * mt - 2 + s; }

// ---------------------------------------------------------------------------
// Kernel 1
// ---------------------------------------------------------------------------
// Inclusive prefix sum over the 64 lanes with DPP: shifts by 1, 2, 4, 8 within
// each 16-lane row, then lane 15 broadcast into rows 1 and 3 and lane 31 into
// rows 2 and 3.  Lanes without a source add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true));
}
__device__ __forceinline__ float wave_inclusive_sum(float v) {
    v += dpp_add_src<0x111, 0xf>(v);  // row_shr:1
    v += dpp_add_src<0x112, 0xf>(v);  // row_shr:2
    v += dpp_add_src<0x114, 0xf>(v);  // row_shr:4
    v += dpp_add_src<0x118, 0xf>(v);  // row_shr:8
    v += dpp_add_src<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_add_src<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

constexpr int kKLD = kDK + 8;  // padded LDS row (bf16) for K and Q tiles
// A is stored by column, de-interleaved: element (i, j) at Ad[j][(i % 4) kAQ + i / 4].
// Rows of 16 + 4 floats keep the 4-row reads 16-byte aligned; the extra 4
// floats per column make the column stride 84 floats, so the 64 lanes of a
// step-3 write (16 columns x 4 row groups) hit 64 different banks.
constexpr int kAQ = kC / 4 + 4;
constexpr int kADS = 4 * kAQ + 4;
constexpr int kBLD = kC + 8;   // padded LDS row (bf16) for 64x64 tiles

// One (chunk, sequence-head) unit of kernel 1.  Unit u maps to head, chunk
// through head_major_xcd when the head count allows (the persistent grid is a
// multiple of 8, so a workgroup's units all share its XCD).
struct IntraUnit {
    SeqInfo sq;
    size_t row_base, wc;
    int c, h, t0, nvalid;
    bool valid;
};
__device__ __forceinline__ IntraUnit intra_unit(const PrefillParams& p, int u) {
    IntraUnit U = {};
    U.valid = false;
    if (u >= p.intra_units) return U;
    int head;
    if (p.xcd_heads) {
        const HeadItem hi = head_major_xcd(u, p.nchunk_grid);
        head = hi.head;
        U.c = hi.item;
    } else {
        head = u / p.nchunk_grid;
        U.c = u % p.nchunk_grid;
    }
    U.h = head % p.H;
    U.sq = seq_info(p, head / p.H);
    U.t0 = U.c * kC;
    if (U.t0 >= U.sq.len) return U;  // varlen: past this sequence's end
    U.valid = true;
    U.nvalid = min(kC, U.sq.len - U.t0);
    U.row_base = static_cast<size_t>(U.sq.b * p.H + U.h) * p.T_stride + U.sq.tok0 + U.t0;
    U.wc = static_cast<size_t>(U.sq.slot0 + U.c) * p.H + U.h;
    return U;
}

// The wave that computes a unit's gates (one token per lane).  It is the wave
// with no work in the last round of the triangular solve, where it computes
// the next unit's gates ahead of time.
constexpr int kGateWave = 2;

// A unit's global inputs that are prefetched into registers: the K tile slice
// this thread stores to LDS (rows past the sequence end zero) and the gate
// wave's inputs (one token per lane, and A_log of the head).
struct IntraLoads {
    u32x4 kv[4];
    float g_m, g_alog;
    uint32_t g_a, g_b;  // bf16 bits, widened at use (a conversion here would wait for the load)
};
__device__ __forceinline__ void intra_load(const PrefillParams& p, const IntraUnit& U, int tid, IntraLoads& L) {
    const int wave = tid >> 6, lane = tid & 63;
    L.g_m = L.g_alog = 0.f;
    L.g_a = L.g_b = 0u;
    if (wave == kGateWave) L.g_alog = p.A_log[U.h];
    if (wave == kGateWave && lane < U.nvalid) {
        const size_t gi = U.row_base + lane;
        L.g_m = p.mask ? p.mask[static_cast<size_t>(U.sq.b) * p.T_stride + U.sq.tok0 + U.t0 + lane] : 1.f;
        L.g_a = p.a[gi];
        L.g_b = p.b[gi];
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = tid + 256 * it, row = idx >> 4, c8 = (idx & 15) * 8;
        L.kv[it] = u32x4{0u, 0u, 0u, 0u};
        if (row < U.nvalid) L.kv[it] = *reinterpret_cast<const u32x4*>(p.k + (U.row_base + row) * kDK + c8);
    }
}

// A unit's gates, one token per lane (the gate wave): log2 of the in-chunk
// decay cumsum, beta m, m scale, and the gate block gamma, m scale gamma,
// gamma_C / gamma.  Tokens past the sequence end: no decay, beta m = m = 0.
struct GateVals {
    float lg2, bm, ms, g0, g1, g2;
};
__device__ __forceinline__ GateVals gate_vals(const PrefillParams& p, const IntraLoads& L, int lane, int nvalid) {
    float lg = 0.f, bm = 0.f, m = 0.f;
    if (lane < nvalid) {
        m = L.g_m;
        lg = -expf(L.g_alog) * softplus_f(__uint_as_float(L.g_a << 16) + p.dt_bias);
        bm = sigmoid_f(__uint_as_float(L.g_b << 16)) * m;
    }
    const float s = wave_inclusive_sum(lg);
    const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), kWave - 1));
    const float gam = expf(s);
    return {s * 1.4426950408889634f, bm, m * p.scale, gam, m * p.scale * gam, expf(last - s)};
}

// Tp fragments (mt, s) = (wave, 0), (wave, 1) of one record: fragments
// (0, 1) and (1, 1) lie above the diagonal and are not stored; the others go
// to slots (0,0) (1,0) (2,0) (2,1) (3,0) (3,1) in that order.
template <int RF>
__device__ __forceinline__ void store_tp(const PrefillParams& p, size_t wc, int wave, int lane, const u32x4 (&tpf)[2]) {
    u32x4* rec = p.wsR + (wc * RF + kRecTp) * 64;
    if (wave < 2) {
        rec[wave * 64 + lane] = tpf[0];
    } else {
        rec[(2 * wave - 2) * 64 + lane] = tpf[0];
        rec[(2 * wave - 1) * 64 + lane] = tpf[1];
    }
}

// Persistent: each workgroup walks units blockIdx.x, + gridDim.x, ...; the
// next unit's K slice and gate inputs are loaded into registers (IntraLoads)
// while the current unit's triangular solve runs, so global latency overlaps
// compute.  Q (MFMA A operands of Q K^T) is read at the start of its unit.
// All global stores of a unit (G, Aq, and the previous unit's Tp, held in
// registers until then) are issued together after step 3: a wait for a load
// issued while stores are in flight waits for the stores as well (the vector
// memory counter does not order reads against writes), so the next wait,
// at the following unit's start, finds them long complete.
// AQ: also form the causal Aq (for the 16-column state kernel; the 32-column
// one forms it itself).  LDS use (about 47 KiB with AQ, 39 KiB without)
// allows three (four) workgroups per CU, i.e. three (four) waves per SIMD:
// saying so lets the scheduler spend registers on hoisting loads.
template <bool AQ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(AQ ? 3 : 4, AQ ? 3 : 4))) void
gdn_prefill_intra_kernel(PrefillParams p) {
    constexpr int RF = AQ ? kRecFull : kRecShort;       // record length (fragments)
    constexpr int RG = AQ ? kRecFull - 1 : kRecGShort;  // gate block
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int m16 = lane & 15;
    const int g4 = lane >> 4;

    // The K tile is dead after step 3: step 5 keeps the fp32 T blocks there.
    // Without AQ the bf16 Tp staging tile (Al) lives in the dead K tile too,
    // after the fp32 T blocks.
    constexpr int kTBytes = sizeof(float) * 6 * 16 * 20;
    __shared__ __attribute__((aligned(16))) bf16 Kl[kC][kKLD];
    __shared__ __attribute__((aligned(16))) float Ad[kC][kADS];
    __shared__ __attribute__((aligned(16))) bf16 Al_own[AQ ? kC : 1][kBLD];
    __shared__ float s_lg2[kC], s_bm[kC], s_ms[kC];  // s_lg2: in-chunk log2 decay cumsum
    static_assert(sizeof(Kl) >= kTBytes + (AQ ? 0 : sizeof(bf16) * kC * kBLD), "the K tile must hold the T blocks");
    bf16 (*const Al)[kBLD] =
        AQ ? Al_own : reinterpret_cast<bf16 (*)[kBLD]>(reinterpret_cast<unsigned char*>(&Kl[0][0]) + kTBytes);

    int u = blockIdx.x;
    IntraUnit U = intra_unit(p, u);
    IntraLoads L;
    if (U.valid) intra_load(p, U, tid, L);
    u32x4 tpf[2];          // the previous unit's Tp fragments 2 wave, 2 wave + 1
    size_t wc_prev = 0;
    bool have_prev = false;
    GateVals gv = {};      // gate wave: this unit's gates, computed ahead during the previous unit
    bool gv_ready = false;
    while (u < p.intra_units) {
    const int u_next = u + static_cast<int>(gridDim.x);
    const IntraUnit N = intra_unit(p, u_next);
    if (!U.valid) {
        if (N.valid) intra_load(p, N, tid, L);
        u = u_next;
        U = N;
        continue;
    }
    const int c = U.c, h = U.h, nvalid = U.nvalid;
    const size_t wc = U.wc;
    (void)c;
    (void)h;

    // 1) K tile into LDS.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = tid + 256 * it;
        *reinterpret_cast<u32x4*>(&Kl[idx >> 4][(idx & 15) * 8]) = L.kv[it];
    }
    // Q row blocks as MFMA A operands: step 3's tiles are dealt so wave w
    // needs block w (qa) and, for w < 2, block 3 (qb).  Rows are clamped to
    // the sequence; those rows get a zero output coefficient.
    bf16x8 qa[4], qb[4];
    constexpr bool want_aq = AQ;
    if constexpr (AQ) {
        const uint16_t* qr = p.q + (U.row_base + min(16 * wave + m16, nvalid - 1)) * kDK + 8 * g4;
#pragma unroll
        for (int s = 0; s < 4; ++s) qa[s] = as_bf16x8(*reinterpret_cast<const u32x4*>(qr + 32 * s));
    }
    if (AQ && wave < 2) {
        const uint16_t* qr = p.q + (U.row_base + min(48 + m16, nvalid - 1)) * kDK + 8 * g4;
#pragma unroll
        for (int s = 0; s < 4; ++s) qb[s] = as_bf16x8(*reinterpret_cast<const u32x4*>(qr + 32 * s));
    }

    // 2) Gates and the in-chunk log-cumsum (the gate wave, one token per
    //    lane; computed during the previous unit's last solve round when that
    //    unit ran here).
    if (wave == kGateWave) {
        if (!gv_ready) gv = gate_vals(p, L, lane, nvalid);
        s_lg2[lane] = gv.lg2;
        s_bm[lane] = gv.bm;
        s_ms[lane] = gv.ms;
    }
    __syncthreads();

    // 3) K K^T and Q K^T on the 10 lower 16x16 tiles (i >= j): tile (ti, tj)
    //    goes to wave ti, except (3,0), (3,1) to wave 0 and (3,2) to wave 1
    //    (three tiles each for waves 0-2); wave 3 takes (3,3) and zeroes the 6
    //    upper tiles of Aq.
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int ti = t >> 2, tj = t & 3;  // tile (row ti, col tj)
        const int col = 16 * tj + m16;
        if (tj > ti) {
            if (wave != 3 || !want_aq) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) Al[16 * ti + 4 * g4 + i][col] = f2bf(0.f);
            continue;
        }
        const int owner = ti < 3 ? ti : (tj < 2 ? 0 : (tj == 2 ? 1 : 3));
        if (owner != wave) continue;
        f32x4 accK = {0.f, 0.f, 0.f, 0.f}, accQ = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 aK = *reinterpret_cast<const bf16x8*>(&Kl[16 * ti + m16][32 * s + 8 * g4]);
            const bf16x8 bK = *reinterpret_cast<const bf16x8*>(&Kl[16 * tj + m16][32 * s + 8 * g4]);
            accK = mfma16x16x32(aK, bK, accK);
            if constexpr (AQ) accQ = mfma16x16x32(ti == wave ? qa[s] : qb[s], bK, accQ);
        }
        const float lg2_col = s_lg2[col];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * ti + 4 * g4 + i;
            const float d = __builtin_amdgcn_exp2f(s_lg2[row] - lg2_col);  // Gamma_{row,col}
            Ad[col][(row & 3) * kAQ + (row >> 2)] = row > col ? s_bm[row] * accK[i] * d : 0.f;
            if constexpr (AQ) Al[row][col] = f2bf(row >= col ? s_ms[row] * accQ[i] * d : 0.f);
        }
    }
    // vmcnt(0): nothing is in flight here (every Q load was consumed above),
    // but the compiler cannot tell on the paths that own no tile and would
    // otherwise wait for the loads issued next before reusing Q's registers.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    // The current unit's inputs are consumed: start the next unit's loads,
    // then this unit's stores.
    if (N.valid) intra_load(p, N, tid, L);
    if (wave == kGateWave) {
        float* G = reinterpret_cast<float*>(p.wsR + (wc * RF + RG) * 64);
        G[lane] = gv.g0;
        G[64 + lane] = gv.g1;
        G[128 + lane] = gv.g2;
        if constexpr (!AQ) {
            float* Hb = reinterpret_cast<float*>(p.wsR + (wc * RF + kRecH) * 64);
            Hb[lane] = gv.lg2;
            Hb[64 + lane] = gv.ms;
        }
    }
    if (have_prev) store_tp<RF>(p, wc_prev, wave, lane, tpf);

    // 4) The six nonzero Aq fragments (mt, s) = (0,0),(1,0),(2,0),(2,1),(3,0),(3,1):
    //    lane holds Aq[16mt + m][32s + pi(g, j)].
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        if (i % 4 != wave || !want_aq) continue;
        const int f = aq_slot(i), mt = f >> 1, s = f & 1;
        const bf16* rp = &Al[16 * mt + m16][32 * s + 4 * g4];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(rp);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(rp + 16);
        p.wsR[(wc * RF + kRecAq + i) * 64 + lane] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }

    // 5) T = (I + A)^-1 in fp32, blocked by 16 (block rows / columns I, J),
    //    and Tp = T diag(beta m) in bf16 into the Aq staging tile (dead after
    //    step 4; the upper blocks are zero):
    //    5a each wave w inverts its diagonal block, T_ww = (I + A_ww)^-1, by
    //       right-looking forward substitution (4 lanes per column, DPP
    //       broadcast of each finished row);
    //    5b T_10 = -T_11 A_10 T_00 (wave 0) and T_32 = -T_33 A_32 T_22
    //       (wave 1), which completes T on each diagonal 32x32 half;
    //    5c the lower left quarter, -T_hi A_hl T_lo: block (2 + r, J) goes to
    //       wave 2J + r, which forms W_2J = A_20 T_0J + A_21 T_1J (and W_3J
    //       for r = 1), then T_2J = -T_22 W_2J or T_3J = -(T_32 W_2J + T_33 W_3J).
    //       What needs only diagonal blocks (all of column J = 1 but T_32 W_21,
    //       the A_x0 T_00 terms of column 0) is done during 5b.
    //    Products run on fp32 MFMA 16x16x4.  A first product's result, in
    //    accumulator layout (lane l: rows 4(l/16)+i of column l%16), is the
    //    B operand of the second product as it stands: slice i then carries
    //    k = 4(l/16) + i, and the A operand is read in the same k order.
    //    The diagonal blocks, T_10 and T_32 (fp32, row stride 20) live in the
    //    dead K tile.
    {
        constexpr int kTS = 20;
        float* const T32 = reinterpret_cast<float*>(&Kl[0][0]);
        // slots: diagonal block I -> I, T_10 -> 4, T_32 -> 5
        auto tblk = [&](int slot) { return T32 + slot * (16 * kTS); };
        int col = lane >> 2;
        int sub = lane & 3;
        int tx = tid;
        // Opaque per unit: otherwise the compiler hoists the per-row selects
        // and per-thread addresses below out of the persistent loop and
        // spills them.
        asm volatile("" : "+v"(col), "+v"(sub), "+v"(tx));
        const int li = tx & 15, lg = (tx >> 4) & 3;  // MFMA lane row / column, k group
        float Tc[4];
        {
            float acc[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) Tc[q] = acc[q] = 0.f;
            // A[16w + 4q + sub][16w + j] for q = 0..3 (this lane's rows) of
            // the columns j = 4g .. 4g + 3, read one group of four steps
            // ahead: each step's row update then waits on no LDS read (a read
            // per step, consumed by the next, exposed its latency 16 times).
            f32x4 colA[2][4];
            auto load_cols = [&](int grp, int slot) {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    colA[slot][t] = *reinterpret_cast<const f32x4*>(&Ad[16 * wave + 4 * grp + t][sub * kAQ + 4 * wave]);
            };
            load_cols(0, 0);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int qj = j >> 2, sj = j & 3;
                if (sj == 0 && qj < 3) load_cols(qj + 1, (qj + 1) & 1);
                const f32x4 a4 = colA[qj & 1][sj];
                const float own = (j == col ? 1.f : 0.f) - acc[qj];  // row j, valid in lane sub == sj
                float tj;
                if (sj == 0) tj = dpp_f<0x00>(own);       // quad_perm [0,0,0,0]
                else if (sj == 1) tj = dpp_f<0x55>(own);  // quad_perm [1,1,1,1]
                else if (sj == 2) tj = dpp_f<0xAA>(own);  // quad_perm [2,2,2,2]
                else tj = dpp_f<0xFF>(own);               // quad_perm [3,3,3,3]
                Tc[qj] = sub == sj ? tj : Tc[qj];
#pragma unroll
                for (int q = qj; q < 4; ++q) {
                    if (q > qj) acc[q] += a4[q] * tj;
                    else if (sj < 3) acc[q] += (sub > sj ? a4[q] : 0.f) * tj;
                }
            }
            float* const tw = tblk(wave);
#pragma unroll
            for (int q = 0; q < 4; ++q) tw[(4 * q + sub) * kTS + col] = Tc[q];
        }
        __syncthreads();  // diagonal blocks visible; step 4 has read Al

        // acc += A_IK T_KJ, T_KJ in slot sKJ.  Slice kk, lane group lg carries
        // k = 4 lg + kk: the 64 lanes' A reads then fall in 64 banks.
        auto mul_at = [&](f32x4 acc, int I, int K, int sKJ) {
            const float* t = tblk(sKJ);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Ad[16 * K + 4 * lg + kk][(li & 3) * kAQ + 4 * I + (li >> 2)],
                                                           t[(4 * lg + kk) * kTS + li], acc, 0, 0, 0);
            return acc;
        };
        // acc += T_slot W, W in accumulator layout
        auto mul_tw = [&](f32x4 acc, int slot, const f32x4& w) {
            const f32x4 t4 = *reinterpret_cast<const f32x4*>(&tblk(slot)[li * kTS + 4 * lg]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(t4[i], w[i], acc, 0, 0, 0);
            return acc;
        };
        // Tp block (I, J) = -x diag(beta m), x in accumulator layout
        auto put_tp = [&](int I, int J, const f32x4& x) {
            const float bm = -s_bm[16 * J + li];
#pragma unroll
            for (int i = 0; i < 4; ++i) Al[16 * I + 4 * lg + i][16 * J + li] = f2bf(x[i] * bm);
        };
        {
            const float bm = s_bm[16 * wave + col];
#pragma unroll
            for (int q = 0; q < 4; ++q) Al[16 * wave + 4 * q + sub][16 * wave + col] = f2bf(Tc[q] * bm);
            // upper blocks (0,1) (0,2) (0,3) (1,2) (1,3) (2,3): waves 0, 1 two, waves 2, 3 one
            const uint2 z = {0u, 0u};
            for (int e = wave; e < 6; e += 4) {
                const int I = e < 3 ? 0 : (e < 5 ? 1 : 2), J = e < 3 ? e + 1 : (e < 5 ? e - 1 : 3);
                *reinterpret_cast<uint2*>(&Al[16 * I + col][16 * J + 4 * sub]) = z;
            }
        }
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        f32x4 w2 = zero, w3 = zero, x = zero;
        if (wave == 0) {
            const f32x4 t = mul_tw(zero, 1, mul_at(zero, 1, 0, 0));
            w2 = mul_at(zero, 2, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) tblk(4)[(4 * lg + i) * kTS + li] = -t[i];
            put_tp(1, 0, t);
        } else if (wave == 1) {
            const f32x4 t = mul_tw(zero, 3, mul_at(zero, 3, 2, 2));
            w2 = mul_at(zero, 2, 0, 0);
            w3 = mul_at(zero, 3, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) tblk(5)[(4 * lg + i) * kTS + li] = -t[i];
            put_tp(3, 2, t);
        } else if (wave == 2) {
            put_tp(2, 1, mul_tw(zero, 2, mul_at(zero, 2, 1, 1)));
        } else {
            w2 = mul_at(zero, 2, 1, 1);
            x = mul_tw(zero, 3, mul_at(zero, 3, 1, 1));
        }
        __syncthreads();  // T_10, T_32 visible
        if (wave == 0) {
            put_tp(2, 0, mul_tw(zero, 2, mul_at(w2, 2, 1, 4)));
        } else if (wave == 1) {
            w2 = mul_at(w2, 2, 1, 4);
            w3 = mul_at(w3, 3, 1, 4);
            put_tp(3, 0, mul_tw(mul_tw(zero, 5, w2), 3, w3));
        } else if (wave == 3) {
            put_tp(3, 1, mul_tw(x, 5, w2));
        } else if (N.valid) {  // the gate wave (no product here): the next unit's gates
            static_assert(kGateWave == 2, "the gate wave is the one idle in this round");
            gv = gate_vals(p, L, lane, N.nvalid);
        }
    }
    gv_ready = N.valid;
    __syncthreads();

    // 6) Tp fragments, two per wave, stored with the next unit's stores.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int mt = wave, s = i;  // fragment f = 2 wave + i
        const bf16* rp = &Al[16 * mt + m16][32 * s + 4 * g4];  // Tp (step 5)
        const u32x2 lo = *reinterpret_cast<const u32x2*>(rp);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(rp + 16);
        tpf[i] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
    wc_prev = wc;
    have_prev = true;
    __syncthreads();  // Tp and T blocks are read before the next unit's K and Aq are stored
    u = u_next;
    U = N;
    }
    if (have_prev) store_tp<RF>(p, wc_prev, wave, lane, tpf);
}

// ---------------------------------------------------------------------------
// Kernel 2
// ---------------------------------------------------------------------------
// Per-chunk operands staged in LDS (one buffer; the kernels double-buffer).
// Every block is a run of 1 KiB "fragments": 64 lanes x 16 bytes, lane l's
// 16 bytes at offset 16 l, i.e. exactly one MFMA operand register quad.
constexpr int kFragB = 1024;
enum { kModeOut = 0, kModeMap = 1 };

// Staging layout of one buffer.  The map pass (no outputs) stages neither Q
// nor Aq.  V is per wave: [64 rows][16 NT columns] bf16.
template <int MODE, int NW, int NT>
struct Stage {
    static constexpr bool out = MODE == kModeOut;
    static constexpr int offK = 0;                                  // 16: (mt, s), lane slots swizzled (kslot)
    static constexpr int offQ = offK + 16 * kFragB;                 // 16 (out only)
    static constexpr int offT = offQ + (out ? 16 : 0) * kFragB;     // 6: nonzero Tp fragments
    static constexpr int offA = offT + 6 * kFragB;                  // 6 (out only): Aq slots used
    static constexpr int offG = offA + (out ? 6 : 0) * kFragB;      // gamma, m scale gamma, gamma_C/gamma
    static constexpr int offV = offG + kFragB;
    static constexpr int vWave = 2 * NT * kFragB;
    static constexpr int bytes = offV + NW * vWave;
    static constexpr int stores = out ? 4 * NT : 0;                 // output stores per chunk per wave
};



// Per-lane byte offsets of the staging copies, fixed for the whole kernel.
struct StageLane {
    uint32_t k;   // K fragment slot `lane`: row kslot_row(lane), k offset 8 (lane >> 4)
    uint32_t q;   // Q fragment: row (lane & 15), k offset 8 (lane >> 4)
    uint32_t fr;  // workspace fragment or gate block: 16 lane
    uint32_t v;   // V tile: row lane / (2 NT), 8 columns (lane % (2 NT))
};

// K fragments are staged with their 16-byte lane slots swizzled: the data of
// fragment lane (m, g) (row m, k group g) sits in slot 16 g + (m ^ 4 g).
// Plain fragment reads stay conflict free, and the transposing reads that
// build K^T (16 lanes reading rows T0..T0+3 of four k groups) hit 16
// different slots modulo 16 instead of 4.
__device__ __forceinline__ int kslot(int m, int g) { return 16 * g + (m ^ (4 * g)); }
__device__ __forceinline__ int kslot_row(int slot) { return (slot & 15) ^ (4 * (slot >> 4)); }

// Copies of one chunk's operands into `buf`, all issued together at the start
// of the previous chunk's work (spreading them between its MFMA phases was
// measured slower: a copy that meets a full memory pipeline stalls the MFMA
// work queued behind it).  Shared jobs (K, Q, Tp, Aq and Kt fragments, the
// gate block) are dealt round robin to the NW waves; each wave copies its own
// V tile when `v_on`.  Full chunks use uniform bases plus the lane offsets;
// the last, partial chunk clamps rows to the sequence (so no load leaves the
// tensors) and its padded rows are zeroed after arrival.

template <int MODE, int NW, int NT>
struct Stager {
    using St = Stage<MODE, NW, NT>;
    static constexpr int nK = 16, nQ = St::out ? 16 : 0, nT = 6, nA = St::out ? 6 : 0;
    static constexpr int NJ = nK + nQ + nT + nA + 1;  // + the gate block
    const PrefillParams* p;
    lds_u8* buf;
    size_t row_base, wc;
    int nvalid, wave, lane, col0_wave;
    bool on, v_on;
    const StageLane* L;

    __device__ __forceinline__ void issue() const {
        if (!on) return;
        const bool full = nvalid == kC;
        const int m = lane & 15, g = lane >> 4;
        const unsigned char* kb = reinterpret_cast<const unsigned char*>(p->k + row_base * kDK);
        const unsigned char* qb = reinterpret_cast<const unsigned char*>(p->q + row_base * kDK);
        // The shared jobs are staged contiguously in job order (K, Q, Tp, Aq,
        // gate block), so job f lands at f KiB.  Each wave walks only its own
        // jobs f = wave, wave + NW, ... (a uniform loop).
        static_assert(St::offK == 0 && St::offQ == nK * kFragB && St::offT == (nK + nQ) * kFragB &&
                          St::offG == (nK + nQ + nT + nA) * kFragB && (!St::out || St::offA == St::offT + nT * kFragB),
                      "staging layout must follow job order");
        for (int f = wave; f < NJ; f += NW) {
            lds_u8* const dst = buf + f * kFragB;
            if (f < nK + nQ) {
                const bool isq = f >= nK;
                const int ff = isq ? f - nK : f;
                const unsigned char* base = isq ? qb : kb;
                if (full) {
                    dma16(base + (ff >> 2) * 16 * kDK * 2 + (ff & 3) * 64, isq ? L->q : L->k, dst);
                } else {
                    const int row = min(16 * (ff >> 2) + (isq ? m : kslot_row(lane)), nvalid - 1);
                    dma16(base, static_cast<uint32_t>((row * kDK + 32 * (ff & 3) + 8 * g) * 2), dst);
                }
            } else {
                // record fragments: Tp, then Aq (output only), then the gate block
                const unsigned char* rec = reinterpret_cast<const unsigned char*>(p->wsR + wc * kRecFull * 64);
                const int j = f - nK - nQ;
                dma16(rec + (j < nT + nA ? j : kRecFull - 1) * kFragB, L->fr, dst);
            }
        }
        if (v_on) {
            constexpr int kRowsPerV = 32 / NT;  // V rows per 1 KiB copy
#pragma unroll
            for (int it = 0; it < 2 * NT; ++it) {
                if (full) {
                    dma16(p->v + (row_base + kRowsPerV * it) * p->dv, L->v,
                          buf + St::offV + wave * St::vWave + it * kFragB);
                } else {
                    const int row = min(kRowsPerV * it + lane / (2 * NT), nvalid - 1);
                    dma16(p->v + row_base * p->dv,
                          static_cast<uint32_t>((row * p->dv + col0_wave + 8 * (lane % (2 * NT))) * 2),
                          buf + St::offV + wave * St::vWave + it * kFragB);
                }
            }
        }
    }
};

// Zero the rows >= nvalid of the staged K, Q and V (partial chunk only).
template <int MODE, int NW, int NT>
__device__ __forceinline__ void zero_pad_rows(lds_u8* buf, int nvalid, int wave, int lane) {
    using St = Stage<MODE, NW, NT>;
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int f = 0; f < (St::out ? 32 : 16); ++f)  // K then Q (contiguous); K slots are swizzled
        if (f % NW == wave && 16 * ((f & 15) >> 2) + (f < 16 ? kslot_row(lane) : (lane & 15)) >= nvalid)
            *reinterpret_cast<lds_u32x4*>(buf + St::offK + f * kFragB + 16 * lane) = z;
#pragma unroll
    for (int it = 0; it < 2 * NT; ++it)
        if ((32 / NT) * it + lane / (2 * NT) >= nvalid)
            *reinterpret_cast<lds_u32x4*>(buf + St::offV + wave * St::vWave + it * kFragB + 16 * lane) = z;
}

__device__ __forceinline__ bf16x8 frag(const lds_u8* buf, int off, int lane) {
    return *reinterpret_cast<const lds_bf16x8*>(buf + off + 16 * lane);
}

// K fragment f = 4 mt + s (rows 16 mt + m, k 32 s + 8 g) from the swizzled slots.
__device__ __forceinline__ bf16x8 kfrag(const lds_u8* kbuf, int f, int lane) {
    return *reinterpret_cast<const lds_bf16x8*>(kbuf + f * kFragB + 16 * kslot(lane & 15, lane >> 4));
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// K^T fragment (r, s), the A operand of the state update: lane (m, g) gets
// K[32 s + pi(g, j)][rho(r, m / 4, m % 4)] for j = 0..7, from the staged K.
// ds_read_b64_tr_b16 hands output lane i of each 16-lane group element i % 4
// of the 8 bytes read by lanes 4 j + i / 4 (j = 0..3); so source lane 4 j + a
// reads row T0 + j at columns base(a) .. base(a) + 3, base(a) = rho(r, a, 0),
// and output lane m = 4 a + p receives column rho(r, a, p) of rows T0 .. T0 + 3.
// Two such reads (T0 = 32 s + 4 g and 32 s + 16 + 4 g) give the pi order.
// Only the K slot depends on the lane (row 4 g + j of the 16-row block,
// k group a): `kt_lane` = 16 kslot(4 g + j, a), computed once; the rest of
// the address is a compile-time offset.
__device__ __forceinline__ uint32_t kt_lane_offset(int lane) {
    return 16u * static_cast<uint32_t>(kslot(4 * (lane >> 4) + ((lane >> 2) & 3), lane & 3));
}
__device__ __forceinline__ bf16x8 ktfrag(const lds_u8* kbuf, uint32_t kt_lane, int r, int s) {
    const lds_u8* base = kbuf + kt_lane + (r >> 1) * kFragB + 8 * (r & 1);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + (2 * s) * 4 * kFragB));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + (2 * s + 1) * 4 * kFragB));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    return as_bf16x8(u32x4{l2[0], l2[1], h2[0], h2[1]});
}

// bf16 of (x - bf16(x)) for a pair of accumulator quads: the low half of a
// two-term bf16 split.
__device__ __forceinline__ bf16x8 pack8_lo(const f32x4 lo, const f32x4 hi, const bf16x8 h) {
    f32x4 dl, dh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dl[i] = lo[i] - bf2f(h[i]);
        dh[i] = hi[i] - bf2f(h[4 + i]);
    }
    return pack8(dl, dh);
}


// One chunk of the state recurrence for a 128 x (16 NT) column tile, operands
// in LDS.  `ob` points at out[row_base][0] (uniform).  Operand fragments are
// read from LDS one phase ahead of their use (none depends on the state), so
// the MFMA chain that does depend on it rarely waits on LDS, without holding
// every fragment in registers at once.  `v_zero`: the tile has no V (identity
// columns of the map pass).  `next` issues the following chunk's copies.
template <int MODE, int NW, int NT>
__device__ __forceinline__ void state_chunk(const lds_u8* buf, f32x4 (&S)[8][NT], uint16_t* ob, int orow, int nvalid,
                                            int wave, int lane, int col0_wave, bool v_zero, uint32_t kt_lane,
                                            const Stager<MODE, NW, NT>& next) {
    using St = Stage<MODE, NW, NT>;
    const int n = lane & 15, g = lane >> 4;
    const lds_f32* G = reinterpret_cast<const lds_f32*>(buf + St::offG);
    const lds_u16* Vs = reinterpret_cast<const lds_u16*>(buf + St::offV + wave * St::vWave);

    next.issue();

    // (a) X = K S (and P = Q S for the output), in two k-halves so only half
    //     of the K and Q fragments is held at a time.
    f32x4 X[4][NT], P[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) X[mt][nt] = P[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        bf16x8 kf[4][2], qf[St::out ? 4 : 1][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int f = 4 * mt + 2 * half + s2;
                kf[mt][s2] = kfrag(buf + St::offK, f, lane);
                if constexpr (St::out) qf[mt][s2] = frag(buf, St::offQ + f * kFragB, lane);
            }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int s = 2 * half + s2;
            bf16x8 Bs[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) Bs[nt] = pack8(S[2 * s][nt], S[2 * s + 1][nt]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    X[mt][nt] = mfma16x16x32(kf[mt][s2], Bs[nt], X[mt][nt]);
                    if constexpr (St::out) P[mt][nt] = mfma16x16x32(Bs[nt], qf[mt][s2], P[mt][nt]);
                }
        }
    }
    bf16x8 tf[6], af[St::out ? 6 : 1], ktf[8][2];
    // With one wave per SIMD (NW <= 4) the Kt fragments are read here, while
    // (a) drains; with two (NW = 8) the other wave covers their latency, so
    // they are read just before (e) to keep this wave within 256 registers.
    constexpr bool kEarlyKt = NW <= 4;
    auto load_kt = [&]() {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            ktf[r][0] = ktfrag(buf + St::offK, kt_lane, r, 0);
            ktf[r][1] = ktfrag(buf + St::offK, kt_lane, r, 1);
        }
    };
#pragma unroll
    for (int f = 0; f < 6; ++f) tf[f] = frag(buf, St::offT + f * kFragB, lane);
    if constexpr (kEarlyKt) load_kt();
    // V in the accumulator layout (column n, rows 16 mt + 4 g + i): one
    // transposing read per (mt, nt) -- source lane 4 j + a of group g reads
    // row 16 mt + 4 g + j at columns 16 nt + 4 a .. + 3.  Kept as bf16 until use.
    i16x4 vv[NT][4];
    const lds_u8* vrow = reinterpret_cast<const lds_u8*>(Vs) + ((4 * g + ((lane >> 2) & 3)) * 16 * NT + 4 * (lane & 3)) * 2;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            vv[nt][mt] = v_zero ? i16x4{0, 0, 0, 0}
                                : __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                      (lds_i16x4*)(vrow + (16 * mt * 16 * NT + 16 * nt) * 2));
    f32x4 gam[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) gam[mt] = *reinterpret_cast<const lds_f32x4*>(G + 16 * mt + 4 * g);
    const float gC = G[kC - 1];
    // (b) Y = V - gamma o X (in place in X).
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                X[mt][nt][i] = bf2f(static_cast<uint16_t>(vv[nt][mt][i])) - gam[mt][i] * X[mt][nt][i];
    // (c) dV = Tp Y.
    f32x4 D[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) D[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Tp is lower triangular: fragments (0, 1) and (1, 1) are zero and absent.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        bf16x8 BY[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) BY[nt] = pack8(X[2 * s][nt], X[2 * s + 1][nt]);
#pragma unroll
        for (int mt = 2 * s; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) D[mt][nt] = mfma16x16x32(tf[aq_index(mt, s)], BY[nt], D[mt][nt]);
    }
    if constexpr (St::out) {
#pragma unroll
        for (int i = 0; i < 6; ++i) af[i] = frag(buf, St::offA + i * kFragB, lane);
    }
    // The state update takes dV with its rows scaled by gamma_C / gamma_t
    // (the decay from token t to the chunk end); the output takes dV as is.
    f32x4 kd[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) kd[mt] = *reinterpret_cast<const lds_f32x4*>(G + 128 + 16 * mt + 4 * g);
    bf16x8 BS0[NT], BS1[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        BS0[nt] = pack8(kd[0] * D[0][nt], kd[1] * D[1][nt]);
        BS1[nt] = pack8(kd[2] * D[2][nt], kd[3] * D[3][nt]);
    }
    if constexpr (!kEarlyKt) load_kt();
    // (e) S <- gamma_C S + K^T (decay o dV)  (issued before (d): the recurrence's critical path).
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            S[r][nt] *= gC;
            S[r][nt] = mfma16x16x32(ktf[r][0], BS0[nt], S[r][nt]);
            S[r][nt] = mfma16x16x32(ktf[r][1], BS1[nt], S[r][nt]);
        }
    if constexpr (St::out) {
        bf16x8 BD0[NT], BD1[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            BD0[nt] = pack8(D[0][nt], D[1][nt]);
            BD1[nt] = pack8(D[2][nt], D[3][nt]);
        }
        // (d) O^T = (m scale gamma) o P^T + dV^T Aq^T, formed transposed so
        //     each lane holds 4 consecutive output columns of one token: the
        //     dV packs are the A operands and the Aq fragments the B operands
        //     as they stand (both carry their k in pi order), and P^T = S^T Q^T
        //     was accumulated with the operands of Q S swapped.  Lane (n, g) of
        //     tile mt stores out[token 16 mt + n][16 nt + 4 g .. + 3] as 8 bytes.
        float co[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) co[mt] = G[64 + 16 * mt + n];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            f32x4 O[4];
            O[0] = mfma16x16x32(BD0[nt], af[0], co[0] * P[0][nt]);
            O[1] = mfma16x16x32(BD0[nt], af[1], co[1] * P[1][nt]);
            O[2] = mfma16x16x32(BD1[nt], af[3], mfma16x16x32(BD0[nt], af[2], co[2] * P[2][nt]));
            O[3] = mfma16x16x32(BD1[nt], af[5], mfma16x16x32(BD0[nt], af[4], co[3] * P[3][nt]));
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int row = 16 * mt + n;
                if (row < nvalid)
                    *reinterpret_cast<u32x2*>(ob + row * orow + col0_wave + 16 * nt + 4 * g) = pack4_bf16(O[mt]);
            }
        }
    }
}

// Work decomposition of the state pass.
struct StateGrid {
    int nvg;         // workgroups per (head, group)
    int ngroups;     // chunk groups per sequence (G)
    int ngroups_run; // groups per sequence this launch covers (map pass: G - 1)
    int nheads;      // sequences x heads
    float* psi;      // [nheads][G][dv/16][8][64][4] fp32 (16-column tile, accumulator tile r,
                     // lane, slot): map pass zero-state results, then (scan) the initial
                     // state of group j + 1 in slot j
    uint16_t* phi;   // map pass: transitions as MFMA A fragments, [nheads][G][8][4][64][8]
                     // bf16 (row tile r, k-step, lane: row rho(r, n/4, n%4), columns 32ks + 8g..)
    // Packed sequences: per-sequence group counts planned on the device
    // (gdn_prefill_plan_kernel), or null for one group count G for all.
    // Table: [0] slots (sum of G_i), [1] map slots (sum of G_i - 1), then
    // (G_i, first slot of sequence i) for every sequence, then kPlanCap
    // entries (sequence << 8 | group) for every slot, then kPlanCap for every
    // map slot.  psi/phi of (sequence, head, group) sit at slot (first + group)
    // x H + head instead of ((sequence H + head) G + group).
    const int32_t* plan;
    int nseq;
};

constexpr int kPlanCap = 256;  // slot table capacity (slots per head never exceed 256 / H)
__device__ __forceinline__ int plan_groups(const StateGrid& sg, int sidx) { return sg.plan[2 + 2 * sidx]; }
__device__ __forceinline__ int plan_first(const StateGrid& sg, int sidx) { return sg.plan[3 + 2 * sidx]; }
// psi/phi unit of (sequence, head, group).
__device__ __forceinline__ size_t group_unit(const StateGrid& sg, int H, int sidx, int h, int grp) {
    return sg.plan ? static_cast<size_t>(plan_first(sg, sidx) + grp) * H + h
                   : static_cast<size_t>(sidx * H + h) * sg.ngroups + grp;
}

// State pass over one chunk group per workgroup (NW waves, NT 16-column tiles
// each, of one (sequence, head)).
//   kModeOut: from the group's initial state (state_in for group 0, else the
//             scan's result), writes the outputs; the last group writes
//             state_out.
//   kModeMap: columns [0, dv) start from zero (psi), columns [dv, dv + 128)
//             from the identity with V = 0 (phi = the group's transition).
//             The last group's map is never needed and is not computed.
// With one group (G = 1) only the output pass runs.  The chunk operands are
// shared by the waves and double-buffered in LDS: the copies for chunk c+1
// are in flight while chunk c is computed.
template <int MODE, int NW, int NT>
__global__ __launch_bounds__(64 * NW) void gdn_prefill_state_kernel(PrefillParams p, StateGrid sg) {
    using St = Stage<MODE, NW, NT>;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2][St::bytes];
    lds_u8* const buf0 = (lds_u8*)&smem[0][0];
    lds_u8* const buf1 = (lds_u8*)&smem[1][0];

    const int wg = blockIdx.x;
    const int nunits = sg.nheads * sg.ngroups_run;
    int head, grp, vg, ngroups;
    if (sg.plan) {
        // ngroups_run = slots per head in the grid: (head, slot, column part)
        vg = wg % sg.nvg;
        const int hh = (wg / sg.nvg) / sg.ngroups_run, q = (wg / sg.nvg) % sg.ngroups_run;
        if (hh >= p.H || q >= sg.plan[MODE == kModeMap ? 1 : 0]) return;  // uniform over the workgroup
        const int e = sg.plan[2 + 2 * sg.nseq + (MODE == kModeMap ? kPlanCap : 0) + q];
        head = (e >> 8) * p.H + hh;
        grp = e & 255;
        ngroups = plan_groups(sg, e >> 8);
    } else {
        if (p.xcd_heads) {
            const HeadItem hi = head_major_xcd(wg, sg.ngroups_run * sg.nvg);
            head = hi.head;
            grp = hi.item / sg.nvg;
            vg = hi.item % sg.nvg;
        } else {
            vg = wg % sg.nvg;
            head = (wg / sg.nvg) / sg.ngroups_run;
            grp = (wg / sg.nvg) % sg.ngroups_run;
        }
        if (head * sg.ngroups_run + grp >= nunits) return;  // uniform over the workgroup
        ngroups = sg.ngroups;
    }
    const int sidx = head / p.H;
    const int h = head % p.H;
    const SeqInfo sq = seq_info(p, sidx);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4;
    const int dv = p.dv;
    const int col0_wave = (vg * NW + wave) * 16 * NT;  // map pass: >= dv means identity columns
    const bool phi_cols = MODE == kModeMap && col0_wave >= dv;
    const int nchunks = (sq.len + kC - 1) / kC;
    const int glen = (nchunks + ngroups - 1) / ngroups;
    const int c_begin = min(grp * glen, nchunks), c_end = min(c_begin + glen, nchunks);
    const StageLane L = {static_cast<uint32_t>(kslot_row(lane) * kDK * 2 + (lane >> 4) * 16),
                         static_cast<uint32_t>((lane & 15) * kDK * 2 + (lane >> 4) * 16),
                         static_cast<uint32_t>(16 * lane),
                         static_cast<uint32_t>((lane / (2 * NT)) * dv * 2 + (lane % (2 * NT)) * 16 +
                                               (phi_cols ? 0 : col0_wave) * 2)};

    const uint32_t kt_lane = kt_lane_offset(lane);

    // State tile: S[r][nt][i] = S[rho(r, g, i)][col0_wave + 16 nt + n].
    f32x4 S[8][NT];
    if constexpr (MODE == kModeMap) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    S[r][nt][i] = (phi_cols && rho_row(r, g, i) == col0_wave - dv + 16 * nt + n) ? 1.f : 0.f;
    } else if (grp > 0) {
        // Initial state of this group, left by the scan in psi slot grp - 1.
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4* Ps = reinterpret_cast<const f32x4*>(
                sg.psi + (group_unit(sg, p.H, sidx, h, grp - 1) * (dv / 16) + col0_wave / 16 + nt) * 2048);
#pragma unroll
            for (int r = 0; r < 8; ++r) S[r][nt] = Ps[r * 64 + lane];
        }
    } else if (p.state_in) {
        const float* sin = p.state_in + static_cast<size_t>(sidx * p.H + h) * kDK * dv;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) S[r][nt][i] = sin[rho_row(r, g, i) * dv + col0_wave + 16 * nt + n];
    } else {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) S[r][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const size_t head_row0 = static_cast<size_t>(sq.b * p.H + h) * p.T_stride + sq.tok0;
    auto rows = [&](int c) { return head_row0 + static_cast<size_t>(c) * kC; };
    // Output rows: head-major out[(sequence, head)][token][dv], or token-major
    // out[sequence][token][head][dv] (row stride H dv), as the caller asked.
    const int orow = p.out_tm ? p.H * dv : dv;
    auto obase = [&](int c) {
        const size_t tok = static_cast<size_t>(sq.b) * p.T_stride + sq.tok0 + static_cast<size_t>(c) * kC;
        return p.out_tm ? (tok * p.H + h) * dv : rows(c) * dv;
    };
    auto nval = [&](int c) { return min(kC, sq.len - c * kC); };
    auto wcof = [&](int c) { return static_cast<size_t>(sq.slot0 + c) * p.H + h; };
    auto step = [&](int c, lds_u8* cur, lds_u8* nxt) {
        // Chunk c's copies were issued before chunk c-1's output stores.
        if (c == c_begin)
            wait_vm<0>();
        else
            wait_vm<St::stores>();
        lds_barrier();  // chunk c staged by every wave; nobody still reads `nxt`
        const Stager<MODE, NW, NT> next = {&p,   nxt,  rows(c + 1), wcof(c + 1),     nval(c + 1), wave,
                                           lane, col0_wave, c + 1 < c_end, !phi_cols, &L};
        const int nv = nval(c);
        if (nv < kC) {
            zero_pad_rows<MODE, NW, NT>(cur, nv, wave, lane);
            lds_barrier();
        }
        state_chunk<MODE, NW, NT>(cur, S, p.out + obase(c), orow, nv, wave, lane, col0_wave, phi_cols, kt_lane,
                                  next);
    };

    {
        const Stager<MODE, NW, NT> first = {&p,   buf0, rows(c_begin), wcof(c_begin),   nval(c_begin), wave,
                                            lane, col0_wave, c_begin < c_end, !phi_cols, &L};
        first.issue();
    }
    for (int c = c_begin; c < c_end; c += 2) {
        step(c, buf0, buf1);
        if (c + 1 < c_end) step(c + 1, buf1, buf0);
    }

    if constexpr (MODE == kModeOut) {
        if (grp != ngroups - 1) return;
        float* so = p.state_out + static_cast<size_t>(sidx * p.H + h) * kDK * dv;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) so[rho_row(r, g, i) * dv + col0_wave + 16 * nt + n] = S[r][nt][i];
    } else if (phi_cols) {
        // phi as A fragments: the accumulator holds 16-column tile T of phi
        // (a column per lane); a fragment lane needs 8 consecutive columns of
        // one row.  Transpose each 16x16 tile through this wave's own V area
        // (unused by identity columns), then store 512 contiguous bytes.
        uint16_t* Ph = sg.phi + group_unit(sg, p.H, sidx, h, grp) * kDK * kDK;
        lds_u16* tt = reinterpret_cast<lds_u16*>(buf0 + St::offV + wave * St::vWave);
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int T = (col0_wave - dv) / 16 + nt;
#pragma unroll
                for (int i = 0; i < 4; ++i) tt[(4 * g + i) * 16 + n] = f2bf_bits(S[r][nt][i]);
                if (lane < 32) {  // fragment lanes 16 (2 (T % 2) + h) + n: row n of the tile, columns 8h..
                    const int h = lane >> 4;
                    const u32x4 v = *reinterpret_cast<const lds_u32x4*>(tt + n * 16 + 8 * h);
                    *reinterpret_cast<u32x4*>(Ph + ((r * 4 + (T >> 1)) * 64 + 16 * (2 * (T & 1) + h) + n) * 8) = v;
                }
            }
    } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            f32x4* Ps = reinterpret_cast<f32x4*>(
                sg.psi + (group_unit(sg, p.H, sidx, h, grp) * (dv / 16) + col0_wave / 16 + nt) * 2048);
#pragma unroll
            for (int r = 0; r < 8; ++r) Ps[r * 64 + lane] = S[r][nt];
        }
    }
}

// ---------------------------------------------------------------------------
// Kernel 2b: the state pass for dv % 128 == 0 -- four compute waves of 32
// columns and one copy wave
// ---------------------------------------------------------------------------
// A workgroup owns 128 state columns of one (sequence, head, chunk group):
// compute wave w owns columns 32 w .. 32 w + 31 as two 16-column MFMA tiles,
// so every operand fragment it reads from LDS feeds two MFMAs (with 16-column
// waves, eight per CU, the LDS reads of a chunk step outlast its MFMAs).
// In the output pass three copy waves do all global memory traffic of the
// chunk loop: waves 4 and 5 stage chunk c + 1 (half of the copies each)
// while the compute waves work on chunk c, and wave 6 writes chunk c - 1's
// outputs, which the compute waves left in LDS, as whole 256-byte rows
// (77 KiB of memory traffic a chunk step): loads and stores from separate
// waves flow at the same time, and no compute wave stalls on a full memory
// queue.  (Staging chunk c + 2 through the loaders' registers, for two steps
// of copy latency instead of one, measured slower: the step is bound by its
// LDS traffic, not by the copies' latency.)  The output pass runs one workgroup per CU
// (one compute wave per SIMD), the map pass two.
// Per chunk, DMA-staged into one of two LDS buffers:
//   K   16 fragments, lane slots swizzled (kslot) for the K^T transposing reads
//   Q   16 fragments (output pass)
//   record: Tp 6, Aq 6 (output pass), gate block 1
//   V   compute wave w's [64 rows][32 columns] bf16 at offV + 4 KiB w (not
//       for phi columns)
// and in the output pass two output tiles [64 rows][128 columns] bf16 (row
// pitch 272 bytes: the compute waves' 8-byte writes then hit all 64 banks).
// Full chunks take a path without per-row checks; a sequence's partial last
// chunk clamps its copies to the sequence and predicates its output rows.
// Rows past the sequence end stay finite copies of the last row, and their Tp
// rows and columns are zero (beta m = 0 there), so they add exact zeros.
constexpr int kObPitch = 272;                // output tile row pitch (bytes)
constexpr int kObBytes = kC * kObPitch;      // one output tile
template <int MODE, int NT = 2>
struct Stage4 {
    static_assert(NT == 2 || (NT == 1 && MODE == kModeOut), "16-column tiles per compute wave");
    static constexpr bool out = MODE == kModeOut;
    static constexpr int cols = 64 * NT;  // state columns of a workgroup (4 compute waves x 16 NT)
    static constexpr int offK = 0;
    static constexpr int offQ = 16 * kFragB;
    static constexpr int offR = offQ + (out ? 16 : 0) * kFragB;
    // copied record fragments: Tp, the gate block and (output pass) the token block
    static constexpr int nRec = out ? kRecShort : kRecGShort + 1;
    static constexpr int offTp = offR;
    static constexpr int offG = offR + kRecGShort * kFragB;
    static constexpr int offH = offR + kRecH * kFragB;
    static constexpr int offAq = offR + nRec * kFragB;  // output pass: Aq, formed by the copy waves
    static constexpr int offV = offAq + (out ? 6 : 0) * kFragB;
    static constexpr int bytes = offV + 8 * NT * kFragB;  // V: [64 rows][32 columns] per 32 columns
    static constexpr int ob_bytes = out ? kObBytes : 0;
    // waves: 4 compute, then (output pass) 2 copying chunks in, a store wave
    // and the Aq wave
    static constexpr int loaders = out ? 2 : 0;
    static constexpr int nWaves = 4 + loaders + (out ? 2 : 0);
    static constexpr int nStores = out ? kC * 256 / kFragB : 0;  // output store instructions per chunk
};

// Per-lane byte offsets of the copies (fixed for the kernel).
struct Lane4 {
    uint32_t k, q, r, v;
};

// Issue chunk `c`'s copies into `buf`: jobs first, first + STRIDE, ... of
// each kind (the output pass's copy wave takes all of them, STRIDE 1; in the
// map pass each compute wave takes a quarter, STRIDE 4).  `row0`: q/k/v row
// of the chunk's first token; `rec`: the chunk's record; `vcol0`: the
// workgroup's first V column.
template <int MODE, int NT, bool FULL, int STRIDE>
__device__ __forceinline__ void stage4_issue(const PrefillParams& p, lds_u8* buf, size_t row0, const u32x4* rec,
                                             int vcol0, int nvalid, int first, int lane, const Lane4& L, bool v_on) {
    using St = Stage4<MODE, NT>;
    // Full chunks: uniform bases, fixed lane offsets.  The partial chunk:
    // base at the chunk's first row and each lane's row clamped to the
    // sequence, so every offset is non-negative and in range.
    const unsigned char* kc = reinterpret_cast<const unsigned char*>(p.k + row0 * kDK);
    const unsigned char* qc = reinterpret_cast<const unsigned char*>(p.q + row0 * kDK);
#pragma unroll
    for (int i = 0; i < 16 / STRIDE; ++i) {  // fragment f = 4 mt + s: rows 16 mt.., k 32 s..
        const int f = first + STRIDE * i, mt = f >> 2, s = f & 3;
        if (FULL) {
            dma16(kc + mt * 16 * kDK * 2 + 64 * s, L.k, buf + St::offK + f * kFragB);
        } else {
            const int row = min(16 * mt + kslot_row(lane), nvalid - 1);
            dma16(kc, static_cast<uint32_t>((row * kDK + 32 * s + 8 * (lane >> 4)) * 2), buf + St::offK + f * kFragB);
        }
    }
    if constexpr (St::out) {
#pragma unroll
        for (int i = 0; i < 16 / STRIDE; ++i) {
            const int f = first + STRIDE * i, mt = f >> 2, s = f & 3;
            if (FULL) {
                dma16(qc + mt * 16 * kDK * 2 + 64 * s, L.q, buf + St::offQ + f * kFragB);
            } else {
                const int row = min(16 * mt + (lane & 15), nvalid - 1);
                dma16(qc, static_cast<uint32_t>((row * kDK + 32 * s + 8 * (lane >> 4)) * 2),
                      buf + St::offQ + f * kFragB);
            }
        }
    }
    const unsigned char* rb = reinterpret_cast<const unsigned char*>(rec);
#pragma unroll
    for (int i = 0; i < (St::nRec + STRIDE - 1) / STRIDE; ++i) {
        const int j = first + STRIDE * i;
        if (j < St::nRec) {
            dma16(rb + j * kFragB, L.r, buf + St::offR + j * kFragB);
        }
    }
    if (v_on) {  // job u: compute wave u / 4's columns, rows 16 (u % 4) ..
        const unsigned char* vb = reinterpret_cast<const unsigned char*>(p.v + row0 * p.dv + vcol0);
#pragma unroll
        for (int i = 0; i < 8 * NT / STRIDE; ++i) {
            const int u = first + STRIDE * i, w = u >> 2, it = u & 3;
            lds_u8* vd = buf + St::offV + u * kFragB;
            if (FULL) {
                dma16(vb + static_cast<size_t>(16 * it) * p.dv * 2 + 64 * w, L.v, vd);
            } else {
                const int row = min(16 * it + (lane >> 2), nvalid - 1);
                dma16(vb, static_cast<uint32_t>((row * p.dv + 32 * w + 8 * (lane & 3)) * 2), vd);
            }
        }
    }
}

// The output pass's copy waves form the six nonzero fragments of the staged
// chunk's causal Aq = (m scale) (Q K^T o Gamma) into the buffer's Aq area,
// from the staged Q and K and the token block, each wave the fragments of
// SLOTS (bit i: fragment i), so that the Aq products are spread over the four
// SIMDs instead of queueing behind one compute wave's products on one.
// Each 16x16 tile (t, s) is formed transposed, as K_s Q_t^T: its accumulator
// (lane (n, g): s rows 4 g + i of token column n) is then, packed, half of a
// fragment (mt, S) as the B operand of dV^T Aq^T reads it (lane (n, g): token
// 16 mt + n, s in pi order).  Rows past a sequence's end are clamped copies;
// their tokens have m scale = 0.
//   fragment: 0      1            2            3      4            5
//   tiles:    (0,0)  (1,0),(1,1)  (2,0),(2,1)  (2,2)  (3,0),(3,1)  (3,2),(3,3)
template <unsigned SLOTS>
__device__ __forceinline__ void stage4_aq(lds_u8* buf, int lane) {
    using St = Stage4<kModeOut>;
    constexpr int t_of[6] = {0, 1, 2, 2, 3, 3};
    constexpr int s_lo[6] = {0, 0, 0, 2, 0, 2};  // first tile's s (the second's is s + 1)
    constexpr bool two[6] = {false, true, true, false, true, true};
    auto needs_q = [](int t) {
        for (int i = 0; i < 6; ++i)
            if (((SLOTS >> i) & 1) && t_of[i] == t) return true;
        return false;
    };
    auto needs_k = [](int s) {
        for (int i = 0; i < 6; ++i)
            if (((SLOTS >> i) & 1) && (s_lo[i] == s || (two[i] && s_lo[i] + 1 == s))) return true;
        return false;
    };
    const int n = lane & 15, g = lane >> 4;
    const lds_f32* Hb = reinterpret_cast<const lds_f32*>(buf + St::offH);
    bf16x8 qf[4][4], kf[4][4];
    float lt[4], mt[4];
    f32x4 ls[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (needs_q(t)) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) qf[t][kk] = frag(buf, St::offQ + (4 * t + kk) * kFragB, lane);
            lt[t] = Hb[16 * t + n];
            mt[t] = Hb[64 + 16 * t + n];
        }
        if (needs_k(t)) {
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) kf[t][kk] = kfrag(buf + St::offK, 4 * t + kk, lane);
            ls[t] = *reinterpret_cast<const lds_f32x4*>(Hb + 16 * t + 4 * g);
        }
    }
    auto tile = [&](int ti, int si) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma16x16x32(kf[si][kk], qf[ti][kk], acc);
        f32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = mt[ti] * acc[i] * __builtin_amdgcn_exp2f(lt[ti] - ls[si][i]);
            v[i] = (ti > si || 4 * g + i <= n) ? x : 0.f;
        }
        return pack4_bf16(v);
    };
    const u32x2 z = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        if ((SLOTS >> i) & 1) {
            const u32x2 lo = tile(t_of[i], s_lo[i]);
            const u32x2 hi = two[i] ? tile(t_of[i], s_lo[i] + 1) : z;
            *reinterpret_cast<lds_u32x4*>(buf + St::offAq + i * kFragB + 16 * lane) = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
    }
}

// The copy wave: chunk c's output tile from LDS to `ob` (row 0, the
// workgroup's first column), rows of RB bytes (the workgroup's columns): 4
// rows of 256 bytes or 8 rows of 128 bytes per instruction.
template <bool FULL, int RB>
__device__ __forceinline__ void stage4_store(const lds_u8* obuf, uint16_t* ob, int orow, int nvalid, int lane) {
    constexpr int LPR = RB / 16;  // lanes per row
    static_assert(LPR == 16 || LPR == 8, "output row bytes");
    // Opaque per call: otherwise the per-lane row offsets are hoisted out of
    // the chunk loop and held in registers that every wave then pays for.
    asm volatile("" : "+s"(orow));
#pragma unroll
    for (int i = 0; i < kC * LPR / 64; ++i) {
        const int row = (64 / LPR) * i + lane / LPR;
        const u32x4 v = *reinterpret_cast<const lds_u32x4*>(obuf + row * kObPitch + (lane % LPR) * 16);
        if (FULL || row < nvalid)  // streamed out: nothing in this pass reads the outputs back
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(ob + static_cast<size_t>(row) * orow + (lane % LPR) * 8));
    }
}

// One chunk of the state recurrence for this wave's 128 x 32 state tile, the
// chunk's operands staged in `buf`; the output pass leaves the chunk's
// outputs in the LDS tile `obuf` for the copy wave.
// LDS reads run one phase ahead of the MFMAs that consume them: K S and
// S^T Q^T go in four k-groups, each group's MFMAs issued after the next
// group's fragment reads, and each later phase's operands (V and the gates,
// Tp, K^T, Aq) are read while the phase before it computes.  Phase fences
// (PHASE()) keep that order: the scheduler would otherwise sink reads to
// their first use (exposing the LDS latency at every one) or hoist all of
// them to the top (past the 256 VGPRs a wave has).
template <int MODE, int NT, typename Mid>
__device__ __forceinline__ void state4_step(const lds_u8* buf, f32x4 (&S)[8][NT], lds_u8* obuf, int wave, int lane,
                                            bool v_zero, uint32_t kt_lane, Mid mid) {
    using St = Stage4<MODE, NT>;
    constexpr bool OUT = St::out;
    const int n = lane & 15, g = lane >> 4;
    const lds_f32* G = reinterpret_cast<const lds_f32*>(buf + St::offG);
    // V is staged per 32 columns ([64 rows][32 columns]): a 32-column wave
    // reads its own tile, two 16-column waves share one (wave 2 i + 1 takes
    // its upper 16 columns).
    const lds_u8* Vs = buf + St::offV + (NT == 2 ? wave : wave >> 1) * 4 * kFragB;
    const int vnt0 = NT == 2 ? 0 : (wave & 1);
#define PHASE() __builtin_amdgcn_sched_barrier(0)

    // (a) X = K S and P^T = S^T Q^T.  The state's bf16 copy is the B operand
    //     of K S and the A operand of S^T Q^T as it stands (k = state rows
    //     32 s + 8 g + j in both).
    bf16x8 kf[2][4], qf[2][OUT ? 4 : 1];
    auto load_a = [&](int s, int slot) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            kf[slot][mt] = kfrag(buf + St::offK, 4 * mt + s, lane);
            if constexpr (OUT) qf[slot][mt] = frag(buf, St::offQ + (4 * mt + s) * kFragB, lane);
        }
    };
    i16x4 vv[NT][4];
    f32x4 gam[4], kd[4];
    float gC = 0.f;
    // (b)'s operands: V in the accumulator layout (column n, rows
    // 16 mt + 4 g + i) -- source lane 4 j + a of group g of a transposing read
    // fetches row 16 mt + 4 g + j, columns 16 nt + 4 a .. -- and the gates.
    auto load_b = [&]() {
        const lds_u8* vrow = Vs + ((4 * g + ((lane >> 2) & 3)) * 32 + 4 * (lane & 3)) * 2;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                vv[nt][mt] = v_zero ? i16x4{0, 0, 0, 0}
                                    : __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                          (lds_i16x4*)(vrow + (16 * mt * 32 + 16 * (nt + vnt0)) * 2));
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            gam[mt] = *reinterpret_cast<const lds_f32x4*>(G + 16 * mt + 4 * g);
            kd[mt] = *reinterpret_cast<const lds_f32x4*>(G + 128 + 16 * mt + 4 * g);
        }
        gC = G[kC - 1];
    };
    f32x4 X[4][NT], P[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) X[mt][nt] = P[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    load_a(0, 0);
    PHASE();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if (s < 3)
            load_a(s + 1, (s + 1) & 1);
        else
            load_b();
        bf16x8 Bs[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) Bs[nt] = pack8(S[2 * s][nt], S[2 * s + 1][nt]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                X[mt][nt] = mfma16x16x32(kf[s & 1][mt], Bs[nt], X[mt][nt]);
                if constexpr (OUT) P[mt][nt] = mfma16x16x32(Bs[nt], qf[s & 1][mt], P[mt][nt]);
            }
        PHASE();
    }
    // (b) Y = V - gamma o X (in place in X), while Tp is read.
    bf16x8 tf[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) tf[i] = frag(buf, St::offTp + i * kFragB, lane);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                X[mt][nt][i] = bf2f(static_cast<uint16_t>(vv[nt][mt][i])) - gam[mt][i] * X[mt][nt][i];
    bf16x8 BY[2][NT];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) BY[s][nt] = pack8(X[2 * s][nt], X[2 * s + 1][nt]);
    PHASE();
    // (c) dV = Tp Y (Tp lower triangular: six nonzero fragments), while the
    //     first half of K^T is read.
    bf16x8 ktf[8][2];
    auto load_kt = [&](int r0) {
#pragma unroll
        for (int r = r0; r < r0 + 4; ++r) {
            ktf[r][0] = ktfrag(buf + St::offK, kt_lane, r, 0);
            ktf[r][1] = ktfrag(buf + St::offK, kt_lane, r, 1);
        }
    };
    load_kt(0);
    f32x4 D[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) D[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int mt = 2 * s; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) D[mt][nt] = mfma16x16x32(tf[aq_index(mt, s)], BY[s][nt], D[mt][nt]);
    PHASE();
    // (d) S <- gamma_C S + K^T ((gamma_C / gamma) o dV) in two halves of
    //     row tiles: the second half of K^T is read during the first, Aq
    //     during the second.
    bf16x8 af[OUT ? 6 : 1];
    float co[4];
    bf16x8 BS0[NT], BS1[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        BS0[nt] = pack8(kd[0] * D[0][nt], kd[1] * D[1][nt]);
        BS1[nt] = pack8(kd[2] * D[2][nt], kd[3] * D[3][nt]);
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if (half == 0) {
            load_kt(4);
        } else if constexpr (OUT) {
            mid();  // the copy waves have formed Aq
#pragma unroll
            for (int i = 0; i < 6; ++i) af[i] = frag(buf, St::offAq + i * kFragB, lane);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) co[mt] = G[64 + 16 * mt + n];
        }
#pragma unroll
        for (int r = 4 * half; r < 4 * half + 4; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                S[r][nt] *= gC;
                S[r][nt] = mfma16x16x32(ktf[r][0], BS0[nt], S[r][nt]);
                S[r][nt] = mfma16x16x32(ktf[r][1], BS1[nt], S[r][nt]);
            }
        PHASE();
    }
    // (e) O^T = (m scale gamma) o P^T + dV^T Aq^T: each lane holds 4
    //     consecutive output columns of token 16 mt + n, written to the
    //     output tile as 8 bytes.
    if constexpr (OUT) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const bf16x8 BD0 = pack8(D[0][nt], D[1][nt]), BD1 = pack8(D[2][nt], D[3][nt]);
            f32x4 O[4];
            O[0] = mfma16x16x32(BD0, af[0], co[0] * P[0][nt]);
            O[1] = mfma16x16x32(BD0, af[1], co[1] * P[1][nt]);
            O[2] = mfma16x16x32(BD1, af[3], mfma16x16x32(BD0, af[2], co[2] * P[2][nt]));
            O[3] = mfma16x16x32(BD1, af[5], mfma16x16x32(BD0, af[4], co[3] * P[3][nt]));
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                *reinterpret_cast<lds_u32x2*>(obuf + (16 * mt + n) * kObPitch + (16 * NT * wave + 16 * nt + 4 * g) * 2) =
                    pack4_bf16(O[mt]);
        }
    }
#undef PHASE
}

// The state pass of one workgroup: 128 columns of one (sequence, head,
// chunk group) in the roles of gdn_prefill_state_kernel (output pass: from
// the group's initial state, outputs and the final state; map pass: psi
// columns from zero with V, phi columns from the identity without V).
// This file is compiled with MFMA results forced into VGPRs (the build's
// -amdgpu-mfma-vgpr-form): with one compute wave per SIMD the compiler would
// otherwise park the accumulators in AGPRs and copy them back for every VALU
// use, about 300 extra instructions per chunk.
// The output pass adds the copy waves.  In the map pass (two workgroups per
// CU, 39 KiB a chunk step each) the compute waves issue a quarter of the
// copies each: dedicated copy waves there measured slower.
template <int MODE, int NT>
__global__ __launch_bounds__((64 * Stage4<MODE, NT>::nWaves)) __attribute__((amdgpu_waves_per_eu(
    MODE == kModeOut ? 1 : 2, 2))) void gdn_prefill_state4_kernel(PrefillParams p, StateGrid sg) {
    using St = Stage4<MODE, NT>;
    constexpr bool OUT = St::out;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * St::bytes + 2 * St::ob_bytes];
    auto buf = [&](int i) { return (lds_u8*)&smem[0] + i * St::bytes; };
    auto obuf = [&](int i) { return (lds_u8*)&smem[0] + 2 * St::bytes + i * St::ob_bytes; };

    const int wg = blockIdx.x;
    int head, grp, vg, ngroups;
    if (sg.plan) {
        vg = wg % sg.nvg;
        const int hh = (wg / sg.nvg) / sg.ngroups_run, q = (wg / sg.nvg) % sg.ngroups_run;
        if (hh >= p.H || q >= sg.plan[MODE == kModeMap ? 1 : 0]) return;  // uniform over the workgroup
        const int e = sg.plan[2 + 2 * sg.nseq + (MODE == kModeMap ? kPlanCap : 0) + q];
        head = (e >> 8) * p.H + hh;
        grp = e & 255;
        ngroups = plan_groups(sg, e >> 8);
    } else {
        if (p.xcd_heads) {
            const HeadItem hi = head_major_xcd(wg, sg.ngroups_run * sg.nvg);
            head = hi.head;
            grp = hi.item / sg.nvg;
            vg = hi.item % sg.nvg;
        } else {
            vg = wg % sg.nvg;
            head = (wg / sg.nvg) / sg.ngroups_run;
            grp = (wg / sg.nvg) % sg.ngroups_run;
        }
        if (head * sg.ngroups_run + grp >= sg.nheads * sg.ngroups_run) return;  // uniform over the workgroup
        ngroups = sg.ngroups;
    }
    const int sidx = head / p.H;
    const int h = head % p.H;
    const SeqInfo sq = seq_info(p, sidx);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Copy waves (output pass): 4 and 5 copy chunk c + 1 in, 6 writes chunk
    // c - 1's outputs, and all four form chunk c's Aq.  In the map pass the
    // compute waves copy (`issuer`).
    const bool loader = OUT && wave >= 4 && wave < 4 + St::loaders;
    const bool storer = OUT && wave == 4 + St::loaders;
    const bool aqw = OUT && wave == 5 + St::loaders;
    const bool issuer = OUT ? loader : true;
    const bool copier = loader || storer || aqw;
    const int cw = copier ? 0 : wave;  // compute wave (column block)
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4;
    const int dv = p.dv;
    const int col0_wave = vg * St::cols + 16 * NT * cw;  // map pass: >= dv means identity columns
    const bool phi_cols = MODE == kModeMap && vg * St::cols >= dv;
    const int vcol0 = phi_cols ? 0 : vg * St::cols;
    const int nchunks = (sq.len + kC - 1) / kC;
    const int glen = (nchunks + ngroups - 1) / ngroups;
    const int c_begin = min(grp * glen, nchunks), c_end = min(c_begin + glen, nchunks);
    const Lane4 L = {static_cast<uint32_t>(kslot_row(lane) * kDK * 2 + (lane >> 4) * 16),
                     static_cast<uint32_t>((lane & 15) * kDK * 2 + (lane >> 4) * 16), static_cast<uint32_t>(16 * lane),
                     static_cast<uint32_t>((lane >> 2) * dv * 2 + (lane & 3) * 16)};
    const uint32_t kt_lane = kt_lane_offset(lane);

    const size_t head_row0 = static_cast<size_t>(sq.b * p.H + h) * p.T_stride + sq.tok0;
    const int orow = p.out_tm ? p.H * dv : dv;
    auto rows = [&](int c) { return head_row0 + static_cast<size_t>(c) * kC; };
    auto obase = [&](int c) {  // out row of chunk c's first token, the workgroup's first column
        const size_t tok = static_cast<size_t>(sq.b) * p.T_stride + sq.tok0 + static_cast<size_t>(c) * kC;
        return p.out + (p.out_tm ? (tok * p.H + h) * dv : rows(c) * dv) + vg * St::cols;
    };
    auto nval = [&](int c) { return min(kC, sq.len - c * kC); };
    auto rec = [&](int c) { return p.wsR + (static_cast<size_t>(sq.slot0 + c) * p.H + h) * kRecShort * 64; };
    auto issue = [&](int c, int bi) {
        // Opaque per call: otherwise the copies' LDS addresses (buffer and
        // fragment constants) are hoisted out of the chunk loop and held in
        // SGPRs, which runs the kernel out of them.
        int first = OUT ? wave - 4 : wave;
        asm volatile("" : "+s"(first));
        lds_u8* b = buf(bi);
        constexpr int STRIDE = OUT ? St::loaders : 4;
        if (nval(c) == kC)
            stage4_issue<MODE, NT, true, STRIDE>(p, b, rows(c), rec(c), vcol0, kC, first, lane, L, !phi_cols);
        else
            stage4_issue<MODE, NT, false, STRIDE>(p, b, rows(c), rec(c), vcol0, nval(c), first, lane, L, !phi_cols);
    };

    // Chunk c = c_begin + k uses buffer k % 2 and output tile k % 2.  Barrier
    // k opens step k: chunk c is staged, nobody reads buffer (k + 1) % 2 any
    // more, and chunk c - 1's outputs are in tile (k - 1) % 2.  In the output
    // pass a second barrier per step, in the middle of the compute waves'
    // state update, publishes chunk c's Aq, formed meanwhile by the copy waves.
    // The copy waves run their own loop (with the same barriers), so the
    // compute waves' state is not live in it.
    if constexpr (OUT) {
        if (copier) {
            if (loader && c_begin < c_end) issue(c_begin, 0);
            for (int c = c_begin; c < c_end; ++c) {
                const int k = c - c_begin;
                if (loader) wait_vm<0>();  // chunk c staged
                lds_barrier();
                if (loader && c + 1 < c_end) issue(c + 1, (k + 1) & 1);
                // Chunk c's Aq: each copy wave (one a SIMD) forms 2 or 3 of its 10 tiles.
                static_assert(St::loaders == 2, "copy waves 4..7");
                if (wave == 4) stage4_aq<0x28>(buf(k & 1), lane);  // (2,2), (3,2), (3,3)
                if (wave == 5) stage4_aq<0x11>(buf(k & 1), lane);  // (0,0), (3,0), (3,1)
                if (wave == 6) stage4_aq<0x04>(buf(k & 1), lane);  // (2,0), (2,1)
                if (wave == 7) stage4_aq<0x02>(buf(k & 1), lane);  // (1,0), (1,1)
                // Chunk c - 1 is never a sequence's partial last chunk here.
                if (storer && k >= 1) stage4_store<true, 2 * St::cols>(obuf((k - 1) & 1), obase(c - 1), orow, kC, lane);
                lds_barrier();  // chunk c's Aq formed
            }
            lds_barrier();  // the last chunk's outputs are in LDS
            if (storer && c_end > c_begin) {
                const int c = c_end - 1, k = c - c_begin;
                if (nval(c) == kC)
                    stage4_store<true, 2 * St::cols>(obuf(k & 1), obase(c), orow, kC, lane);
                else
                    stage4_store<false, 2 * St::cols>(obuf(k & 1), obase(c), orow, nval(c), lane);
            }
            return;
        }
    }

    // State tile: S[r][nt][i] = S[rho(r, g, i)][col0_wave + 16 nt + n].
    f32x4 S[8][NT];
    if constexpr (MODE == kModeMap) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    S[r][nt][i] = (phi_cols && rho_row(r, g, i) == col0_wave - dv + 16 * nt + n) ? 1.f : 0.f;
    } else if (grp > 0) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f32x4* Ps = reinterpret_cast<const f32x4*>(
                sg.psi + (group_unit(sg, p.H, sidx, h, grp - 1) * (dv / 16) + col0_wave / 16 + nt) * 2048);
#pragma unroll
            for (int r = 0; r < 8; ++r) S[r][nt] = Ps[r * 64 + lane];
        }
    } else if (p.state_in) {
        const float* sin = p.state_in + static_cast<size_t>(sidx * p.H + h) * kDK * dv;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) S[r][nt][i] = sin[rho_row(r, g, i) * dv + col0_wave + 16 * nt + n];
    } else {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) S[r][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    if (!OUT && c_begin < c_end) issue(c_begin, 0);
    for (int c = c_begin; c < c_end; ++c) {
        const int k = c - c_begin;
        if (!OUT) wait_vm<0>();  // chunk c staged (the map pass's compute waves copy)
        lds_barrier();
        if (!OUT && c + 1 < c_end) issue(c + 1, (k + 1) & 1);
        state4_step<MODE, NT>(buf(k & 1), S, obuf(k & 1), cw, lane, phi_cols, kt_lane, [] { lds_barrier(); });
    }

    if constexpr (OUT) {
        lds_barrier();  // the last chunk's outputs are in LDS (matches the copy waves' final barrier)
        if (grp != ngroups - 1) return;
        float* so = p.state_out + static_cast<size_t>(sidx * p.H + h) * kDK * dv;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) so[rho_row(r, g, i) * dv + col0_wave + 16 * nt + n] = S[r][nt][i];
    } else if (phi_cols) {
        // phi as A fragments, transposed 16x16 tile by tile through this
        // wave's V area of buffer 0 (unused by identity columns): no copy is
        // in flight any more, and no other wave reads that area.
        uint16_t* Ph = sg.phi + group_unit(sg, p.H, sidx, h, grp) * kDK * kDK;
        lds_u16* tt = reinterpret_cast<lds_u16*>(buf(0) + St::offV + cw * 4 * kFragB);
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int T = (col0_wave - dv) / 16 + nt;
#pragma unroll
                for (int i = 0; i < 4; ++i) tt[(4 * g + i) * 16 + n] = f2bf_bits(S[r][nt][i]);
                if (lane < 32) {  // fragment lanes 16 (2 (T % 2) + h2) + n: row n of the tile, columns 8 h2 ..
                    const int h2 = lane >> 4;
                    const u32x4 v = *reinterpret_cast<const lds_u32x4*>(tt + n * 16 + 8 * h2);
                    *reinterpret_cast<u32x4*>(Ph + ((r * 4 + (T >> 1)) * 64 + 16 * (2 * (T & 1) + h2) + n) * 8) = v;
                }
            }
    } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            f32x4* Ps = reinterpret_cast<f32x4*>(sg.psi +
                                                 (group_unit(sg, p.H, sidx, h, grp) * (dv / 16) + col0_wave / 16 + nt) * 2048);
#pragma unroll
            for (int r = 0; r < 8; ++r) Ps[r * 64 + lane] = S[r][nt];
        }
    }
}

// Initial states of the chunk groups: S_in(0) = state_in (or 0) and
// S_in(j + 1) = phi_j S_in(j) + psi_j, written over psi_j.  One workgroup of
// 8 waves per (sequence-head, 16-column tile); wave w owns accumulator row
// tile r = w (state rows rho(w, g, i)).  Row tiles 2s and 2s + 1 make up
// MFMA k-step s, so wave w publishes its rows as one 8-byte half of k-step
// w / 2's B operand (bf16 high and low parts of the fp32 state, which give
// two independent accumulation chains) and every wave reads all four k-steps
// back.  The steps are a dependent chain, so what bounds a step is latency:
// each wave holds its phi fragments and psi quad for the next kScanDepth
// steps in registers (20 VGPRs a step), loaded kScanDepth steps before use,
// which covers the memory latency that a shallower LDS ring (limited to 3
// steps by LDS capacity) did not.
constexpr int kScanDepth = 6;
constexpr int kMaxGroups = 16;  // chunk groups per sequence (plan_state caps G here)

__device__ __forceinline__ u32x2 pack4_hi(const f32x4 v) { return pack4_bf16(v); }
// bf16 of (x - bf16(x)): the low part of a two-term bf16 split.
__device__ __forceinline__ u32x2 pack4_lo(const f32x4 v, const u32x2 hi) {
    f32x4 d;
    d[0] = v[0] - __uint_as_float(hi[0] << 16);
    d[1] = v[1] - __uint_as_float(hi[0] & 0xffff0000u);
    d[2] = v[2] - __uint_as_float(hi[1] << 16);
    d[3] = v[3] - __uint_as_float(hi[1] & 0xffff0000u);
    return pack4_hi(d);
}

// STEPS = G - 1 is a template parameter so that the step loop unrolls
// completely with static register slots and exact wait counts (a rolled
// loop makes the compiler wait for every outstanding load at its header).
// PLANNED: per-sequence group counts (sg.plan); STEPS is then the most any
// sequence can have and each workgroup stops after its own G_i - 1 steps.
template <int STEPS, bool PLANNED>
__global__ __launch_bounds__(512) void gdn_prefill_scan_kernel(PrefillParams p, StateGrid sg) {
    static_assert(STEPS >= 1 && STEPS < kMaxGroups, "scan steps");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * 8 * kFragB];
    const int dv = p.dv, ntile = dv / 16;
    const int nunits = sg.nheads * ntile;
    if (static_cast<int>(blockIdx.x) >= nunits) return;  // uniform over the workgroup
    int head, tile;
    if (p.xcd_heads) {
        const HeadItem hi = head_major_xcd(blockIdx.x, ntile);
        head = hi.head;
        tile = hi.item;
    } else {
        head = blockIdx.x / ntile;
        tile = blockIdx.x % ntile;
    }
    const int sidx = head / p.H, h = head % p.H;
    const int nsteps = PLANNED ? plan_groups(sg, sidx) - 1 : STEPS;
    if (PLANNED && nsteps <= 0) return;  // one group: nothing to compose
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // = row tile r
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4;
    const int col = 16 * tile + n;
    lds_u8* const sbuf = (lds_u8*)&smem[0];

    f32x4 S;
    if (p.state_in) {
        const float* sin = p.state_in + static_cast<size_t>(sidx * p.H + h) * kDK * dv;
#pragma unroll
        for (int i = 0; i < 4; ++i) S[i] = sin[rho_row(wave, g, i) * dv + col];
    } else {
        S = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // psi/phi unit of group j: unit0 + j ustride (group_unit, with the plan
    // table read once here: a table read inside the step loop would come with
    // a wait for every load in flight, the prefetched steps included).
    const size_t unit0 = PLANNED ? static_cast<size_t>(plan_first(sg, sidx)) * p.H + h
                                 : static_cast<size_t>(sidx * p.H + h) * sg.ngroups;
    const size_t ustride = PLANNED ? static_cast<size_t>(p.H) : 1;
    auto unit = [&](int j) { return unit0 + static_cast<size_t>(j) * ustride; };
    auto psi_at = [&](int j) {
        return reinterpret_cast<f32x4*>(sg.psi + (unit(j) * ntile + tile) * 2048) + wave * 64 + lane;
    };
    // This wave's phi fragments (row tile r, k-steps 0..3: 4 contiguous KiB)
    // and psi quad r of step j, into register slot j % kScanDepth.
    constexpr int D = STEPS < kScanDepth ? STEPS : kScanDepth;
    u32x4 ph[D][4];
    f32x4 ps[D];
    auto load = [&](int j) {
        const u32x4* src = reinterpret_cast<const u32x4*>(sg.phi + unit(j) * kDK * kDK) + 4 * wave * 64 + lane;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) ph[j % D][ks] = src[ks * 64];
        ps[j % D] = *psi_at(j);
        // Keep each step's loads together and in step order: the wait for
        // step j then only covers what was issued up to step j.
        __builtin_amdgcn_sched_barrier(0);
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (!PLANNED || j < nsteps) load(j);
    const int half = (wave & 1) * 8;  // this row tile's bytes in its k-step's B fragment
    auto publish = [&](lds_u8* buf) {
        const u32x2 hi = pack4_hi(S);
        *reinterpret_cast<lds_u32x2*>(buf + (2 * (wave >> 1)) * kFragB + 16 * lane + half) = hi;
        *reinterpret_cast<lds_u32x2*>(buf + (2 * (wave >> 1) + 1) * kFragB + 16 * lane + half) = pack4_lo(S, hi);
    };
    // From a zero initial state the first step is S_in(1) = psi_0 (phi_0 0 +
    // psi_0 adds exact zeros), which psi_0's slot already holds: it is taken
    // as is, one dependent step shorter.
    const bool zero_start = p.state_in == nullptr;
    if (!zero_start) publish(sbuf);
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        if (PLANNED && j >= nsteps) continue;  // uniform over the workgroup (the loop still unrolls)
        if (j == 0 && zero_start) {
            S = ps[0];
            if (D < STEPS && (!PLANNED || D < nsteps)) load(D);
            publish(sbuf + 8 * kFragB);
            continue;
        }
        lds_u8* const buf = sbuf + (j & 1) * 8 * kFragB;
        lds_barrier();
        f32x4 acc_h = ps[j % D];
        f32x4 acc_l = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const bf16x8 a = as_bf16x8(ph[j % D][ks]);
            acc_h = mfma16x16x32(a, frag(buf, (2 * ks) * kFragB, lane), acc_h);
            acc_l = mfma16x16x32(a, frag(buf, (2 * ks + 1) * kFragB, lane), acc_l);
        }
        if (j + D < STEPS && (!PLANNED || j + D < nsteps)) load(j + D);
        S = acc_h + acc_l;
        *psi_at(j) = S;
        publish(sbuf + ((j + 1) & 1) * 8 * kFragB);
    }
}

template <int STEPS>
int launch_scan(const PrefillParams& p, const StateGrid& sg, unsigned nblocks, hipStream_t stream, int steps) {
    if constexpr (STEPS < kMaxGroups) {
        if (steps == STEPS) {
            if (sg.plan)
                hipLaunchKernelGGL((gdn_prefill_scan_kernel<STEPS, true>), dim3(nblocks), dim3(512), 0, stream, p, sg);
            else
                hipLaunchKernelGGL((gdn_prefill_scan_kernel<STEPS, false>), dim3(nblocks), dim3(512), 0, stream, p, sg);
            return gdn_host::check_launch("gdn_prefill_scan_kernel");
        }
        return launch_scan<STEPS + 1>(p, sg, nblocks, stream, steps);
    } else {
        return gdn_host::fail(GDN_ERR_UNSUPPORTED, "prefill: %d chunk groups", steps + 1);
    }
}

// Chunk groups of packed sequences, balanced by length: the smallest group
// length L (at least 4 chunks) for which sum_i min(16, ceil(n_i / L)) groups
// fit `target` slots per head, n_i the chunks of sequence i (an empty
// sequence keeps one group, which passes its state through).  Every group of
// a sequence then has ceil(n_i / G_i) chunks (the last may have fewer), so the
// longest chain is about L wherever the long sequences sit, instead of the
// longest sequence over one group count shared by all.  One wave; writes the
// StateGrid::plan table.  Requires nseq <= target <= kPlanCap.
__global__ __launch_bounds__(64) void gdn_prefill_plan_kernel(const int32_t* __restrict__ cu, int nseq, int target,
                                                              int32_t* __restrict__ tab) {
    const int lane = threadIdx.x;
    auto nchunks = [&](int i) { return (cu[i + 1] - cu[i] + kC - 1) / kC; };
    auto gcount = [&](int n, int L) { return min(kMaxGroups, max(1, (n + L - 1) / L)); };
    // Chunk counts of sequences lane + 64 u (nseq <= target <= kPlanCap = 256).
    int nc[kPlanCap / 64];
    int nmax = 0;
#pragma unroll
    for (int u = 0; u < kPlanCap / 64; ++u) {
        const int i = lane + 64 * u;
        nc[u] = i < nseq ? nchunks(i) : -1;
        nmax = max(nmax, nc[u]);
    }
    for (int off = 32; off > 0; off >>= 1) nmax = max(nmax, __shfl_xor(nmax, off));
    auto total = [&](int L) {
        int t = 0;
#pragma unroll
        for (int u = 0; u < kPlanCap / 64; ++u) t += nc[u] >= 0 ? gcount(nc[u], L) : 0;
        for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off);
        return t;
    };
    int lo = 4, hi = max(4, nmax);  // total(hi) = nseq <= target
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (total(mid) <= target)
            hi = mid;
        else
            lo = mid + 1;
    }
    // Slots in sequence order: sequence i = lane + 64 u takes slots from the
    // sum of G over the sequences before it (exclusive wave scans per u).
    int base = 0, mbase = 0;
#pragma unroll
    for (int u = 0; u < kPlanCap / 64; ++u) {
        const int i = lane + 64 * u;
        const int G = nc[u] >= 0 ? gcount(nc[u], lo) : 0, M = G > 0 ? G - 1 : 0;
        int x = G, y = M;  // inclusive scans
        for (int off = 1; off < 64; off <<= 1) {
            const int xs = __shfl_up(x, off), ys = __shfl_up(y, off);
            if (lane >= off) {
                x += xs;
                y += ys;
            }
        }
        const int first = base + x - G, mfirst = mbase + y - M;
        if (i < nseq) {
            tab[2 + 2 * i] = G;
            tab[3 + 2 * i] = first;
            for (int g = 0; g < G; ++g) {
                tab[2 + 2 * nseq + first + g] = (i << 8) | g;
                if (g < M) tab[2 + 2 * nseq + kPlanCap + mfirst + g] = (i << 8) | g;
            }
        }
        base += __shfl(x, 63);
        mbase += __shfl(y, 63);
    }
    if (lane == 0) {
        tab[0] = base;
        tab[1] = mbase;
    }
}

// ---------------------------------------------------------------------------
// Zero fill used for the T == 0 state (a kernel rather than a memset node, so
// the call stays safe to capture in a HIP graph).
__global__ void gdn_fill_zero_kernel(float* __restrict__ p, size_t n) {
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr size_t kFragBytes = 64 * 16;  // one record fragment

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// How the state pass is split: NT 16-column tiles per wave; NW waves per
// workgroup; G chunk groups per sequence when (sequence, head) pairs alone
// cannot fill the chip (each group then runs its own chain of chunks, joined
// through the groups' affine maps).
struct StatePlan {
    int NT_out, NW_out, nvg_out, NT_map, NW_map, nvg_map, G;
    bool wide;  // dv % 128 == 0: gdn_prefill_state4_kernel (4 waves x 32 columns, 128 columns a workgroup)
    bool half;  // wide, output pass in 64-column workgroups (4 compute waves x 16): one group, few pairs
};

// `exact`: max_chunks is the exact chunk count of every sequence, so the
// group count is trimmed until no group is empty.  Workspace sizing uses the
// untrimmed count, which never decreases as sequences grow.
// `varlen`: packed sequences of unequal lengths.
StatePlan plan_state(long long nheads, int dv, long long max_chunks, bool exact, bool varlen) {
    StatePlan s;
    s.wide = dv % 128 == 0;
    s.half = false;
    if (s.wide) {
        s.NT_out = s.NT_map = 2;
        s.NW_out = s.NW_map = 4;
        s.nvg_out = dv / 128;
        s.nvg_map = (dv + kDK) / 128;
        // Chunk groups when the output pass alone would leave CUs idle: below
        // 256 output workgroups for packed sequences (groups also balance
        // their unequal lengths), below 128 for equal lengths (measured at
        // T = 8192: 128 (sequence, head) pairs run 1.2x faster as one group
        // each than as two, where the map pass and scan cost more than the
        // idle half of the chip).  Groups of at least 4 chunks; of 2 when
        // there are at most 16 (sequence, head) pairs and at most 16 chunks,
        // where the map pass's chain is most of the call (measured: B=1,
        // H=16, T=512 27.7 -> 23.9 us, T=1024 29.9 -> 28.4; H=4, T=900 34.6
        // -> 30.7; B=2, H=8, T=1024 30.1 -> 28.6; H=2, T=600 33.2 -> 27.4;
        // slower at 32 or more pairs, and at T=2048).
        const long long base = nheads * s.nvg_out;  // output-pass workgroups (one per CU) with one group
        long long G = 1;
        if (base < (varlen ? 256 : 128) && max_chunks >= 8) {
            const long long min_chunks = (!varlen && base <= 16 && max_chunks <= 16) ? 2 : 4;
            G = std::min<long long>(std::min<long long>(kMaxGroups, 256 / base), max_chunks / min_chunks);
        }
        if (exact && G > 1) G = (max_chunks + (max_chunks + G - 1) / G - 1) / ((max_chunks + G - 1) / G);
        s.G = G < 2 ? 1 : static_cast<int>(G);
        // At most half the CUs busy in the output pass (equal lengths, or
        // one group): split each head's 128 columns over two workgroups of
        // four 16-column compute waves (the state columns update
        // independently; the halves of a head share K and Q through the L2
        // of their XCD).  Packed sequences with planned groups keep whole
        // heads (their plan targets a full round of 128-column workgroups).
        s.half = (s.G == 1 || !varlen) && base * s.G <= 128;
        if (s.half) s.nvg_out = dv / 64;
        return s;
    }
    // dv not a multiple of 128: the 16-column state kernel.  Output pass:
    // 32-column waves where dv allows, as many waves (up to 4) as divide the
    // tiles.  Map pass (dv + 128 columns): two waves per SIMD (8-wave
    // workgroups of 32-column waves) where the tiling allows, so the waves
    // hide each other's LDS and copy latency; otherwise wider or fewer waves.
    s.NT_out = (dv % 32 == 0) ? 2 : 1;
    {
        const int tiles = dv / (16 * s.NT_out);
        s.NW_out = (tiles % 4 == 0) ? 4 : (tiles % 2 == 0) ? 2 : 1;
    }
    s.nvg_out = dv / (16 * s.NT_out * s.NW_out);
    if ((dv + kDK) % 256 == 0) {
        s.NT_map = 2;
        s.NW_map = 8;
        s.nvg_map = (dv + kDK) / 256;
    } else if ((dv + kDK) % 64 == 0 && (dv + kDK) / 64 <= 4) {
        // One workgroup of 64-column waves for all dv + 128 columns (dv = 64).
        s.NT_map = 4;
        s.NW_map = (dv + kDK) / 64;
        s.nvg_map = 1;
    } else {
        s.NT_map = (dv % 32 == 0) ? 2 : 1;
        const int mtiles = (dv + kDK) / (16 * s.NT_map);
        s.NW_map = (mtiles % 4 == 0) ? 4 : (mtiles % 2 == 0) ? 2 : 1;
        s.nvg_map = mtiles / s.NW_map;
    }
    const long long base = nheads * s.nvg_out;  // output-pass workgroups with one group
    long long G = 1;
    if (base < 256 && max_chunks >= 8)
        G = std::min<long long>(std::min<long long>(kMaxGroups, 256 / base), max_chunks / 4);
    if (exact && G > 1) G = (max_chunks + (max_chunks + G - 1) / G - 1) / ((max_chunks + G - 1) / G);
    s.G = G < 2 ? 1 : static_cast<int>(G);
    // A map pass that would fill at most half the CUs (few groups, e.g. G = 2
    // at 128 (sequence, head) pairs) splits each group's dv + 128 columns over
    // workgroups of 8 waves x 16 columns instead (psi and phi apart).
    if (s.G > 1 && s.NT_map == 2 && s.NW_map == 8 && nheads * (s.G - 1) * s.nvg_map * 2 <= 256) {
        s.NT_map = 1;
        s.nvg_map = (dv + kDK) / 128;
    }
    return s;
}

// Record length: the 32-column state kernel forms Aq itself.
int rec_frags(const StatePlan& sp) { return sp.wide ? kRecShort : kRecFull; }

struct WsLayout {
    size_t offR, offPsi, offPhi, offPlan, total;
};

// Packed sequences with chunk groups plan them per sequence on the device
// (gdn_prefill_plan_kernel): target slots per head, at most 256 / (H nvg_out)
// (one round of the output pass), which also bounds the group maps.
bool planned_groups(const StatePlan& sp, bool varlen) { return varlen && sp.G > 1; }
int plan_target(const StatePlan& sp, int H) { return std::max(1, 256 / (H * sp.nvg_out)); }

WsLayout ws_layout(long long slots, int H, long long nheads, int dv, const StatePlan& sp, bool varlen, int nseq) {
    const size_t ch = static_cast<size_t>(slots) * H;
    const bool planned = planned_groups(sp, varlen);
    WsLayout L;
    L.offR = 0;
    L.offPsi = align256(L.offR + ch * rec_frags(sp) * kFragBytes);
    const size_t units = planned      ? static_cast<size_t>(H) * plan_target(sp, H)
                         : sp.G > 1 ? static_cast<size_t>(nheads) * sp.G
                                    : 0;
    L.offPhi = align256(L.offPsi + units * kDK * dv * 4);
    L.offPlan = align256(L.offPhi + units * kDK * kDK * 2);
    L.total = align256(L.offPlan + (planned ? (2 + 2 * static_cast<size_t>(nseq) + 2 * kPlanCap) * 4 : 0));
    return L;
}

int check_common(const char* who, int H, int dk, int dv) {
    using gdn_host::fail;
    if (H <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "%s: H=%d", who, H);
    if (dk != kDK) return fail(GDN_ERR_UNSUPPORTED, "%s: dk=%d, only dk=128 is built", who, dk);
    if (dv < 16 || dv > 512 || dv % 16 != 0)
        return fail(GDN_ERR_UNSUPPORTED, "%s: dv=%d must be a multiple of 16 in [16, 512]", who, dv);
    return GDN_OK;
}

template <int MODE, int NT>
int launch_state4(const PrefillParams& p, const StateGrid& sg, hipStream_t stream) {
    const long long nwg = static_cast<long long>(sg.nheads) * sg.ngroups_run * sg.nvg;
    if (nwg > 0x7fffffffLL) return gdn_host::fail(GDN_ERR_UNSUPPORTED, "prefill: grid too large");
    hipLaunchKernelGGL((gdn_prefill_state4_kernel<MODE, NT>), dim3(static_cast<unsigned>(nwg)),
                       dim3(64 * Stage4<MODE, NT>::nWaves), 0, stream, p, sg);
    return gdn_host::check_launch(MODE == kModeMap ? "gdn_prefill_state4_kernel<map>" : "gdn_prefill_state4_kernel");
}

template <int MODE>
int launch_state_plan(const PrefillParams& p, const StateGrid& sg, const StatePlan& sp, hipStream_t stream);

template <int MODE, int NT>
int launch_state(const PrefillParams& p, const StateGrid& sg, int NW, hipStream_t stream) {
    const long long nwg = static_cast<long long>(sg.nheads) * sg.ngroups_run * sg.nvg;
    if (nwg > 0x7fffffffLL) return gdn_host::fail(GDN_ERR_UNSUPPORTED, "prefill: grid too large");
    const dim3 grid(static_cast<unsigned>(nwg));
    switch (NW) {
        case 1: hipLaunchKernelGGL((gdn_prefill_state_kernel<MODE, 1, NT>), grid, dim3(64), 0, stream, p, sg); break;
        case 2: hipLaunchKernelGGL((gdn_prefill_state_kernel<MODE, 2, NT>), grid, dim3(128), 0, stream, p, sg); break;
        case 4: hipLaunchKernelGGL((gdn_prefill_state_kernel<MODE, 4, NT>), grid, dim3(256), 0, stream, p, sg); break;
        case 3:
            if constexpr (MODE == kModeMap && NT == 4) {
                hipLaunchKernelGGL((gdn_prefill_state_kernel<MODE, 3, NT>), grid, dim3(192), 0, stream, p, sg);
                break;
            }
            return gdn_host::fail(GDN_ERR_UNSUPPORTED, "prefill: no state kernel for %d waves", NW);
        case 8:
            if constexpr (MODE == kModeMap && NT <= 2) {
                hipLaunchKernelGGL((gdn_prefill_state_kernel<MODE, 8, NT>), grid, dim3(512), 0, stream, p, sg);
                break;
            }
            return gdn_host::fail(GDN_ERR_UNSUPPORTED, "prefill: no state kernel for %d waves", NW);
        default:
            return gdn_host::fail(GDN_ERR_UNSUPPORTED, "prefill: no state kernel for %d waves", NW);
    }
    return gdn_host::check_launch(MODE == kModeMap ? "gdn_prefill_state_kernel<map>" : "gdn_prefill_state_kernel");
}

template <int MODE>
int launch_state_plan(const PrefillParams& p, const StateGrid& sg, const StatePlan& sp, hipStream_t stream) {
    if (sp.wide) {
        if constexpr (MODE == kModeOut)
            if (sp.half) return launch_state4<MODE, 1>(p, sg, stream);
        return launch_state4<MODE, 2>(p, sg, stream);
    }
    if (MODE == kModeMap)
        return sp.NT_map == 4   ? launch_state<MODE, 4>(p, sg, sp.NW_map, stream)
               : sp.NT_map == 2 ? launch_state<MODE, 2>(p, sg, sp.NW_map, stream)
                                : launch_state<MODE, 1>(p, sg, sp.NW_map, stream);
    return sp.NT_out == 2 ? launch_state<MODE, 2>(p, sg, sp.NW_out, stream)
                          : launch_state<MODE, 1>(p, sg, sp.NW_out, stream);
}

// phases: bit 0 = chunk-parallel intra kernel, bit 1 = state pass (map pass
// and scan when chunk groups are used, then the output pass).
int launch(PrefillParams& p, int nseq, int nchunk_grid, bool exact, void* workspace, size_t ws_bytes,
           long long slots, hipStream_t stream, int phases) {
    using gdn_host::fail;
    const long long nheads = static_cast<long long>(nseq) * p.H;
    const StatePlan sp = plan_state(nheads, p.dv, nchunk_grid, exact, p.cu != nullptr);
    const bool varlen = p.cu != nullptr;
    const WsLayout L = ws_layout(slots, p.H, nheads, p.dv, sp, varlen, nseq);
    if (!workspace || ws_bytes < L.total)
        return fail(GDN_ERR_WORKSPACE, "prefill: workspace of %zu bytes given, %zu needed", ws_bytes, L.total);
    if (!gdn_host::aligned(workspace, 256))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    p.wsR = reinterpret_cast<u32x4*>(ws + L.offR);
    p.intra_aq = sp.wide ? 0 : 1;

    p.xcd_heads = (nheads % 8 == 0) ? 1 : 0;
    p.nchunk_grid = nchunk_grid;
    if ((phases & 1) && nchunk_grid > 0) {
        const long long units = nheads * nchunk_grid;
        if (units > 0x7fffffffLL) return fail(GDN_ERR_UNSUPPORTED, "prefill: grid too large");
        p.intra_units = static_cast<int>(units);
        // Persistent grid: three or four workgroups per CU (LDS-limited), a
        // multiple of 8 so each workgroup's units stay on its XCD.
        int dev = 0, ncu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
            ncu = 256;
        long long nwg = std::min<long long>(units, (p.intra_aq ? 3LL : 4LL) * ncu);
        if (nwg >= 8) nwg &= ~7LL;
        if (p.intra_aq)
            hipLaunchKernelGGL(gdn_prefill_intra_kernel<true>, dim3(static_cast<unsigned>(nwg)), dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(gdn_prefill_intra_kernel<false>, dim3(static_cast<unsigned>(nwg)), dim3(256), 0, stream, p);
        const int st = gdn_host::check_launch("gdn_prefill_intra_kernel");
        if (st != GDN_OK) return st;
    }
    if (!(phases & 2)) return GDN_OK;
    StateGrid sg = {};
    sg.ngroups = sp.G;
    sg.nheads = static_cast<int>(nheads);
    sg.psi = reinterpret_cast<float*>(ws + L.offPsi);
    sg.phi = reinterpret_cast<uint16_t*>(ws + L.offPhi);
    sg.nseq = nseq;
    int st;
    if (planned_groups(sp, varlen)) {
        // Per-sequence group counts, planned on the device from cu_seqlens.
        const int target = plan_target(sp, p.H);
        if (target > kPlanCap || nseq > target) return fail(GDN_ERR_UNSUPPORTED, "prefill: group plan");
        int32_t* tab = reinterpret_cast<int32_t*>(ws + L.offPlan);
        hipLaunchKernelGGL(gdn_prefill_plan_kernel, dim3(1), dim3(64), 0, stream, p.cu, nseq, target, tab);
        st = gdn_host::check_launch("gdn_prefill_plan_kernel");
        if (st != GDN_OK) return st;
        sg.plan = tab;
        const int map_cap = target - nseq;  // sum of G_i - 1
        if (map_cap > 0) {
            StateGrid sm = sg;
            sm.nheads = p.H;  // grid: (head, map slot, column part)
            sm.nvg = sp.nvg_map;
            sm.ngroups_run = map_cap;
            st = launch_state_plan<kModeMap>(p, sm, sp, stream);
            if (st != GDN_OK) return st;
            const long long nscan = nheads * (p.dv / 16);
            if (nscan > 0x7fffffffLL) return fail(GDN_ERR_UNSUPPORTED, "prefill: grid too large");
            st = launch_scan<1>(p, sg, static_cast<unsigned>(nscan), stream, std::min(kMaxGroups - 1, map_cap));
            if (st != GDN_OK) return st;
        }
        StateGrid so = sg;
        so.nheads = p.H;  // grid: (head, slot, column part)
        so.nvg = sp.nvg_out;
        so.ngroups_run = target;
        return launch_state_plan<kModeOut>(p, so, sp, stream);
    }
    if (sp.G > 1) {
        sg.nvg = sp.nvg_map;
        sg.ngroups_run = sp.G - 1;
        st = launch_state_plan<kModeMap>(p, sg, sp, stream);
        if (st != GDN_OK) return st;
        const long long nscan = nheads * (p.dv / 16);
        if (nscan > 0x7fffffffLL) return fail(GDN_ERR_UNSUPPORTED, "prefill: grid too large");
        st = launch_scan<1>(p, sg, static_cast<unsigned>(nscan), stream, sp.G - 1);
        if (st != GDN_OK) return st;
    }
    sg.nvg = sp.nvg_out;
    sg.ngroups_run = sp.G;
    return launch_state_plan<kModeOut>(p, sg, sp, stream);
}

}  // namespace

extern "C" {

size_t gdn_prefill_workspace_bytes(int B, int H, int T, int dk, int dv) {
    (void)dk;
    if (B <= 0 || H <= 0 || T <= 0 || dv <= 0) return 0;
    const long long nch = (T + kC - 1) / kC;
    const long long slots = static_cast<long long>(B) * nch;
    const long long nheads = static_cast<long long>(B) * H;
    return ws_layout(slots, H, nheads, dv, plan_state(nheads, dv, nch, false, false), false, B).total;
}

size_t gdn_prefill_varlen_workspace_bytes(int num_seqs, int H, int T_total, int dk, int dv) {
    (void)dk;
    if (num_seqs <= 0 || H <= 0 || T_total < 0 || dv <= 0) return 0;
    const long long slots = static_cast<long long>(T_total) / kC + num_seqs + 1;
    const long long nheads = static_cast<long long>(num_seqs) * H;
    // Whether chunk groups are used only grows with the longest sequence: size
    // for T_total (the per-sequence plan then fits in H x 256 / (H nvg) maps).
    return ws_layout(slots, H, nheads, dv, plan_state(nheads, dv, (T_total + kC - 1) / kC, false, true), true, num_seqs)
        .total;
}

}  // extern "C"

namespace {

int prefill_batch(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                  const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                  const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H, int T,
                  int dk, int dv, void* workspace, size_t workspace_bytes, void* stream, int phases,
                  int out_tm = 0) {
    using gdn_host::aligned;
    using gdn_host::fail;
    int st = check_common("prefill", H, dk, dv);
    if (st != GDN_OK) return st;
    if (B < 0 || T < 0) return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: B=%d T=%d", B, T);
    if (B == 0) return GDN_OK;
    if (!q || !k || !v || !A_log || !a || !b_logits || !state_out || (T > 0 && !out))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || (out && !aligned(out, 16)) ||
        !aligned(state_out, 4) || (state_in && !aligned(state_in, 4)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: q/k/v/out need 16-byte alignment");
    if (static_cast<long long>(B) * H * T * dv >= (1LL << 40))
        return fail(GDN_ERR_UNSUPPORTED, "prefill: problem too large");
    PrefillParams p = {};
    p.q = q;
    p.k = k;
    p.v = v;
    p.a = a;
    p.b = b_logits;
    p.A_log = A_log;
    p.mask = mask;
    p.state_in = state_in;
    p.out = out;
    p.state_out = state_out;
    p.cu = nullptr;
    p.out_tm = out_tm;
    p.dt_bias = dt_bias;
    p.scale = scale == 0.f ? 1.f / sqrtf(static_cast<float>(dk)) : scale;
    p.H = H;
    p.dv = dv;
    p.T_stride = T;
    p.T_len = T;
    p.chunks_per_seq = (T + kC - 1) / kC;
    const long long slots = static_cast<long long>(B) * p.chunks_per_seq;
    if (slots == 0) {
        // T == 0: the state passes through unchanged.
        if (!(phases & 2)) return GDN_OK;
        if (state_in)
            return hipMemcpyAsync(state_out, state_in, static_cast<size_t>(B) * H * dk * dv * 4,
                                  hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)) == hipSuccess
                       ? GDN_OK
                       : fail(GDN_ERR_HIP, "prefill: state copy failed");
        hipLaunchKernelGGL(gdn_fill_zero_kernel, dim3(1024), dim3(256), 0, static_cast<hipStream_t>(stream),
                           state_out, static_cast<size_t>(B) * H * dk * dv);
        return gdn_host::check_launch("gdn_fill_zero_kernel");
    }
    return launch(p, B, p.chunks_per_seq, true, workspace, workspace_bytes, slots, static_cast<hipStream_t>(stream),
                  phases);
}

}  // namespace

extern "C" {

int gdn_prefill_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                    const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                    const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H,
                    int T, int dk, int dv, void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_batch(q, k, v, A_log, a, dt_bias, b_logits, mask, state_in, scale, out, state_out, B, H, T, dk,
                         dv, workspace, workspace_bytes, stream, 3);
}

int gdn_prefill_tm_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                       const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                       const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H,
                       int T, int dk, int dv, void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_batch(q, k, v, A_log, a, dt_bias, b_logits, mask, state_in, scale, out, state_out, B, H, T, dk,
                         dv, workspace, workspace_bytes, stream, 3, 1);
}

int gdn_prefill_intra_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                          const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                          const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H,
                          int T, int dk, int dv, void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_batch(q, k, v, A_log, a, dt_bias, b_logits, mask, state_in, scale, out, state_out, B, H, T, dk,
                         dv, workspace, workspace_bytes, stream, 1);
}

int gdn_prefill_state_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                          const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                          const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H,
                          int T, int dk, int dv, void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_batch(q, k, v, A_log, a, dt_bias, b_logits, mask, state_in, scale, out, state_out, B, H, T, dk,
                         dv, workspace, workspace_bytes, stream, 2);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// No-allocation prefill: the workspace is a static device array, one copy per
// GPU (each device that loads this code object holds it until the process
// ends).  Its device address is looked up once per device, with that device
// current, on the first call there; host code uses only that address (the
// array's own name is a host-side stand-in, not a device pointer); the
// stream must belong to the current device.  Nothing in
// the workspace has to start zeroed: every chunk slot and group map that a
// kernel reads was written earlier in the same call.  Calls that overlap on
// one GPU (e.g. on two streams) share the array and race.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = static_cast<size_t>(GDN_PREFILL_NOALLOC_MAX_BYTES);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
// Device address of `scratch` per device, set once a lookup has succeeded (a
// failed lookup is not cached: the next call on that device tries again).
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// `scratch`'s address on the current device `dev`, or null with *err set.
void* scratch_ptr(int dev, hipError_t* err) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (*err != hipSuccess) return nullptr;
        g_scratch[dev] = ptr;
    }
    return g_scratch[dev];
}

}  // namespace

extern "C" {

int gdn_prefill_noalloc_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                            const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                            const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H,
                            int T, int dk, int dv, void* stream) {
    using gdn_host::fail;
    // Sizes first: a request that cannot fit is refused before any HIP call.
    const int st = check_common("prefill_noalloc", H, dk, dv);
    if (st != GDN_OK) return st;
    if (B < 0 || T < 0) return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_noalloc: B=%d T=%d", B, T);
    const size_t need = gdn_prefill_workspace_bytes(B, H, T, dk, dv);
    if (need > kScratchBytes)
        return fail(GDN_ERR_WORKSPACE,
                    "prefill_noalloc: B=%d H=%d T=%d dv=%d needs %zu bytes of scratch, the static buffer holds %zu "
                    "(use gdn_prefill_hip with a caller workspace)",
                    B, H, T, dv, need, kScratchBytes);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(GDN_ERR_HIP, "prefill_noalloc: hipGetDevice failed");
    if (dev < 0 || dev >= kMaxDevices) return fail(GDN_ERR_UNSUPPORTED, "prefill_noalloc: device %d", dev);
    // The buffer is the current device's: a stream of another device would
    // run the kernels there against this device's address.
    if (stream) {
        int sdev = -1;
        if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess)
            return fail(GDN_ERR_HIP, "prefill_noalloc: hipStreamGetDevice failed");
        if (sdev != dev)
            return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_noalloc: stream is on device %d, the current device is %d",
                        sdev, dev);
    }
    hipError_t err = hipSuccess;
    void* const ws = scratch_ptr(dev, &err);
    if (!ws) return fail(GDN_ERR_HIP, "prefill_noalloc: scratch address lookup failed: %s", hipGetErrorString(err));
    return prefill_batch(q, k, v, A_log, a, dt_bias, b_logits, mask, state_in, scale, out, state_out, B, H, T, dk,
                         dv, ws, kScratchBytes, stream, 3);
}

}  // extern "C"

namespace {

int prefill_varlen(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                   const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                   const int32_t* cu_seqlens, int num_seqs, int max_seqlen, const float* state_in, float scale,
                   gdn_bf16_t* out, float* state_out, int H, int T_total, int dk, int dv, void* workspace,
                   size_t workspace_bytes, void* stream, int out_tm) {
    using gdn_host::aligned;
    using gdn_host::fail;
    int st = check_common("prefill_varlen", H, dk, dv);
    if (st != GDN_OK) return st;
    if (num_seqs < 0 || T_total < 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_varlen: num_seqs=%d T_total=%d", num_seqs, T_total);
    if (num_seqs == 0) return GDN_OK;
    if (!q || !k || !v || !A_log || !a || !b_logits || !cu_seqlens || !state_out || (T_total > 0 && !out))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_varlen: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || (out && !aligned(out, 16)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_varlen: q/k/v/out need 16-byte alignment");
    if (static_cast<long long>(H) * T_total * dv >= (1LL << 40))
        return fail(GDN_ERR_UNSUPPORTED, "prefill_varlen: problem too large");
    PrefillParams p = {};
    p.q = q;
    p.k = k;
    p.v = v;
    p.a = a;
    p.b = b_logits;
    p.A_log = A_log;
    p.mask = mask;
    p.state_in = state_in;
    p.out = out;
    p.state_out = state_out;
    p.cu = cu_seqlens;
    p.out_tm = out_tm;
    p.dt_bias = dt_bias;
    p.scale = scale == 0.f ? 1.f / sqrtf(static_cast<float>(dk)) : scale;
    p.H = H;
    p.dv = dv;
    p.T_stride = T_total;
    p.T_len = 0;
    p.chunks_per_seq = 0;
    const int maxlen = (max_seqlen > 0 && max_seqlen < T_total) ? max_seqlen : T_total;
    const int nchunk_grid = (maxlen + kC - 1) / kC;
    const long long slots = static_cast<long long>(T_total) / kC + num_seqs + 1;
    return launch(p, num_seqs, nchunk_grid, false, workspace, workspace_bytes, slots, static_cast<hipStream_t>(stream), 3);
}

}  // namespace

extern "C" {

int gdn_prefill_varlen_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                           const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                           const int32_t* cu_seqlens, int num_seqs, int max_seqlen, const float* state_in,
                           float scale, gdn_bf16_t* out, float* state_out, int H, int T_total, int dk, int dv,
                           void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_varlen(q, k, v, A_log, a, dt_bias, b_logits, mask, cu_seqlens, num_seqs, max_seqlen, state_in,
                          scale, out, state_out, H, T_total, dk, dv, workspace, workspace_bytes, stream, 0);
}

int gdn_prefill_varlen_tm_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                              const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                              const int32_t* cu_seqlens, int num_seqs, int max_seqlen, const float* state_in,
                              float scale, gdn_bf16_t* out, float* state_out, int H, int T_total, int dk, int dv,
                              void* workspace, size_t workspace_bytes, void* stream) {
    return prefill_varlen(q, k, v, A_log, a, dt_bias, b_logits, mask, cu_seqlens, num_seqs, max_seqlen, state_in,
                          scale, out, state_out, H, T_total, dk, dv, workspace, workspace_bytes, stream, 1);
}

}  // extern "C"
