// GDN chunked prefill (chunk C = 64, dk = 128), two kernels.
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
// per chunk (bf16 unless noted), already in the register order kernel 2's
// MFMA operands need (one 16-byte load per lane per fragment):
//   Tp  = T diag(beta m)                       8 fragments  (8 KiB)
//   Aq  = m scale (Q K^T o Gamma), t >= s      8 fragments  (8 KiB)
//   Kt  = (K o gamma_C/gamma)^T                16 fragments (16 KiB)
//   G   = [gamma_t, m_t scale gamma_t]         128 fp32
// Kernel 2, gdn_prefill_state_kernel — one wave per (sequence, head, 16*NT
// state columns) walks the chunks in order.  The fp32 state tile lives in
// MFMA accumulator registers the whole time; its bf16 copy feeds the next
// chunk's products directly (no LDS), because the k order inside an MFMA
// operand is free: the state rows are assigned to accumulator slots so that
// the accumulator of the state update IS the B operand of K S and Q S.
//
// Fragment k-order conventions (lane l: m = l%16 row/column, g = l/16 group):
//   pi(g, j)   = j < 4 ? 4g + j : 16 + 4g + (j-4)   chunk position inside a
//                32-wide k-step, the order produced by two stacked accumulators
//   rho(r,g,i) = 32(r/2) + 8g + 4(r%2) + i          state row held in
//                accumulator tile r, slot i, of lane group g
#include "gdn_common.hpp"

namespace {

using namespace gdn;

constexpr int kC = 64;    // chunk length
constexpr int kDK = 128;  // key / query dim

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
    u32x4* wsT;
    u32x4* wsA;
    u32x4* wsK;
    float* wsG;
    float dt_bias;
    float scale;
    int H;
    int dv;
    int T_stride;        // tokens per (b, h) row block of q/k/v/a/b/out
    int T_len;           // batch mode: sequence length
    int chunks_per_seq;  // batch mode: ceil(T_len / 64)
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

// ---------------------------------------------------------------------------
// Kernel 1
// ---------------------------------------------------------------------------
constexpr int kKLD = kDK + 8;  // padded LDS row (bf16) for K and Q tiles
constexpr int kALD = kC + 4;   // padded LDS row (fp32) for A
constexpr int kBLD = kC + 8;   // padded LDS row (bf16) for 64x64 tiles

__global__ __launch_bounds__(256) void gdn_prefill_intra_kernel(PrefillParams p) {
    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int sidx = blockIdx.z;
    const SeqInfo sq = seq_info(p, sidx);
    const int t0 = c * kC;
    if (t0 >= sq.len) return;  // uniform over the workgroup
    const int nvalid = min(kC, sq.len - t0);
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int m16 = lane & 15;
    const int g4 = lane >> 4;
    const size_t row_base = static_cast<size_t>(sq.b * p.H + h) * p.T_stride + sq.tok0 + t0;
    const size_t wc = static_cast<size_t>(sq.slot0 + c) * p.H + h;

    __shared__ __attribute__((aligned(16))) bf16 Kl[kC][kKLD];
    __shared__ __attribute__((aligned(16))) bf16 Ql[kC][kKLD];
    __shared__ __attribute__((aligned(16))) float Am[kC][kALD];
    __shared__ __attribute__((aligned(16))) bf16 Al[kC][kBLD];
    __shared__ __attribute__((aligned(16))) bf16 Tl[kC][kBLD];
    __shared__ float s_lgc[kC], s_bm[kC], s_ms[kC], s_kdec[kC];

    // 1) K and Q tiles into LDS; rows past the sequence end are zero.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = tid + 256 * it;
        const int row = idx >> 4;
        const int c8 = (idx & 15) * 8;
        u32x4 kv = {0u, 0u, 0u, 0u}, qv = {0u, 0u, 0u, 0u};
        if (row < nvalid) {
            kv = *reinterpret_cast<const u32x4*>(p.k + (row_base + row) * kDK + c8);
            qv = *reinterpret_cast<const u32x4*>(p.q + (row_base + row) * kDK + c8);
        }
        *reinterpret_cast<u32x4*>(&Kl[row][c8]) = kv;
        *reinterpret_cast<u32x4*>(&Ql[row][c8]) = qv;
    }

    // 2) Gates (wave 0, one token per lane) and the in-chunk log-cumsum.
    if (wave == 0) {
        const int t = lane;
        float lg = 0.f, bm = 0.f, m = 0.f;
        if (t < nvalid) {
            const size_t gi = row_base + t;
            m = p.mask ? p.mask[static_cast<size_t>(sq.b) * p.T_stride + sq.tok0 + t0 + t] : 1.f;
            lg = -expf(p.A_log[h]) * softplus_f(bf2f(p.a[gi]) + p.dt_bias);
            bm = sigmoid_f(bf2f(p.b[gi])) * m;
        }
        float s = lg;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const float u = __shfl_up(s, off);
            if (lane >= off) s += u;
        }
        const float last = __shfl(s, kWave - 1);
        s_lgc[t] = s;
        s_bm[t] = bm;
        s_ms[t] = m * p.scale;
        s_kdec[t] = expf(last - s);
        const float gam = expf(s);
        float* G = p.wsG + wc * 128;
        G[t] = gam;
        G[64 + t] = m * p.scale * gam;
    }
    __syncthreads();

    // 3) K K^T and Q K^T: wave w owns row tile w and the column tiles j <= w.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = 16 * j + m16;
        if (j > wave) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * wave + 4 * g4 + i;
                Am[row][col] = 0.f;
                Al[row][col] = f2bf(0.f);
            }
            continue;
        }
        f32x4 accK = {0.f, 0.f, 0.f, 0.f}, accQ = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 aK = *reinterpret_cast<const bf16x8*>(&Kl[16 * wave + m16][32 * s + 8 * g4]);
            const bf16x8 aQ = *reinterpret_cast<const bf16x8*>(&Ql[16 * wave + m16][32 * s + 8 * g4]);
            const bf16x8 bK = *reinterpret_cast<const bf16x8*>(&Kl[16 * j + m16][32 * s + 8 * g4]);
            accK = mfma16x16x32(aK, bK, accK);
            accQ = mfma16x16x32(aQ, bK, accQ);
        }
        const float lgc_col = s_lgc[col];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * wave + 4 * g4 + i;
            const float d = expf(s_lgc[row] - lgc_col);
            Am[row][col] = row > col ? s_bm[row] * accK[i] * d : 0.f;
            Al[row][col] = f2bf(row >= col ? s_ms[row] * accQ[i] * d : 0.f);
        }
    }
    __syncthreads();

    if (wave == 0) {
        // 4a) T = (I + A)^-1 by forward substitution, fp32.  Lane c owns
        // column c: T[i][c] = [i == c] - sum_{j<i} A[i][j] T[j][c]; rows of A
        // are broadcast reads from LDS.
        float Tc[kC];
#pragma unroll
        for (int i = 0; i < kC; ++i) {
            float acc = (i == lane) ? 1.f : 0.f;
#pragma unroll
            for (int j4 = 0; j4 < i; j4 += 4) {
                const f32x4 arow = *reinterpret_cast<const f32x4*>(&Am[i][j4]);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (j4 + u < i) acc -= arow[u] * Tc[j4 + u];
            }
            Tc[i] = acc;
        }
        const float bmc = s_bm[lane];
#pragma unroll
        for (int i = 0; i < kC; ++i) Tl[i][lane] = f2bf(Tc[i] * bmc);
    } else if (wave == 1) {
        // 4b) Aq fragments (mt, s): lane holds Aq[16mt + m][32s + pi(g, j)].
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const int mt = f >> 1, s = f & 1;
            const bf16* rp = &Al[16 * mt + m16][32 * s + 4 * g4];
            const u32x2 lo = *reinterpret_cast<const u32x2*>(rp);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(rp + 16);
            p.wsA[(wc * 8 + f) * 64 + lane] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
    } else {
        // 4c) Kt fragments (r, s): lane holds K[32s + pi(g,j)][rho(r, m/4, m%4)]
        // times gamma_C / gamma_t.  Waves 2 and 3 take eight fragments each.
        const int f0 = (wave - 2) * 8;
#pragma unroll
        for (int f = f0; f < f0 + 8; ++f) {
            const int r = f >> 1, s = f & 1;
            const int krow = rho_row(r, m16 >> 2, m16 & 3);
            bf16x8 frag;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int t = 32 * s + pi_pos(g4, jj);
                frag[jj] = f2bf(bf2f(Kl[t][krow]) * s_kdec[t]);
            }
            p.wsK[(wc * 16 + f) * 64 + lane] = __builtin_bit_cast(u32x4, frag);
        }
    }
    __syncthreads();

    // 5) Tp fragments, two per wave.
#pragma unroll
    for (int f = 2 * wave; f < 2 * wave + 2; ++f) {
        const int mt = f >> 1, s = f & 1;
        const bf16* rp = &Tl[16 * mt + m16][32 * s + 4 * g4];
        const u32x2 lo = *reinterpret_cast<const u32x2*>(rp);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(rp + 16);
        p.wsT[(wc * 8 + f) * 64 + lane] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
}

// ---------------------------------------------------------------------------
// Kernel 2
// ---------------------------------------------------------------------------
template <int NT>
__global__ __launch_bounds__(64) void gdn_prefill_state_kernel(PrefillParams p, int nvt, int nheads,
                                                               int xcd_map) {
    // blockIdx -> (head, column tile).  With xcd_map the column tiles of one
    // head land on the same XCD (workgroups are dealt to the 8 XCDs round
    // robin), so the per-chunk operands they all read share one L2.
    const int wg = blockIdx.x;
    int head, vt;
    if (xcd_map) {
        const int xcd = wg & 7, j = wg >> 3;
        vt = j % nvt;
        head = (j / nvt) * 8 + xcd;
    } else {
        vt = wg % nvt;
        head = wg / nvt;
    }
    if (head >= nheads) return;
    const int sidx = head / p.H;
    const int h = head % p.H;
    const SeqInfo sq = seq_info(p, sidx);
    const int lane = threadIdx.x;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int dv = p.dv;
    const int colbase = vt * 16 * NT + n;

    // State tile: S[r][nt][i] = S[rho(r, g, i)][colbase + 16 nt].
    f32x4 S[8][NT];
    {
        const float* sin = p.state_in ? p.state_in + static_cast<size_t>(sidx * p.H + h) * kDK * dv : nullptr;
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    S[r][nt][i] = sin ? sin[static_cast<size_t>(rho_row(r, g, i)) * dv + colbase + 16 * nt] : 0.f;
    }

    const int nchunks = (sq.len + kC - 1) / kC;
    const size_t head_row0 = static_cast<size_t>(sq.b * p.H + h) * p.T_stride + sq.tok0;
    for (int c = 0; c < nchunks; ++c) {
        const int nvalid = min(kC, sq.len - c * kC);
        const size_t row_base = head_row0 + static_cast<size_t>(c) * kC;
        const size_t wc = static_cast<size_t>(sq.slot0 + c) * p.H + h;
        const float* G = p.wsG + wc * 128;

        // (a) X = K S and P = Q S; B operand = bf16 of the state accumulators.
        f32x4 X[4][NT], P[4][NT];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                X[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                P[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            bf16x8 Bs[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) Bs[nt] = pack8(S[2 * s][nt], S[2 * s + 1][nt]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int row = 16 * mt + n;
                u32x4 kw = {0u, 0u, 0u, 0u}, qw = {0u, 0u, 0u, 0u};
                if (row < nvalid) {
                    kw = *reinterpret_cast<const u32x4*>(p.k + (row_base + row) * kDK + 32 * s + 8 * g);
                    qw = *reinterpret_cast<const u32x4*>(p.q + (row_base + row) * kDK + 32 * s + 8 * g);
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    X[mt][nt] = mfma16x16x32(as_bf16x8(kw), Bs[nt], X[mt][nt]);
                    P[mt][nt] = mfma16x16x32(as_bf16x8(qw), Bs[nt], P[mt][nt]);
                }
            }
        }

        // (b) Y = V - gamma o X, in the accumulator layout (reuses X).
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const f32x4 gam = *reinterpret_cast<const f32x4*>(G + 16 * mt + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * mt + 4 * g + i;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const float vv = row < nvalid ? bf2f(p.v[(row_base + row) * dv + colbase + 16 * nt]) : 0.f;
                    X[mt][nt][i] = vv - gam[i] * X[mt][nt][i];
                }
            }
        }

        // (c) dV = Tp Y.
        f32x4 D[4][NT];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) D[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            bf16x8 BY[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) BY[nt] = pack8(X[2 * s][nt], X[2 * s + 1][nt]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const bf16x8 aT = as_bf16x8(p.wsT[(wc * 8 + mt * 2 + s) * 64 + lane]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) D[mt][nt] = mfma16x16x32(aT, BY[nt], D[mt][nt]);
            }
        }
        bf16x8 BD[2][NT];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) BD[s][nt] = pack8(D[2 * s][nt], D[2 * s + 1][nt]);

        // (d) O = (m scale gamma) o P + Aq dV  -> bf16 out.
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const f32x4 co = *reinterpret_cast<const f32x4*>(G + 64 + 16 * mt + 4 * g);
            f32x4 O[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) O[nt] = co * P[mt][nt];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                if (s == 1 && mt < 2) continue;  // columns 32..63 are above the diagonal
                const bf16x8 aA = as_bf16x8(p.wsA[(wc * 8 + mt * 2 + s) * 64 + lane]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) O[nt] = mfma16x16x32(aA, BD[s][nt], O[nt]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * mt + 4 * g + i;
                if (row < nvalid) {
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        p.out[(row_base + row) * dv + colbase + 16 * nt] = f2bf_bits(O[nt][i]);
                }
            }
        }

        // (e) S <- gamma_C S + Kt dV.
        const float gC = G[kC - 1];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) S[r][nt] *= gC;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const bf16x8 aK = as_bf16x8(p.wsK[(wc * 16 + r * 2 + s) * 64 + lane]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) S[r][nt] = mfma16x16x32(aK, BD[s][nt], S[r][nt]);
            }
        }
    }

    float* so = p.state_out + static_cast<size_t>(sidx * p.H + h) * kDK * dv;
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                so[static_cast<size_t>(rho_row(r, g, i)) * dv + colbase + 16 * nt] = S[r][nt][i];
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr size_t kBytesT = 8 * 64 * 16;
constexpr size_t kBytesA = 8 * 64 * 16;
constexpr size_t kBytesK = 16 * 64 * 16;
constexpr size_t kBytesG = 128 * 4;

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct WsLayout {
    size_t offT, offA, offK, offG, total;
};

WsLayout ws_layout(long long slots, int H) {
    const size_t ch = static_cast<size_t>(slots) * H;
    WsLayout L;
    L.offT = 0;
    L.offA = align256(L.offT + ch * kBytesT);
    L.offK = align256(L.offA + ch * kBytesA);
    L.offG = align256(L.offK + ch * kBytesK);
    L.total = align256(L.offG + ch * kBytesG);
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

int launch(PrefillParams& p, int nseq, int nchunk_grid, void* workspace, size_t ws_bytes,
           long long slots, hipStream_t stream) {
    using gdn_host::fail;
    const WsLayout L = ws_layout(slots, p.H);
    if (!workspace || ws_bytes < L.total)
        return fail(GDN_ERR_WORKSPACE, "prefill: workspace of %zu bytes given, %zu needed", ws_bytes, L.total);
    if (!gdn_host::aligned(workspace, 256))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: workspace must be 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    p.wsT = reinterpret_cast<u32x4*>(ws + L.offT);
    p.wsA = reinterpret_cast<u32x4*>(ws + L.offA);
    p.wsK = reinterpret_cast<u32x4*>(ws + L.offK);
    p.wsG = reinterpret_cast<float*>(ws + L.offG);

    if (nchunk_grid > 0) {
        hipLaunchKernelGGL(gdn_prefill_intra_kernel, dim3(nchunk_grid, p.H, nseq), dim3(256), 0, stream, p);
        const int st = gdn_host::check_launch("gdn_prefill_intra_kernel");
        if (st != GDN_OK) return st;
    }
    const int nheads = nseq * p.H;
    const long long waves16 = static_cast<long long>(nheads) * (p.dv / 16);
    const int NT = (waves16 >= 4096 && p.dv % 32 == 0) ? 2 : 1;
    const int nvt = p.dv / (16 * NT);
    const int xcd_map = (nheads % 8 == 0) ? 1 : 0;
    const long long nwg = static_cast<long long>(nheads) * nvt;
    if (nwg > 0x7fffffffLL) return fail(GDN_ERR_UNSUPPORTED, "prefill: grid too large");
    if (NT == 2)
        hipLaunchKernelGGL(gdn_prefill_state_kernel<2>, dim3(static_cast<unsigned>(nwg)), dim3(64), 0, stream, p,
                           nvt, nheads, xcd_map);
    else
        hipLaunchKernelGGL(gdn_prefill_state_kernel<1>, dim3(static_cast<unsigned>(nwg)), dim3(64), 0, stream, p,
                           nvt, nheads, xcd_map);
    return gdn_host::check_launch("gdn_prefill_state_kernel");
}

}  // namespace

extern "C" {

size_t gdn_prefill_workspace_bytes(int B, int H, int T, int dk, int dv) {
    (void)dk;
    (void)dv;
    if (B <= 0 || H <= 0 || T <= 0) return 0;
    const long long slots = static_cast<long long>(B) * ((T + kC - 1) / kC);
    return ws_layout(slots, H).total;
}

size_t gdn_prefill_varlen_workspace_bytes(int num_seqs, int H, int T_total, int dk, int dv) {
    (void)dk;
    (void)dv;
    if (num_seqs <= 0 || H <= 0 || T_total < 0) return 0;
    const long long slots = static_cast<long long>(T_total) / kC + num_seqs + 1;
    return ws_layout(slots, H).total;
}

int gdn_prefill_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                    const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                    const float* state_in, float scale, gdn_bf16_t* out, float* state_out, int B, int H,
                    int T, int dk, int dv, void* workspace, size_t workspace_bytes, void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    int st = check_common("prefill", H, dk, dv);
    if (st != GDN_OK) return st;
    if (B < 0 || T < 0) return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: B=%d T=%d", B, T);
    if (B == 0) return GDN_OK;
    if (!q || !k || !v || !A_log || !a || !b_logits || !state_out || (T > 0 && !out))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(state_out, 4) || (state_in && !aligned(state_in, 4)))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill: q/k need 16-byte alignment");
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
        if (state_in)
            return hipMemcpyAsync(state_out, state_in, static_cast<size_t>(B) * H * dk * dv * 4,
                                  hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)) == hipSuccess
                       ? GDN_OK
                       : fail(GDN_ERR_HIP, "prefill: state copy failed");
        return hipMemsetAsync(state_out, 0, static_cast<size_t>(B) * H * dk * dv * 4,
                              static_cast<hipStream_t>(stream)) == hipSuccess
                   ? GDN_OK
                   : fail(GDN_ERR_HIP, "prefill: state clear failed");
    }
    return launch(p, B, p.chunks_per_seq, workspace, workspace_bytes, slots, static_cast<hipStream_t>(stream));
}

int gdn_prefill_varlen_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v, const float* A_log,
                           const gdn_bf16_t* a, float dt_bias, const gdn_bf16_t* b_logits, const float* mask,
                           const int32_t* cu_seqlens, int num_seqs, int max_seqlen, const float* state_in,
                           float scale, gdn_bf16_t* out, float* state_out, int H, int T_total, int dk, int dv,
                           void* workspace, size_t workspace_bytes, void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    int st = check_common("prefill_varlen", H, dk, dv);
    if (st != GDN_OK) return st;
    if (num_seqs < 0 || T_total < 0)
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_varlen: num_seqs=%d T_total=%d", num_seqs, T_total);
    if (num_seqs == 0) return GDN_OK;
    if (!q || !k || !v || !A_log || !a || !b_logits || !cu_seqlens || !state_out || (T_total > 0 && !out))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_varlen: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "prefill_varlen: q/k need 16-byte alignment");
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
    return launch(p, num_seqs, nchunk_grid, workspace, workspace_bytes, slots, static_cast<hipStream_t>(stream));
}

}  // extern "C"
