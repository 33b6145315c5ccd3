// GDN decode: one token per sequence, fp32 state streamed through registers.
//
// Reference: kernels/decode.cu:48-128 (gdn_decode_kernel) and its launcher
// gdn_decode_cuda (:131-162); semantics of reference/decode_ref.py:36-59.
//
// Work split (MI355X, wave64).  The state of one head is S[dk=128][dv] fp32,
// dv contiguous.  One workgroup of 4 waves owns a 128 x CW column slice of
// one (sequence, head), CW = 128 where it divides dv (else 64, else 32):
//   wave w            -> state rows 32w .. 32w+31
//   lane = LPR rp + c -> columns 4c .. 4c+3 of the slice (LPR = CW/4 lanes
//                        per row), rows 32w + RPI i + rp, i < NI
// (RPI = 64/LPR rows per instruction, NI = 32/RPI instructions).  Every
// load/store instruction of a wave moves RPI whole row pieces of CW floats:
// at CW = 128, two full 512-byte state rows.  Each lane keeps its NI float4
// of S in VGPRs between the read-reduce pass and the update-write pass, so S
// is read once and written once (the HBM floor).  The reductions over dk
// (r = k^T S, o = q^T S') are a per-lane partial, a lane-group sum and one
// LDS exchange between the 4 waves.
//
// Measured at B=256, H=32, dv=128 (512 MiB state, in place, one MI355X):
//  * Full-row accesses beat 128-byte row pieces (a wave per 128 x 32 tile):
//    185 -> 175 us per step.
//  * At most two workgroups per CU (8 waves; 128 KiB of the state in flight
//    per CU) beats letting the register budget admit four: 175 -> 169 us
//    (80% of 8 TB/s; a plain in-place float4 stream of the same 512 MiB
//    takes 162 us on the same box).  More heads in flight at once spread
//    the DRAM accesses over more pages.  The cap is the LDS reduction buffer
//    sized to 72 KiB, so that no third workgroup fits in the CU's 160 KiB.
//  * Persistent workgroups (with or without loading the next head early)
//    measured 181-211 us.
//
// The state stream uses nontemporal loads and stores (the 'nt' cache policy):
// it is touched once per step and is larger than L2 and the 256 MB MALL, so
// keeping it out of the caches measured ~10% faster than default loads.
//
// In place: S_out may equal S_in.  Each element is read and later written by
// the same lane, so no other lane can observe a half-updated state.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

constexpr int kDK = 128;
constexpr int kWavesPerWG = 4;
constexpr int kRowsPerWave = kDK / kWavesPerWG;
// LDS per workgroup: the reduction buffer, sized so two workgroups fit in a
// CU's 160 KiB and a third does not.
constexpr int kRedSlots = 72 * 1024 / 16;

// OBF16: o is written as bf16 (round to nearest even of the fp32 value) into
// a [B, H, dv] bf16 buffer, for the decode step's out-projection.
template <int CW, bool OBF16>
__global__ __launch_bounds__(kWave* kWavesPerWG) void gdn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ bg, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* S_in, float scale,
    float* __restrict__ o, float* S_out, int H, int dv) {
    constexpr int LPR = CW / 4;
    constexpr int RPI = kWave / LPR;
    constexpr int NI = kRowsPerWave / RPI;
    static_assert(2 * kWavesPerWG * LPR <= kRedSlots, "reduction buffer");
    // [0][wave][c]: partial r; [1][wave][c]: partial o.
    __shared__ f32x4 red[kRedSlots];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int slices = dv / CW;
    const int bh = blockIdx.x / slices;
    const int h = bh % H;
    const int c = lane % LPR, rp = lane / LPR;
    const int col = (blockIdx.x % slices) * CW + 4 * c;
    const int row0 = kRowsPerWave * wave + rp;  // this lane's rows: row0 + RPI i

    const size_t sbase = (static_cast<size_t>(bh) * kDK + row0) * dv + col;
    f32x4 s[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
        s[i] = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4*>(S_in + sbase + static_cast<size_t>(RPI * i) * dv));

    float kf[NI], qf[NI];
    {
        const uint16_t* kp = k + static_cast<size_t>(bh) * kDK + row0;
        const uint16_t* qp = q + static_cast<size_t>(bh) * kDK + row0;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            kf[i] = bf2f(kp[RPI * i]);
            qf[i] = bf2f(qp[RPI * i]);
        }
    }
    // Gates: g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b).
    const float gdec = expf(-expf(A_log[h]) * softplus_f(bf2f(a[bh]) + dt_bias[h]));
    const float beta = sigmoid_f(bf2f(bg[bh]));
    const u32x2 vw = *reinterpret_cast<const u32x2*>(v + static_cast<size_t>(bh) * dv + col);
    const f32x4 vv = {__uint_as_float(vw[0] << 16), __uint_as_float(vw[0] & 0xffff0000u),
                      __uint_as_float(vw[1] << 16), __uint_as_float(vw[1] & 0xffff0000u)};

    // r = k^T S: this lane's rows, the RPI lanes of the column, the 4 waves.
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NI; ++i) r += kf[i] * s[i];
#pragma unroll
    for (int m = LPR; m < kWave; m <<= 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] += __shfl_xor(r[j], m);
    if (rp == 0) red[wave * LPR + c] = r;
    __syncthreads();
    f32x4 rt = red[c];
#pragma unroll
    for (int w = 1; w < kWavesPerWG; ++w) rt += red[w * LPR + c];
    const f32x4 delta = beta * (vv - gdec * rt);

    // S' = g S + k delta^T, written back; o = q^T S' accumulated on the way.
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const f32x4 sn = gdec * s[i] + kf[i] * delta;
        __builtin_nontemporal_store(sn, reinterpret_cast<f32x4*>(S_out + sbase + static_cast<size_t>(RPI * i) * dv));
        acc += qf[i] * sn;
    }
#pragma unroll
    for (int m = LPR; m < kWave; m <<= 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] += __shfl_xor(acc[j], m);
    if (rp == 0) red[(kWavesPerWG + wave) * LPR + c] = acc;
    __syncthreads();
    if (wave == 0 && rp == 0) {
        f32x4 ot = red[kWavesPerWG * LPR + c];
#pragma unroll
        for (int w = 1; w < kWavesPerWG; ++w) ot += red[(kWavesPerWG + w) * LPR + c];
        if constexpr (OBF16)
            *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(o) + static_cast<size_t>(bh) * dv + col) =
                pack4_bf16(scale * ot);
        else
            *reinterpret_cast<f32x4*>(o + static_cast<size_t>(bh) * dv + col) = scale * ot;
    }
}

}  // namespace

namespace gdn_host {

int decode_check(const void* q, const void* k, const void* v, const void* a, const void* b, const void* A_log,
                 const void* dt_bias, const void* S_in, const void* o, const void* S_out, int B, int H, int dk,
                 int dv) {
    if (B < 0 || H <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "decode: B=%d H=%d", B, H);
    if (dk != kDK) return fail(GDN_ERR_UNSUPPORTED, "decode: dk=%d, only dk=128 is built", dk);
    if (dv < 32 || dv > 1024 || dv % 32 != 0)
        return fail(GDN_ERR_UNSUPPORTED, "decode: dv=%d must be a multiple of 32 in [32, 1024]", dv);
    if (B == 0) return GDN_OK;
    if (!q || !k || !v || !a || !b || !A_log || !dt_bias || !S_in || !o || !S_out)
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 8) || !aligned(S_in, 16) ||
        !aligned(S_out, 16) || !aligned(o, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode: q/k/S/o need 16-byte, v 8-byte alignment");
    return GDN_OK;
}

}  // namespace gdn_host

int gdn_host::decode_launch(const void* q, const void* k, const void* v, const void* a, const void* b,
                           const float* A_log, const float* dt_bias, const float* S_in, float scale, void* o,
                           bool o_bf16, float* S_out, int B, int H, int dv, hipStream_t st) {
    // Column slice: the widest of 128 / 64 / 32 dividing dv, halved while the
    // grid would leave CUs idle (a small batch splits each head's columns
    // over more workgroups; columns of the state update independently).
    constexpr long long kCUs = 256;
    int cw = dv % 128 == 0 ? 128 : (dv % 64 == 0 ? 64 : 32);
    while (cw > 32 && static_cast<long long>(B) * H * (dv / cw) < kCUs) cw /= 2;
    const long long nwg_ll = static_cast<long long>(B) * H * (dv / cw);
    if (nwg_ll > 0x7fffffffLL) return fail(GDN_ERR_UNSUPPORTED, "decode: grid too large");
    const dim3 grid(static_cast<unsigned>(nwg_ll)), block(kWave * kWavesPerWG);
    const auto* qp = static_cast<const uint16_t*>(q);
    const auto* kp = static_cast<const uint16_t*>(k);
    const auto* vp = static_cast<const uint16_t*>(v);
    const auto* ap = static_cast<const uint16_t*>(a);
    const auto* bp = static_cast<const uint16_t*>(b);
    auto* op = static_cast<float*>(o);
    auto launch = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, st, qp, kp, vp, ap, bp, A_log, dt_bias, S_in, scale, op, S_out, H, dv);
    };
    if (cw == 128)
        o_bf16 ? launch(gdn_decode_kernel<128, true>) : launch(gdn_decode_kernel<128, false>);
    else if (cw == 64)
        o_bf16 ? launch(gdn_decode_kernel<64, true>) : launch(gdn_decode_kernel<64, false>);
    else
        o_bf16 ? launch(gdn_decode_kernel<32, true>) : launch(gdn_decode_kernel<32, false>);
    return gdn_host::check_launch("gdn_decode_kernel");
}

extern "C" int gdn_decode_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                              const gdn_bf16_t* a, const gdn_bf16_t* b, const float* A_log,
                              const float* dt_bias, const float* S_in, float scale, float* o,
                              float* S_out, int B, int H, int dk, int dv, void* stream) {
    const int chk = gdn_host::decode_check(q, k, v, a, b, A_log, dt_bias, S_in, o, S_out, B, H, dk, dv);
    if (chk != GDN_OK || B == 0) return chk;
    return gdn_host::decode_launch(q, k, v, a, b, A_log, dt_bias, S_in, scale, o, false, S_out, B, H, dv,
                                   static_cast<hipStream_t>(stream));
}
