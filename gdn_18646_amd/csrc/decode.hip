// GDN decode: one token per sequence, fp32 state streamed through registers.
//
// Reference: kernels/decode.cu:48-128 (gdn_decode_kernel) and its launcher
// gdn_decode_cuda (:131-162); semantics of reference/decode_ref.py:36-59.
//
// Work split (MI355X, wave64).  The state of one head is S[dk=128][dv] fp32,
// dv contiguous.  One wave owns a 128 x 32 column tile (16 KiB):
//   lane = 8 * cg + rg,  cg = 0..7 -> columns col0 + 4cg .. +3 (one float4)
//                        rg = 0..7 -> rows 16rg .. 16rg+15
// Every load/store instruction of the wave moves 8 rows x 128 contiguous
// bytes (one 128-byte line per row).  Each lane keeps its 16 float4 of S in
// VGPRs between the read-reduce pass and the update-write pass, so S is read
// once and written once (the HBM floor).  The two reductions over dk
// (r = k^T S and o = q^T S') are a per-lane partial over 16 rows followed by
// an 8-lane DPP sum (no LDS, no barrier).  Four waves form a workgroup and
// cover 128 columns; dv > 128 uses more workgroups per head.
//
// The state stream uses nontemporal loads and stores (the 'nt' cache policy):
// it is touched once per step and is larger than L2 and the 256 MB MALL, so
// keeping it out of the caches measured ~10% faster than default loads
// (188 vs 207 us per step at B=256, H=32).
//
// In place: S_out may equal S_in.  Each element is read and later written by
// the same lane, so no other lane can observe a half-updated state.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

constexpr int kDK = 128;
constexpr int kColsPerWave = 32;
constexpr int kWavesPerWG = 4;

__global__ __launch_bounds__(kWave* kWavesPerWG) void gdn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ bg, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const float* S_in, float scale,
    float* __restrict__ o, float* S_out, int H, int dv, int wgs_per_head) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int bh = blockIdx.x / wgs_per_head;
    const int col0 = ((blockIdx.x % wgs_per_head) * kWavesPerWG + wave) * kColsPerWave;
    if (col0 >= dv) return;  // whole wave leaves together; no barriers below
    const int h = bh % H;
    const int cg = lane >> 3;
    const int rg = lane & 7;
    const int col = col0 + 4 * cg;
    const int row0 = 16 * rg;

    // Gates: g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b).
    const float gdec = expf(-expf(A_log[h]) * softplus_f(bf2f(a[bh]) + dt_bias[h]));
    const float beta = sigmoid_f(bf2f(bg[bh]));

    const size_t sbase = (static_cast<size_t>(bh) * kDK + row0) * dv + col;
    f32x4 s[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        s[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(S_in + sbase + static_cast<size_t>(i) * dv));

    float kf[16], qf[16];
    {
        const u32x4* kp = reinterpret_cast<const u32x4*>(k + static_cast<size_t>(bh) * kDK + row0);
        const u32x4* qp = reinterpret_cast<const u32x4*>(q + static_cast<size_t>(bh) * kDK + row0);
        unpack8(kp[0], kf);
        unpack8(kp[1], kf + 8);
        unpack8(qp[0], qf);
        unpack8(qp[1], qf + 8);
    }
    const u32x2 vw = *reinterpret_cast<const u32x2*>(v + static_cast<size_t>(bh) * dv + col);
    const float vv[4] = {__uint_as_float(vw[0] << 16), __uint_as_float(vw[0] & 0xffff0000u),
                         __uint_as_float(vw[1] << 16), __uint_as_float(vw[1] & 0xffff0000u)};

    // r = k^T S over this lane's 16 rows, then across the 8 row groups.
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) r += kf[i] * s[i];
    f32x4 delta;
#pragma unroll
    for (int c = 0; c < 4; ++c) delta[c] = beta * (vv[c] - gdec * sum8(r[c]));

    // S' = g S + k delta^T, written back; o = q^T S' accumulated on the way.
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const f32x4 sn = gdec * s[i] + kf[i] * delta;
        __builtin_nontemporal_store(sn, reinterpret_cast<f32x4*>(S_out + sbase + static_cast<size_t>(i) * dv));
        acc += qf[i] * sn;
    }
    f32x4 out;
#pragma unroll
    for (int c = 0; c < 4; ++c) out[c] = scale * sum8(acc[c]);
    if (rg == 0) *reinterpret_cast<f32x4*>(o + static_cast<size_t>(bh) * dv + col) = out;
}

}  // namespace

extern "C" int gdn_decode_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                              const gdn_bf16_t* a, const gdn_bf16_t* b, const float* A_log,
                              const float* dt_bias, const float* S_in, float scale, float* o,
                              float* S_out, int B, int H, int dk, int dv, void* stream) {
    using gdn_host::aligned;
    using gdn_host::fail;
    if (B < 0 || H <= 0) return fail(GDN_ERR_INVALID_ARGUMENT, "decode: B=%d H=%d", B, H);
    if (dk != kDK) return fail(GDN_ERR_UNSUPPORTED, "decode: dk=%d, only dk=128 is built", dk);
    if (dv < 32 || dv > 1024 || dv % kColsPerWave != 0)
        return fail(GDN_ERR_UNSUPPORTED, "decode: dv=%d must be a multiple of 32 in [32, 1024]", dv);
    if (B == 0) return GDN_OK;
    if (!q || !k || !v || !a || !b || !A_log || !dt_bias || !S_in || !o || !S_out)
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode: null pointer argument");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 8) || !aligned(S_in, 16) ||
        !aligned(S_out, 16) || !aligned(o, 16))
        return fail(GDN_ERR_INVALID_ARGUMENT, "decode: q/k/S/o need 16-byte, v 8-byte alignment");
    const long long nwg_ll = static_cast<long long>(B) * H * ((dv + 127) / 128);
    if (nwg_ll > 0x7fffffffLL) return fail(GDN_ERR_UNSUPPORTED, "decode: grid too large");
    const int wgs_per_head = (dv + 127) / 128;
    hipLaunchKernelGGL(gdn_decode_kernel, dim3(static_cast<unsigned>(nwg_ll)),
                       dim3(kWave * kWavesPerWG), 0, static_cast<hipStream_t>(stream), q, k, v, a,
                       b, A_log, dt_bias, S_in, scale, o, S_out, H, dv, wgs_per_head);
    return gdn_host::check_launch("gdn_decode_kernel");
}
