// Shared device helpers and host-side error plumbing for libgdn_amd.so.
// gfx950 (CDNA4) only: wave64, bf16 MFMA 16x16x32, 160 KiB LDS per CU.
#pragma once

#include <type_traits>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/gdn_amd.h"

namespace gdn {

// ---------------------------------------------------------------------------
// Vector types used as MFMA operands and for 128-bit memory traffic.
// ---------------------------------------------------------------------------
typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
__device__ __forceinline__ float bf2f(bf16 x) { return static_cast<float>(x); }

// Round-to-nearest-even float -> bf16 (gfx950 has a native convert).
__device__ __forceinline__ bf16 f2bf(float x) { return static_cast<bf16>(x); }

__device__ __forceinline__ uint16_t f2bf_bits(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<bf16>(x));
}

// Unpack 8 bf16 held in a 128-bit word into floats.
__device__ __forceinline__ void unpack8(const u32x4 w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

// softplus(x) = log(1 + e^x), linear above 20 as in the reference
// (kernels/decode.cu:36-38); log1pf/expf are the ROCm device library's.
__device__ __forceinline__ float softplus_f(float x) {
    return x > 20.f ? x : log1pf(expf(x));
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }
// x * sigmoid(x) with the hardware exp2 and reciprocal (about 1 ulp each).
__device__ __forceinline__ float silu_f(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// ---------------------------------------------------------------------------
// Cross-lane sums over groups of 8 consecutive lanes, all DPP (no LDS).
// quad_perm [1,0,3,2] and [2,3,0,1] give the sum over each quad; the
// half-row mirror (lane i <-> 7-i inside each 8-lane half row) adds the
// other quad of the group.  Every lane of the group ends with the total.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    return v;
}
// Sum over the whole wave, the same in every lane: sum8, the row mirror
// (lane i <-> 15-i of each 16-lane row) for the row sums, then the four row
// sums read into scalars and added in row order.  No LDS round trips.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = sum8(v);
    v += dpp_f<0x140>(v);  // row_mirror
    const int b = __float_as_int(v);
    return (__int_as_float(__builtin_amdgcn_readlane(b, 0)) + __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
           (__int_as_float(__builtin_amdgcn_readlane(b, 32)) + __int_as_float(__builtin_amdgcn_readlane(b, 48)));
}

// MFMA 16x16x32 bf16 -> fp32.  Operand layout used throughout (the k order
// inside a lane is free as long as A and B agree on it):
//   A (16 x 32): lane l supplies row l%16, eight k values of group l/16
//   B (32 x 16): lane l supplies column l%16, the same eight k values
//   C (16 x 16): lane l holds column l%16, rows 4*(l/16) + i, i = 0..3
__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8 a, const bf16x8 b, const f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two floats -> two round-to-nearest-even bf16 in one word: one
// v_cvt_pk_bf16_f32 (converting element by element costs a convert per value
// plus the shifts and ors that merge the halves).
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Four floats -> four bf16, as 8 bytes.
__device__ __forceinline__ u32x2 pack4_bf16(const f32x4 v) {
    return u32x2{pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])};
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 w) { return __builtin_bit_cast(bf16x8, w); }
__device__ __forceinline__ u32x4 as_u32x4(const bf16x8 w) { return __builtin_bit_cast(u32x4, w); }

// Compile-time loop: f(integral_constant<int, I>) for I in [B, E).  Keeps
// register-array indices constant from the first optimisation pass on.
template <int B, int E, typename Fn>
__device__ __forceinline__ void static_for(Fn&& fn) {
    if constexpr (B < E) {
        fn(std::integral_constant<int, B>{});
        static_for<B + 1, E>(fn);
    }
}

__device__ __forceinline__ bf16x8 pack8(const f32x4 lo, const f32x4 hi) {
    return as_bf16x8(u32x4{pack2_bf16(lo[0], lo[1]), pack2_bf16(lo[2], lo[3]), pack2_bf16(hi[0], hi[1]),
                           pack2_bf16(hi[2], hi[3])});
}

// ---------------------------------------------------------------------------
// LDS staging by DMA (global_load_lds) and the waits that order it.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) uint16_t lds_u16;

// 16 bytes per lane from sbase + voff (sbase uniform over the wave, voff the
// lane's 32-bit byte offset) to lds_base + 16 lane (lds_base uniform).
// Asynchronous: completion is vmcnt.  The scalar-base form keeps source
// addresses to one 32-bit register per lane: 64-bit per-lane pointers spill
// in the state kernels, and a spill reload between copies makes the compiler
// wait for every copy issued before it.  Issued as inline asm so the
// compiler's wait-count pass does not drain the copy before unrelated LDS
// reads of the other buffer (it cannot prove they do not alias); the kernels
// order copies with their own vmcnt waits and barriers.  M0 is otherwise
// unused on gfx950 (LDS instructions do not read it), so the clobber is safe.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, lds_u8* lds_base) {
    const uint32_t m0v = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0v), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier for LDS producer/consumer hand-off: LDS writes of this
// wave complete, then all waves meet.  (Async copies are covered by the
// vmcnt wait that precedes it.)
// Raw buffer resource over [base, base + bytes) (base uniform over the wave):
// a load past the end returns zeros.  A buffer load addresses with the
// resource (SGPRs), one 32-bit lane offset and a scalar offset, so a run of
// loads in flight holds no 64-bit address per load in VGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// vmcnt(N) with the other counters open (gfx9 layout: vmcnt[3:0] | expcnt[6:4]
// | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).  Vector memory ops retire in issue
// order, so vmcnt(N) means "all but the last N issued have completed".
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

}  // namespace gdn

// ---------------------------------------------------------------------------
// Host-side helpers shared by the entry points (defined in abi.cpp).
// ---------------------------------------------------------------------------
namespace gdn_host {
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* kernel);
inline bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }
// Argument checks of gdn_decode_hip (defined in decode.hip): GDN_OK when the
// call would launch (or, for B == 0, do nothing), else the error status.
int decode_check(const void* q, const void* k, const void* v, const void* a, const void* b, const void* A_log,
                 const void* dt_bias, const void* S_in, const void* o, const void* S_out, int B, int H, int dk,
                 int dv);
// The decode recurrence launch behind gdn_decode_hip (defined in decode.hip;
// arguments already checked by decode_check).  o_bf16: o is written as bf16
// [B, H, dv] (RNE of the fp32 value) into the buffer o points to.
int decode_launch(const void* q, const void* k, const void* v, const void* a, const void* b, const float* A_log,
                  const float* dt_bias, const float* S_in, float scale, void* o, bool o_bf16, float* S_out, int B,
                  int H, int dv, hipStream_t stream);
// RMSNorm of R rows (defined in rmsnorm.hip; arguments already checked as
// gdn_rmsnorm_hip checks them).  hist (nc > 0): the rows' x_n history
// [R, nc, D] (nc <= 3), shifted one token older with y appended, in place.
int rmsnorm_launch(const void* x, const void* gamma, void* y, void* hist, int nc, int R, int D, float eps,
                   hipStream_t stream);
}  // namespace gdn_host
