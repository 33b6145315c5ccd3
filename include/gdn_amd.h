/*
 * gdn_amd.h — C ABI of the MI355X (gfx950) Gated DeltaNet hot-path library
 * (libgdn_amd.so).
 *
 * Plain pointers and sizes only.  All data pointers are DEVICE pointers unless
 * a parameter says otherwise; every call is asynchronous on `stream` (a
 * hipStream_t passed as void*, NULL = the null stream) and returns a status
 * code.  On failure nothing is launched and gdn_last_error() returns a message
 * for the calling thread.  bf16 tensors are passed as their 16-bit patterns.
 *
 * Reference interfaces replaced (paths into diacccc/GDN_18646):
 *   gdn_decode_hip            <- extern "C" gdn_decode_cuda, kernels/decode.cu:131-162
 *                                (and gdn_decode_forward, kernels/decode.cu:172-214)
 *   gdn_prefill_hip           <- gdn_prefill, kernels/prefill_chunked.cu:422-504
 *   gdn_prefill_noalloc_hip   <- no reference counterpart (gdn_prefill_hip with a static
 *                                scratch buffer, for callers that cannot allocate)
 *   gdn_prefill_varlen_hip    <- no reference counterpart (packed cu_seqlens prefill);
 *                                semantics = gdn_prefill per sequence
 *   gdn_rmsnorm_hip           <- rmsnorm_forward_impl / launch_rmsnorm,
 *                                kernels/rmsnorm.cu:112-131,251-276
 *   gdn_proj_conv_silu_hip    <- fused_proj_conv_silu, kernels/fused_proj_conv_silu.cu:298-355
 *   gdn_in_proj_hip           <- GDNLayerCustom.forward's projections, gdn_layer.py:240-252
 *   gdn_in_proj_varlen_hip,   <- no reference counterpart (packed sequences through the layer;
 *   gdn_prefill_varlen_tm_hip    the reference layer has no cu_seqlens path, gdn_layer.py:222-263)
 *   gdn_decode_conv_step_hip  <- _decode_conv_step / _decode_fused_proj_step, gdn_layer.py:43-69
 *   gdn_decode_in_proj_hip    <- GDNLayerCustom.decode's RMSNorm, projections and conv step,
 *                                gdn_layer.py:280-299 (with 43-69)
 *   gdn_decode_out_proj_hip   <- GDNLayerCustom.decode's output projection, gdn_layer.py:309
 *   gdn_layer_decode_step_hip <- GDNLayerCustom.decode as a whole, gdn_layer.py:265-316
 */
#ifndef GDN_AMD_H
#define GDN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t gdn_bf16_t; /* bfloat16 bit pattern */

enum {
    GDN_OK = 0,
    GDN_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, misaligned buffer */
    GDN_ERR_UNSUPPORTED = 2,      /* shape outside what the kernels are built for */
    GDN_ERR_WORKSPACE = 3,        /* workspace missing or smaller than required */
    GDN_ERR_HIP = 4               /* a HIP runtime call or launch failed */
};

/* Library version, e.g. 1 for this interface revision. */
int gdn_abi_version(void);

/* Human-readable text for a status code, and the last error of this thread. */
const char* gdn_status_string(int status);
const char* gdn_last_error(void);

/*
 * Decode: one token per sequence, state updated as
 *   S <- g S ; r = k^T S ; S <- S + k (beta (v - r))^T ; o = scale q^T S
 * with g = exp(-exp(A_log[h]) softplus(a + dt_bias[h])), beta = sigmoid(b).
 *   q, k     [B, H, dk]   bf16        v        [B, H, dv] bf16
 *   a, b     [B, H]       bf16        A_log, dt_bias [H] fp32
 *   S_in     [B, H, dk, dv] fp32      o        [B, H, dv] fp32
 *   S_out    [B, H, dk, dv] fp32 — may be the same buffer as S_in (in place)
 * Supported: dk == 128, dv % 32 == 0, 32 <= dv <= 1024.  Buffers 16-byte aligned.
 * Replaces gdn_decode_cuda (kernels/decode.cu:131-162), which took no stream,
 * returned nothing and silently did nothing for an unsupported dv.
 */
int gdn_decode_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                   const gdn_bf16_t* a, const gdn_bf16_t* b,
                   const float* A_log, const float* dt_bias,
                   const float* S_in, float scale,
                   float* o, float* S_out,
                   int B, int H, int dk, int dv, void* stream);

/*
 * Chunked prefill (chunk size 64) of B equal-length sequences.
 *   q, k [B, H, T, dk] bf16; v [B, H, T, dv] bf16; a, b_logits [B, H, T] bf16
 *   A_log [H] fp32; dt_bias scalar; mask [B, T] fp32 or NULL (all ones)
 *   state_in [B, H, dk, dv] fp32 or NULL (zero state)
 *   out [B, H, T, dv] bf16; state_out [B, H, dk, dv] fp32
 * scale == 0 means dk^-0.5.  Any T >= 1.  Supported: dk == 128, dv % 16 == 0,
 * 16 <= dv <= 512.  Masked tokens decay the state but write nothing, and their
 * outputs are zero (reference/prefill_ref.py:79-80,130).
 * workspace: device buffer of at least gdn_prefill_workspace_bytes(B, H, T,
 * dk, dv) bytes, 256-byte aligned; it holds per-chunk intermediates.
 * Replaces gdn_prefill (kernels/prefill_chunked.cu:422-504), which required
 * H == 16, dv == 256 and T % 64 == 0 and allocated its outputs itself.
 */
size_t gdn_prefill_workspace_bytes(int B, int H, int T, int dk, int dv);

int gdn_prefill_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                    const float* A_log, const gdn_bf16_t* a, float dt_bias,
                    const gdn_bf16_t* b_logits, const float* mask,
                    const float* state_in, float scale,
                    gdn_bf16_t* out, float* state_out,
                    int B, int H, int T, int dk, int dv,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * gdn_prefill_hip with the output written token-major: out [B, T, H, dv]
 * (the layout the output projection consumes, so the caller's
 * transpose(1, 2).contiguous() copy disappears); all else identical.
 * Replaces the transposes around the prefill call in the reference layer
 * (gdn_layer.py:256-263), which has no kernel-level counterpart.
 */
int gdn_prefill_tm_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                       const float* A_log, const gdn_bf16_t* a, float dt_bias,
                       const gdn_bf16_t* b_logits, const float* mask,
                       const float* state_in, float scale,
                       gdn_bf16_t* out, float* state_out,
                       int B, int H, int T, int dk, int dv,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * gdn_prefill_hip without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.
 * The per-chunk intermediates go to a static device buffer of
 * GDN_PREFILL_NOALLOC_MAX_BYTES that the library holds per GPU until the
 * process ends; the call allocates nothing.  A shape whose
 * gdn_prefill_workspace_bytes() exceeds that size is refused with
 * GDN_ERR_WORKSPACE before any HIP call (e.g. B=1, H=16, T=8192, dk=dv=128
 * needs 40 MiB and B=4, H=16, T=4096 56 MiB, which fit; B=4, H=16, T=8192
 * needs 88 MiB and does not).
 * The buffer used is the current device's, so `stream` (when not null) must
 * belong to the current device (else GDN_ERR_INVALID_ARGUMENT).
 * All calls on one GPU share the buffer: calls that overlap on one GPU (two
 * streams, two threads) race, so serialise them.  Nothing in it needs to
 * start zeroed.  Outputs are bit-identical to gdn_prefill_hip's.
 */
#define GDN_PREFILL_NOALLOC_MAX_BYTES (64u << 20)

int gdn_prefill_noalloc_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                            const float* A_log, const gdn_bf16_t* a, float dt_bias,
                            const gdn_bf16_t* b_logits, const float* mask,
                            const float* state_in, float scale,
                            gdn_bf16_t* out, float* state_out,
                            int B, int H, int T, int dk, int dv, void* stream);

/*
 * The two phases of gdn_prefill_hip, same arguments, for callers that overlap
 * them with other work (and for per-phase timing):
 *   intra — every chunk in parallel: reads q, k, a, b_logits, mask, A_log,
 *           dt_bias, scale; fills `workspace` (out/state pointers unused);
 *   state — chunks in order per (sequence, head): reads the workspace, q, k,
 *           v, state_in; writes out and state_out.
 * gdn_prefill_hip is intra followed by state on the same stream.  No
 * reference counterpart (the reference runs one fused kernel).
 */
int gdn_prefill_intra_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                          const float* A_log, const gdn_bf16_t* a, float dt_bias,
                          const gdn_bf16_t* b_logits, const float* mask,
                          const float* state_in, float scale,
                          gdn_bf16_t* out, float* state_out,
                          int B, int H, int T, int dk, int dv,
                          void* workspace, size_t workspace_bytes, void* stream);

int gdn_prefill_state_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                          const float* A_log, const gdn_bf16_t* a, float dt_bias,
                          const gdn_bf16_t* b_logits, const float* mask,
                          const float* state_in, float scale,
                          gdn_bf16_t* out, float* state_out,
                          int B, int H, int T, int dk, int dv,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Packed variable-length prefill: num_seqs sequences concatenated along T.
 *   q, k [H, T_total, dk]; v [H, T_total, dv]; a, b_logits [H, T_total]
 *   cu_seqlens: DEVICE int32 [num_seqs + 1], non-decreasing, cu[0] = 0,
 *               cu[num_seqs] = T_total
 *   max_seqlen: upper bound on any sequence length (<= 0: T_total is used)
 *   mask [T_total] fp32 or NULL; state_in [num_seqs, H, dk, dv] or NULL
 *   out [H, T_total, dv] bf16; state_out [num_seqs, H, dk, dv] fp32
 * Each sequence is an independent prefill (state does not cross sequences).
 */
size_t gdn_prefill_varlen_workspace_bytes(int num_seqs, int H, int T_total, int dk, int dv);

int gdn_prefill_varlen_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                           const float* A_log, const gdn_bf16_t* a, float dt_bias,
                           const gdn_bf16_t* b_logits, const float* mask,
                           const int32_t* cu_seqlens, int num_seqs, int max_seqlen,
                           const float* state_in, float scale,
                           gdn_bf16_t* out, float* state_out,
                           int H, int T_total, int dk, int dv,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * gdn_prefill_varlen_hip with the output written token-major: out
 * [T_total, H, dv] (the layout the output projection consumes); all else
 * identical.  No reference counterpart (the layer's packed-sequence forward).
 */
int gdn_prefill_varlen_tm_hip(const gdn_bf16_t* q, const gdn_bf16_t* k, const gdn_bf16_t* v,
                              const float* A_log, const gdn_bf16_t* a, float dt_bias,
                              const gdn_bf16_t* b_logits, const float* mask,
                              const int32_t* cu_seqlens, int num_seqs, int max_seqlen,
                              const float* state_in, float scale,
                              gdn_bf16_t* out, float* state_out,
                              int H, int T_total, int dk, int dv,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * RMSNorm: y[r, :] = bf16(x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * gamma).
 *   x, y [R, D] bf16 (may not alias); gamma [D] bf16.  D % 8 == 0, D <= 16384.
 */
int gdn_rmsnorm_hip(const gdn_bf16_t* x, const gdn_bf16_t* gamma, gdn_bf16_t* y,
                    int R, int D, float eps, void* stream);

/*
 * Projection + causal depthwise conv (taps conv_k) + SiLU, fp32 accumulation:
 *   out[b, t, c] = bf16(SiLU(sum_j conv_w[c, j] * P[b, t - conv_k + 1 + j, c]))
 *   P = x W^T with P[b, t<0, :] = 0.
 *   x [B, T, D] bf16; W [D_out, D] bf16; conv_w [D_out, conv_k] bf16;
 *   out [B, T, D_out] bf16.  D % 64 == 0, D_out % 16 == 0, conv_k in 1..4.
 */
int gdn_proj_conv_silu_hip(const gdn_bf16_t* x, const gdn_bf16_t* W,
                           const gdn_bf16_t* conv_w, gdn_bf16_t* out,
                           int B, int T, int D, int D_out, int conv_k, void* stream);

/*
 * Layer in-projection for a prefill: P = xn [B, T, D] x W^T with
 * W = [W_q; W_k; W_v; W_a; W_b] ([2 H dk + H dv + 2 H, D] bf16), causal
 * depthwise conv (conv_w_qkv [2 H dk + H dv, conv_k]) + SiLU on the q/k/v
 * columns, written head-major: q, k [B, H, T, dk]; v [B, H, T, dv];
 * a, b [B, H, T] (no conv).  Optional conv caches [B, H d, conv_k - 1] bf16
 * of projected tokens (oldest first): *_in (NULL = zeros) precede t = 0,
 * *_out (NULL = not written, must not alias *_in) receive the last conv_k - 1
 * projected tokens.  D % 64 == 0, conv_k in 1..4.
 * Replaces the three fused_proj_conv_silu launches, the a/b GEMMs and the
 * transposes of GDNLayerCustom.forward (gdn_layer.py:240-252).
 */
int gdn_in_proj_hip(const gdn_bf16_t* xn, const gdn_bf16_t* W_qkvab, const gdn_bf16_t* conv_w_qkv,
                    const gdn_bf16_t* cache_q_in, const gdn_bf16_t* cache_k_in, const gdn_bf16_t* cache_v_in,
                    gdn_bf16_t* cache_q_out, gdn_bf16_t* cache_k_out, gdn_bf16_t* cache_v_out,
                    gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b,
                    int B, int T, int D, int H, int dk, int dv, int conv_k, void* stream);

/*
 * gdn_in_proj_hip for num_seqs packed sequences: xn [T_total, D];
 * cu_seqlens is a HOST int32 array [num_seqs + 1] (0 = cu[0] <= cu[1] <= ...
 * <= cu[num_seqs] = T_total).  Each sequence's causal conv starts from its
 * own cache (cache_*_in [num_seqs, H d, conv_k - 1], NULL = zeros) and
 * cache_*_out [num_seqs, H d, conv_k - 1] (NULL = not written) receives its
 * last conv_k - 1 projected tokens; outputs are packed head-major:
 * q, k [H, T_total, dk]; v [H, T_total, dv]; a, b [H, T_total], as
 * gdn_prefill_varlen_hip reads them.  One launch per non-empty sequence.
 * No reference counterpart (the layer's packed-sequence forward; the
 * reference layer has no cu_seqlens path, gdn_layer.py:222-263).
 */
int gdn_in_proj_varlen_hip(const gdn_bf16_t* xn, const gdn_bf16_t* W_qkvab, const gdn_bf16_t* conv_w_qkv,
                           const int32_t* cu_seqlens, int num_seqs,
                           const gdn_bf16_t* cache_q_in, const gdn_bf16_t* cache_k_in, const gdn_bf16_t* cache_v_in,
                           gdn_bf16_t* cache_q_out, gdn_bf16_t* cache_k_out, gdn_bf16_t* cache_v_out,
                           gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b,
                           int T_total, int D, int H, int dk, int dv, int conv_k, void* stream);

/*
 * Decode-step conv: P [B, 2 H dk + H dv + 2 H] bf16 holds xn W^T of the new
 * token (columns q|k|v|a|b).  q/k/v columns go through the causal conv over
 * the cached previous conv_k - 1 projections (cache_* [B, H d, conv_k - 1],
 * updated in place) and SiLU; a/b pass through.  Outputs in the decode
 * kernel's layouts: q, k [B, H, dk]; v [B, H, dv]; a, b [B, H].  With
 * xn_hist [B, conv_k - 1, D] (nullable) the same launch also moves the x_n
 * history one token older and appends xn [B, D] (the layer's decode-state
 * `xn`).  B <= 65535.
 * Replaces _decode_conv_step / _decode_fused_proj_step (gdn_layer.py:43-69).
 */
int gdn_decode_conv_step_hip(const gdn_bf16_t* P, const gdn_bf16_t* conv_w_qkv,
                             gdn_bf16_t* cache_q, gdn_bf16_t* cache_k, gdn_bf16_t* cache_v,
                             const gdn_bf16_t* xn, gdn_bf16_t* xn_hist,
                             gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b,
                             int B, int D, int H, int dk, int dv, int conv_k, void* stream);

/*
 * One decode step's input side for B <= 16 sequences: x_n = RMSNorm(x)
 * (x [B, D] bf16, gamma [D], eps; the same numbers as gdn_rmsnorm_hip),
 * P = x_n W_qkvab^T kept in fp32, then the conv step of
 * gdn_decode_conv_step_hip on P (conv caches updated in place; they receive
 * bf16(P)) and SiLU.  Outputs q, k [B, H, dk]; v [B, H, dv]; a, b [B, H].
 * xn_hist [B, conv_k - 1, D] (NULL = skipped) is shifted one token and x_n
 * appended, in place.  D % 32 == 0, D <= 4096, conv_k in 1..4.  Caches and
 * xn_hist must not alias the outputs.
 * Replaces GDNLayerCustom.decode's rmsnorm, projection GEMM and conv step
 * (gdn_layer.py:280-299 and 43-69).
 */
int gdn_decode_in_proj_hip(const gdn_bf16_t* x, const gdn_bf16_t* gamma, float eps, const gdn_bf16_t* W_qkvab,
                           const gdn_bf16_t* conv_w_qkv, gdn_bf16_t* cache_q, gdn_bf16_t* cache_k,
                           gdn_bf16_t* cache_v, gdn_bf16_t* xn_hist, gdn_bf16_t* q, gdn_bf16_t* k, gdn_bf16_t* v,
                           gdn_bf16_t* a, gdn_bf16_t* b, int B, int D, int H, int dk, int dv, int conv_k,
                           void* stream);

/*
 * y [B, N] bf16 = bf16(o) W^T for o [B, K] fp32 (the decode kernel's output,
 * rounded to bf16 as the reference's o.to(bf16)), W [N, K] bf16, fp32
 * accumulation.  B <= 16, K % 32 == 0, K <= 4096.
 * Replaces GDNLayerCustom.decode's output projection (gdn_layer.py:309).
 */
int gdn_decode_out_proj_hip(const float* o, const gdn_bf16_t* W, gdn_bf16_t* y, int B, int K, int N,
                            void* stream);

/*
 * One whole decode step of the layer, on `stream`: gdn_decode_in_proj_hip
 * (RMSNorm, projections, conv step, x_n history), gdn_decode_hip (state S,
 * in place when S_out == S_in) and gdn_decode_out_proj_hip, so a serving loop
 * pays one host call per step.  q, k, v, a, b ([B, H dk] x2, [B, H dv],
 * [B, H] x2 bf16) and o ([B, H dv] fp32) are caller-owned scratch; y is
 * [B, D] bf16.  B <= 16: gdn_decode_in_proj_hip, the recurrence and
 * gdn_decode_out_proj_hip, whose constraints and errors apply.
 * 16 < B <= 65535: RMSNorm (x_n written to y, which
 * is then scratch until the out-projection overwrites it, and the x_n
 * history shifted), a tiled in-projection with the conv step in its
 * epilogue, the recurrence, a tiled out-projection; D % 64 == 0, D <= 16384,
 * H dk and H dv multiples of 64, conv_k in 1..4, x/gamma/W/W_o/y/q/k/v/o/
 * caches/xn_hist 16-byte aligned.  Every argument is checked before the first
 * launch, so a refused call leaves the caches and state untouched.
 * Replaces GDNLayerCustom.decode (gdn_layer.py:265-316) as a whole.
 */
int gdn_layer_decode_step_hip(const gdn_bf16_t* x, const gdn_bf16_t* gamma, float eps, const gdn_bf16_t* W_qkvab,
                              const gdn_bf16_t* conv_w_qkv, gdn_bf16_t* cache_q, gdn_bf16_t* cache_k,
                              gdn_bf16_t* cache_v, gdn_bf16_t* xn_hist, const float* A_log, const float* dt_bias,
                              const float* S_in, float* S_out, float scale, const gdn_bf16_t* W_o, gdn_bf16_t* q,
                              gdn_bf16_t* k, gdn_bf16_t* v, gdn_bf16_t* a, gdn_bf16_t* b, float* o, gdn_bf16_t* y,
                              int B, int D, int H, int dk, int dv, int conv_k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_AMD_H */
