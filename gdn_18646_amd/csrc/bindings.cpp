// Thin torch binding over libgdn_amd.so's C ABI.
//
// Exposes four submodules with the reference's pybind API (names, positional
// argument order, dtypes, return conventions), so a caller written against the
// reference's torch.utils.cpp_extension.load() modules works unchanged:
//   prefill.prefill(q, k, v, A_log, a, dt_bias, b_logits, mask, state_in, scale)
//       -> (out bf16 [B,H,T,V], state_out fp32 [B,H,K,V])
//       + attrs H_DIM K_DIM V_DIM C_DIM     (kernels/prefill_chunked.cu:422-527)
//   decode.forward(q, k, v, a, b, A_log, dt_bias, S_in, scale, o_out, S_out)
//                                           (kernels/decode.cu:172-218)
//   rmsnorm.forward(x, gamma, eps, block_threads, rows_per_block) -> y
//                                           (kernels/rmsnorm.cu:133-153,278-298)
//   proj.forward(input, weight, conv_w) -> out (kernels/fused_proj_conv_silu.cu:298-361)
// Errors surface as RuntimeError, like the reference's TORCH_CHECK.  Launches
// go to torch's current HIP stream of the tensors' device.
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include "../../include/gdn_amd.h"

namespace {

using at::Tensor;

void* stream_of(const Tensor& t) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

#define GDN_CHECK_STATUS(call, who)                                                    \
    do {                                                                                \
        const int _st = (call);                                                         \
        TORCH_CHECK(_st == GDN_OK, who, ": ", gdn_status_string(_st), ": ", gdn_last_error()); \
    } while (0)

void check_gpu(const Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

void check_bf16(const Tensor& t, const char* name) {
    check_gpu(t, name);
    TORCH_CHECK(t.scalar_type() == at::kBFloat16, name, " must be bfloat16");
}

void check_f32(const Tensor& t, const char* name) {
    check_gpu(t, name);
    TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be float32");
}

const gdn_bf16_t* bf(const Tensor& t) { return reinterpret_cast<const gdn_bf16_t*>(t.data_ptr()); }
gdn_bf16_t* bf_mut(const Tensor& t) { return reinterpret_cast<gdn_bf16_t*>(t.data_ptr()); }

// ---------------------------------------------------------------------------
// prefill
// ---------------------------------------------------------------------------
std::tuple<Tensor, Tensor> prefill(Tensor q, Tensor k, Tensor v, Tensor A_log, Tensor a, double dt_bias,
                                   Tensor b_logits, Tensor mask, Tensor state_in, double scale, bool token_major) {
    check_bf16(q, "q");
    check_bf16(k, "k");
    check_bf16(v, "v");
    check_bf16(a, "a");
    check_bf16(b_logits, "b_logits");
    check_f32(A_log, "A_log");
    TORCH_CHECK(q.dim() == 4 && k.sizes() == q.sizes(), "q, k must be [B, H, T, K] of equal shape");
    const int64_t B = q.size(0), H = q.size(1), T = q.size(2), K = q.size(3);
    TORCH_CHECK(v.dim() == 4 && v.size(0) == B && v.size(1) == H && v.size(2) == T, "v must be [B, H, T, V]");
    const int64_t V = v.size(3);
    TORCH_CHECK(a.dim() == 3 && a.size(0) == B && a.size(1) == H && a.size(2) == T, "a must be [B, H, T]");
    TORCH_CHECK(b_logits.sizes() == a.sizes(), "b_logits must be [B, H, T]");
    TORCH_CHECK(A_log.numel() == H, "A_log must have H entries");
    const float* mask_ptr = nullptr;
    if (mask.defined() && mask.numel() > 0) {
        check_f32(mask, "mask");
        TORCH_CHECK(mask.dim() == 2 && mask.size(0) == B && mask.size(1) == T, "mask must be [B, T]");
        mask_ptr = mask.data_ptr<float>();
    }
    const float* sin_ptr = nullptr;
    if (state_in.defined() && state_in.numel() > 0) {
        check_f32(state_in, "state_in");
        TORCH_CHECK(state_in.dim() == 4 && state_in.size(0) == B && state_in.size(1) == H &&
                        state_in.size(2) == K && state_in.size(3) == V,
                    "state_in must be [B, H, K, V] or empty");
        sin_ptr = state_in.data_ptr<float>();
    }
    const c10::DeviceGuard guard(q.device());
    auto out = token_major ? at::empty({B, T, H, V}, q.options()) : at::empty({B, H, T, V}, q.options());
    auto state_out = at::empty({B, H, K, V}, q.options().dtype(at::kFloat));
    const size_t ws_bytes = gdn_prefill_workspace_bytes(B, H, T, K, V);
    auto ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, q.options().dtype(at::kByte));
    auto fn = token_major ? &gdn_prefill_tm_hip : &gdn_prefill_hip;
    GDN_CHECK_STATUS(fn(bf(q), bf(k), bf(v), A_log.data_ptr<float>(), bf(a), static_cast<float>(dt_bias),
                        bf(b_logits), mask_ptr, sin_ptr, static_cast<float>(scale), bf_mut(out),
                        state_out.data_ptr<float>(), B, H, T, K, V, ws.data_ptr(), ws_bytes, stream_of(q)),
                     "prefill");
    return {out, state_out};
}

// Packed variable-length prefill (no reference counterpart).
// q, k [1, H, Ttot, K]; v [1, H, Ttot, V]; a, b_logits [1, H, Ttot];
// cu_seqlens int32/int64 [N+1] on CPU or GPU; state_in [N, H, K, V] or empty.
std::tuple<Tensor, Tensor> prefill_varlen(Tensor q, Tensor k, Tensor v, Tensor A_log, Tensor a, double dt_bias,
                                          Tensor b_logits, Tensor cu_seqlens, Tensor state_in, double scale,
                                          std::optional<Tensor> mask_opt, int64_t max_seqlen, bool token_major) {
    check_bf16(q, "q");
    check_bf16(k, "k");
    check_bf16(v, "v");
    check_bf16(a, "a");
    check_bf16(b_logits, "b_logits");
    check_f32(A_log, "A_log");
    TORCH_CHECK(q.dim() == 4 && q.size(0) == 1 && k.sizes() == q.sizes(), "q, k must be [1, H, T_total, K]");
    const int64_t H = q.size(1), Ttot = q.size(2), K = q.size(3);
    TORCH_CHECK(v.dim() == 4 && v.size(0) == 1 && v.size(1) == H && v.size(2) == Ttot, "v must be [1, H, T_total, V]");
    const int64_t V = v.size(3);
    TORCH_CHECK(a.dim() == 3 && a.size(0) == 1 && a.size(1) == H && a.size(2) == Ttot, "a must be [1, H, T_total]");
    TORCH_CHECK(b_logits.sizes() == a.sizes(), "b_logits must be [1, H, T_total]");
    TORCH_CHECK(A_log.numel() == H, "A_log must have H entries");
    TORCH_CHECK(cu_seqlens.dim() == 1 && cu_seqlens.numel() >= 2, "cu_seqlens must be [N + 1]");
    const int64_t N = cu_seqlens.numel() - 1;
    // Validate offsets on the host: kernels index with them.
    auto cu_host = cu_seqlens.to(at::kCPU).to(at::kLong).contiguous();
    const int64_t* cu = cu_host.data_ptr<int64_t>();
    TORCH_CHECK(cu[0] == 0 && cu[N] == Ttot, "cu_seqlens must start at 0 and end at T_total");
    int64_t maxlen = 0;
    for (int64_t i = 0; i < N; ++i) {
        TORCH_CHECK(cu[i + 1] >= cu[i], "cu_seqlens must be non-decreasing");
        maxlen = std::max(maxlen, cu[i + 1] - cu[i]);
    }
    if (max_seqlen > 0) TORCH_CHECK(max_seqlen >= maxlen, "max_seqlen is smaller than a sequence");
    const float* mask_ptr = nullptr;
    const Tensor mask = mask_opt.has_value() ? *mask_opt : Tensor();
    if (mask.defined() && mask.numel() > 0) {
        check_f32(mask, "mask");
        TORCH_CHECK(mask.numel() == Ttot, "mask must have T_total entries");
        mask_ptr = mask.data_ptr<float>();
    }
    const float* sin_ptr = nullptr;
    if (state_in.defined() && state_in.numel() > 0) {
        check_f32(state_in, "state_in");
        TORCH_CHECK(state_in.dim() == 4 && state_in.size(0) == N && state_in.size(1) == H &&
                        state_in.size(2) == K && state_in.size(3) == V,
                    "state_in must be [N, H, K, V] or empty");
        sin_ptr = state_in.data_ptr<float>();
    }
    const c10::DeviceGuard guard(q.device());
    // Offsets given on the GPU are used in place (validating them above took
    // one read back); offsets given on the host go up through pinned memory
    // without blocking the host on the stream.
    Tensor cu_dev;
    if (cu_seqlens.is_cuda()) {
        TORCH_CHECK(cu_seqlens.device() == q.device(), "cu_seqlens must be on q's device");
        cu_dev = cu_seqlens.to(at::kInt).contiguous();
    } else {
        cu_dev = cu_host.to(at::kInt).pin_memory().to(q.device(), /*non_blocking=*/true);
    }
    auto out = token_major ? at::empty({1, Ttot, H, V}, q.options()) : at::empty({1, H, Ttot, V}, q.options());
    auto state_out = at::empty({N, H, K, V}, q.options().dtype(at::kFloat));
    const size_t ws_bytes = gdn_prefill_varlen_workspace_bytes(N, H, Ttot, K, V);
    auto ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, q.options().dtype(at::kByte));
    auto fn = token_major ? &gdn_prefill_varlen_tm_hip : &gdn_prefill_varlen_hip;
    GDN_CHECK_STATUS(fn(bf(q), bf(k), bf(v), A_log.data_ptr<float>(), bf(a),
                                            static_cast<float>(dt_bias), bf(b_logits), mask_ptr,
                                            cu_dev.data_ptr<int32_t>(), N, static_cast<int>(maxlen), sin_ptr,
                                            static_cast<float>(scale), bf_mut(out), state_out.data_ptr<float>(), H,
                                            Ttot, K, V, ws.data_ptr(), ws_bytes, stream_of(q)),
                     "prefill_varlen");
    return {out, state_out};
}

// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------
void decode_forward(Tensor q, Tensor k, Tensor v, Tensor a, Tensor b, Tensor A_log, Tensor dt_bias, Tensor S_in,
                    double scale, Tensor o_out, Tensor S_out) {
    check_bf16(q, "q");
    check_bf16(k, "k");
    check_bf16(v, "v");
    check_bf16(a, "a");
    check_bf16(b, "b");
    check_f32(A_log, "A_log");
    check_f32(dt_bias, "dt_bias");
    check_f32(S_in, "S_in");
    check_f32(o_out, "o_out");
    check_f32(S_out, "S_out");
    TORCH_CHECK(q.dim() == 3 && k.sizes() == q.sizes(), "q, k must be [B, H, K]");
    const int64_t B = q.size(0), H = q.size(1), K = q.size(2);
    TORCH_CHECK(v.dim() == 3 && v.size(0) == B && v.size(1) == H, "v must be [B, H, V]");
    const int64_t V = v.size(2);
    TORCH_CHECK(a.numel() == B * H && b.numel() == B * H, "a, b must be [B, H]");
    TORCH_CHECK(A_log.numel() == H && dt_bias.numel() == H, "A_log, dt_bias must be [H]");
    TORCH_CHECK(S_in.numel() == B * H * K * V && S_out.numel() == B * H * K * V, "S_in, S_out must be [B, H, K, V]");
    TORCH_CHECK(o_out.numel() == B * H * V, "o_out must be [B, H, V]");
    const c10::DeviceGuard guard(q.device());
    GDN_CHECK_STATUS(gdn_decode_hip(bf(q), bf(k), bf(v), bf(a), bf(b), A_log.data_ptr<float>(),
                                    dt_bias.data_ptr<float>(), S_in.data_ptr<float>(), static_cast<float>(scale),
                                    o_out.data_ptr<float>(), S_out.data_ptr<float>(), B, H, K, V, stream_of(q)),
                     "decode");
}

// ---------------------------------------------------------------------------
// rmsnorm
// ---------------------------------------------------------------------------
Tensor rmsnorm_forward(Tensor x, Tensor gamma, double eps, int64_t block_threads, int64_t rows_per_block) {
    // Launch-shape arguments are validated with the reference's rules
    // (kernels/rmsnorm.cu:140-151); the kernel picks its own shape.
    TORCH_CHECK(rows_per_block >= 1, "rows_per_block must be >= 1");
    TORCH_CHECK(block_threads >= 32, "block_threads must be >= 32");
    TORCH_CHECK(block_threads <= 1024, "block_threads must be <= 1024");
    TORCH_CHECK(block_threads % rows_per_block == 0, "block_threads must be divisible by rows_per_block");
    const int64_t tpr = block_threads / rows_per_block;
    TORCH_CHECK(tpr >= 32, "threads_per_row must be >= 32");
    TORCH_CHECK(tpr % 32 == 0, "threads_per_row must be a multiple of 32");
    check_bf16(x, "x");
    check_bf16(gamma, "gamma");
    TORCH_CHECK(x.dim() == 2, "x must be [R, D]");
    TORCH_CHECK(gamma.dim() == 1 && gamma.size(0) == x.size(1), "gamma must be [D]");
    TORCH_CHECK(x.get_device() == gamma.get_device(), "x and gamma must be on the same device");
    const c10::DeviceGuard guard(x.device());
    auto y = at::empty_like(x);
    GDN_CHECK_STATUS(gdn_rmsnorm_hip(bf(x), bf(gamma), bf_mut(y), x.size(0), x.size(1), static_cast<float>(eps),
                                     stream_of(x)),
                     "rmsnorm");
    return y;
}

// ---------------------------------------------------------------------------
// proj
// ---------------------------------------------------------------------------
Tensor proj_forward(Tensor input, Tensor weight, Tensor conv_w) {
    check_bf16(input, "input");
    check_bf16(weight, "weight");
    check_bf16(conv_w, "conv_w");
    TORCH_CHECK(input.dim() == 3, "input must be [B, T, D]");
    TORCH_CHECK(weight.dim() == 2 && weight.size(1) == input.size(2), "weight dim-1 must equal D");
    TORCH_CHECK(conv_w.dim() == 2 && conv_w.size(0) == weight.size(0), "conv_w dim-0 must equal D_out");
    const int64_t B = input.size(0), T = input.size(1), D = input.size(2), Dout = weight.size(0);
    const c10::DeviceGuard guard(input.device());
    auto out = at::empty({B, T, Dout}, input.options());
    GDN_CHECK_STATUS(gdn_proj_conv_silu_hip(bf(input), bf(weight), bf(conv_w), bf_mut(out), B, T, D, Dout,
                                            conv_w.size(1), stream_of(input)),
                     "proj");
    return out;
}

// ---------------------------------------------------------------------------
// layer helpers (no reference counterpart; used by gdn_layer.GDNLayerCustom)
// ---------------------------------------------------------------------------
const gdn_bf16_t* opt_bf(const std::optional<Tensor>& t, const char* name, int64_t numel) {
    if (!t.has_value() || !t->defined() || t->numel() == 0) return nullptr;
    check_bf16(*t, name);
    TORCH_CHECK(t->numel() == numel, name, " has ", t->numel(), " elements, expected ", numel);
    return bf(*t);
}

// Returns (q, k, v, a, b) head-major, plus new conv caches (q, k, v) when want_cache.
std::vector<Tensor> in_proj(Tensor xn, Tensor W_qkvab, Tensor conv_w_qkv, int64_t H, int64_t dk, int64_t dv,
                            std::optional<Tensor> cache_q, std::optional<Tensor> cache_k,
                            std::optional<Tensor> cache_v, bool want_cache) {
    check_bf16(xn, "xn");
    check_bf16(W_qkvab, "W_qkvab");
    check_bf16(conv_w_qkv, "conv_w_qkv");
    TORCH_CHECK(xn.dim() == 3, "xn must be [B, T, D]");
    const int64_t B = xn.size(0), T = xn.size(1), D = xn.size(2);
    TORCH_CHECK(W_qkvab.dim() == 2 && W_qkvab.size(0) == 2 * H * dk + H * dv + 2 * H && W_qkvab.size(1) == D,
                "W_qkvab must be [2 H dk + H dv + 2 H, D]");
    TORCH_CHECK(conv_w_qkv.dim() == 2 && conv_w_qkv.size(0) == 2 * H * dk + H * dv, "conv_w_qkv must be [2 H dk + H dv, K]");
    const int64_t ck = conv_w_qkv.size(1);
    const c10::DeviceGuard guard(xn.device());
    auto o = xn.options();
    auto q = at::empty({B, H, T, dk}, o), k = at::empty({B, H, T, dk}, o), v = at::empty({B, H, T, dv}, o);
    auto a = at::empty({B, H, T}, o), b = at::empty({B, H, T}, o);
    std::vector<Tensor> res = {q, k, v, a, b};
    gdn_bf16_t *cq = nullptr, *ckk = nullptr, *cv = nullptr;
    if (want_cache) {
        auto nq = at::empty({B, H * dk, ck - 1}, o), nk = at::empty({B, H * dk, ck - 1}, o),
             nv = at::empty({B, H * dv, ck - 1}, o);
        cq = bf_mut(nq);
        ckk = bf_mut(nk);
        cv = bf_mut(nv);
        res.push_back(nq);
        res.push_back(nk);
        res.push_back(nv);
    }
    GDN_CHECK_STATUS(gdn_in_proj_hip(bf(xn), bf(W_qkvab), bf(conv_w_qkv), opt_bf(cache_q, "cache_q", B * H * dk * (ck - 1)),
                                     opt_bf(cache_k, "cache_k", B * H * dk * (ck - 1)),
                                     opt_bf(cache_v, "cache_v", B * H * dv * (ck - 1)), cq, ckk, cv, bf_mut(q),
                                     bf_mut(k), bf_mut(v), bf_mut(a), bf_mut(b), B, T, D, H, dk, dv, ck, stream_of(xn)),
                     "in_proj");
    return res;
}

// Packed sequences: xn [T_total, D] (or [1, T_total, D]) with host offsets
// cu_seqlens [N + 1]; returns q, k [1, H, T_total, dk], v [1, H, T_total, dv],
// a, b [1, H, T_total], plus new conv caches [N, H d, K - 1] when want_cache.
// Caches in (optional): [N, H d, K - 1].
std::vector<Tensor> in_proj_varlen(Tensor xn, Tensor W_qkvab, Tensor conv_w_qkv, int64_t H, int64_t dk, int64_t dv,
                                   Tensor cu_seqlens, std::optional<Tensor> cache_q, std::optional<Tensor> cache_k,
                                   std::optional<Tensor> cache_v, bool want_cache) {
    check_bf16(xn, "xn");
    check_bf16(W_qkvab, "W_qkvab");
    check_bf16(conv_w_qkv, "conv_w_qkv");
    TORCH_CHECK(xn.dim() == 2 || (xn.dim() == 3 && xn.size(0) == 1), "xn must be [T_total, D] or [1, T_total, D]");
    const int64_t Ttot = xn.size(-2), D = xn.size(-1);
    TORCH_CHECK(W_qkvab.dim() == 2 && W_qkvab.size(0) == 2 * H * dk + H * dv + 2 * H && W_qkvab.size(1) == D,
                "W_qkvab must be [2 H dk + H dv + 2 H, D]");
    TORCH_CHECK(conv_w_qkv.dim() == 2 && conv_w_qkv.size(0) == 2 * H * dk + H * dv, "conv_w_qkv must be [2 H dk + H dv, K]");
    TORCH_CHECK(cu_seqlens.dim() == 1 && cu_seqlens.numel() >= 2, "cu_seqlens must be [N + 1]");
    TORCH_CHECK(!cu_seqlens.is_cuda(), "in_proj_varlen takes host offsets (cu_seqlens on the CPU)");
    const int64_t N = cu_seqlens.numel() - 1;
    auto cu = cu_seqlens.to(at::kInt).contiguous();
    const int64_t ck = conv_w_qkv.size(1);
    const c10::DeviceGuard guard(xn.device());
    auto o = xn.options();
    auto q = at::empty({1, H, Ttot, dk}, o), k = at::empty({1, H, Ttot, dk}, o), v = at::empty({1, H, Ttot, dv}, o);
    auto a = at::empty({1, H, Ttot}, o), b = at::empty({1, H, Ttot}, o);
    std::vector<Tensor> res = {q, k, v, a, b};
    gdn_bf16_t *cq = nullptr, *ckk = nullptr, *cv = nullptr;
    if (want_cache) {
        auto nq = at::empty({N, H * dk, ck - 1}, o), nk = at::empty({N, H * dk, ck - 1}, o),
             nv = at::empty({N, H * dv, ck - 1}, o);
        cq = bf_mut(nq);
        ckk = bf_mut(nk);
        cv = bf_mut(nv);
        res.push_back(nq);
        res.push_back(nk);
        res.push_back(nv);
    }
    GDN_CHECK_STATUS(gdn_in_proj_varlen_hip(bf(xn), bf(W_qkvab), bf(conv_w_qkv), cu.data_ptr<int32_t>(), N,
                                            opt_bf(cache_q, "cache_q", N * H * dk * (ck - 1)),
                                            opt_bf(cache_k, "cache_k", N * H * dk * (ck - 1)),
                                            opt_bf(cache_v, "cache_v", N * H * dv * (ck - 1)), cq, ckk, cv, bf_mut(q),
                                            bf_mut(k), bf_mut(v), bf_mut(a), bf_mut(b), Ttot, D, H, dk, dv, ck,
                                            stream_of(xn)),
                     "in_proj_varlen");
    return res;
}

// Decode conv step on P = xn W^T of one token; caches updated in place, and,
// with xn and xn_hist [B, K - 1, D], the x_n history shifted in place.
std::vector<Tensor> decode_conv_step(Tensor P, Tensor conv_w_qkv, Tensor cache_q, Tensor cache_k, Tensor cache_v,
                                     int64_t H, int64_t dk, int64_t dv, std::optional<Tensor> xn,
                                     std::optional<Tensor> xn_hist) {
    check_bf16(P, "P");
    check_bf16(conv_w_qkv, "conv_w_qkv");
    const int64_t B = P.size(0);
    TORCH_CHECK(P.dim() == 2 && P.size(1) == 2 * H * dk + H * dv + 2 * H, "P must be [B, 2 H dk + H dv + 2 H]");
    const int64_t ck = conv_w_qkv.size(1);
    TORCH_CHECK(conv_w_qkv.dim() == 2 && conv_w_qkv.size(0) == 2 * H * dk + H * dv, "conv_w_qkv must be [2 H dk + H dv, K]");
    check_bf16(cache_q, "cache_q");
    check_bf16(cache_k, "cache_k");
    check_bf16(cache_v, "cache_v");
    TORCH_CHECK(cache_q.numel() == B * H * dk * (ck - 1) && cache_k.numel() == B * H * dk * (ck - 1) &&
                    cache_v.numel() == B * H * dv * (ck - 1),
                "conv caches must be [B, H d, K - 1]");
    const gdn_bf16_t* xn_ptr = nullptr;
    gdn_bf16_t* hist = nullptr;
    int64_t D = 0;
    if (xn_hist.has_value() && xn_hist->defined() && xn_hist->numel() > 0) {
        TORCH_CHECK(xn.has_value() && xn->defined(), "xn_hist needs xn");
        check_bf16(*xn, "xn");
        check_bf16(*xn_hist, "xn_hist");
        D = xn->size(-1);
        TORCH_CHECK(xn->numel() == B * D, "xn must be [B, D]");
        TORCH_CHECK(xn_hist->numel() == B * (ck - 1) * D, "xn_hist must be [B, K - 1, D]");
        xn_ptr = bf(*xn);
        hist = bf_mut(*xn_hist);
    }
    const c10::DeviceGuard guard(P.device());
    auto o = P.options();
    auto q = at::empty({B, H, dk}, o), k = at::empty({B, H, dk}, o), v = at::empty({B, H, dv}, o);
    auto a = at::empty({B, H}, o), b = at::empty({B, H}, o);
    GDN_CHECK_STATUS(gdn_decode_conv_step_hip(bf(P), bf(conv_w_qkv), bf_mut(cache_q), bf_mut(cache_k), bf_mut(cache_v),
                                              xn_ptr, hist, bf_mut(q), bf_mut(k), bf_mut(v), bf_mut(a), bf_mut(b), B, D,
                                              H, dk, dv, ck, stream_of(P)),
                     "decode_conv_step");
    return {q, k, v, a, b};
}

// Decode step, B <= 16: RMSNorm + projection + conv step + SiLU in one launch.
// x [B, D]; caches and xn_hist (optional, [B, K - 1, D]) updated in place.
std::vector<Tensor> decode_in_proj(Tensor x, Tensor gamma, double eps, Tensor W_qkvab, Tensor conv_w_qkv,
                                   Tensor cache_q, Tensor cache_k, Tensor cache_v, std::optional<Tensor> xn_hist,
                                   int64_t H, int64_t dk, int64_t dv) {
    check_bf16(x, "x");
    check_bf16(gamma, "gamma");
    check_bf16(W_qkvab, "W_qkvab");
    check_bf16(conv_w_qkv, "conv_w_qkv");
    TORCH_CHECK(x.dim() == 2, "x must be [B, D]");
    const int64_t B = x.size(0), D = x.size(1);
    TORCH_CHECK(gamma.numel() == D, "gamma must have D entries");
    TORCH_CHECK(W_qkvab.dim() == 2 && W_qkvab.size(0) == 2 * H * dk + H * dv + 2 * H && W_qkvab.size(1) == D,
                "W_qkvab must be [2 H dk + H dv + 2 H, D]");
    TORCH_CHECK(conv_w_qkv.dim() == 2 && conv_w_qkv.size(0) == 2 * H * dk + H * dv, "conv_w_qkv must be [2 H dk + H dv, K]");
    const int64_t ck = conv_w_qkv.size(1);
    check_bf16(cache_q, "cache_q");
    check_bf16(cache_k, "cache_k");
    check_bf16(cache_v, "cache_v");
    TORCH_CHECK(cache_q.numel() == B * H * dk * (ck - 1) && cache_k.numel() == B * H * dk * (ck - 1) &&
                    cache_v.numel() == B * H * dv * (ck - 1),
                "conv caches must be [B, H d, K - 1]");
    gdn_bf16_t* hist = nullptr;
    if (xn_hist.has_value() && xn_hist->defined() && xn_hist->numel() > 0) {
        check_bf16(*xn_hist, "xn_hist");
        TORCH_CHECK(xn_hist->numel() == B * (ck - 1) * D, "xn_hist must be [B, K - 1, D]");
        hist = bf_mut(*xn_hist);
    }
    const c10::DeviceGuard guard(x.device());
    auto o = x.options();
    auto q = at::empty({B, H, dk}, o), k = at::empty({B, H, dk}, o), v = at::empty({B, H, dv}, o);
    auto a = at::empty({B, H}, o), b = at::empty({B, H}, o);
    GDN_CHECK_STATUS(gdn_decode_in_proj_hip(bf(x), bf(gamma), static_cast<float>(eps), bf(W_qkvab), bf(conv_w_qkv),
                                            bf_mut(cache_q), bf_mut(cache_k), bf_mut(cache_v), hist, bf_mut(q),
                                            bf_mut(k), bf_mut(v), bf_mut(a), bf_mut(b), B, D, H, dk, dv, ck,
                                            stream_of(x)),
                     "decode_in_proj");
    return {q, k, v, a, b};
}

// Decode step output projection: o [B, K] fp32 -> bf16(o) W^T [B, N] bf16.
Tensor decode_out_proj(Tensor o, Tensor W) {
    check_f32(o, "o");
    check_bf16(W, "W");
    TORCH_CHECK(o.dim() == 2 && W.dim() == 2 && W.size(1) == o.size(1), "o must be [B, K] and W [N, K]");
    const int64_t B = o.size(0), K = o.size(1), N = W.size(0);
    const c10::DeviceGuard guard(o.device());
    auto y = at::empty({B, N}, o.options().dtype(at::kBFloat16));
    GDN_CHECK_STATUS(gdn_decode_out_proj_hip(o.data_ptr<float>(), bf(W), bf_mut(y), B, K, N, stream_of(o)),
                     "decode_out_proj");
    return y;
}

// One whole decode step (in place on the caches, the x_n history and S):
// x [B, D] -> y [B, D] bf16; q..o are caller-owned scratch.
void decode_step(Tensor x, Tensor gamma, double eps, Tensor W_qkvab, Tensor conv_w_qkv, Tensor cache_q,
                 Tensor cache_k, Tensor cache_v, std::optional<Tensor> xn_hist, Tensor A_log, Tensor dt_bias,
                 Tensor S_in, Tensor S_out, double scale, Tensor W_o, Tensor q, Tensor k, Tensor v, Tensor a, Tensor b,
                 Tensor o, Tensor y, int64_t H, int64_t dk, int64_t dv) {
    for (const Tensor* t : {&x, &gamma, &W_qkvab, &conv_w_qkv, &cache_q, &cache_k, &cache_v, &W_o, &q, &k, &v, &a, &b, &y})
        check_bf16(*t, "decode_step bf16 argument");
    for (const Tensor* t : {&A_log, &dt_bias, &S_in, &S_out, &o}) check_f32(*t, "decode_step fp32 argument");
    TORCH_CHECK(x.dim() == 2, "x must be [B, D]");
    const int64_t B = x.size(0), D = x.size(1);
    const int64_t ck = conv_w_qkv.size(1);
    TORCH_CHECK(W_qkvab.dim() == 2 && W_qkvab.size(0) == 2 * H * dk + H * dv + 2 * H && W_qkvab.size(1) == D,
                "W_qkvab must be [2 H dk + H dv + 2 H, D]");
    TORCH_CHECK(conv_w_qkv.dim() == 2 && conv_w_qkv.size(0) == 2 * H * dk + H * dv, "conv_w_qkv must be [2 H dk + H dv, K]");
    TORCH_CHECK(gamma.numel() == D, "gamma must have D entries");
    TORCH_CHECK(cache_q.numel() == B * H * dk * (ck - 1) && cache_k.numel() == B * H * dk * (ck - 1) &&
                    cache_v.numel() == B * H * dv * (ck - 1),
                "conv caches must be [B, H d, K - 1]");
    TORCH_CHECK(A_log.numel() == H && dt_bias.numel() == H, "A_log, dt_bias must be [H]");
    TORCH_CHECK(S_in.numel() == B * H * dk * dv && S_out.numel() == B * H * dk * dv, "S must be [B, H, dk, dv]");
    TORCH_CHECK(W_o.dim() == 2 && W_o.size(0) == D && W_o.size(1) == H * dv, "W_o must be [D, H dv]");
    TORCH_CHECK(q.numel() == B * H * dk && k.numel() == B * H * dk && v.numel() == B * H * dv && a.numel() == B * H &&
                    b.numel() == B * H && o.numel() == B * H * dv && y.numel() == B * D,
                "scratch q, k [B, H dk], v [B, H dv], a, b [B, H], o [B, H dv] fp32, y [B, D]");
    gdn_bf16_t* hist = nullptr;
    if (xn_hist.has_value() && xn_hist->defined() && xn_hist->numel() > 0) {
        check_bf16(*xn_hist, "xn_hist");
        TORCH_CHECK(xn_hist->numel() == B * (ck - 1) * D, "xn_hist must be [B, K - 1, D]");
        hist = bf_mut(*xn_hist);
    }
    const c10::DeviceGuard guard(x.device());
    GDN_CHECK_STATUS(gdn_layer_decode_step_hip(bf(x), bf(gamma), static_cast<float>(eps), bf(W_qkvab), bf(conv_w_qkv),
                                               bf_mut(cache_q), bf_mut(cache_k), bf_mut(cache_v), hist,
                                               A_log.data_ptr<float>(), dt_bias.data_ptr<float>(),
                                               S_in.data_ptr<float>(), S_out.data_ptr<float>(),
                                               static_cast<float>(scale), bf(W_o), bf_mut(q), bf_mut(k), bf_mut(v),
                                               bf_mut(a), bf_mut(b), o.data_ptr<float>(), bf_mut(y), B, D, H, dk, dv,
                                               ck, stream_of(x)),
                     "decode_step");
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "MI355X (gfx950) Gated DeltaNet kernels: torch binding over libgdn_amd.so";
    m.attr("ABI_VERSION") = gdn_abi_version();

    auto mp = m.def_submodule("prefill", "GDN chunked prefill (chunk 64)");
    mp.def("prefill", &prefill,
           "Args: q,k [B,H,T,K] bf16 | v [B,H,T,V] bf16 | A_log [H] fp32 | a,b_logits [B,H,T] bf16 | "
           "dt_bias float | mask [B,T] fp32 (empty = ones) | state_in [B,H,K,V] fp32 (empty = zeros) | "
           "scale float (0 = K^-0.5) | token_major (keyword, default False)\n"
           "Returns: (out [B,H,T,V] bf16, or [B,T,H,V] with token_major, state_out [B,H,K,V] fp32)",
           py::arg("q"), py::arg("k"), py::arg("v"), py::arg("A_log"), py::arg("a"), py::arg("dt_bias"),
           py::arg("b_logits"), py::arg("mask"), py::arg("state_in"), py::arg("scale"), py::kw_only(),
           py::arg("token_major") = false);
    mp.def("prefill_varlen", &prefill_varlen,
           "Packed varlen prefill: q,k [1,H,Ttot,K] | v [1,H,Ttot,V] | a,b_logits [1,H,Ttot] | cu_seqlens [N+1] | "
           "state_in [N,H,K,V] or empty.  Returns (out [1,H,Ttot,V] bf16, or [1,Ttot,H,V] with token_major, "
           "state_out [N,H,K,V] fp32)",
           py::arg("q"), py::arg("k"), py::arg("v"), py::arg("A_log"), py::arg("a"), py::arg("dt_bias"),
           py::arg("b_logits"), py::arg("cu_seqlens"), py::arg("state_in"), py::arg("scale"),
           py::arg("mask") = py::none(), py::arg("max_seqlen") = 0, py::arg("token_major") = false);
    // Reference attribute values; H and V are runtime parameters here (any H,
    // V % 16 == 0), K is 128 and the chunk is 64 as in the reference.
    mp.attr("H_DIM") = 16;
    mp.attr("K_DIM") = 128;
    mp.attr("V_DIM") = 256;
    mp.attr("C_DIM") = 64;

    auto md = m.def_submodule("decode", "GDN decode step");
    md.def("forward", &decode_forward, "GDN decode forward (S_out may alias S_in)", py::arg("q"), py::arg("k"),
           py::arg("v"), py::arg("a"), py::arg("b"), py::arg("A_log"), py::arg("dt_bias"), py::arg("S_in"),
           py::arg("scale"), py::arg("o_out"), py::arg("S_out"));

    auto mr = m.def_submodule("rmsnorm", "RMSNorm (bf16)");
    mr.def("forward", &rmsnorm_forward, "RMSNorm forward (bf16, any D % 8 == 0)", py::arg("x"), py::arg("gamma"),
           py::arg("eps"), py::arg("block_threads"), py::arg("rows_per_block"));

    auto ml = m.def_submodule("layer", "Layer-level fused projection and decode conv step");
    ml.def("in_proj", &in_proj, "Fused q/k/v/a/b projection + conv + SiLU, head-major outputs (+ conv caches)",
           py::arg("xn"), py::arg("W_qkvab"), py::arg("conv_w_qkv"), py::arg("H"), py::arg("dk"), py::arg("dv"),
           py::arg("cache_q") = py::none(), py::arg("cache_k") = py::none(), py::arg("cache_v") = py::none(),
           py::arg("want_cache") = false);
    ml.def("in_proj_varlen", &in_proj_varlen,
           "in_proj for packed sequences (host cu_seqlens): each sequence's conv starts from its own cache",
           py::arg("xn"), py::arg("W_qkvab"), py::arg("conv_w_qkv"), py::arg("H"), py::arg("dk"), py::arg("dv"),
           py::arg("cu_seqlens"), py::arg("cache_q") = py::none(), py::arg("cache_k") = py::none(),
           py::arg("cache_v") = py::none(), py::arg("want_cache") = false);
    ml.def("decode_conv_step", &decode_conv_step,
           "Decode conv step with projected-token caches (in place); with xn and xn_hist also shifts the x_n history",
           py::arg("P"), py::arg("conv_w_qkv"), py::arg("cache_q"), py::arg("cache_k"), py::arg("cache_v"),
           py::arg("H"), py::arg("dk"), py::arg("dv"), py::arg("xn") = py::none(), py::arg("xn_hist") = py::none());
    ml.def("decode_in_proj", &decode_in_proj,
           "Decode step (B <= 16): RMSNorm + q/k/v/a/b projection + conv step + SiLU; caches and xn_hist in place",
           py::arg("x"), py::arg("gamma"), py::arg("eps"), py::arg("W_qkvab"), py::arg("conv_w_qkv"),
           py::arg("cache_q"), py::arg("cache_k"), py::arg("cache_v"), py::arg("xn_hist") = py::none(),
           py::arg("H"), py::arg("dk"), py::arg("dv"));
    ml.def("decode_out_proj", &decode_out_proj, "Decode step output projection (B <= 16): bf16(o) W^T",
           py::arg("o"), py::arg("W"));
    ml.def("decode_step", &decode_step,
           "Whole decode step (B <= 16: skinny projections; larger B: tiled projections): in-projection, "
           "recurrence, out-projection in one call; caches, xn_hist and S_out updated in place, y written; q, k, v, a, b, "
           "o are scratch",
           py::arg("x"), py::arg("gamma"), py::arg("eps"), py::arg("W_qkvab"), py::arg("conv_w_qkv"),
           py::arg("cache_q"), py::arg("cache_k"), py::arg("cache_v"), py::arg("xn_hist"), py::arg("A_log"),
           py::arg("dt_bias"), py::arg("S_in"), py::arg("S_out"), py::arg("scale"), py::arg("W_o"), py::arg("q"),
           py::arg("k"), py::arg("v"), py::arg("a"), py::arg("b"), py::arg("o"), py::arg("y"), py::arg("H"),
           py::arg("dk"), py::arg("dv"));

    auto mj = m.def_submodule("proj", "Projection + causal conv + SiLU");
    mj.def("forward", &proj_forward, "Fused linear projection + causal depthwise conv1d + SiLU (bf16)",
           py::arg("input"), py::arg("weight"), py::arg("conv_w"));
}
