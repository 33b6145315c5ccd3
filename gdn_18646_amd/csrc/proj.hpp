// Parameter block of the projection + conv + SiLU kernel (proj.hip), shared
// with the layer-level fused in-projection entry point.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn_proj {

constexpr int kMaxGroups = 5;
constexpr int kPackMax = 256;  // packed sequences per launch of the MFMA kernel

// Columns [col0, col0 + width) of P = x W^T go to dst.  head_dim > 0 writes
// [B, width / head_dim, T, head_dim]; head_dim == 0 writes [B, T, width].
// conv != 0 applies the causal depthwise conv (weights conv_w rows cw_row0 +
// column-in-group) and SiLU; conv == 0 stores the current token's P.
// Conv groups may carry a projected-token cache [B, width, conv_k - 1] (bf16,
// oldest first): cache_in (nullable) supplies P for the tokens before t = 0
// (zeros when null), cache_out (nullable) receives bf16(P) of the last
// conv_k - 1 tokens of the extended sequence cache_in ++ P.
struct ProjGroup {
    int col0;
    int width;
    int head_dim;
    int conv;
    int cw_row0;
    uint16_t* dst;
    const uint16_t* cache_in;
    uint16_t* cache_out;
};

struct ProjParams {
    const uint16_t* x;       // [B, T, D]
    const uint16_t* W;       // [D_out, D]
    const uint16_t* conv_w;  // [rows, conv_k]
    int B, T, D, D_out, conv_k;
    int T_out;    // token stride of the outputs (>= T; 0 = T): a sequence written into a longer packed buffer
    int ngroups;  // groups sorted by col0, groups[0].col0 == 0
    ProjGroup groups[kMaxGroups];
    // Packed sequences (MFMA kernel only): packed > 0 sequences of unequal
    // lengths, x [T_total, D] and outputs [.., T_out, ..] token-packed, caches
    // [packed, width, conv_k - 1].  Sequence i owns rows row_off[i] ..
    // row_off[i + 1] - 1 of the kernel's row space (3 cache rows, then its
    // tokens), so row_off[i] = (token offset of sequence i) + 3 i.  The kernel
    // reads the table from its argument block.
    int packed;
    int32_t row_off[kPackMax + 1];
};

constexpr int kCacheRows = 3;  // rows of the MFMA kernel's row space ahead of each sequence's tokens

// Whether the MFMA kernel takes these parameters (group alignment, sizes).
bool mfma_path_ok(const ProjParams& p);
int launch_proj(const ProjParams& p, hipStream_t stream);

}  // namespace gdn_proj
