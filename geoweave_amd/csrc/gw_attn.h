// Internal interface between the gather forward (sparse_attn_fwd.hip) and the masked-dense
// forward (sparse_attn_dense.hip).
#pragma once

#include "gw_common.h"

namespace gw {

// The gather forward restricted to the 32-query blocks flagged in blk_flags
// ([B][nqb][nchunk] ints, a block runs when any of its nchunk entries is non-zero) and to
// every block of a batch element b with batch_flags[b] != 0 (batch_flags nullable); every
// other block is left untouched. attn_sum (nullable; workspace as for gw_sparse_attn_fwd)
// and the fused KL loss (logits nullable) as in gw_sparse_attn_fwd_kl.
int attn_fwd_flagged_blocks(int dtype, const void* q, const int64_t* q_strides, const void* k,
                            const int64_t* k_strides, const void* v, const int64_t* v_strides,
                            const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t, void* o,
                            const int64_t* o_strides, float* lse, float* attn_sum, int64_t B, int64_t T, int64_t S,
                            int64_t H, int64_t D, int64_t K, float softmax_scale, const void* logits,
                            int logits_dtype, int64_t logits_stride_b, int64_t logits_stride_t, float eps,
                            float* row_loss, void* workspace, size_t workspace_bytes, const int* blk_flags,
                            const int* batch_flags, int nqb, int nchunk, void* stream);

}  // namespace gw
