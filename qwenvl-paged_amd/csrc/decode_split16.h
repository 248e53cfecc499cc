// Matrix-core split decode for 16-bit caches at head_dim 64 (decode_split16.hip).
#pragma once

#include "decode_common.h"

namespace qvp {

// bf16 or fp16 cache, head_dim 64, GQA group <= 16, a positive scale,
// power-of-two tokens_per_block >= 16, splits a multiple of 32 tokens, and
// 16-byte aligned query, pool and strides: one workgroup per (split, kv head)
// on the bf16 / fp16 matrix cores, in the generic workspace layout (the
// generic split merge finishes). Returns a qvp_status.
bool split16_supported(const DecodeGeometry& g, uint32_t kv_dtype, uint32_t split_tokens, uintptr_t query_addr);
int launch_split16_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t kv_dtype, uint32_t out_dtype,
                          void* out, void* workspace, hipEvent_t split_event, hipStream_t stream);

}  // namespace qvp
