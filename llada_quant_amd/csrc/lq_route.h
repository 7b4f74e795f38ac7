// lq_route.h -- routing pieces shared with the MoE forward.
#pragma once

#include "lq_common.h"

namespace lq {

constexpr int kMaxExperts = 256;

// Stable expert permutation (the plan kernel of lq_moe.hip without its work
// list).  Assignments whose id lies outside [0, E) are not routed.
int launch_permute(const int32_t *ids, int64_t N, int E, int32_t *counts, int32_t *offsets, int32_t *sorted,
                   hipStream_t st);

// Top-k softmax router launch (validates its arguments).  With xperm !=
// nullptr it also writes x [T, H] (H % 8 == 0) into xperm in the MoE
// kernel's K-slot order (permute_kslots).
int launch_route_topk(const void *logits, int logits_dtype, int64_t T, int E, int k, int renormalize,
                      int32_t *topk_ids, float *topk_weights, hipStream_t st, const uint16_t *x = nullptr,
                      int H = 0, uint16_t *xperm = nullptr);

}  // namespace lq
