// lq_route.h -- routing pieces shared with the MoE forward.
#pragma once

#include "lq_common.h"

namespace lq {

constexpr int kMaxExperts = 256;

// Stable expert permutation (see lq_route.hip); unit_rows > 0 also emits the
// (expert, first sorted position, rows) work units and their count.
// Assignments whose id lies outside [0, E) are not routed.
int launch_permute(const int32_t *ids, int64_t N, int E, int32_t *counts, int32_t *offsets, int32_t *sorted,
                   int unit_rows, int32_t *units, int32_t *n_units, hipStream_t st);

// Top-k softmax router launch (validates its arguments).
int launch_route_topk(const void *logits, int logits_dtype, int64_t T, int E, int k, int renormalize,
                      int32_t *topk_ids, float *topk_weights, hipStream_t st);

}  // namespace lq
