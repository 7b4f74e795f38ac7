// lq_route.h -- routing pieces shared with the MoE forward.
#pragma once

#include "lq_common.h"

namespace lq {

constexpr int kMaxExperts = 256;

// Route token t with one wavefront: fp32 softmax over its E logits, top-k by
// rank counting.  Lane l holds experts l, l+64, ... (EPL of them); each
// expert's rank is rank(e) = #{e' : x[e'] > x[e], or x[e'] == x[e] and
// e' < e} over the token's logits (broadcast lane by lane), so
// ids come out in descending-logit order with ties to the lower expert id --
// the order of descending probability, softmax being monotone -- with no
// serial selection rounds.  Experts of rank < k write their id and fp32
// softmax probability (renormalized over the k when renorm) to slot `rank`
// of ids / weights, and the id also to ids_lds when it is not null.
// Restates softmax(logits, -1, dtype=float32).topk(k) of
// trajectory/llada.py:228-234.
template <int LDT, int EPL>
__device__ __forceinline__ void route_token(const void *__restrict__ logits, int64_t t, int E, int k, int renorm,
                                            int32_t *__restrict__ ids, float *__restrict__ weights,
                                            int32_t *ids_lds) {
  const int lane = threadIdx.x & 63;
  float v[EPL];
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? load_f32<LDT>(logits, t * E + e) : -__builtin_inff();
    m = fmaxf(m, v[j]);
  }
  m = wave_max(m);
  float p[EPL];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? expf(v[j] - m) : 0.0f;
    s += p[j];
  }
  s = wave_sum(s);
  int rank[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) rank[j] = 0;
  // every logit is broadcast from its lane (v_readlane: no LDS round trip)
#pragma unroll
  for (int jc = 0; jc < EPL; ++jc) {
#pragma unroll
    for (int l = 0; l < 64; ++l) {
      const int c = 64 * jc + l;
      if (c < E) {
        const float xc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[jc]), l));
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
          const int e = lane + 64 * j;
          rank[j] += (xc > v[j] || (xc == v[j] && c < e)) ? 1 : 0;
        }
      }
    }
  }
  float wsel = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    if (e < E && rank[j] < k) wsel += p[j] / s;
  }
  const float wsum = renorm ? wave_sum(wsel) : 1.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    if (e < E && rank[j] < k) {
      const float pw = p[j] / s;
      ids[t * k + rank[j]] = e;
      weights[t * k + rank[j]] = renorm ? pw / wsum : pw;
      if (ids_lds) ids_lds[t * k + rank[j]] = e;
    }
  }
}

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
