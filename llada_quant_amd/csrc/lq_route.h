// lq_route.h -- routing pieces shared with the MoE forward.
#pragma once

#include "lq_common.h"

namespace lq {

constexpr int kMaxExperts = 256;

// Routing of one token over E <= 64 experts with one wavefront (lane e holds
// expert e's logit v; lanes past E hold -inf): fp32 softmax as route_values
// below.  The top-k set comes from a radix select on orderable 32-bit keys
// of the logits (-0.0 keyed as +0.0, so equal logits have equal keys; lanes
// past E key 0, below every logit): 32 ballots of key >= c build the k-th
// largest key from the top bit down, and the set is every key above it plus
// the lowest-numbered lanes equal to it.  Each selected lane's rank is then
// counted against the k selected ones only: (greater key) or (equal key and
// lower expert id).  The ids, their order and the weights are those of the
// rank count in route_values.
template <class Put>
__device__ __forceinline__ void route_values64(float v, int E, int k, int renorm, Put put) {
  const int lane = threadIdx.x & 63;
  const float m = wave_max(v);
  const float p = lane < E ? expf(v - m) : 0.0f;
  const float s = wave_sum(p);
  const uint32_t u = __builtin_bit_cast(uint32_t, v == 0.0f ? 0.0f : v);
  const uint32_t key = lane < E ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
  uint32_t thr = 0;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = thr | (1u << b);
    thr = __popcll(__ballot(key >= c)) >= k ? c : thr;
  }
  const uint64_t gt = __ballot(key > thr);
  uint64_t eq = __ballot(key == thr);
  uint64_t sel = gt;
  for (int need = k - __popcll(gt); need > 0; --need) {
    const uint64_t low = eq & (~eq + 1);
    sel |= low;
    eq ^= low;
  }
  int rank = 0;
  for (uint64_t rem = sel; rem; rem &= rem - 1) {
    const int c = __builtin_ctzll(rem);
    const uint32_t kc = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), c));
    rank += static_cast<int>(kc > key) + (static_cast<int>(kc == key) & static_cast<int>(c < lane));
  }
  const bool mine = (sel >> lane) & 1;
  const float pw = p / s;
  const float wsum = renorm ? wave_sum(mine ? pw : 0.0f) : 1.0f;
  if (mine) put(rank, lane, renorm ? pw / wsum : pw);
}

// Route one token with one wavefront from its logits v (lane l holds experts
// l, l+64, ...: EPL of them; lanes past E hold -inf): fp32 softmax over the
// E logits, top-k by rank counting.  Each expert's rank is rank(e) =
// #{e' : x[e'] > x[e], or x[e'] == x[e] and e' < e} over the token's logits
// (broadcast lane by lane), so ids come out in descending-logit order with
// ties to the lower expert id -- the order of descending probability,
// softmax being monotone -- with no serial selection rounds.  Experts of
// rank < k call put(rank, e, p) with their fp32 softmax probability p
// (renormalized over the k when renorm).  Restates
// softmax(logits, -1, dtype=float32).topk(k) of trajectory/llada.py:228-234.
// One logit per lane (EPL == 1) takes route_values64.
template <int EPL, class Put>
__device__ __forceinline__ void route_values(const float (&v)[EPL], int E, int k, int renorm, Put put) {
  if constexpr (EPL == 1) {
    route_values64(v[0], E, k, renorm, put);
    return;
  }
  const int lane = threadIdx.x & 63;
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; ++j) m = fmaxf(m, v[j]);
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
  // every logit is broadcast from its lane (v_readlane: no LDS round trip).
  // No test of c < E: a lane past E holds -inf, which is greater than no
  // logit, and equal ones count only for a lower index, which c >= E is
  // not for any e < E.  The terms are combined without short-circuiting so
  // the loop stays straight-line.
#pragma unroll
  for (int jc = 0; jc < EPL; ++jc) {
#pragma unroll
    for (int l = 0; l < 64; ++l) {
      const int c = 64 * jc + l;
      const float xc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[jc]), l));
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        rank[j] += static_cast<int>(xc > v[j]) + (static_cast<int>(xc == v[j]) & static_cast<int>(c < e));
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
      put(rank[j], e, renorm ? pw / wsum : pw);
    }
  }
}

// Token t's logits of [T, E] (dtype LDT) in the lane layout of route_values
// (lane l holds experts l, l+64, ...; -inf past E).
template <int LDT, int EPL>
__device__ __forceinline__ void route_logits(const void *__restrict__ logits, int64_t t, int E, float (&v)[EPL]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? load_f32<LDT>(logits, t * E + e) : -__builtin_inff();
  }
}

// Route token t from its logits v (route_logits) with one wavefront: writes
// its k ids and weights to slots t*k .. t*k + k-1 of ids / weights, and the
// ids also to ids_lds when it is not null (route_values).
template <int EPL>
__device__ __forceinline__ void route_store(const float (&v)[EPL], int64_t t, int E, int k, int renorm,
                                            int32_t *__restrict__ ids, float *__restrict__ weights,
                                            int32_t *ids_lds) {
  route_values<EPL>(v, E, k, renorm, [&](int rank, int e, float w) __attribute__((always_inline)) {
    ids[t * k + rank] = e;
    weights[t * k + rank] = w;
    if (ids_lds) ids_lds[t * k + rank] = e;
  });
}

// route_logits then route_store
template <int LDT, int EPL>
__device__ __forceinline__ void route_token(const void *__restrict__ logits, int64_t t, int E, int k, int renorm,
                                            int32_t *__restrict__ ids, float *__restrict__ weights,
                                            int32_t *ids_lds) {
  float v[EPL];
  route_logits<LDT, EPL>(logits, t, E, v);
  route_store<EPL>(v, t, E, k, renorm, ids, weights, ids_lds);
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
