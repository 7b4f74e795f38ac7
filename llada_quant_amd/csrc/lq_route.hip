// lq_route.hip -- routing front end for gfx950: top-k softmax router and the
// stable expert permutation of the T*k assignments.
//
// Routing restates TritonFusedMoEBlock.forward as trajectory/llada.py:228-234
// records it: softmax(logits, dim=-1, dtype=float32).topk(k).indices.
// The permutation orders assignments by expert and, within an expert, by
// flat index t*k + j -- the bit-identical order of moe_align_block_size
// (INFERENCE_REPO_CHANGES.md:274-278).
#include "lq_common.h"
#include "lq_route.h"

namespace lq {
namespace {

constexpr int kRouteBlock = 256;  // 4 tokens per block, one wave each

// One wavefront per token; lane l holds experts l, l+64, ... (EPL of them).
// ids are chosen by descending logit with ties to the lower expert id (the
// order of descending probability: softmax is monotone).  Weights are the
// fp32 softmax probabilities of the chosen experts.
template <int LDT, int EPL>
__global__ __launch_bounds__(kRouteBlock) void route_topk_kernel(const void *__restrict__ logits, int64_t T,
                                                                 int E, int k, int renorm,
                                                                 int32_t *__restrict__ ids,
                                                                 float *__restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (t >= T) return;  // uniform per wave
  float x[EPL];
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    x[j] = e < E ? load_f32<LDT>(logits, t * E + e) : -__builtin_inff();
    m = fmaxf(m, x[j]);
  }
  m = wave_max(m);
  float p[EPL];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? expf(x[j] - m) : 0.0f;
    s += p[j];
  }
  s = wave_sum(s);
#pragma unroll
  for (int j = 0; j < EPL; ++j) p[j] = p[j] / s;

  uint32_t taken = 0;  // bit j: slot j of this lane already chosen
  float wsum = 0.0f;
  for (int r = 0; r < k; ++r) {
    float bv = -__builtin_inff();
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !((taken >> j) & 1u) && (x[j] > bv || (x[j] == bv && e < bi))) {
        bv = x[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    // every lane now holds the winner bi; its owner marks it taken
    float pw = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      if (lane + 64 * j == bi) {
        taken |= 1u << j;
        pw = p[j];
      }
    }
    pw = __shfl(pw, bi & 63, 64);
    wsum += pw;
    if (lane == 0) {
      ids[t * k + r] = bi;
      weights[t * k + r] = pw;
    }
  }
  if (renorm && lane == 0) {
    for (int r = 0; r < k; ++r) weights[t * k + r] = weights[t * k + r] / wsum;
  }
}

// weights[t, j] = probs[t, ids[t, j]], ids copied out as int32
template <typename IdT>
__global__ void gather_weights_kernel(const float *__restrict__ probs, const IdT *__restrict__ ids, int64_t T, int E,
                                      int k, int renorm, int32_t *__restrict__ ids32, float *__restrict__ weights) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= T) return;
  float s = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int64_t e = static_cast<int64_t>(ids[t * k + j]);
    const float v = (e >= 0 && e < E) ? probs[t * E + e] : 0.0f;
    ids32[t * k + j] = static_cast<int32_t>(e);
    weights[t * k + j] = v;
    s += v;
  }
  if (renorm)
    for (int j = 0; j < k; ++j) weights[t * k + j] = weights[t * k + j] / s;
}

constexpr int kPermBlock = 1024;
constexpr int kPermWaves = kPermBlock / 64;

// exclusive scan of v over the E (<= kMaxExperts) entries, by wave 0; lane l
// owns entries 4l..4l+3.  Returns the total through *total.
__device__ void wave0_exclusive_scan(const int *in, int *out, int E, int *total) {
  const int lane = threadIdx.x & 63;
  int v[4];
  int local = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * lane + i;
    v[i] = e < E ? in[e] : 0;
    local += v[i];
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  int run = incl - local;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * lane + i;
    if (e < E) out[e] = run;
    run += v[i];
  }
  const int tot = __shfl(incl, 63, 64);
  if (lane == 0) *total = tot;
}

// Single-block stable counting sort of the N = T*k assignments.
// Optionally (unit_rows > 0) also emits the GEMM work units: each expert's
// sorted run split into chunks of unit_rows rows, as (expert, first sorted
// position, rows) triples, expert-major; n_units receives their count.
__global__ __launch_bounds__(kPermBlock) void permute_kernel(const int32_t *__restrict__ ids, int64_t N, int E,
                                                             int32_t *__restrict__ counts,
                                                             int32_t *__restrict__ offsets,
                                                             int32_t *__restrict__ sorted, int unit_rows,
                                                             int32_t *__restrict__ units,
                                                             int32_t *__restrict__ n_units) {
  __shared__ int hist[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int ustart[kMaxExperts];
  __shared__ int wcnt[kPermWaves][kMaxExperts];
  __shared__ int total;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  for (int e = tid; e < kMaxExperts; e += kPermBlock) hist[e] = 0;
  for (int i = tid; i < kPermWaves * kMaxExperts; i += kPermBlock) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  for (int64_t a = tid; a < N; a += kPermBlock) {
    const int id = ids[a];
    if (id >= 0 && id < E) atomicAdd(&hist[id], 1);
  }
  __syncthreads();
  if (wave == 0) wave0_exclusive_scan(hist, base, E, &total);
  __syncthreads();
  for (int e = tid; e < E; e += kPermBlock) {
    counts[e] = hist[e];
    offsets[e] = base[e];
  }
  if (tid == 0) offsets[E] = total;
  if (unit_rows > 0) {
    // per-expert unit counts, then their exclusive scan
    __syncthreads();
    for (int e = tid; e < E; e += kPermBlock) wcnt[0][e] = (hist[e] + unit_rows - 1) / unit_rows;
    __syncthreads();
    if (wave == 0) wave0_exclusive_scan(wcnt[0], ustart, E, n_units);
    __syncthreads();
    for (int e = tid; e < E; e += kPermBlock) {
      const int nu = wcnt[0][e];
      for (int u = 0; u < nu; ++u) {
        const int row0 = base[e] + u * unit_rows;
        const int rows = min(unit_rows, hist[e] - u * unit_rows);
        int32_t *dst = units + 3 * (ustart[e] + u);
        dst[0] = e;
        dst[1] = row0;
        dst[2] = rows;
      }
    }
    __syncthreads();
    for (int e = tid; e < E; e += kPermBlock) wcnt[0][e] = 0;
  }
  __syncthreads();

  // key bits: experts are < E <= 256, invalid lanes use key E
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t chunk = 0; chunk < N; chunk += kPermBlock) {
    const int64_t a = chunk + tid;
    const int raw = a < N ? ids[a] : -1;
    const bool valid = raw >= 0 && raw < E;
    const int key = valid ? raw : E;
    unsigned long long peers = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1;
      const unsigned long long bal = __ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    const int rank = __popcll(peers & lt_mask);
    if (valid && rank == 0) wcnt[wave][key] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pos = base[key] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][key];
      sorted[pos] = static_cast<int32_t>(a);
    }
    __syncthreads();
    for (int e = tid; e < E; e += kPermBlock) {
      int s = 0;
      for (int w = 0; w < kPermWaves; ++w) {
        s += wcnt[w][e];
        wcnt[w][e] = 0;
      }
      base[e] += s;
    }
    __syncthreads();
  }
}

}  // namespace

int launch_permute(const int32_t *ids, int64_t N, int E, int32_t *counts, int32_t *offsets, int32_t *sorted,
                   int unit_rows, int32_t *units, int32_t *n_units, hipStream_t st) {
  permute_kernel<<<1, kPermBlock, 0, st>>>(ids, N, E, counts, offsets, sorted, unit_rows, units, n_units);
  return check_launch("moe_permute");
}

}  // namespace lq

using namespace lq;

namespace lq {
int launch_route_topk(const void *logits, int logits_dtype, int64_t T, int E, int k, int renormalize,
                      int32_t *topk_ids, float *topk_weights, hipStream_t st) {
  if (logits_dtype != LQ_F32 && logits_dtype != LQ_BF16 && logits_dtype != LQ_F16)
    return fail(LQ_ERR_VALUE, "route_topk: logits must be float32, float16 or bfloat16");
  if (E < 1 || E > kMaxExperts)
    return fail(LQ_ERR_UNSUPPORTED, "route_topk: 1 <= num_experts <= " + std::to_string(kMaxExperts));
  if (k < 1 || k > E) return fail(LQ_ERR_VALUE, "route_topk: need 1 <= k <= num_experts");
  if (T < 0) return fail(LQ_ERR_VALUE, "route_topk: negative token count");
  if (T == 0) return LQ_OK;
  if (!logits || !topk_ids || !topk_weights) return fail(LQ_ERR_VALUE, "route_topk: null pointer");
  const int64_t blocks = ceil_div(T * 64, kRouteBlock);
  if (blocks > 0x7FFFFFFF) return fail(LQ_ERR_UNSUPPORTED, "route_topk: too many tokens");
#define LQ_ROUTE_LAUNCH(EPL)                                                                         \
  LQ_DISPATCH_DTYPE(logits_dtype, LDT, {                                                             \
    route_topk_kernel<LDT, EPL><<<static_cast<int>(blocks), kRouteBlock, 0, st>>>(                   \
        logits, T, E, k, renormalize, topk_ids, topk_weights);                                       \
  })
  if (E <= 64) {
    LQ_ROUTE_LAUNCH(1);
  } else if (E <= 128) {
    LQ_ROUTE_LAUNCH(2);
  } else {
    LQ_ROUTE_LAUNCH(4);
  }
#undef LQ_ROUTE_LAUNCH
  return check_launch("route_topk");
}
}  // namespace lq

extern "C" int lq_route_topk(const void *logits, int logits_dtype, int64_t T, int E, int k, int renormalize,
                             int32_t *topk_ids, float *topk_weights, lq_stream_t stream) {
  return launch_route_topk(logits, logits_dtype, T, E, k, renormalize, topk_ids, topk_weights, as_stream(stream));
}

extern "C" int lq_gather_topk_weights(const float *probs, const void *ids, int ids_int64, int64_t T, int E, int k,
                                      int renormalize, int32_t *ids32_out, float *topk_weights,
                                      lq_stream_t stream) {
  if (T < 0 || E < 1 || k < 1 || k > E) return fail(LQ_ERR_VALUE, "gather_topk_weights: bad shape");
  if (T == 0) return LQ_OK;
  if (!probs || !ids || !ids32_out || !topk_weights) return fail(LQ_ERR_VALUE, "gather_topk_weights: null pointer");
  const int64_t blocks = ceil_div(T, 256);
  const hipStream_t st = as_stream(stream);
  if (ids_int64)
    gather_weights_kernel<int64_t><<<static_cast<int>(blocks), 256, 0, st>>>(
        probs, static_cast<const int64_t *>(ids), T, E, k, renormalize, ids32_out, topk_weights);
  else
    gather_weights_kernel<int32_t><<<static_cast<int>(blocks), 256, 0, st>>>(
        probs, static_cast<const int32_t *>(ids), T, E, k, renormalize, ids32_out, topk_weights);
  return check_launch("gather_topk_weights");
}

extern "C" int lq_moe_permute(const int32_t *topk_ids, int64_t T, int k, int E, int32_t *counts, int32_t *offsets,
                              int32_t *sorted, lq_stream_t stream) {
  if (E < 1 || E > kMaxExperts)
    return fail(LQ_ERR_UNSUPPORTED, "moe_permute: 1 <= num_experts <= " + std::to_string(kMaxExperts));
  if (T < 0 || k < 1) return fail(LQ_ERR_VALUE, "moe_permute: bad shape");
  if (T * k > 0x7FFFFFFF) return fail(LQ_ERR_UNSUPPORTED, "moe_permute: too many assignments");
  if (!counts || !offsets || (T > 0 && (!topk_ids || !sorted))) return fail(LQ_ERR_VALUE, "moe_permute: null pointer");
  return launch_permute(topk_ids, T * k, E, counts, offsets, sorted, 0, nullptr, nullptr, as_stream(stream));
}
