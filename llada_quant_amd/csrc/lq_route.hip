// lq_route.hip -- routing front end for gfx950: top-k softmax router, the
// gathered top-k weights, and the entry point of the stable expert
// permutation of the T*k assignments (its kernel is lq_moe.hip's plan).
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
constexpr int kRouteRowRegs = 8;  // 16-byte pieces of x a lane holds: rows up to 8 * 64 * 8 = 4096 wide

// One wavefront per token (route_token).  With xperm != nullptr the wave
// also copies its token's row of x into xperm in the MoE kernel's K-slot
// order.  Rows up to 4096 wide are read into registers before the routing,
// so their loads overlap the logits load and the top-k instead of following
// it one round trip per 1 KB; wider rows are copied afterwards in a loop.
template <int LDT, int EPL>
__global__ __launch_bounds__(kRouteBlock) void route_topk_kernel(const void *__restrict__ logits, int64_t T,
                                                                 int E, int k, int renorm,
                                                                 int32_t *__restrict__ ids,
                                                                 float *__restrict__ weights,
                                                                 const uint16_t *__restrict__ x, int H,
                                                                 uint16_t *__restrict__ xperm) {
  const int lane = threadIdx.x & 63;
  // the wave's token, uniform (a scalar) so the row's buffer descriptor is too
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (kRouteBlock / 64) +
                    __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  if (t >= T) return;  // uniform per wave; no block-wide barrier below
  float v[EPL];
  route_logits<LDT, EPL>(logits, t, E, v);  // first, so the routing waits on it alone
  const int nc = H >> 3;                    // 16-byte pieces per row
  const bool held = xperm != nullptr && nc <= 64 * kRouteRowRegs;
  // bounded to the row (to nothing when the row is not held): pieces past H
  // read zeros without touching memory and are never stored.  No branch, so
  // the routing's wait covers the logits load alone.
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(held ? x + t * H : x), 0, held ? H * 2 : 0, 0x00020000);
  uint4 row[kRouteRowRegs];
#pragma unroll
  for (int i = 0; i < kRouteRowRegs; ++i)
    row[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (lane + 64 * i) * 16, 0, 0));
  __builtin_amdgcn_sched_barrier(0);  // keeps the row loads ahead of the routing's wait
  route_store<EPL>(v, t, E, k, renorm, ids, weights, nullptr);
  if (xperm != nullptr) {
    uint4 *dst = reinterpret_cast<uint4 *>(xperm + t * H);
    if (held) {
#pragma unroll
      for (int i = 0; i < kRouteRowRegs; ++i)
        if (lane + 64 * i < nc) dst[lane + 64 * i] = permute_kslots(row[i]);
    } else {
      const uint4 *src = reinterpret_cast<const uint4 *>(x + t * H);
      for (int c = lane; c < nc; c += 64) dst[c] = permute_kslots(src[c]);
    }
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

}  // namespace

}  // namespace lq

using namespace lq;

namespace lq {
// Router GEMM fused with the top-k (trajectory/llada.py:228-234 with the
// gate in front: router_logits = gate(x) in bf16, then softmax(fp32).topk).
// One wave per 16 tokens: the 16 x E logits (E <= 64, four 16-expert tiles)
// accumulate in fp32 with v_mfma_f32_16x16x32_bf16 over K = H, the A (x
// rows) and B (gate rows) fragments loaded straight from memory -- lane l
// holds 8 consecutive K values of row l % 16 at K offset 8 (l / 16) of each
// 32-wide step, the same K order on both sides -- then are rounded to bf16
// as nn.Linear's bf16 output is, staged in LDS and routed token by token
// with route_token (the unfused path's routine).  Rows past T and gate rows
// past E read zeros (bounded buffer descriptors) and are never routed.
typedef __bf16 rg_bf16x8 __attribute__((ext_vector_type(8)));
typedef float rg_floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t rg_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kRgWaves = 4;
constexpr int kRgRows = 16;

__global__ __launch_bounds__(64 * kRgWaves) void route_gemm_topk_kernel(const uint16_t *__restrict__ x,
                                                                       const uint16_t *__restrict__ wg, int64_t T,
                                                                       int H, int E, int k, int renorm,
                                                                       int32_t *__restrict__ ids,
                                                                       float *__restrict__ weights,
                                                                       uint16_t *__restrict__ logits_out) {
  __shared__ float lg[kRgWaves][kRgRows * 64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int lc = lane & 15, lgp = lane >> 4;
  const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kRgWaves + wave) * kRgRows;
  if (t0 >= T) return;  // uniform per wave; no block-wide barrier below
  const int rows = static_cast<int>(T - t0 < kRgRows ? T - t0 : kRgRows);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(x + t0 * H), 0, rows * H * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(wg), 0, E * H * 2, 0x00020000);
  rg_floatx4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = rg_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const int xoff = (lc * H + 8 * lgp) * 2;
  int woff[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) woff[n] = ((16 * n + lc) * H + 8 * lgp) * 2;
  for (int k0 = 0; k0 < H; k0 += 32) {
    const rg_u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff, k0 * 2, 0);
    rg_u32x4 b[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) b[n] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff[n], k0 * 2, 0);
#pragma unroll
    for (int n = 0; n < 4; ++n)
      acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rg_bf16x8, a),
                                                        __builtin_bit_cast(rg_bf16x8, b[n]), acc[n], 0, 0, 0);
  }
  // lane l holds logits of tokens 4 (l / 16) + j, expert 16 n + l % 16
  float *L = lg[wave];
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * lgp + j, e = 16 * n + lc;
      const uint16_t hb = f32_to_bf16_bits(acc[n][j]);
      L[r * 64 + e] = bf16_bits_to_f32(hb);
      if (logits_out && r < rows && e < E) logits_out[(t0 + r) * E + e] = hb;
    }
  // the other lanes' logits: LDS writes complete and ordered before the reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  for (int r = 0; r < rows; ++r)
    route_token<LQ_F32, 1>(L + r * 64 - static_cast<int64_t>(r) * E, r, E, k, renorm, ids + t0 * k, weights + t0 * k,
                           nullptr);
}

int launch_route_topk(const void *logits, int logits_dtype, int64_t T, int E, int k, int renormalize,
                      int32_t *topk_ids, float *topk_weights, hipStream_t st, const uint16_t *x, int H,
                      uint16_t *xperm) {
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
        logits, T, E, k, renormalize, topk_ids, topk_weights, x, H, xperm);                          \
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
  return launch_permute(topk_ids, T * k, E, counts, offsets, sorted, as_stream(stream));
}

extern "C" int lq_route_gemm_topk(const void *x, const void *gate_weight, int64_t T, int H, int E, int k,
                                  int renormalize, int32_t *topk_ids, float *topk_weights, void *logits_out,
                                  lq_stream_t stream) {
  if (E < 1 || E > 64) return fail(LQ_ERR_UNSUPPORTED, "route_gemm_topk: 1 <= num_experts <= 64");
  if (k < 1 || k > E) return fail(LQ_ERR_VALUE, "route_gemm_topk: need 1 <= k <= num_experts");
  if (T < 0 || H <= 0) return fail(LQ_ERR_VALUE, "route_gemm_topk: bad shape");
  if (H % 32 != 0) return fail(LQ_ERR_UNSUPPORTED, "route_gemm_topk: hidden must be a multiple of 32");
  if (int64_t{64} * H * 2 > 0x7FFFFFF0) return fail(LQ_ERR_UNSUPPORTED, "route_gemm_topk: hidden too large");
  if (T == 0) return LQ_OK;
  if (!x || !gate_weight || !topk_ids || !topk_weights) return fail(LQ_ERR_VALUE, "route_gemm_topk: null pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gate_weight)) & 15)
    return fail(LQ_ERR_VALUE, "route_gemm_topk: x and gate_weight must be 16-byte aligned");
  const int64_t blocks = ceil_div(T, kRgWaves * kRgRows);
  if (blocks > 0x7FFFFFFF) return fail(LQ_ERR_UNSUPPORTED, "route_gemm_topk: too many tokens");
  route_gemm_topk_kernel<<<static_cast<int>(blocks), 64 * kRgWaves, 0, as_stream(stream)>>>(
      static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(gate_weight), T, H, E, k, renormalize, topk_ids,
      topk_weights, static_cast<uint16_t *>(logits_out));
  return check_launch("route_gemm_topk");
}
