// lq_quant.hip -- packing, unpacking, dequantization and the groupwise
// symmetric quantizer (amax or MSE clip search) for gfx950.
//
// Numerical contract: algorithms/symmetric.py of Ahmed-Hedhili-se/LLaDA_Quant
// v0.2.0 evaluated by torch on the CPU.  Every float operation below is the
// IEEE one the reference performs, in the same order (the library is built
// with -ffp-contract=off so `v * safe - x` stays two roundings).
#include "lq_common.h"

namespace lq {
namespace {

constexpr int kBlock = 256;

inline int grid_1d(int64_t items, int64_t per_block) {
  int64_t g = ceil_div(items, per_block);
  if (g < 1) g = 1;
  if (g > (int64_t)1 << 20) g = (int64_t)1 << 20;  // grid-stride beyond this
  return static_cast<int>(g);
}

__device__ __forceinline__ int64_t gtid() {
  return static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
}
__device__ __forceinline__ int64_t gstride() {
  return static_cast<int64_t>(gridDim.x) * blockDim.x;
}

// ---------------------------------------------------------------------------
// pack / unpack (algorithms/symmetric.py:296-346)
// ---------------------------------------------------------------------------

// one output byte per pair: low nibble = even element, high = odd element
__global__ void pack_int4_kernel(const int8_t *__restrict__ q, int64_t n_out,
                                 int8_t *__restrict__ out, int32_t *__restrict__ range_flag) {
  for (int64_t i = gtid(); i < n_out; i += gstride()) {
    const int lo = q[2 * i], hi = q[2 * i + 1];
    if (lo < -8 || lo > 7 || hi < -8 || hi > 7) range_flag[0] = 1;
    out[i] = static_cast<int8_t>(static_cast<uint8_t>((lo & 0x0F) | ((hi & 0x0F) << 4)));
  }
}

// low = (b << 4) >> 4, high = b >> 4, arithmetic shifts on int8
__global__ void unpack_int4_kernel(const int8_t *__restrict__ packed, int64_t n_bytes,
                                   int8_t *__restrict__ out) {
  for (int64_t i = gtid(); i < n_bytes; i += gstride()) {
    const int32_t b = packed[i];
    out[2 * i] = static_cast<int8_t>((b << 28) >> 28);
    out[2 * i + 1] = static_cast<int8_t>(b >> 4);
  }
}

// ---------------------------------------------------------------------------
// dequantize: out = cast(fp32(q) * fp32(s[row, col / g]))  (symmetric.py:272-293)
// ---------------------------------------------------------------------------

template <int SDT, int ODT>
__device__ __forceinline__ void store8(void *out, int64_t idx, const float (&v)[8]) {
  if constexpr (ODT == LQ_F32) {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + idx);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint16_t a, b;
      if constexpr (ODT == LQ_BF16) {
        a = f32_to_bf16_bits(v[2 * i]);
        b = f32_to_bf16_bits(v[2 * i + 1]);
      } else {
        a = f32_to_f16_bits(v[2 * i]);
        b = f32_to_f16_bits(v[2 * i + 1]);
      }
      p[i] = static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
    }
    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + idx) = make_uint4(p[0], p[1], p[2], p[3]);
  }
}

// 8 consecutive elements of one row per thread; needs k % 8 == 0, g % 8 == 0
// and 8-element-aligned operands (checked by the host).
template <int BITS, int SDT, int ODT>
__global__ __launch_bounds__(kBlock) void dequant8_kernel(
    const int8_t *__restrict__ q, const void *__restrict__ s, int64_t rows, int64_t k,
    int64_t g, int64_t ng, void *__restrict__ out) {
  const int64_t cpr = k >> 3;
  const int64_t total = rows * cpr;
  for (int64_t c = gtid(); c < total; c += gstride()) {
    const int64_t row = c / cpr;
    const int64_t col = (c - row * cpr) << 3;
    const float sc = load_f32<SDT>(s, row * ng + col / g);
    // the products come from the same routine the MoE GEMMs feed their
    // matrix cores with (dq_int4x8 / dq_int8x4)
    float v[8];
    if constexpr (BITS == 4) {
      const uint32_t w = *reinterpret_cast<const uint32_t *>(q + row * (k >> 1) + (col >> 1));
      if (dq_fast_ok(sc))
        dq_int4x8(w, dq_scale<4>(sc), v);
      else
        dq_slow_int4x8(w, sc, v);
    } else {
      const uint2 w = *reinterpret_cast<const uint2 *>(q + row * k + col);
      float lo[4], hi[4];
      if (dq_fast_ok(sc)) {
        const DqScale d = dq_scale<8>(sc);
        dq_int8x4(w.x, d, lo);
        dq_int8x4(w.y, d, hi);
      } else {
        dq_slow_int8x4(w.x, sc, lo);
        dq_slow_int8x4(w.y, sc, hi);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = lo[i];
        v[4 + i] = hi[i];
      }
    }
    store8<SDT, ODT>(out, row * k + col, v);
  }
}

// any shape: one element per thread
template <int BITS, int SDT, int ODT>
__global__ __launch_bounds__(kBlock) void dequant1_kernel(
    const int8_t *__restrict__ q, const void *__restrict__ s, int64_t rows, int64_t k,
    int64_t g, int64_t ng, void *__restrict__ out) {
  const int64_t total = rows * k;
  for (int64_t e = gtid(); e < total; e += gstride()) {
    const int64_t row = e / k;
    const int64_t col = e - row * k;
    int32_t n;
    if constexpr (BITS == 4) {
      const int32_t b = q[row * (k >> 1) + (col >> 1)];
      n = (col & 1) ? (b >> 4) : ((b << 28) >> 28);
    } else {
      n = q[e];
    }
    store_f32<ODT>(out, e, static_cast<float>(n) * load_f32<SDT>(s, row * ng + col / g));
  }
}

// ---------------------------------------------------------------------------
// quantizer (symmetric.py:117-119 _amax_scale, :122-204 search_group_scale,
// :207-269 quantize_tensor)
//
// The MSE search keeps, per group, the first candidate scale whose squared
// error is strictly smallest; the error is an fp32 sum whose order must be
// torch's CPU order for `x.sum(dim=-1)` (8-wide vectors, 4 accumulators,
// 4-level cascade) so that near ties resolve as in the reference.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float candidate_ratio(double max_shrink, int step, int grid) {
  // python: 1.0 - max_shrink * step / grid, then fp32 when it scales the tensor
  return static_cast<float>(1.0 - max_shrink * static_cast<double>(step) / static_cast<double>(grid));
}

// Code of x for scale s: clamp(rint(RN(x / s)), qmin, qmax), rint rounding
// half to even.  Only the integer rint(RN(x / s)) matters, so no quotient is
// rounded correctly unless it has to be.  Once per scale of a group whose
// largest magnitude is amax: y ~ 1/s (the hardware reciprocal and one Newton
// step, relative error <= 2^-23) and Q = RN(amax y), which no |q0| of the
// group exceeds.  Per weight: q0 = RN(x y) and r = rint(q0).
//
// Bound: with s and 1/s normal, |q0 - x/s| + |RN(x/s) - x/s| <= |q0| 2^-21 +
// 2^-148.  The weight keeps r when |q0 - r| (exact) < t = RN(0.5 - Q 2^-18):
// then q0 lies more than Q 2^-18 - 2^-26 >= |q0| 2^-18 - 2^-26 from the
// nearest half-integer, above that bound for |q0| >= 2^-7, and below that
// 0.5 - |q0| > 0.49 dominates it; so RN(x/s) lies in the same open interval
// (r - 1/2, r + 1/2) as q0 and rounds to r as well.  Otherwise (near a
// half-integer, a non-finite q0, t <= 0 once Q >= 2^17) the weight divides.
// Scales outside [2^-100, 2^126] always divide (t = -1); from 2^-100 up a
// subnormal x has |x/s| < 2^-26 and code 0 whether the product flushes it or
// not.  The clamp of a kept r, finite and below 2^17, is one v_med3.
struct QuotScale {
  float s, y, t;
};
__device__ __forceinline__ QuotScale quot_scale(float s, float amax) {
  const float y0 = __builtin_amdgcn_rcpf(s);
  const float y = fmaf(fmaf(-s, y0, 1.0f), y0, y0);
  const bool fast = s >= 0x1p-100f && s <= 0x1p126f;
  return {s, y, fast ? fmaf(amax * y, -0x1p-18f, 0.5f) : -1.0f};
}
// The code from the product alone; sets redo when the weight must divide
// (the code returned is then meaningless).
__device__ __forceinline__ float quot_code_fast(float x, const QuotScale &d, float qmin, float qmax, bool &redo) {
  const float q0 = x * d.y;
  const float r = rintf(q0);
  redo |= !(fabsf(q0 - r) < d.t);
  return __builtin_amdgcn_fmed3f(r, qmin, qmax);
}
__device__ __forceinline__ float quot_code_div(float x, const QuotScale &d, float qmin, float qmax) {
  return fminf(fmaxf(rintf(x / d.s), qmin), qmax);
}
// code from quot_code_fast, replaced by the division's where that applies
__device__ __forceinline__ float quot_code_fix(float x, const QuotScale &d, float qmin, float qmax, float code) {
  bool redo = false;
  quot_code_fast(x, d, qmin, qmax, redo);
  return redo ? quot_code_div(x, d, qmin, qmax) : code;
}
__device__ __forceinline__ float quot_code(float x, const QuotScale &d, float qmin, float qmax) {
  bool redo = false;
  const float c = quot_code_fast(x, d, qmin, qmax, redo);
  return redo ? quot_code_div(x, d, qmin, qmax) : c;
}

// the reference's squared error of one weight, from its code
__device__ __forceinline__ float sq_err_code(float x, float code, float safe) {
  float v = code * safe;  // mul_(safe)
  v = v - x;              // sub_(wf)
  return v * v;           // pow_(2)
}
__device__ __forceinline__ float sq_err(float x, const QuotScale &d, float qmin, float qmax) {
  // (wf / safe).round_().clamp_(qmin, qmax)
  return sq_err_code(x, quot_code(x, d, qmin, qmax), d.s);
}

// Lane 8j of a row of 16 gets p of lane 8j + N (row_shl:N; N <= 7 stays
// inside the row).  Other lanes get values they do not use.
template <int N>
__device__ __forceinline__ float row_shl(float p) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, p), 0x100 | N, 0xF, 0xF,
                                                               false));
}

__device__ __forceinline__ float round_scale(float v, int sdt) {
  if (sdt == LQ_BF16) return round_through<LQ_BF16>(v);
  if (sdt == LQ_F16) return round_through<LQ_F16>(v);
  return v;
}

__device__ __forceinline__ void store_scale(void *p, int64_t i, float v, int sdt) {
  if (sdt == LQ_BF16)
    store_f32<LQ_BF16>(p, i, v);
  else if (sdt == LQ_F16)
    store_f32<LQ_F16>(p, i, v);
  else
    store_f32<LQ_F32>(p, i, v);
}

struct QuantArgs {
  const void *w;
  int64_t n_groups;
  int64_t n;  // group length
  int bits;
  int pack;  // bits == 4: two values per byte
  int mse;
  int grid;
  double max_shrink;
  int write_q;
  int8_t *q;
  void *scale;
  int scale_dtype;
};

// Fast path: 8 lanes per group, group length n with n % 8 == 0 and
// n / 8 <= MAXV (n <= 256 covers every group size the expert path uses).
// Lane l of a group holds elements 8*i + l: exactly the lanes of torch's
// 8-float vectors, so each lane forms its vector lane's partial sums and the
// 8 partials are added in lane order, as the CPU reduction does.  For
// n <= 256 the cascade of multi_row_sum never triggers (it needs >= 16 rows
// of 4 vectors), so per lane the order is:
//   acc[k] = sum over rows r of e[(4r + k)*8 + l]      (k = 0..3)
//   acc[0] += tail vectors;  p = ((acc0 + acc1) + acc2) + acc3
//   err = 0 + (((0 + p_0) + p_1) + ... + p_7)
// EXACT: n is exactly 8 * MAXV, so every vector test below folds away.
template <int WDT, int MAXV, bool EXACT>
__global__ __launch_bounds__(kBlock) void quant_group8_kernel(QuantArgs a) {
  const int lane = threadIdx.x & 63;
  const int l8 = lane & 7;
  const int64_t gi = gtid() >> 3;
  const bool active = gi < a.n_groups;
  const int vs = EXACT ? MAXV : static_cast<int>(a.n >> 3);
  const int64_t base = (active ? gi : 0) * a.n;
  const float qmax = static_cast<float>((1 << (a.bits - 1)) - 1);
  const float qmin = -static_cast<float>(1 << (a.bits - 1));

  float x[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) x[i] = (i < vs) ? load_f32<WDT>(a.w, base + 8 * i + l8) : 0.0f;

  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i)
    if (i < vs) m = fmaxf(m, fabsf(x[i]));
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  m = fmaxf(m, __shfl_xor(m, 4, 64));
  const float amax_s = m / qmax;

  float chosen = amax_s;
  if (a.mse) {
    const int rows4 = (vs >> 2) << 2;
    // candidate ratios of steps 0..63, one per lane, read back by step
    const float lane_ratio = candidate_ratio(a.max_shrink, lane, a.grid);
    float best = amax_s;
    float best_err = __builtin_inff();
    for (int step = 0; step < a.grid; ++step) {
      const float ratio =
          step < 64 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lane_ratio), step))
                    : candidate_ratio(a.max_shrink, step, a.grid);
      const float cand = amax_s * ratio;
      const float safe = cand > 0.0f ? cand : 1.0f;
      const QuotScale rs = quot_scale(safe, m);
      // codes from the products; a lane with a quotient too near a
      // half-integer (rare) then redoes those weights by division
      float code[MAXV];
      bool redo = false;
#pragma unroll
      for (int i = 0; i < MAXV; ++i)
        if (i < vs) code[i] = quot_code_fast(x[i], rs, qmin, qmax, redo);
      if (redo) {
#pragma unroll
        for (int i = 0; i < MAXV; ++i)
          if (i < vs) code[i] = quot_code_fix(x[i], rs, qmin, qmax, code[i]);
      }
      float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
#pragma unroll
      for (int i = 0; i < MAXV; ++i) {
        if (i < vs) {
          const float e = sq_err_code(x[i], code[i], safe);
          if (i < rows4) {
            if ((i & 3) == 0) acc0 += e;
            else if ((i & 3) == 1) acc1 += e;
            else if ((i & 3) == 2) acc2 += e;
            else acc3 += e;
          } else {
            acc0 += e;  // tail vectors go to partial 0 after the rows
          }
        }
      }
      const float p = ((acc0 + acc1) + acc2) + acc3;
      // the group's first lane adds the 8 partials in lane order; the
      // other lanes' err and best are never used
      float f = 0.0f + p;
      f += row_shl<1>(p);
      f += row_shl<2>(p);
      f += row_shl<3>(p);
      f += row_shl<4>(p);
      f += row_shl<5>(p);
      f += row_shl<6>(p);
      f += row_shl<7>(p);
      const float err = 0.0f + f;
      if (err < best_err) {
        best_err = err;
        best = cand;
      }
    }
    best = __shfl(best, lane & ~7, 64);
    chosen = amax_s > 0.0f ? best : 0.0f;
  }

  const float stored = round_scale(chosen, a.scale_dtype);
  if (active && l8 == 0) store_scale(a.scale, gi, stored, a.scale_dtype);
  if (!a.write_q) return;

  const QuotScale qs = quot_scale(stored > 0.0f ? stored : 1.0f, m);
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    if (i < vs) {
      const int qi = static_cast<int>(quot_code(x[i], qs, qmin, qmax));
      const int64_t e = base + 8 * i + l8;
      if (!a.pack) {
        if (active) a.q[e] = static_cast<int8_t>(qi);
      } else {
        const int hi = __shfl_down(qi, 1, 64);
        if (active && (l8 & 1) == 0)
          a.q[e >> 1] = static_cast<int8_t>(static_cast<uint8_t>((qi & 0x0F) | ((hi & 0x0F) << 4)));
      }
    }
  }
}

// ---- generic path: one thread per group, any length, torch's full order ----

__device__ __forceinline__ int64_t ceil_log2_dev(int64_t x) {
  if (x <= 1) return 0;
  return 64 - __clzll(static_cast<unsigned long long>(x - 1));
}

// multi_row_sum restricted to one vector lane: `size` rows of 4 units; unit
// (i, k) has value elem(i * 4 + k).  Returns the 4 partials in ps.
template <class Elem>
__device__ void multi_row_sum_1(const Elem &elem, int64_t size, float ps[4]) {
  float acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[j][k] = 0.0f;
  int64_t lp = ceil_log2_dev(size) / 4;
  if (lp < 4) lp = 4;
  const int64_t step = static_cast<int64_t>(1) << lp;
  const int64_t mask = step - 1;
  int64_t i = 0;
  for (; i + step <= size;) {
    for (int64_t j = 0; j < step; ++j, ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[0][k] += elem(i * 4 + k);
#pragma unroll
    for (int j = 1; j < 4; ++j) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[j][k] += acc[j - 1][k];
        acc[j - 1][k] = 0.0f;
      }
      if ((i & (mask << (j * lp))) != 0) break;
    }
  }
  for (; i < size; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[0][k] += elem(i * 4 + k);
#pragma unroll
  for (int j = 1; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[0][k] += acc[j][k];
#pragma unroll
  for (int k = 0; k < 4; ++k) ps[k] = acc[0][k];
}

// row_sum over `size` units (one vector lane, or scalars)
template <class Elem>
__device__ float row_sum_1(const Elem &elem, int64_t size) {
  float ps[4];
  const int64_t size_ilp = size / 4;
  multi_row_sum_1(elem, size_ilp, ps);
  for (int64_t u = size_ilp * 4; u < size; ++u) ps[0] += elem(u);
  ps[0] += ps[1];
  ps[0] += ps[2];
  ps[0] += ps[3];
  return ps[0];
}

template <class Err>
__device__ float torch_cpu_sum(const Err &err, int64_t n) {
  if (n >= 8) {
    const int64_t vs = n / 8;
    float vacc[8];
    for (int l = 0; l < 8; ++l) {
      auto col = [&](int64_t u) { return err(u * 8 + l); };
      vacc[l] = row_sum_1(col, vs);
    }
    float f = 0.0f;
    for (int64_t t = vs * 8; t < n; ++t) f += err(t);
#pragma unroll
    for (int l = 0; l < 8; ++l) f += vacc[l];
    return 0.0f + f;
  }
  return 0.0f + row_sum_1(err, n);
}

template <int WDT>
__global__ __launch_bounds__(kBlock) void quant_generic_kernel(QuantArgs a) {
  const int64_t gi = gtid();
  if (gi >= a.n_groups) return;
  const int64_t base = gi * a.n;
  const float qmax = static_cast<float>((1 << (a.bits - 1)) - 1);
  const float qmin = -static_cast<float>(1 << (a.bits - 1));
  float m = 0.0f;
  for (int64_t i = 0; i < a.n; ++i) m = fmaxf(m, fabsf(load_f32<WDT>(a.w, base + i)));
  const float amax_s = m / qmax;
  float chosen = amax_s;
  if (a.mse) {
    float best = amax_s;
    float best_err = __builtin_inff();
    for (int step = 0; step < a.grid; ++step) {
      const float cand = amax_s * candidate_ratio(a.max_shrink, step, a.grid);
      const float safe = cand > 0.0f ? cand : 1.0f;
      const QuotScale rs = quot_scale(safe, m);
      auto err = [&](int64_t i) { return sq_err(load_f32<WDT>(a.w, base + i), rs, qmin, qmax); };
      const float e = torch_cpu_sum(err, a.n);
      if (e < best_err) {
        best_err = e;
        best = cand;
      }
    }
    chosen = amax_s > 0.0f ? best : 0.0f;
  }
  const float stored = round_scale(chosen, a.scale_dtype);
  store_scale(a.scale, gi, stored, a.scale_dtype);
  if (!a.write_q) return;
  const float safe = stored > 0.0f ? stored : 1.0f;
  auto qval = [&](int64_t i) {
    float v = rintf(load_f32<WDT>(a.w, base + i) / safe);
    return static_cast<int>(fminf(fmaxf(v, qmin), qmax));
  };
  if (!a.pack) {
    for (int64_t i = 0; i < a.n; ++i) a.q[base + i] = static_cast<int8_t>(qval(i));
  } else {
    for (int64_t i = 0; i < a.n; i += 2)
      a.q[(base + i) >> 1] =
          static_cast<int8_t>(static_cast<uint8_t>((qval(i) & 0x0F) | ((qval(i + 1) & 0x0F) << 4)));
  }
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int launch_quant(const QuantArgs &a, int w_dtype, hipStream_t st) {
  if (a.n_groups == 0) return LQ_OK;
  const bool fast = (a.n % 8 == 0) && (a.n / 8 <= 32);
  if (fast) {
    const int vs = static_cast<int>(a.n / 8);
    const int grid = grid_1d(a.n_groups * 8, kBlock);
    if (a.n_groups * 8 > static_cast<int64_t>(grid) * kBlock)
      return fail(LQ_ERR_UNSUPPORTED, "quantize: too many groups for one launch");
    LQ_DISPATCH_DTYPE(w_dtype, WDT, {
      if (vs == 4)
        quant_group8_kernel<WDT, 4, true><<<grid, kBlock, 0, st>>>(a);
      else if (vs == 8)
        quant_group8_kernel<WDT, 8, true><<<grid, kBlock, 0, st>>>(a);
      else if (vs == 16)
        quant_group8_kernel<WDT, 16, true><<<grid, kBlock, 0, st>>>(a);
      else if (vs == 32)
        quant_group8_kernel<WDT, 32, true><<<grid, kBlock, 0, st>>>(a);
      else if (vs < 4)
        quant_group8_kernel<WDT, 4, false><<<grid, kBlock, 0, st>>>(a);
      else if (vs < 16)
        quant_group8_kernel<WDT, 16, false><<<grid, kBlock, 0, st>>>(a);
      else
        quant_group8_kernel<WDT, 32, false><<<grid, kBlock, 0, st>>>(a);
    });
  } else {
    const int grid = grid_1d(a.n_groups, kBlock);
    if (a.n_groups > static_cast<int64_t>(grid) * kBlock)
      return fail(LQ_ERR_UNSUPPORTED, "quantize: too many groups for one launch");
    LQ_DISPATCH_DTYPE(w_dtype, WDT, { quant_generic_kernel<WDT><<<grid, kBlock, 0, st>>>(a); });
  }
  return check_launch("quantize");
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" int lq_pack_int4(const int8_t *q, int64_t rows, int64_t k, int8_t *packed,
                            int32_t *range_flag, lq_stream_t stream) {
  if (rows < 0 || k < 0) return fail(LQ_ERR_VALUE, "pack_int4: negative size");
  if (k % 2 != 0) return fail(LQ_ERR_VALUE, "last dim must be even for int4 packing");
  const int64_t n_out = rows * (k / 2);
  if (n_out == 0) return LQ_OK;
  if (!q || !packed || !range_flag) return fail(LQ_ERR_VALUE, "pack_int4: null pointer");
  pack_int4_kernel<<<grid_1d(n_out, kBlock), kBlock, 0, as_stream(stream)>>>(q, n_out, packed, range_flag);
  return check_launch("pack_int4");
}

extern "C" int lq_unpack_int4(const int8_t *packed, int64_t rows, int64_t k_packed, int8_t *out,
                              lq_stream_t stream) {
  if (rows < 0 || k_packed < 0) return fail(LQ_ERR_VALUE, "unpack_int4: negative size");
  const int64_t n = rows * k_packed;
  if (n == 0) return LQ_OK;
  if (!packed || !out) return fail(LQ_ERR_VALUE, "unpack_int4: null pointer");
  unpack_int4_kernel<<<grid_1d(n, kBlock), kBlock, 0, as_stream(stream)>>>(packed, n, out);
  return check_launch("unpack_int4");
}

extern "C" int lq_dequant(const int8_t *q, const void *scale, int scale_dtype, int64_t rows, int64_t k,
                          int bits, int64_t group_size, void *out, int out_dtype, lq_stream_t stream) {
  if (bits != 4 && bits != 8) return fail(LQ_ERR_VALUE, "bits must be 8 or 4, got " + std::to_string(bits));
  if (!valid_dtype(scale_dtype) || !valid_dtype(out_dtype)) return fail(LQ_ERR_VALUE, "dequant: bad dtype code");
  if (rows < 0 || k < 0) return fail(LQ_ERR_VALUE, "dequant: negative size");
  if (bits == 4 && k % 2 != 0) return fail(LQ_ERR_VALUE, "dequant: packed int4 needs an even last dimension");
  if (rows * k == 0) return LQ_OK;
  if (!q || !scale || !out) return fail(LQ_ERR_VALUE, "dequant: null pointer");
  const int64_t g = effective_group(k, group_size);
  const int64_t ng = k / g;
  const hipStream_t st = as_stream(stream);
  const bool fast = (k % 8 == 0) && (g % 8 == 0) && aligned(q, bits == 4 ? 4 : 8) &&
                    aligned(out, out_dtype == LQ_F32 ? 16 : 16);
  const int grid = fast ? grid_1d(rows * (k / 8), kBlock) : grid_1d(rows * k, kBlock);
#define LQ_DEQ_LAUNCH(B)                                                                           \
  LQ_DISPATCH_DTYPE(scale_dtype, SDT, {                                                            \
    LQ_DISPATCH_DTYPE(out_dtype, ODT, {                                                            \
      if (fast)                                                                                    \
        dequant8_kernel<B, SDT, ODT><<<grid, kBlock, 0, st>>>(q, scale, rows, k, g, ng, out);      \
      else                                                                                         \
        dequant1_kernel<B, SDT, ODT><<<grid, kBlock, 0, st>>>(q, scale, rows, k, g, ng, out);      \
    });                                                                                            \
  })
  if (bits == 4) {
    LQ_DEQ_LAUNCH(4);
  } else {
    LQ_DEQ_LAUNCH(8);
  }
#undef LQ_DEQ_LAUNCH
  return check_launch("dequant");
}

static int validate_search(int grid, double max_shrink) {
  if (grid < 1) return fail(LQ_ERR_VALUE, "grid must be >= 1, got " + std::to_string(grid));
  if (!(max_shrink >= 0.0 && max_shrink < 1.0))
    return fail(LQ_ERR_VALUE, "max_shrink must lie in [0, 1), got " + std::to_string(max_shrink));
  return LQ_OK;
}

extern "C" int lq_quantize(const void *w, int w_dtype, int64_t rows, int64_t k, int bits, int pack,
                           int64_t group_size, int scale_search, int grid, double max_shrink, int8_t *q,
                           void *scale, int scale_dtype, lq_stream_t stream) {
  if (bits != 4 && bits != 8) return fail(LQ_ERR_VALUE, "bits must be 8 or 4, got " + std::to_string(bits));
  if (rows <= 0 || k <= 0) return fail(LQ_ERR_VALUE, "cannot quantize an empty tensor");
  pack = (bits == 4 && pack) ? 1 : 0;
  if (pack && k % 2 != 0)
    return fail(LQ_ERR_VALUE, "int4 packing needs an even last dimension");
  if (pack && group_size != -1 && group_size % 2 != 0)
    return fail(LQ_ERR_VALUE, "int4 packing needs an even group_size so groups stay byte-aligned");
  if (!valid_dtype(w_dtype) || !valid_dtype(scale_dtype)) return fail(LQ_ERR_VALUE, "quantize: bad dtype code");
  if (scale_search != LQ_SCALE_AMAX && scale_search != LQ_SCALE_MSE)
    return fail(LQ_ERR_VALUE, "scale_search must be one of ['amax', 'mse']");
  if (scale_search == LQ_SCALE_MSE) {
    const int rc = validate_search(grid, max_shrink);
    if (rc) return rc;
  }
  if (!w || !q || !scale) return fail(LQ_ERR_VALUE, "quantize: null pointer");
  QuantArgs a;
  a.w = w;
  a.n = effective_group(k, group_size);
  a.n_groups = rows * (k / a.n);
  a.bits = bits;
  a.pack = pack;
  a.mse = scale_search == LQ_SCALE_MSE;
  a.grid = grid;
  a.max_shrink = max_shrink;
  a.write_q = 1;
  a.q = q;
  a.scale = scale;
  a.scale_dtype = scale_dtype;
  return launch_quant(a, w_dtype, as_stream(stream));
}

extern "C" int lq_search_group_scale(const void *w, int w_dtype, int64_t n_groups, int64_t group_len, int bits,
                                     int grid, double max_shrink, float *scale, lq_stream_t stream) {
  {
    const int rc = validate_search(grid, max_shrink);
    if (rc) return rc;
  }
  if (bits != 4 && bits != 8) return fail(LQ_ERR_VALUE, "bits must be 8 or 4, got " + std::to_string(bits));
  if (!valid_dtype(w_dtype)) return fail(LQ_ERR_VALUE, "search_group_scale: bad dtype code");
  if (n_groups < 0 || group_len <= 0) return fail(LQ_ERR_VALUE, "search_group_scale: bad size");
  if (n_groups == 0) return LQ_OK;
  if (!w || !scale) return fail(LQ_ERR_VALUE, "search_group_scale: null pointer");
  QuantArgs a;
  a.w = w;
  a.n = group_len;
  a.n_groups = n_groups;
  a.bits = bits;
  a.pack = 0;
  a.mse = 1;
  a.grid = grid;
  a.max_shrink = max_shrink;
  a.write_q = 0;
  a.q = nullptr;
  a.scale = scale;
  a.scale_dtype = LQ_F32;
  return launch_quant(a, w_dtype, as_stream(stream));
}
