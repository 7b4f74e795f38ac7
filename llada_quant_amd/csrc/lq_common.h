// lq_common.h -- shared definitions of liblladaq.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstddef>
#include <string>

#include "../../include/lladaq.h"

namespace lq {

// ---------------------------------------------------------------------------
// error reporting across the C ABI: a thread-local message + status code
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
int fail(int status, const std::string &msg);
int check_launch(const char *what);

#define LQ_HIP_CHECK(expr)                                                   \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess)                                                    \
      return ::lq::fail(LQ_ERR_RUNTIME, std::string(#expr " failed: ") +     \
                                            hipGetErrorString(_e));          \
  } while (0)

inline hipStream_t as_stream(lq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// the reference's grouping (algorithms/symmetric.py:85-90): G divides k ->
// groups of G, otherwise (or G == -1) one group spanning the whole row.
inline int64_t effective_group(int64_t k, int64_t group_size) {
  if (group_size == -1 || group_size <= 0 || k % group_size != 0) return k;
  return group_size;
}

inline bool valid_dtype(int d) { return d == LQ_F32 || d == LQ_F16 || d == LQ_BF16; }

// ---------------------------------------------------------------------------
// scalar conversions (device)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// torch's float -> bfloat16 (round half to even, NaN -> 0x7FC0).  Used where
// the result must equal the reference bit for bit for every input.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// IEEE round-to-nearest-even float -> half (what c10::Half does).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT>
__device__ __forceinline__ float load_f32(const void *p, int64_t i);
template <>
__device__ __forceinline__ float load_f32<LQ_F32>(const void *p, int64_t i) {
  return static_cast<const float *>(p)[i];
}
template <>
__device__ __forceinline__ float load_f32<LQ_F16>(const void *p, int64_t i) {
  return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
}
template <>
__device__ __forceinline__ float load_f32<LQ_BF16>(const void *p, int64_t i) {
  return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_f32(void *p, int64_t i, float v);
template <>
__device__ __forceinline__ void store_f32<LQ_F32>(void *p, int64_t i, float v) {
  static_cast<float *>(p)[i] = v;
}
template <>
__device__ __forceinline__ void store_f32<LQ_F16>(void *p, int64_t i, float v) {
  static_cast<uint16_t *>(p)[i] = f32_to_f16_bits(v);
}
template <>
__device__ __forceinline__ void store_f32<LQ_BF16>(void *p, int64_t i, float v) {
  static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
}

// value.to(dtype).float(): the rounding a scale goes through when the
// reference stores it in scale_dtype (algorithms/symmetric.py:244-245).
template <int DT>
__device__ __forceinline__ float round_through(float v) {
  if constexpr (DT == LQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if constexpr (DT == LQ_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

// ---------------------------------------------------------------------------
// wavefront helpers (wave64)
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// exact dequantization fp32(q) * s of packed codes (algorithms/symmetric.py:
// 272-293), shared by the dequant kernel and the MoE GEMMs.
//
// A code enters as n = q + 2^(b-1) (nibble ^ 8, byte ^ 0x80) in the low bits
// of a binary16 half: the half is the subnormal n * 2^-24 (or 16 n * 2^-24),
// which v_fma_mix_f32 widens exactly.  fma(n 2^-24, s 2^24, -2^(b-1) s) is
// then (n - 2^(b-1)) s = q s rounded once -- the rounding of the IEEE
// product fp32(q) * s.  This needs s * 2^24 finite: dq_fast_ok(s) says so
// (s < 2^103); callers take dq_slow_* otherwise.
// ---------------------------------------------------------------------------
struct DqScale {
  float s24;  // s * 2^24
  float s20;  // s * 2^20
  float c;    // -2^(b-1) * s
};

template <int BITS>
__device__ __forceinline__ DqScale dq_scale(float s) {
  return {s * 16777216.0f, s * 1048576.0f, (BITS == 4 ? -8.0f : -128.0f) * s};
}

__device__ __forceinline__ bool dq_fast_ok(float s) { return s < 0x1p103f; }

__device__ __forceinline__ float half_lo_f32(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xFFFFu)));
}
__device__ __forceinline__ float half_hi_f32(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v >> 16)));
}

// 8 INT4 codes of one dword (element i in nibble i) -> e[i] = fp32(q_i) * s
__device__ __forceinline__ void dq_int4x8(uint32_t w, const DqScale &d, float (&e)[8]) {
  // each (x ^ c) & m is one v_bitop3_b32; the shift is the only other op
  const uint32_t ws = w >> 8;
  const uint32_t t0 = (w ^ 0x00080008u) & 0x000F000Fu;   // n0, n4
  const uint32_t t1 = (w ^ 0x00800080u) & 0x00F000F0u;   // 16 n1, 16 n5
  const uint32_t t2 = (ws ^ 0x00080008u) & 0x000F000Fu;  // n2, n6
  const uint32_t t3 = (ws ^ 0x00800080u) & 0x00F000F0u;  // 16 n3, 16 n7
  e[0] = fmaf(half_lo_f32(t0), d.s24, d.c);
  e[4] = fmaf(half_hi_f32(t0), d.s24, d.c);
  e[1] = fmaf(half_lo_f32(t1), d.s20, d.c);
  e[5] = fmaf(half_hi_f32(t1), d.s20, d.c);
  e[2] = fmaf(half_lo_f32(t2), d.s24, d.c);
  e[6] = fmaf(half_hi_f32(t2), d.s24, d.c);
  e[3] = fmaf(half_lo_f32(t3), d.s20, d.c);
  e[7] = fmaf(half_hi_f32(t3), d.s20, d.c);
}

// 4 INT8 codes of one dword (element i in byte i) -> e[i] = fp32(q_i) * s
__device__ __forceinline__ void dq_int8x4(uint32_t w, const DqScale &d, float (&e)[4]) {
  const uint32_t t0 = (w ^ 0x00800080u) & 0x00FF00FFu;         // n0, n2 (one v_bitop3_b32)
  const uint32_t t1 = ((w >> 8) ^ 0x00800080u) & 0x00FF00FFu;  // n1, n3
  e[0] = fmaf(half_lo_f32(t0), d.s24, d.c);
  e[2] = fmaf(half_hi_f32(t0), d.s24, d.c);
  e[1] = fmaf(half_lo_f32(t1), d.s24, d.c);
  e[3] = fmaf(half_hi_f32(t1), d.s24, d.c);
}

// the same products by plain conversion (any finite or non-finite scale)
__device__ __forceinline__ void dq_slow_int4x8(uint32_t w, float s, float (&e)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = static_cast<float>(static_cast<int32_t>(w << (28 - 4 * i)) >> 28) * s;
}
__device__ __forceinline__ void dq_slow_int8x4(uint32_t w, float s, float (&e)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) e[i] = static_cast<float>(static_cast<int32_t>(w << (24 - 8 * i)) >> 24) * s;
}

// 8 consecutive bf16 (dwords = element pairs 01 23 45 67) -> the K-slot order
// [0,4,1,5,2,6,3,7] of the MoE kernel's MFMA fragments (dwords 04 15 26 37)
__device__ __forceinline__ uint4 permute_kslots(uint4 v) {
  return make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                    __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
}

// storage column of K index f in a permuted row: slot order [0,4,1,5,2,6,3,7]
// within each group of 8, i.e. element e of a group lands in slot 2e (e < 4)
// or 2(e - 4) + 1
__device__ __forceinline__ int kslot(int f) {
  const int e = f & 7;
  return (f & ~7) | (e < 4 ? 2 * e : 2 * (e - 4) + 1);
}

// dispatch a runtime dtype code to a template parameter
#define LQ_DISPATCH_DTYPE(code, NAME, ...)        \
  switch (code) {                                 \
    case LQ_F32: {                                \
      constexpr int NAME = LQ_F32;                \
      __VA_ARGS__;                                \
    } break;                                      \
    case LQ_F16: {                                \
      constexpr int NAME = LQ_F16;                \
      __VA_ARGS__;                                \
    } break;                                      \
    default: {                                    \
      constexpr int NAME = LQ_BF16;               \
      __VA_ARGS__;                                \
    } break;                                      \
  }

}  // namespace lq
