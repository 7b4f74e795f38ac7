// lq_moe.hip -- the quantized MoE expert layer on gfx950: grouped W4A16 /
// W8A16 GEMMs that read packed weights straight from HBM, dequantize them in
// registers (bit-exact to the reference's bf16(fp32(q) * s)) and feed
// v_mfma_f32_16x16x32_bf16, with the SwiGLU activation fused into GEMM1 and
// the routed-weight scaling fused into GEMM2.
//
// Replaces dequantize_tensor (runtime/moe.py:199-216) feeding the external
// fused_moe (INFERENCE_REPO_CHANGES.md:37-63, 259-265, 296-309).
//
// Data flow of one forward (all on one stream, no host sync):
//   permute   ids -> counts/offsets/sorted + work units (expert, rows)
//   GEMM1     act[p, :]  = swiglu(x[t(p)] . W1[e]^T)          p = sorted pos
//   GEMM2     y[a, :]    = w[a] * (act[p] . W2[e]^T)          a = assignment
//   combine   out[t, :]  = bf16(sum_j y[t*k + j, :])
//
// Work decomposition: a unit is up to 16*NRT consecutive sorted rows of one
// expert.  A workgroup (4 waves) computes one unit against 8 column tiles of
// 16 weight rows (GEMM1: 4 gate + 4 up tiles, 64 output features; GEMM2: 8
// tiles, 128 output features), over the full reduction axis split across the
// 4 waves; the 4 partials are summed through LDS in fixed order, so results
// are deterministic.
//
// Fragment layout (v_mfma_f32_16x16x32_bf16, A = tokens 16 x 32, B = weights
// 32 x 16): lane l supplies row/column (l & 15) and 8 reduction elements of
// its lane group g = l >> 4.  One 16-byte load per lane of a packed INT4 row
// holds 32 consecutive K values: lane group g of a 128-wide K block loads the
// 32 values [32g, 32g + 32), which feed 4 MFMA steps (8 values each).  The A
// fragments are loaded with the same K assignment, so the products pair up.
#include "lq_common.h"
#include "lq_route.h"

namespace lq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kCols = 8;       // column tiles of 16 weight rows per workgroup

struct MoeArgs {
  const uint16_t *x;        // [T, H] bf16
  const int8_t *q1;         // [E, 2I, H] int8 or [E, 2I, H/2] packed
  const float *s1;          // [E, 2I, ng1]
  const int8_t *q2;         // [E, H, I] or [E, H, I/2]
  const float *s2;          // [E, H, ng2]
  const int32_t *ids;       // [T*k]
  const float *topk_w;      // [T*k]
  const int32_t *sorted;    // [N] assignment ids by expert
  const int32_t *units;     // [max_units][3] (expert, first sorted position, rows)
  const int32_t *n_units;   // [1]
  uint16_t *act;            // [N, I] bf16, by sorted position
  float *ybuf;              // [N, H] fp32, by assignment
  uint16_t *out;            // [T, H] bf16
  int64_t T;
  int H, I, E, k;
  int g1, ng1, g2, ng2;     // effective group length and groups per row
};

// torch's fp32 -> bf16 rounding, back to fp32
__device__ __forceinline__ float bf16_round(float v) {
  return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(v)) << 16);
}

// 8 INT4 values (value j in nibble j of w) -> bf16(fp32(q) * s)
__device__ __forceinline__ bf16x8 deq_int4x8(uint32_t w, float s) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int32_t n = static_cast<int32_t>(w << (28 - 4 * j)) >> 28;
    r[j] = static_cast<__bf16>(static_cast<float>(n) * s);
  }
  return r;
}

// 8 INT8 values (little-endian bytes of lo, hi) -> bf16(fp32(q) * s)
__device__ __forceinline__ bf16x8 deq_int8x8(uint32_t lo, uint32_t hi, float s) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w = j < 4 ? lo : hi;
    const int32_t n = static_cast<int32_t>(w << (24 - 8 * (j & 3))) >> 24;
    r[j] = static_cast<__bf16>(static_cast<float>(n) * s);
  }
  return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// Packed weight bytes of one lane for one 128-wide K block (4 chunks of 32):
// INT4: 16 bytes; INT8: 32 bytes.
template <int BITS>
struct BFrag;
template <>
struct BFrag<4> {
  uint4 v;
};
template <>
struct BFrag<8> {
  uint4 v0, v1;
};

template <int BITS, int NRT, bool FIRST>
__global__ __launch_bounds__(kThreads) void moe_gemm_kernel(MoeArgs a) {
  __shared__ float red[4][kCols][4][64];  // split-K partials, one row tile

  const int nunits = *a.n_units;
  const int ntiles = FIRST ? (a.I >> 6) : (a.H >> 7);
  const int total = nunits * ntiles;
  const int bid = blockIdx.x;
  if (bid >= total) return;
  // blocks are dealt to the 8 XCDs round-robin (block b -> XCD b % 8); give
  // each XCD a contiguous range of logical tiles so the tiles that share a
  // unit's activations or an expert's weights share an L2
  const int xcd = bid & 7, idx = bid >> 3;
  const int per = total >> 3, rem = total & 7;
  const int L = xcd * per + min(xcd, rem) + idx;
  const int u = L / ntiles;
  const int nt = L - u * ntiles;

  const int e = a.units[3 * u];
  const int row0 = a.units[3 * u + 1];
  const int rows = a.units[3 * u + 2];
  const int nrt = (rows + 15) >> 4;

  const int K = FIRST ? a.H : a.I;
  const int64_t rowbytes = BITS == 4 ? (K >> 1) : K;
  const int nrows_w = FIRST ? 2 * a.I : a.H;
  const int G = FIRST ? a.g1 : a.g2;
  const int ng = FIRST ? a.ng1 : a.ng2;
  const int8_t *W = (FIRST ? a.q1 : a.q2) + static_cast<int64_t>(e) * nrows_w * rowbytes;
  const float *S = (FIRST ? a.s1 : a.s2) + static_cast<int64_t>(e) * nrows_w * ng;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lc = lane & 15;
  const int lg = lane >> 4;

  const int8_t *wrow[kCols];
  const float *srow[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) {
    const int r = FIRST ? ((c < 4 ? 0 : a.I) + nt * 64 + 16 * (c & 3) + lc) : (nt * 128 + 16 * c + lc);
    wrow[c] = W + static_cast<int64_t>(r) * rowbytes;
    srow[c] = S + static_cast<int64_t>(r) * ng;
  }
  const uint16_t *arow[NRT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    const int m = rt * 16 + lc;
    const int pos = row0 + (m < rows ? m : 0);
    arow[rt] = FIRST ? a.x + static_cast<int64_t>(a.sorted[pos] / a.k) * a.H
                     : a.act + static_cast<int64_t>(pos) * a.I;
  }

  floatx4 acc[NRT][kCols];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[rt][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // this wave's range of 32-wide K chunks
  const int nck = K >> 5;
  const int c0 = (wave * nck) >> 2;
  const int c1 = ((wave + 1) * nck) >> 2;
  int kc = c0;

  auto load_b = [&](int kchunk, BFrag<BITS>(&b)[kCols], float(&s)[kCols]) {
    const int kelem = 32 * (kchunk + lg);  // first K element of this lane group
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      if constexpr (BITS == 4) {
        b[c].v = *reinterpret_cast<const uint4 *>(wrow[c] + (kelem >> 1));
      } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(wrow[c] + kelem);
        b[c].v0 = p[0];
        b[c].v1 = p[1];
      }
      s[c] = srow[c][kelem / G];
    }
  };

  if (kc + 4 <= c1) {
    BFrag<BITS> bcur[kCols];
    float scur[kCols];
    load_b(kc, bcur, scur);
    for (; kc + 4 <= c1; kc += 4) {
      BFrag<BITS> bnxt[kCols];
      float snxt[kCols];
      const bool more = kc + 8 <= c1;
      if (more) load_b(kc + 4, bnxt, snxt);
      uint4 af[NRT][4];
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        if (rt < nrt) {
          const uint4 *p = reinterpret_cast<const uint4 *>(arow[rt] + 32 * (kc + lg));
#pragma unroll
          for (int s = 0; s < 4; ++s) af[rt][s] = p[s];
        }
      }
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          bf16x8 b;
          if constexpr (BITS == 4) {
            const uint32_t w = s == 0 ? bcur[c].v.x : s == 1 ? bcur[c].v.y : s == 2 ? bcur[c].v.z : bcur[c].v.w;
            b = deq_int4x8(w, scur[c]);
          } else {
            const uint4 &v = s < 2 ? bcur[c].v0 : bcur[c].v1;
            const uint32_t lo = (s & 1) ? v.z : v.x;
            const uint32_t hi = (s & 1) ? v.w : v.y;
            b = deq_int8x8(lo, hi, scur[c]);
          }
#pragma unroll
          for (int rt = 0; rt < NRT; ++rt)
            if (rt < nrt)
              acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af[rt][s]), b, acc[rt][c], 0, 0, 0);
        }
      }
      if (more) {
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
          bcur[c] = bnxt[c];
          scur[c] = snxt[c];
        }
      }
    }
  }
  // remaining single 32-wide chunks: lane group g takes values [8g, 8g + 8)
  for (; kc < c1; ++kc) {
    const int kelem = 32 * kc + 8 * lg;
    uint4 af[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
      if (rt < nrt) af[rt] = *reinterpret_cast<const uint4 *>(arow[rt] + kelem);
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      const float sc = srow[c][(32 * kc) / G];
      bf16x8 b;
      if constexpr (BITS == 4) {
        b = deq_int4x8(*reinterpret_cast<const uint32_t *>(wrow[c] + (kelem >> 1)), sc);
      } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(wrow[c] + kelem);
        b = deq_int8x8(v.x, v.y, sc);
      }
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
        if (rt < nrt) acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af[rt]), b, acc[rt][c], 0, 0, 0);
    }
  }

  // split-K reduction and epilogue, one row tile at a time
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    if (rt >= nrt) break;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kCols; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][c][r][lane] = acc[rt][c][r];
    __syncthreads();
    if constexpr (FIRST) {
      // 16 rows x 64 features: thread -> feature j, rows 4q .. 4q+3
      const int j = threadIdx.x & 63;
      const int q = threadIdx.x >> 6;
      const int c = j >> 4;
      const int src = q * 16 + (j & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = rt * 16 + 4 * q + r;
        const float g = ((red[0][c][r][src] + red[1][c][r][src]) + red[2][c][r][src]) + red[3][c][r][src];
        const float up =
            ((red[0][c + 4][r][src] + red[1][c + 4][r][src]) + red[2][c + 4][r][src]) + red[3][c + 4][r][src];
        if (m < rows) {
          // reference op order: g, u -> bf16; silu in fp32 -> bf16; bf16 product
          const float gb = bf16_round(g);
          const float ub = bf16_round(up);
          const float sb = bf16_round(gb / (1.0f + expf(-gb)));
          a.act[static_cast<int64_t>(row0 + m) * a.I + nt * 64 + j] = f32_to_bf16_bits(sb * ub);
        }
      }
    } else {
      // 16 rows x 128 features: thread -> feature j, rows 8h .. 8h+7
      const int j = threadIdx.x & 127;
      const int h = threadIdx.x >> 7;
      const int c = j >> 4;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int grp = 2 * h + (i >> 2);
        const int r = i & 3;
        const int src = grp * 16 + (j & 15);
        const int m = rt * 16 + 4 * grp + r;
        const float y = ((red[0][c][r][src] + red[1][c][r][src]) + red[2][c][r][src]) + red[3][c][r][src];
        if (m < rows) {
          const int asg = a.sorted[row0 + m];
          a.ybuf[static_cast<int64_t>(asg) * a.H + nt * 128 + j] = y * a.topk_w[asg];
        }
      }
    }
  }
}

// out[t, h] = bf16(sum_j y[t*k + j, h]) over the routed slots, j ascending
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ ybuf, const int32_t *__restrict__ ids,
                                                      int64_t T, int H, int k, int E, uint16_t *__restrict__ out) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int hq = H >> 2;
  if (q >= T * hq) return;
  const int64_t t = q / hq;
  const int h = static_cast<int>(q - t * hq) << 2;
  float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int j = 0; j < k; ++j) {
    const int id = ids[t * k + j];
    if (id < 0 || id >= E) continue;
    const float4 v = *reinterpret_cast<const float4 *>(ybuf + (t * k + j) * H + h);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  const uint32_t lo = f32_to_bf16_bits(s.x) | (static_cast<uint32_t>(f32_to_bf16_bits(s.y)) << 16);
  const uint32_t hi = f32_to_bf16_bits(s.z) | (static_cast<uint32_t>(f32_to_bf16_bits(s.w)) << 16);
  *reinterpret_cast<uint2 *>(out + t * H + h) = make_uint2(lo, hi);
}

struct WsLayout {
  size_t counts, offsets, sorted, units, n_units, ids, weights, act, ybuf, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

int unit_rows_for(int64_t N, int E) {
  const int64_t avg = N / (E > 0 ? E : 1);
  if (avg <= 16) return 16;
  if (avg <= 32) return 32;
  return 64;
}

int64_t max_units_for(int64_t N, int E, int mc) { return E + N / mc; }

WsLayout ws_layout(int64_t T, int H, int I, int E, int k) {
  const int64_t N = T * k;
  const int mc = unit_rows_for(N, E);
  WsLayout w;
  size_t off = 0;
  auto take = [&](size_t &field, size_t bytes) {
    field = off;
    off = align256(off + bytes);
  };
  take(w.counts, sizeof(int32_t) * E);
  take(w.offsets, sizeof(int32_t) * (E + 1));
  take(w.sorted, sizeof(int32_t) * N);
  take(w.units, sizeof(int32_t) * 3 * max_units_for(N, E, mc));
  take(w.n_units, sizeof(int32_t));
  take(w.ids, sizeof(int32_t) * N);
  take(w.weights, sizeof(float) * N);
  take(w.act, sizeof(uint16_t) * N * I);
  take(w.ybuf, sizeof(float) * N * H);
  w.total = off;
  return w;
}

template <int BITS, int NRT>
void launch_gemm1(const MoeArgs &a, int64_t max_units, hipStream_t st) {
  moe_gemm_kernel<BITS, NRT, true><<<static_cast<int>(max_units * (a.I >> 6)), kThreads, 0, st>>>(a);
}
template <int BITS, int NRT>
void launch_gemm2(const MoeArgs &a, int64_t max_units, hipStream_t st) {
  moe_gemm_kernel<BITS, NRT, false><<<static_cast<int>(max_units * (a.H >> 7)), kThreads, 0, st>>>(a);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Measurement hook (lq_moe_profile_events): caller-owned hipEvent_t handles
// recorded on the call's stream at the kernel boundaries of the next layer
// call on this thread.
thread_local void *const *t_prof_events = nullptr;
thread_local int t_prof_n = 0;

struct ProfileMarks {
  void *const *ev;
  int n;
  hipStream_t st;
  int rc = LQ_OK;
  void mark(int i) {
    if (ev && i < n && ev[i] && rc == LQ_OK) {
      hipError_t e = hipEventRecord(static_cast<hipEvent_t>(ev[i]), st);
      if (e != hipSuccess) rc = fail(LQ_ERR_RUNTIME, std::string("hipEventRecord failed: ") + hipGetErrorString(e));
    }
  }
};

int validate_layer(const void *x, int64_t T, int H, int I, int E, int k, const int8_t *q1, const float *s1,
                   const int8_t *q2, const float *s2, int bits, int64_t group_w1, int64_t group_w2,
                   void *workspace, size_t ws_bytes, void *out) {
  if (bits != 4 && bits != 8) return fail(LQ_ERR_VALUE, "bits must be 8 or 4, got " + std::to_string(bits));
  if (T < 0 || H <= 0 || I <= 0 || k <= 0) return fail(LQ_ERR_VALUE, "moe_forward: bad shape");
  if (E < 1 || E > kMaxExperts)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: 1 <= num_experts <= " + std::to_string(kMaxExperts));
  if (k > E) return fail(LQ_ERR_VALUE, "moe_forward: top_k exceeds num_experts");
  if (H % 128 != 0 || I % 64 != 0)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: needs hidden % 128 == 0 and intermediate % 64 == 0");
  const int64_t g1 = effective_group(H, group_w1);
  const int64_t g2 = effective_group(I, group_w2);
  if (g1 % 32 != 0 || g2 % 32 != 0)
    return fail(LQ_ERR_UNSUPPORTED,
                "moe_forward: the group length along K must be a multiple of 32 (got " + std::to_string(g1) +
                    " for w1, " + std::to_string(g2) + " for w2)");
  const int64_t N = T * k;
  if (N > 0x7FFFFFFF / (H > I ? H : I)) return fail(LQ_ERR_UNSUPPORTED, "moe_forward: too many tokens");
  if (T == 0) return LQ_OK;
  if (!x || !q1 || !s1 || !q2 || !s2 || !workspace || !out) return fail(LQ_ERR_VALUE, "moe_forward: null pointer");
  if (!aligned16(x) || !aligned16(q1) || !aligned16(q2) || !aligned16(workspace) || !aligned16(out))
    return fail(LQ_ERR_VALUE, "moe_forward: x, q1, q2, workspace and out must be 16-byte aligned");
  const size_t need = ws_layout(T, H, I, E, k).total;
  if (ws_bytes < need)
    return fail(LQ_ERR_VALUE, "moe_forward: workspace too small (" + std::to_string(ws_bytes) + " < " +
                                  std::to_string(need) + ")");
  return LQ_OK;
}

// permute -> GEMM1 -> GEMM2 -> combine, marks[first_mark ..] at each boundary
int moe_forward_impl(const void *x, int64_t T, int H, int I, int E, int k, const int8_t *q1, const float *s1,
                     const int8_t *q2, const float *s2, int bits, int64_t group_w1, int64_t group_w2,
                     const int32_t *topk_ids, const float *topk_weights, char *ws, void *out, hipStream_t st,
                     ProfileMarks &pm, int first_mark) {
  const WsLayout w = ws_layout(T, H, I, E, k);
  const int64_t N = T * k;
  const int mc = unit_rows_for(N, E);
  const int64_t max_units = max_units_for(N, E, mc);
  const int64_t g1 = effective_group(H, group_w1);
  const int64_t g2 = effective_group(I, group_w2);

  MoeArgs a;
  a.x = static_cast<const uint16_t *>(x);
  a.q1 = q1;
  a.s1 = s1;
  a.q2 = q2;
  a.s2 = s2;
  a.ids = topk_ids;
  a.topk_w = topk_weights;
  a.sorted = reinterpret_cast<const int32_t *>(ws + w.sorted);
  a.units = reinterpret_cast<const int32_t *>(ws + w.units);
  a.n_units = reinterpret_cast<const int32_t *>(ws + w.n_units);
  a.act = reinterpret_cast<uint16_t *>(ws + w.act);
  a.ybuf = reinterpret_cast<float *>(ws + w.ybuf);
  a.out = static_cast<uint16_t *>(out);
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.k = k;
  a.g1 = static_cast<int>(g1);
  a.ng1 = static_cast<int>(H / g1);
  a.g2 = static_cast<int>(g2);
  a.ng2 = static_cast<int>(I / g2);

  int rc = launch_permute(topk_ids, N, E, reinterpret_cast<int32_t *>(ws + w.counts),
                          reinterpret_cast<int32_t *>(ws + w.offsets), reinterpret_cast<int32_t *>(ws + w.sorted),
                          mc, reinterpret_cast<int32_t *>(ws + w.units), reinterpret_cast<int32_t *>(ws + w.n_units),
                          st);
  if (rc) return rc;
  pm.mark(first_mark);
#define LQ_GEMM(WHICH)                                       \
  if (bits == 4) {                                           \
    if (mc == 16) WHICH<4, 1>(a, max_units, st);             \
    else if (mc == 32) WHICH<4, 2>(a, max_units, st);        \
    else WHICH<4, 4>(a, max_units, st);                      \
  } else {                                                   \
    if (mc == 16) WHICH<8, 1>(a, max_units, st);             \
    else if (mc == 32) WHICH<8, 2>(a, max_units, st);        \
    else WHICH<8, 4>(a, max_units, st);                      \
  }
  LQ_GEMM(launch_gemm1);
  pm.mark(first_mark + 1);
  LQ_GEMM(launch_gemm2);
#undef LQ_GEMM
  rc = check_launch("moe_gemm");
  if (rc) return rc;
  pm.mark(first_mark + 2);
  const int64_t nthreads = T * (H >> 2);
  combine_kernel<<<static_cast<int>(ceil_div(nthreads, 256)), 256, 0, st>>>(a.ybuf, topk_ids, T, H, k, E, a.out);
  rc = check_launch("moe_combine");
  if (rc) return rc;
  pm.mark(first_mark + 3);
  return pm.rc;
}

ProfileMarks take_profile(hipStream_t st) {
  ProfileMarks pm{t_prof_events, t_prof_n, st};
  t_prof_events = nullptr;
  t_prof_n = 0;
  return pm;
}

}  // namespace

}  // namespace lq

using namespace lq;

extern "C" size_t lq_moe_workspace_bytes(int64_t T, int H, int I, int E, int k) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return ws_layout(T, H, I, E, k).total;
}

extern "C" int lq_moe_profile_events(void *const *events, int n_events) {
  if (n_events < 0) return fail(LQ_ERR_VALUE, "moe_profile_events: negative count");
  t_prof_events = n_events ? events : nullptr;
  t_prof_n = n_events;
  return LQ_OK;
}

extern "C" int lq_moe_forward(const void *x, int64_t T, int H, int I, int E, int k, const int8_t *q1,
                              const float *s1, const int8_t *q2, const float *s2, int bits, int64_t group_w1,
                              int64_t group_w2, const int32_t *topk_ids, const float *topk_weights,
                              void *workspace, size_t ws_bytes, void *out, lq_stream_t stream) {
  const hipStream_t st = as_stream(stream);
  ProfileMarks pm = take_profile(st);
  int rc = validate_layer(x, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, workspace, ws_bytes, out);
  if (rc || T == 0) return rc;
  if (!topk_ids || !topk_weights) return fail(LQ_ERR_VALUE, "moe_forward: null routing pointer");
  pm.mark(0);
  return moe_forward_impl(x, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, topk_ids, topk_weights,
                          static_cast<char *>(workspace), out, st, pm, 1);
}

extern "C" int lq_moe_layer(const void *x, const void *logits, int logits_dtype, int64_t T, int H, int I, int E,
                            int k, int renormalize, const int8_t *q1, const float *s1, const int8_t *q2,
                            const float *s2, int bits, int64_t group_w1, int64_t group_w2, void *workspace,
                            size_t ws_bytes, void *out, int32_t *topk_ids_out, lq_stream_t stream) {
  const hipStream_t st = as_stream(stream);
  ProfileMarks pm = take_profile(st);
  int rc = validate_layer(x, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, workspace, ws_bytes, out);
  if (rc || T == 0) return rc;
  if (!logits) return fail(LQ_ERR_VALUE, "moe_layer: null logits");
  char *ws = static_cast<char *>(workspace);
  const WsLayout w = ws_layout(T, H, I, E, k);
  int32_t *ids = topk_ids_out ? topk_ids_out : reinterpret_cast<int32_t *>(ws + w.ids);
  float *weights = reinterpret_cast<float *>(ws + w.weights);
  pm.mark(0);
  rc = launch_route_topk(logits, logits_dtype, T, E, k, renormalize, ids, weights, st);
  if (rc) return rc;
  pm.mark(1);
  return moe_forward_impl(x, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, ids, weights, ws, out, st,
                          pm, 2);
}
