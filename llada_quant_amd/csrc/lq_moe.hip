// lq_moe.hip -- the quantized MoE expert layer on gfx950.
//
// Replaces dequantize_tensor (runtime/moe.py:199-216) feeding the external
// fused_moe (INFERENCE_REPO_CHANGES.md:37-63, 259-265, 296-309): packed
// INT4/INT8 expert weights are read straight from HBM, unpacked in registers
// and fed to v_mfma_f32_16x16x32_bf16; no BF16 copy of a weight is written.
//
// One forward is a few launches on one stream, with no host synchronisation:
//
//   plan     (one workgroup) stable counting sort of the T*k assignments by
//            expert, and the work list of the layer:
//              G1 items  (expert, 64-feature slice, block of <= 32 rows)
//              G2 items  (expert, 128-row output slice, block of <= 32 rows)
//   G1       (persistent, items in ticket order)
//              act[p, f] = swiglu(x[t(p)] . W1[e]^T)      p = sorted row
//   G2       (persistent, items in ticket order)
//              y[a, h]   = w[a] * (act[p] . W2[e]^T)      a = assignment
//   combine  out[t, h] = bf16(sum_j y[t*k + j, h])        j ascending
// The phases communicate through the stream order only: a dependency inside
// one launch would need an agent-scope release/acquire per item, and on a
// multi-XCD device those write back / invalidate a whole L2 each time.
//
// Workgroup: 4 compute waves + 1 staging wave.  The staging wave copies the
// token rows of the current 128-wide K chunk into LDS (double buffered, one
// barrier per chunk); each compute wave owns two 16-row weight tiles (G1: the
// gate and up rows of the same 16 features, so SwiGLU is lane-local; G2: 32
// output rows) over the full K and keeps kDepth chunks of its packed weights
// in flight in registers.  The staging loads sit in another wave's memory
// counter, so waiting for them never drains the weight prefetch.
//
// Weight arithmetic (per 128-wide K chunk, lane group g holds K [32g, 32g+32)):
//   default: B = bf16_rne(fp32(q) * s), computed as fma(q + 2^(b-1), s,
//     -2^(b-1) s) (one rounding, as fp32(q) * s) then RNE to bf16 -- the
//     reference's dequantized BF16 weight bit for bit, for any group length
//     % 32 == 0.  The layer is then the reference's dequantize-then-matmul up
//     to the fp32 summation order.
//   folded (LQ_MOE_FOLDED_SCALES): B = bf16(q + c), an exact small integer
//     (INT4: c = 136, one AND-OR per two values; INT8: c = 128); the chunk's
//     MFMA sum S = sum x*(q + c) and X = sum x (an MFMA against ones) give
//     sum x*q = S - c X, scaled in fp32 by the group scale: the products use
//     q * s without rounding each weight to bf16, which moves the output by
//     about the reference tolerance (mean-relative ~5e-3), so it is opt-in.
// Both feed the same K order to A and B: within each 8-value MFMA slot the K
// order is [0,4,1,5,2,6,3,7]; the staging wave permutes the token rows to
// match.
#include <mutex>
#include <type_traits>

#include "lq_common.h"
#include "lq_route.h"

namespace lq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
// a plain vector type (not HIP's uint4 struct) so staged copies stay in registers
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsMax = 32;                    // token rows per item (2 row tiles)
constexpr int kKC = 128;                        // K per pipeline chunk
constexpr int kRowBytes = kKC * 2;              // one staged row of a chunk (bf16)

// LDS slot of 16-byte piece p of staged row r: p ^ lds_swizzle(r).  The mask
// is linear in the row's low four bits.  An MFMA A-fragment read (lane
// 16*lg + lc takes row 16*rt + lc, piece 4*lg + s) then hits no LDS bank
// twice in one pass: on MI355X, timing every linear mask of 4 bits for that
// read put this one among the fastest, 1.7x faster than the plain r & 15,
// whose reads conflict two ways.  Staging writes cost the same either way.
__device__ __forceinline__ int lds_swizzle(int r) {
  return static_cast<int>((0x59a659a63fc03fc0ull >> (4 * (r & 15))) & 15);
}
constexpr int kStageBytes = kRowsMax * kRowBytes;  // one LDS stage
constexpr int kStages = 2;                      // LDS stages (double buffer)
constexpr int kF1 = 64;                         // G1 features per item (128 weight rows)
constexpr int kR2 = 128;                        // G2 output rows per item
constexpr int kCombineBlock = 256;             // combine: threads per workgroup

// 128-wide K chunks of weights in flight per wave: 8 KB per wave either way
// (INT4: 2 tiles x 1 KB per chunk; INT8: 2 tiles x 2 KB)
template <int BITS>
constexpr int depth_for() {
  return BITS == 4 ? 4 : 2;
}

struct alignas(16) PlanHeader {
  int32_t n_blk;  // row blocks in the block table
  int32_t pad[3];
};

struct MoeArgs {
  const uint16_t *x;       // [T, H] bf16
  const uint16_t *xperm;   // [T, H] bf16, K slots permuted (kslot)
  const int8_t *q1;        // [E, 2I, H] int8 or [E, 2I, H/2] packed
  const float *s1;         // [E, 2I, ng1]
  const int8_t *q2;        // [E, H, I] or [E, H, I/2]
  const float *s2;         // [E, H, ng2]
  const int32_t *ids;      // [T*k]
  const float *topk_w;     // [T*k]
  const int32_t *offsets;  // [E+1]
  const int32_t *sorted;   // [T*k] assignment ids by expert
  const int32_t *srow;     // [T*k] token of each sorted row (sorted / k)
  const int4 *blocks;      // row blocks {expert, first sorted row, rows, 0}
  const PlanHeader *hdr;
  int4 *slotplan;          // streaming, in-kernel plan: per CU slot {expert, first row, rows, i << 16 | m}
  int32_t *slotasg;        // ... and the assignment of each of its block's rows [slot][kRowsMax]
  uint16_t *act;           // [T*k, I] bf16, by sorted row
  float *ybuf;             // QuantLinear: [M*ksplit, N] fp32 K-slice partial sums (MoE layers: unused)
  uint16_t *ybf;           // MoE layers: [T*k, H] bf16 slot outputs by assignment (QuantLinear: nullptr)
  uint16_t *out;           // [T, H] bf16
  int64_t T;
  int H, I, E, k;
  int g1, ng1, g2, ng2;    // group length and groups per row of w1 / w2
  int ksplit;              // general G2 only: K slices per item (partial sums to ybuf slot asg * ksplit + ks)
  // fused layer kernel only
  const void *logits;      // [T, E] router logits (dtype ldt), or nullptr: ids / topk_w are inputs
  int ldt, renorm;
  int32_t *ids_out;        // routed ids / weights written back (logits != nullptr); ids_out may be nullptr
  float *w_out;
  int32_t *g1_done;        // per row block: GEMM1 tiles finished           } zero on entry,
  int32_t *g1_seen;        // per row block: workgroups that saw them all   } zero again on exit
  int32_t *bar;            // [0] arrived at / [1] left the barrier before the combine, [2] tokens routed
  uint32_t *status;        // sticky error bits (kStatus*), or nullptr
};

// status bits a kernel sets when a bounded wait gives up (its output is then
// not to be trusted); the host reads them with lq_moe_status
constexpr uint32_t kStatusHandOver = 1u;   // a wave's hand-over of partial sums inside a workgroup
constexpr uint32_t kStatusGemm1Wait = 2u;  // GEMM2 waiting for the GEMM1 tiles of its row block
constexpr uint32_t kStatusGridWait = 4u;   // the fused kernel's barrier before the combine
constexpr uint32_t kStatusRouteWait = 8u;  // the fused kernel waiting for the routing of every token

// ---------------------------------------------------------------------------
// weights -> MFMA B fragments (8 bf16 in K slot order [0,4,1,5,2,6,3,7])
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t cvt2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){lo, hi}, bf16x2));
}

// SwiGLU of gate / up values that are already bf16 (held as floats), in
// the reference op order (INFERENCE_REPO_CHANGES.md:296-309): silu in fp32,
// rounded to bf16, times up, rounded to bf16.  exp and the reciprocal are
// the hardware's (v_exp_f32, v_rcp_f32), so silu is within two fp32 ulps of
// g / (1 + e^-g) before its rounding; both GEMM families use these, so
// they agree bit for bit.
__device__ __forceinline__ float silu_f32(float gb) { return gb * __builtin_amdgcn_rcpf(1.0f + __expf(-gb)); }
// two features at once: g0/u0 -> low half, g1/u1 -> high half
__device__ __forceinline__ uint32_t swiglu_pk(float g0, float g1, float u0, float u1) {
  const uint32_t sb = cvt2(silu_f32(g0), silu_f32(g1));
  return cvt2(__uint_as_float(sb << 16) * u0, __uint_as_float(sb & 0xFFFF0000u) * u1);
}

// INT4 folded: 8 nibbles of w -> bf16(128 + (q + 8)) = 136 + q, exact; (q ^ 8) is q + 8
__device__ __forceinline__ uint4 b_int4_folded(uint32_t w) {
  const uint32_t v = w ^ 0x88888888u;
  uint4 r;
  r.x = (v & 0x000F000Fu) | 0x43004300u;
  r.y = ((v >> 4) & 0x000F000Fu) | 0x43004300u;
  r.z = ((v >> 8) & 0x000F000Fu) | 0x43004300u;
  r.w = ((v >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// weights of one lane's 8 K slots -> B fragment dwords (e0,e4) (e1,e5) (e2,e6) (e3,e7)
__device__ __forceinline__ uint4 pack_kslots(const float (&e)[8]) {
  return make_uint4(cvt2(e[0], e[4]), cvt2(e[1], e[5]), cvt2(e[2], e[6]), cvt2(e[3], e[7]));
}

// INT4 exact: bf16_rne(fp32(q) * s) (dq_int4x8; FAST needs dq_fast_ok(s))
template <bool FAST>
__device__ __forceinline__ uint4 b_int4_exact(uint32_t w, float s, const DqScale &d) {
  float e[8];
  if constexpr (FAST)
    dq_int4x8(w, d, e);
  else
    dq_slow_int4x8(w, s, e);
  return pack_kslots(e);
}

__device__ __forceinline__ uint4 b_int8_folded(uint32_t d0, uint32_t d1) {
  const uint32_t u = d0 ^ 0x80808080u, v = d1 ^ 0x80808080u;  // q + 128
  return make_uint4(cvt2(static_cast<float>(u & 0xFF), static_cast<float>(v & 0xFF)),
                    cvt2(static_cast<float>((u >> 8) & 0xFF), static_cast<float>((v >> 8) & 0xFF)),
                    cvt2(static_cast<float>((u >> 16) & 0xFF), static_cast<float>((v >> 16) & 0xFF)),
                    cvt2(static_cast<float>(u >> 24), static_cast<float>(v >> 24)));
}

// INT8 exact: elements 0-3 in d0, 4-7 in d1
template <bool FAST>
__device__ __forceinline__ uint4 b_int8_exact(uint32_t d0, uint32_t d1, float s, const DqScale &d) {
  float lo[4], hi[4];
  if constexpr (FAST) {
    dq_int8x4(d0, d, lo);
    dq_int8x4(d1, d, hi);
  } else {
    dq_slow_int8x4(d0, s, lo);
    dq_slow_int8x4(d1, s, hi);
  }
  return make_uint4(cvt2(lo[0], hi[0]), cvt2(lo[1], hi[1]), cvt2(lo[2], hi[2]), cvt2(lo[3], hi[3]));
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// cache-policy operand of the raw buffer loads / stores: sc1 (agent scope) --
// a load misses stale lines of this XCD's L2, a store writes through to the
// agent's point of coherence
constexpr int kCpolSc1 = 16;

// raw buffer resource over [base, base + bytes) (gfx9 descriptor word 3);
// loads at offsets >= bytes return zeros and touch no memory
constexpr int kOutOfRange = 0x7FFFFFF0;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           static_cast<int>(bytes < kOutOfRange ? bytes : kOutOfRange), 0x00020000);
}


__device__ __forceinline__ float bf16_round(float v) {
  return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(v)) << 16);
}

// packed weight bytes of one lane for one 128-wide K chunk of one tile
template <int BITS>
struct WChunk;
template <>
struct WChunk<4> {
  uint4 v;
};
template <>
struct WChunk<8> {
  uint4 v0, v1;
};

// One 128-wide K chunk: dequantize this lane's codes of NT 16-row weight
// tiles into B fragments and multiply them with NRT 16-row tiles of token
// rows staged in LDS at `buf` (row r at buf + r * 256, its 16-byte pieces
// at slots p ^ lds_swizzle(r)).  FAST: every lane's scales pass dq_fast_ok
// (wave-uniform choice).  In the partial last chunk of a K that is not a
// multiple of 128, lanes past K hold zero codes (out-of-range loads), which
// dequantize to +0 and meet finite token values; the folded form never sees
// such a chunk (it needs group lengths that are multiples of 128).
// afrag(rt, s): this lane's A fragment (8 bf16 of row rt*16 + lc, K piece
// 4*lg + s of the chunk, K-slot order) from LDS
// AHEAD: every A fragment of the chunk is read first, so each step's MFMAs
// find theirs in registers instead of waiting on a read issued just ahead of
// them (same arithmetic in the same order; 16 * NRT more registers)
template <int BITS, bool FOLDED, bool FAST, int NRT, int NT, bool AHEAD = false, class AFrag>
__device__ __forceinline__ void chunk_mfma_f(const WChunk<BITS> (&w)[NT], const float (&sc)[NT], AFrag afrag,
                                             floatx4 (&tot)[NRT][NT]) {
  const uint4 ones4 = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);  // bf16 1.0
  floatx4 acc[NRT][NT];
  floatx4 xs[NRT];
  uint4 afr[AHEAD ? 4 : 1][NRT];
  if constexpr (AHEAD) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) afr[s][rt] = afrag(rt, s);
    __builtin_amdgcn_sched_barrier(0);
  }
  DqScale dqs[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) dqs[c] = dq_scale<BITS>(sc[c]);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint4 b[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      if constexpr (BITS == 4) {
        const uint32_t q = s == 0 ? w[c].v.x : s == 1 ? w[c].v.y : s == 2 ? w[c].v.z : w[c].v.w;
        if constexpr (FOLDED)
          b[c] = b_int4_folded(q);
        else
          b[c] = b_int4_exact<FAST>(q, sc[c], dqs[c]);
      } else {
        const uint4 &v = s < 2 ? w[c].v0 : w[c].v1;
        const uint32_t d0 = (s & 1) ? v.z : v.x;
        const uint32_t d1 = (s & 1) ? v.w : v.y;
        if constexpr (FOLDED)
          b[c] = b_int8_folded(d0, d1);
        else
          b[c] = b_int8_exact<FAST>(d0, d1, sc[c], dqs[c]);
      }
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      const uint4 af = AHEAD ? afr[AHEAD ? s : 0][rt] : afrag(rt, s);
      if constexpr (!FOLDED) {
#pragma unroll
        for (int c = 0; c < NT; ++c)
          tot[rt][c] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(b[c]), tot[rt][c], 0, 0, 0);
      } else {
        const floatx4 z = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NT; ++c)
          acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(b[c]),
                                                               s == 0 ? z : acc[rt][c], 0, 0, 0);
        xs[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(ones4), s == 0 ? z : xs[rt],
                                                         0, 0, 0);
      }
    }
  }
  if constexpr (FOLDED) {
    // sum x*q = S - bias * X, then the column's group scale
    constexpr float kBias = BITS == 4 ? 136.0f : 128.0f;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int c = 0; c < NT; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          tot[rt][c][j] = fmaf(sc[c], fmaf(-kBias, xs[rt][j], acc[rt][c][j]), tot[rt][c][j]);
  }
}

template <int BITS, bool FOLDED, bool FAST, int NRT, int NT>
__device__ __forceinline__ void chunk_mfma(const WChunk<BITS> (&w)[NT], const float (&sc)[NT],
                                           const unsigned char *buf, int lc, int lg, floatx4 (&tot)[NRT][NT]) {
  chunk_mfma_f<BITS, FOLDED, FAST, NRT, NT>(
      w, sc,
      [&](int rt, int s) __attribute__((always_inline)) {
        // row rt*16 + lc (its low 4 bits are lc), K piece 4*lg + s of this 128-wide chunk
        return *reinterpret_cast<const uint4 *>(buf + (rt * 16 + lc) * kRowBytes + 16 * ((4 * lg + s) ^ lds_swizzle(lc)));
      },
      tot);
}

// ---------------------------------------------------------------------------
// one G1 / G2 item
// ---------------------------------------------------------------------------

template <int BITS, bool FOLDED, int NRT, bool FIRST, bool G128>
__device__ __forceinline__ void gemm_item(const MoeArgs &a, int e, int slice, int row0, int rows, int ks,
                                          unsigned char *lds) {
  constexpr int kD = depth_for<BITS>();
  static_assert(kD == 2 || kD == 4, "the K loop is unrolled for depth 2 or 4");
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lc = lane & 15;
  const int lg = lane >> 4;
  const int K = FIRST ? a.H : a.I;
  // split K (G2, ksplit > 1, K / ksplit a multiple of 128): this item sums
  // chunks [c0, c0 + nk) of the full K; chunk i below is chunk c0 + i
  const int ksplit = FIRST ? 1 : a.ksplit;
  const int nk = ksplit > 1 ? K / kKC / ksplit : (K + kKC - 1) / kKC;
  const int c0 = ks * nk;

  // ---- token rows (all four waves stage them): a chunk is NRT*16 rows x 16
  // pieces of 16 bytes; wave w, lane l owns pieces w*64 + l + 256q (q < NRT):
  // row (w*64 + l + 256q) >> 4, piece c = l & 15, stored at LDS slot
  // c ^ lds_swizzle(row) of the row (conflict-free fragment reads).
  // Rows arrive already K-slot permuted (xperm, act).
  // Every load below is a raw buffer load.  The per-lane byte offset is
  // fixed for the item; the chunk's offset rides in the wave-uniform soffset.
  // Steps past the last chunk load through an empty descriptor (size 0),
  // which the hardware answers with zeros without touching memory, so the K
  // loop issues the same loads in every step (straight-line code: the
  // compiler counts the loads in flight exactly) and never reads outside its
  // operands.  Only the partial last chunk of a K that is not a multiple of
  // 128 takes per-lane offsets (ktail).
  const bool ktail = ksplit == 1 && (K % kKC) != 0;
  const __amdgpu_buffer_rsrc_t arsrc = make_rsrc(FIRST ? static_cast<const void *>(a.xperm) : a.act,
                                                 FIRST ? a.T * a.H * 2 : a.T * a.k * a.I * 2);
  int avoff[NRT];    // byte offset of each owned row piece in chunk 0 (row 0 for padding rows)
  int avoff_t[NRT];  // the same for the partial last chunk, clamped into the row
  int ldsoff[NRT];   // byte offset of each owned piece within a stage
#pragma unroll
  for (int q = 0; q < NRT; ++q) {
    const int piece = wave * 64 + lane + 256 * q;
    const int r = piece >> 4;
    const int rr = r < rows ? r : 0;
    const int rowelem = FIRST ? a.srow[row0 + rr] * a.H : (row0 + rr) * a.I;
    avoff[q] = 2 * (rowelem + 8 * (lane & 15));
    // lanes past the row end read its last 8 values (finite; their B is zero)
    avoff_t[q] = 2 * (rowelem + min(8 * (lane & 15), K - 8 - (nk - 1) * kKC));
    ldsoff[q] = r * kRowBytes + 16 * ((lane & 15) ^ lds_swizzle(r));
  }
  const __amdgpu_buffer_rsrc_t empty = make_rsrc(a.out, 0);
  auto load_a = [&](int i, u32x4(&v)[NRT]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = i < nk ? arsrc : empty;
    const bool tail = ktail && i == nk - 1;
#pragma unroll
    for (int q = 0; q < NRT; ++q)
      v[q] = __builtin_amdgcn_raw_buffer_load_b128(r, tail ? avoff_t[q] : avoff[q], (c0 + i) * kKC * 2, 0);
  };
  auto store_a = [&](int i, const u32x4(&v)[NRT]) __attribute__((always_inline)) {
    unsigned char *buf = lds + (i % kStages) * kStageBytes;
#pragma unroll
    for (int q = 0; q < NRT; ++q) *reinterpret_cast<u32x4 *>(buf + ldsoff[q]) = v[q];
  };

  // ---- weights: wave w owns two 16-row tiles
  const int rowbytes = BITS == 4 ? (K >> 1) : K;
  const int G = FIRST ? a.g1 : a.g2;
  const int ng = FIRST ? a.ng1 : a.ng2;
  const int nrows_w = FIRST ? 2 * a.I : a.H;
  const __amdgpu_buffer_rsrc_t wrsrc =
      make_rsrc((FIRST ? a.q1 : a.q2) + static_cast<int64_t>(e) * nrows_w * rowbytes,
                static_cast<int64_t>(nrows_w) * rowbytes);
  const __amdgpu_buffer_rsrc_t srsrc = make_rsrc((FIRST ? a.s1 : a.s2) + static_cast<int64_t>(e) * nrows_w * ng,
                                                 static_cast<int64_t>(nrows_w) * ng * 4);
  int wr[2];
  if (FIRST) {
    wr[0] = slice * kF1 + 16 * wave + lc;        // gate row
    wr[1] = a.I + slice * kF1 + 16 * wave + lc;  // up row of the same feature
  } else {
    wr[0] = slice * kR2 + 32 * wave + lc;
    wr[1] = wr[0] + 16;
  }
  constexpr int kLaneBytes = BITS == 4 ? 16 : 32;  // one lane's 32 codes of a chunk
  constexpr int kChunkBytes = BITS == 4 ? 64 : 128;
  // lanes whose 32 K values of the partial last chunk lie past K read zeros
  const bool lane_in_tail = (nk - 1) * kKC + 32 * lg < K;
  int wvoff[2], wvoff_t[2], svoff[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    wvoff[c] = wr[c] * rowbytes + kLaneBytes * lg;
    wvoff_t[c] = lane_in_tail ? wvoff[c] : kOutOfRange;
    svoff[c] = wr[c] * ng * 4;
  }

  auto load_w = [&](int i, WChunk<BITS>(&w)[2], float(&sc)[2]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rw = i < nk ? wrsrc : empty;
    const __amdgpu_buffer_rsrc_t rs = i < nk ? srsrc : empty;
    const bool tail = ktail && i == nk - 1;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int vo = tail ? wvoff_t[c] : wvoff[c];
      if constexpr (BITS == 4) {
        w[c].v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo, (c0 + i) * kChunkBytes, 0));
      } else {
        w[c].v0 =
            __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo, (c0 + i) * kChunkBytes, 0));
        w[c].v1 =
            __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo + 16, (c0 + i) * kChunkBytes, 0));
      }
      if constexpr (G128) {
        sc[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, svoff[c], (c0 + i) * 4, 0));
      } else {
        // group of this lane's K values (FOLDED: of the chunk, G % 128 == 0)
        const int sidx = (FOLDED ? (c0 + i) * kKC : min((c0 + i) * kKC + 32 * lg, K - 1)) / G;
        sc[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, svoff[c] + 4 * sidx, 0, 0));
      }
    }
  };

  floatx4 tot[NRT][2];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int c = 0; c < 2; ++c) tot[rt][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int i, const WChunk<BITS>(&w)[2], const float(&sc)[2]) __attribute__((always_inline)) {
    const unsigned char *buf = lds + (i % kStages) * kStageBytes;
    if constexpr (FOLDED) {
      chunk_mfma<BITS, FOLDED, true, NRT, 2>(w, sc, buf, lc, lg, tot);
    } else {
      if (__all(dq_fast_ok(sc[0]) && dq_fast_ok(sc[1])))
        chunk_mfma<BITS, FOLDED, true, NRT, 2>(w, sc, buf, lc, lg, tot);
      else
        chunk_mfma<BITS, FOLDED, false, NRT, 2>(w, sc, buf, lc, lg, tot);
    }
  };

  // Prefetch schedule.  Every vector load of a wave completes in issue order
  // (one vmcnt counter), so waiting for a token chunk also waits for every
  // weight load issued before it.  Token chunk i+1 (stored to LDS in step i)
  // is therefore issued together with, and just before, weight chunk i
  // (consumed in step i): kD steps ahead, in the register slot that step i
  // frees.  Waiting for either never drains the kD - 1 younger weight chunks.
  //   step i: compute chunk i (weights slot i % kD, tokens LDS stage i % 2);
  //           tokens i+1: slot -> LDS stage (i+1) % 2; issue tokens i+1+kD
  //           into that slot; issue weights i+kD into slot i % kD; barrier.
  WChunk<BITS> wb[kD][2];
  float sb[kD][2];
  u32x4 av[kD][NRT];
  // The prologue is kD load-only steps -kD .. -1 issuing exactly what a
  // steady step issues, in the same order (tokens j+1+kD, weights j+kD), so
  // every load has the same number of younger loads behind it in the first
  // loop iteration as in later ones: the compiler's wait counts (one per
  // instruction, valid on every path into the loop) then never drain the
  // prefetch.
  // (sched_barrier keeps the machine scheduler from regrouping the loads.)
  load_a(0, av[0]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = -kD; j < 0; ++j) {
    if (j == -1) store_a(0, av[0]);
    load_a(j + 1 + kD, av[(j + 1 + kD) % kD]);
    __builtin_amdgcn_sched_barrier(0);
    load_w(j + kD, wb[(j + kD) % kD], sb[(j + kD) % kD]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // chunk 0 staged

  // One step per chunk, kD steps per loop iteration (static register slots).
  // Steps past the last chunk (nk % kD != 0) compute nothing; their loads
  // are out of range.  The branches below contain no loads.
  auto step = [&](int i, auto d_tag) __attribute__((always_inline)) {
    constexpr int d = decltype(d_tag)::value;
    constexpr int dn = (d + 1) % kD;
    if (i < nk) compute(i, wb[d], sb[d]);
    __builtin_amdgcn_sched_barrier(0);
    store_a(i + 1, av[dn]);
    load_a(i + 1 + kD, av[dn]);
    __builtin_amdgcn_sched_barrier(0);
    load_w(i + kD, wb[d], sb[d]);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();  // chunk i consumed by every wave, chunk i + 1 staged
  };
  for (int i0 = 0; i0 < nk; i0 += kD) {
    step(i0 + 0, std::integral_constant<int, 0>{});
    step(i0 + 1, std::integral_constant<int, 1>{});
    if constexpr (kD > 2) {
      step(i0 + 2, std::integral_constant<int, 2>{});
      step(i0 + 3, std::integral_constant<int, 3>{});
    }
  }

  if constexpr (FIRST) {
    // reference op order (INFERENCE_REPO_CHANGES.md:296-309): g, u -> bf16;
    // silu in fp32 -> bf16; bf16 product.  act is stored K-slot permuted for
    // the G2 items that stage it.
    const int f = kslot(slice * kF1 + 16 * wave + lc);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = rt * 16 + 4 * lg + j;
        if (m < rows) {
          const float gb = bf16_round(tot[rt][0][j]);
          const float ub = bf16_round(tot[rt][1][j]);
          a.act[static_cast<int64_t>(row0 + m) * a.I + f] = static_cast<uint16_t>(swiglu_pk(gb, 0.0f, ub, 0.0f));
        }
      }
  } else {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = rt * 16 + 4 * lg + j;
        if (m < rows) {
          const int asg = a.sorted[row0 + m];
          const float wt = a.topk_w[asg];
          if (a.ybf) {  // MoE slot output, rounded to bf16 (ksplit is 1)
            uint16_t *yrow = a.ybf + static_cast<int64_t>(asg) * a.H;
            yrow[wr[0]] = static_cast<uint16_t>(cvt2(tot[rt][0][j] * wt, 0.0f));
            yrow[wr[1]] = static_cast<uint16_t>(cvt2(tot[rt][1][j] * wt, 0.0f));
          } else {
            float *yrow = a.ybuf + (static_cast<int64_t>(asg) * ksplit + ks) * a.H;
            yrow[wr[0]] = tot[rt][0][j] * wt;
            yrow[wr[1]] = tot[rt][1][j] * wt;
          }
        }
      }
  }
}

template <int BITS, bool FOLDED, bool FIRST, bool G128>
__device__ __forceinline__ void gemm_dispatch(const MoeArgs &a, int e, int slice, int row0, int rows, int ks,
                                              unsigned char *lds) {
  if (rows <= 16)
    gemm_item<BITS, FOLDED, 1, FIRST, G128>(a, e, slice, row0, rows, ks, lds);
  else
    gemm_item<BITS, FOLDED, 2, FIRST, G128>(a, e, slice, row0, rows, ks, lds);
}

// out[t, h..h+V) = bf16(sum_j y[t*k + j, h..h+V)) over the routed slots, j
// ascending, summed in fp32.  BF: the slot outputs are bf16 (MoE layers),
// V = 8 outputs per thread (one 16-byte load per slot); else fp32
// (QuantLinear's K-slice partial sums), V = 2.  The slot ids and slot
// outputs of a run of 8 slots are loaded together -- one memory round trip --
// and the outputs of slots whose id is out of range (never written) are left
// out of the sum.
template <bool BF>
__global__ __launch_bounds__(kCombineBlock) void combine_kernel(const void *__restrict__ ybuf,
                                                                const int32_t *__restrict__ ids, int64_t T,
                                                                int H, int k, int E, uint16_t *__restrict__ out) {
  constexpr int V = BF ? 8 : 2;
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kCombineBlock + threadIdx.x) * V;
  if (base >= T * H) return;  // H % V == 0 (H % 128 == 0), so a thread's outputs share one row
  const int64_t t = base / H;
  const int h = static_cast<int>(base - t * H);
  const int32_t *idr = ids + t * k;
  const int64_t y0 = t * k * H + h;  // element offset of slot 0's outputs
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  for (int j0 = 0; j0 < k; j0 += 8) {
    int id[8];
    float y[8][V];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = j0 + jj < k ? j0 + jj : k - 1;
      id[jj] = idr[j];
      const int64_t off = y0 + static_cast<int64_t>(j) * H;
      if constexpr (BF) {
        const uint4 p = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(ybuf) + off);
        const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          y[jj][2 * q] = __uint_as_float(w[q] << 16);
          y[jj][2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
        }
      } else {
        const float2 p = *reinterpret_cast<const float2 *>(static_cast<const float *>(ybuf) + off);
        y[jj][0] = p.x;
        y[jj][1] = p.y;
      }
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if (j0 + jj < k && id[jj] >= 0 && id[jj] < E) {
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] += y[jj][v];
      }
    }
  }
  uint32_t o[V / 2];
#pragma unroll
  for (int q = 0; q < V / 2; ++q)
    o[q] = static_cast<uint32_t>(f32_to_bf16_bits(acc[2 * q])) |
           (static_cast<uint32_t>(f32_to_bf16_bits(acc[2 * q + 1])) << 16);
  if constexpr (BF)
    *reinterpret_cast<uint4 *>(out + base) = make_uint4(o[0], o[1], o[2], o[3]);
  else
    *reinterpret_cast<uint32_t *>(out + base) = o[0];
}

// Persistent G1 (FIRST) or G2 kernel.  Items are (row block, slice) pairs,
// block-major: item t is slice t % per of block t / per.  The list is cut
// into 8 contiguous ranges, one per XCD (workgroup g runs on XCD g % 8), so
// the slices of one row block -- which stage the same token rows -- and the
// row blocks of one expert -- which read the same weights at about the same
// time -- meet in one L2.  Workgroups of an XCD take its items round-robin;
// the grid is a multiple of 8.  G128: the group length along K is 128 (the
// scale of a chunk is its group), else any multiple of 32.
template <int BITS, bool FOLDED, bool FIRST, bool G128>
__global__ __launch_bounds__(kThreads, 3) void moe_gemm_kernel(MoeArgs a) {
  __shared__ __align__(16) unsigned char lds[kStages * kStageBytes];
  const int nb = __builtin_amdgcn_readfirstlane(a.hdr->n_blk);
  const int ksplit = FIRST ? 1 : a.ksplit;
  const int per = (FIRST ? a.I / kF1 : a.H / kR2) * ksplit;  // items per block: slices x K slices
  const int n = nb * per;
  const int xcd = blockIdx.x & 7;
  const int gx = gridDim.x >> 3;
  const int n8 = (n + 7) >> 3;
  const int end = min(n, (xcd + 1) * n8);
  // every value below is wave-uniform (scalar): the item body contains barriers
  for (int t = xcd * n8 + static_cast<int>(blockIdx.x >> 3); t < end; t += gx) {
    const int blk = t / per;
    const int rem = t - blk * per;
    const int slice = rem / ksplit;
    const int ks = rem - slice * ksplit;
    const int4 bi = a.blocks[blk];
    const int e = __builtin_amdgcn_readfirstlane(bi.x);
    const int row0 = __builtin_amdgcn_readfirstlane(bi.y);
    const int rows = __builtin_amdgcn_readfirstlane(bi.z);
    gemm_dispatch<BITS, FOLDED, FIRST, G128>(a, e, slice, row0, rows, ks, lds);
  }
}

// ---------------------------------------------------------------------------
// wide G1 / G2 kernels (the matrix-core regime: hundreds of rows per expert)
//
// An item is (row block of up to 128 sorted rows of one expert, slice of
// weight rows).  Eight waves, two per SIMD, so one wave's weight arithmetic
// runs while the other's MFMAs do; wave w owns two 16-row weight tiles over
// the whole K -- G1: the gate and up rows of features [16w, 16w + 16) of
// the slice (128 features per item), so SwiGLU stays lane-local; G2: output
// rows [32w, 32w + 32) of the slice (256 per item) -- and multiplies each
// dequantized B fragment with up to 8 row tiles staged in LDS.  One
// dequantization then feeds 128 rows instead of 32, which keeps the weight
// arithmetic (17 VALU per 8 weights, 4 cycles each) below the matrix-core
// time of the fragment (8 x v_mfma_f32_16x16x32_bf16, 16 cycles each).
// Token rows are staged one 128-wide K chunk at a time by all 512 threads
// (double buffered, 32 KB per stage, one barrier per chunk), one chunk
// ahead; weight codes are loaded two chunks ahead into registers.  The
// per-chunk arithmetic and its order are chunk_mfma's (wide_chunk), as in
// the other GEMM families, so all of them agree bit for bit.
// Items are cut into 8 contiguous ranges, one per XCD, block-major: the
// slices of one block (the same token rows) and the blocks of one expert
// (the same weights) run at about the same time on one L2.
// ---------------------------------------------------------------------------
constexpr int kWWaves = 8;
constexpr int kWThreads = 64 * kWWaves;
constexpr int kWRows = 128;                  // sorted rows per wide row block
constexpr int kWT = 2;                       // weight tiles per wave
constexpr int kWF1 = kWWaves * 16 * kWT / 2;  // G1 features per item (gate + up tiles)
constexpr int kWR2 = kWWaves * 16 * kWT;      // G2 output rows per item
constexpr int kWStage = kWRows * kRowBytes;  // one LDS stage: 128 rows x 128 K bf16

// One 128-wide K chunk of the wide kernels: chunk_mfma's arithmetic in
// chunk_mfma's order, software-pipelined for one wave per SIMD.  The four
// 32-wide K steps s run with the A fragments of step s + 1 read from LDS
// and the B fragments of step s + 1 dequantized while the MFMAs of step s
// execute (two register sets, ping-pong), so neither the LDS latency nor the
// weight arithmetic stalls the matrix core; sched_group_barrier interleaves
// one MFMA with a share of the reads and VALU work.
template <int BITS, bool FAST, int NRT, int NT>
__device__ __forceinline__ void wide_chunk(const WChunk<BITS> (&w)[NT], const float (&sc)[NT],
                                           const unsigned char *buf, int lc, int lg, floatx4 (&tot)[NRT][NT]) {
  DqScale dqs[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) dqs[c] = dq_scale<BITS>(sc[c]);
  auto bfrag = [&](int s, uint4(&b)[NT]) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      if constexpr (BITS == 4) {
        const uint32_t q = s == 0 ? w[c].v.x : s == 1 ? w[c].v.y : s == 2 ? w[c].v.z : w[c].v.w;
        b[c] = b_int4_exact<FAST>(q, sc[c], dqs[c]);
      } else {
        const uint4 &v = s < 2 ? w[c].v0 : w[c].v1;
        b[c] = b_int8_exact<FAST>((s & 1) ? v.z : v.x, (s & 1) ? v.w : v.y, sc[c], dqs[c]);
      }
    }
  };
  auto afrag = [&](int s, uint4(&a)[NRT]) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
      a[rt] = *reinterpret_cast<const uint4 *>(buf + (rt * 16 + lc) * kRowBytes + 16 * ((4 * lg + s) ^ lds_swizzle(lc)));
  };
  // VALU instructions to place after each MFMA (the dequant of one step is
  // 17 (INT4) or 18 (INT8) per tile)
  constexpr int kValuPer = (18 * NT + NRT * NT - 1) / (NRT * NT);
  auto step = [&](int s, const uint4(&ac)[NRT], const uint4(&bc)[NT], uint4(&an)[NRT], uint4(&bn)[NT])
                  __attribute__((always_inline)) {
    if (s < 3) {
      afrag(s + 1, an);
      bfrag(s + 1, bn);
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int c = 0; c < NT; ++c)
        tot[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ac[rt]), as_bf16x8(bc[c]), tot[rt][c], 0, 0, 0);
    if (s < 3) {
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);
#pragma unroll
        for (int c = 1; c < NT; ++c) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  uint4 a0[NRT], a1[NRT], b0[NT], b1[NT];
  afrag(0, a0);
  bfrag(0, b0);
  // every step-0 A read goes out before step 0's interleaved schedule (which
  // would otherwise place them one by one just ahead of their MFMAs)
  __builtin_amdgcn_sched_barrier(0);
  step(0, a0, b0, a1, b1);
  step(1, a1, b1, a0, b0);
  step(2, a0, b0, a1, b1);
  step(3, a1, b1, a0, b0);
}

template <int BITS, int NRT, bool FIRST, bool G128>
__device__ __forceinline__ void wide_item(const MoeArgs &a, int e, int slice, int row0, int rows, int ks,
                                          unsigned char *lds, int *r_asg, float *r_wt) {
  static_assert(NRT == 2 || NRT == 4 || NRT == 8, "row tiles per block");
  constexpr int NQ = NRT * 256 / kWThreads;  // staged pieces per thread and chunk: NRT * 16 rows x 16 pieces
  constexpr int NT = kWT;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lc = lane & 15;
  const int lg = lane >> 4;
  const int K = FIRST ? a.H : a.I;
  // G2 may split K (ksplit > 1): this item sums chunks [c0, c0 + nk) of the
  // full K, nk even (host-checked), and writes its partial sums to slot
  // asg * ksplit + ks; chunk i below is chunk c0 + i
  const int ksplit = FIRST ? 1 : a.ksplit;
  const int nk = K / kKC / ksplit;  // K / ksplit is a multiple of 256 on this path (host-checked): nk is even
  const int c0 = ks * nk;

  // ---- token rows: piece tid + 512 q of a chunk is row r = piece >> 4,
  // 16-byte piece lc of the row's 128 K values, stored at slot
  // lc ^ lds_swizzle(r) (the layout chunk_mfma reads).  Rows arrive K-slot permuted (xperm,
  // act); rows past the block re-read its first row and are never stored out.
  const __amdgpu_buffer_rsrc_t arsrc = make_rsrc(FIRST ? static_cast<const void *>(a.xperm) : a.act,
                                                 FIRST ? a.T * a.H * 2 : a.T * a.k * a.I * 2);
  const __amdgpu_buffer_rsrc_t empty = make_rsrc(a.out, 0);
  int avoff[NQ], ldsoff[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int r = (tid + kWThreads * q) >> 4;
    const int rr = r < rows ? r : 0;
    const int rowelem = FIRST ? a.srow[row0 + rr] * a.H : (row0 + rr) * a.I;
    avoff[q] = 2 * (rowelem + 8 * lc);
    ldsoff[q] = r * kRowBytes + 16 * (lc ^ lds_swizzle(r));
  }
  auto load_a = [&](int i, u32x4(&v)[NQ]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = i < nk ? arsrc : empty;
#pragma unroll
    for (int q = 0; q < NQ; ++q) v[q] = __builtin_amdgcn_raw_buffer_load_b128(r, avoff[q], (c0 + i) * kKC * 2, 0);
  };
  auto store_a = [&](int i, const u32x4(&v)[NQ]) __attribute__((always_inline)) {
    unsigned char *buf = lds + (i & 1) * kWStage;
#pragma unroll
    for (int q = 0; q < NQ; ++q) *reinterpret_cast<u32x4 *>(buf + ldsoff[q]) = v[q];
  };

  // ---- weights: tile 0 holds the gate rows of the wave's 16 features
  // (G1), tile 1 the up rows of the same features; G2: output rows
  // 16c + lc of the wave's 32
  const int rowbytes = BITS == 4 ? (K >> 1) : K;
  const int G = FIRST ? a.g1 : a.g2;
  const int ng = FIRST ? a.ng1 : a.ng2;
  const int nrows_w = FIRST ? 2 * a.I : a.H;
  const __amdgpu_buffer_rsrc_t wrsrc =
      make_rsrc((FIRST ? a.q1 : a.q2) + static_cast<int64_t>(e) * nrows_w * rowbytes,
                static_cast<int64_t>(nrows_w) * rowbytes);
  const __amdgpu_buffer_rsrc_t srsrc = make_rsrc((FIRST ? a.s1 : a.s2) + static_cast<int64_t>(e) * nrows_w * ng,
                                                 static_cast<int64_t>(nrows_w) * ng * 4);
  constexpr int kLaneBytes = BITS == 4 ? 16 : 32;  // one lane's 32 codes of a chunk
  constexpr int kChunkBytes = BITS == 4 ? 64 : 128;
  const int fbase = slice * kWF1 + 16 * wave;  // G1: the wave's first feature
  const int obase = slice * kWR2 + 32 * wave;  // G2: the wave's first output row
  int wvoff[NT], svoff[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) {
    const int wr = FIRST ? (c == 0 ? 0 : a.I) + fbase + lc : obase + 16 * c + lc;
    wvoff[c] = wr * rowbytes + kLaneBytes * lg;
    svoff[c] = wr * ng * 4;
  }
  auto load_w = [&](int i, WChunk<BITS>(&w)[NT], float(&sc)[NT]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rw = i < nk ? wrsrc : empty;
    const __amdgpu_buffer_rsrc_t rs = i < nk ? srsrc : empty;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      if constexpr (BITS == 4) {
        w[c].v = __builtin_bit_cast(uint4,
                                    __builtin_amdgcn_raw_buffer_load_b128(rw, wvoff[c], (c0 + i) * kChunkBytes, 0));
      } else {
        w[c].v0 = __builtin_bit_cast(uint4,
                                     __builtin_amdgcn_raw_buffer_load_b128(rw, wvoff[c], (c0 + i) * kChunkBytes, 0));
        w[c].v1 = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wvoff[c] + 16, (c0 + i) * kChunkBytes, 0));
      }
      if constexpr (G128) {
        sc[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, svoff[c], (c0 + i) * 4, 0));
      } else {
        const int sidx = ((c0 + i) * kKC + 32 * lg) / G;  // group of this lane's 32 K values
        sc[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, svoff[c] + 4 * sidx, 0, 0));
      }
    }
  };

  floatx4 tot[NRT][NT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int c = 0; c < NT; ++c) tot[rt][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // Schedule (loads of a wave complete in issue order):
  //   first:    the item's scales, for the dequant choice (below), then
  //             tokens 0 and weights 0, which do not depend on the choice
  //   prologue: tokens 0 -> LDS stage 0; tokens 1 -> registers, weights 1
  //   step i:   compute chunk i (weights slot i & 1, LDS stage i & 1);
  //             tokens i+1: registers -> LDS stage (i+1) & 1 (waits for them only:
  //             weights i+1 were issued after them); issue tokens i+2 and
  //             weights i+2 (into slot i & 1); barrier.
  // The chunk count is even (host-checked), so the loop is straight-line;
  // the two steps past the last chunk load out of range.
  // Dequant choice: one per item and wave (FAST needs dq_fast_ok for every
  // scale the wave meets), so each K loop holds one form only.  Lane group
  // lg checks groups g0 + lg, g0 + lg + 4, ... of the item's K range in its
  // tiles' rows, up to 4 * kChk groups; longer ranges take the exact-slow
  // form throughout.
  constexpr int kChk = G128 ? 4 : 8;
  // G2: the assignment and routing weight of each row (thread r < rows),
  // fetched before the K loop and kept in LDS for the epilogue: their two
  // dependent loads overlap the item's first loads instead of following
  // the last chunk
  int asg_r = 0;
  float wt_r = 0.0f;
  if constexpr (!FIRST) {
    if (tid < rows) asg_r = a.sorted[row0 + tid];
  }
  // (the groups of this item's K range [c0, c0 + nk) chunks: [g0, g1))
  const int g0 = c0 * kKC / G, g1 = min(ng, ((c0 + nk) * kKC + G - 1) / G);
  bool ok = g1 - g0 <= 4 * kChk;
  float chk[NT][kChk];
  {
    // groups past the range read as 0 (fast) through an out-of-range offset,
    // so the descriptor stays uniform
    const __amdgpu_buffer_rsrc_t rs = ok ? srsrc : empty;
#pragma unroll
    for (int c = 0; c < NT; ++c)
#pragma unroll
      for (int j = 0; j < kChk; ++j)
        chk[c][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  rs, g0 + lg + 4 * j < g1 ? svoff[c] + 4 * (g0 + lg + 4 * j) : kOutOfRange,
                                                  0, 0));
  }
  // chunk 0's loads do not depend on the dequant form: they go out behind
  // the scale checks, so the choice waits for the checks only
  WChunk<BITS> wb[2][NT];
  float sb[2][NT];
  u32x4 av[NQ];
  if constexpr (!FIRST) {
    if (tid < rows) wt_r = a.topk_w[asg_r];
  }
  __builtin_amdgcn_sched_barrier(0);
  load_a(0, av);
  __builtin_amdgcn_sched_barrier(0);
  load_w(0, wb[0], sb[0]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < NT; ++c)
#pragma unroll
    for (int j = 0; j < kChk; ++j) ok = ok && dq_fast_ok(chk[c][j]);
  // the rest of the prologue and the K loop, one copy per dequant form
  auto kloop = [&](auto fast_tag) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast_tag)::value;
    if constexpr (!FIRST) {
      if (tid < rows) {
        r_asg[tid] = asg_r;
        r_wt[tid] = wt_r;
      }
    }
    store_a(0, av);
    load_a(1, av);
    __builtin_amdgcn_sched_barrier(0);
    load_w(1, wb[1], sb[1]);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();  // chunk 0 staged
    auto step = [&](int i, auto d_tag) __attribute__((always_inline)) {
      constexpr int d = decltype(d_tag)::value;
      wide_chunk<BITS, FAST, NRT, NT>(wb[d], sb[d], lds + (i & 1) * kWStage, lc, lg, tot);
      __builtin_amdgcn_sched_barrier(0);
      store_a(i + 1, av);
      load_a(i + 2, av);
      __builtin_amdgcn_sched_barrier(0);
      load_w(i + 2, wb[d], sb[d]);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // chunk i consumed by every wave, chunk i + 1 staged
    };
    for (int i0 = 0; i0 < nk; i0 += 2) {
      step(i0, std::integral_constant<int, 0>{});
      step(i0 + 1, std::integral_constant<int, 1>{});
    }
  };
  if (__all(ok))
    kloop(std::true_type{});
  else
    kloop(std::false_type{});

  if constexpr (FIRST) {
    // reference op order (INFERENCE_REPO_CHANGES.md:296-309): g, u -> bf16;
    // silu in fp32 -> bf16; bf16 product; act stored K-slot permuted
    const int f = kslot(fbase + lc);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = rt * 16 + 4 * lg + j;
        if (m < rows) {
          const float gb = bf16_round(tot[rt][0][j]);
          const float ub = bf16_round(tot[rt][1][j]);
          a.act[static_cast<int64_t>(row0 + m) * a.I + f] = static_cast<uint16_t>(swiglu_pk(gb, 0.0f, ub, 0.0f));
        }
      }
  } else {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = rt * 16 + 4 * lg + j;
        if (m < rows) {
          const int asg = r_asg[m];
          const float wt = r_wt[m];
          if (a.ybf) {  // MoE slot output, rounded to bf16 (ksplit is 1)
            uint16_t *yrow = a.ybf + static_cast<int64_t>(asg) * a.H + obase + lc;
#pragma unroll
            for (int c = 0; c < NT; ++c) yrow[16 * c] = static_cast<uint16_t>(cvt2(tot[rt][c][j] * wt, 0.0f));
          } else {
            float *yrow = a.ybuf + (static_cast<int64_t>(asg) * ksplit + ks) * a.H + obase + lc;
#pragma unroll
            for (int c = 0; c < NT; ++c) yrow[16 * c] = tot[rt][c][j] * wt;
          }
        }
      }
  }
}

// Persistent wide G1 (FIRST) or G2 kernel over (row block, slice) items,
// block-major, 8 contiguous ranges (one per XCD; workgroup g runs on XCD
// g % 8, the grid is a multiple of 8), taken round-robin by the XCD's
// workgroups.
template <int BITS, bool FIRST, bool G128>
__global__ __launch_bounds__(kWThreads, 1) void moe_wide_kernel(MoeArgs a) {
  static_assert(kWT == 2, "G1 pairs the gate and up tile of each wave");
  __shared__ __align__(16) unsigned char lds[2 * kWStage];
  // G2: assignment and routing weight of each row of the item, two copies
  // used by alternate items.  Item n's epilogue reads its copy after the
  // item's last barrier; item n+1 writes the other copy in its prologue, and
  // item n+2 -- the next writer of this copy -- starts only after every
  // wave has passed item n+1's barriers, so no wave overwrites rows another
  // wave still reads.
  __shared__ int r_asg[2][kWRows];
  __shared__ float r_wt[2][kWRows];
  const int nb = __builtin_amdgcn_readfirstlane(a.hdr->n_blk);
  const int ksplit = FIRST ? 1 : a.ksplit;
  const int per = (FIRST ? a.I / kWF1 : a.H / kWR2) * ksplit;  // items per block: slices x K slices
  const int n = nb * per;
  const int xcd = blockIdx.x & 7;
  const int gx = gridDim.x >> 3;
  const int n8 = (n + 7) >> 3;
  const int end = min(n, (xcd + 1) * n8);
  int parity = 0;
  for (int t = xcd * n8 + static_cast<int>(blockIdx.x >> 3); t < end; t += gx, parity ^= 1) {
    const int blk = t / per;
    const int rem = t - blk * per;
    const int slice = rem / ksplit;
    const int ks = rem - slice * ksplit;
    // a scalar load: the block table was written by an earlier launch
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    const i32x4 bi = *reinterpret_cast<const __attribute__((address_space(4))) i32x4 *>(
        reinterpret_cast<uintptr_t>(a.blocks + blk));
    const int e = __builtin_amdgcn_readfirstlane(bi.x);
    const int row0 = __builtin_amdgcn_readfirstlane(bi.y);
    const int rows = __builtin_amdgcn_readfirstlane(bi.z);
    int *ra = r_asg[parity];
    float *rw = r_wt[parity];
    if (rows <= 32)
      wide_item<BITS, 2, FIRST, G128>(a, e, slice, row0, rows, ks, lds, ra, rw);
    else if (rows <= 64)
      wide_item<BITS, 4, FIRST, G128>(a, e, slice, row0, rows, ks, lds, ra, rw);
    else
      wide_item<BITS, 8, FIRST, G128>(a, e, slice, row0, rows, ks, lds, ra, rw);
  }
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP lane moves:
// row_shr 1, 2, 4, 8 within each row of 16 lanes (lanes without a source
// add 0), then row_bcast 15 and 31 carry the row totals into later rows.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// exclusive scan of in[0..E) by wave 0 (lane l owns entries 4l..4l+3)
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

// ---------------------------------------------------------------------------
// streaming G1 / G2 kernels (the weight-bandwidth regime)
//
// One 12-wave workgroup per CU (3 waves per SIMD).  A unit is one 16-row
// weight tile of one row block over the whole K: G1 has 2I / 16 units per
// block (gate rows, then up rows), G2 H / 16.  With no more blocks than
// CUs, every block gets floor or ceil(CUs / blocks) CUs and each of them a
// contiguous, equal share of the block's units, so every CU stages one block
// and streams the same number of weight bytes (+-1 tile); with more blocks
// than CUs each CU takes a contiguous range of whole blocks.  For each block
// it handles, a CU stages the block's token rows for the whole K into LDS
// once (up to 32 rows x K bf16 = K * 64 bytes, in 128-wide chunks laid out
// as gemm_item's per-stage tiles); its waves then take the units round-robin
// and stream each as one flat sequence of 128-wide K chunks with kD chunks
// of codes and scales in flight and no barriers.
//
// G1 stores bf16(x . w) of each tile -- the gate and up pre-activations,
// rounded as the reference rounds them -- into gu [T*k, 2I] (sorted rows);
// G2's staging applies SwiGLU while it copies the rows into LDS, so gate
// and up tiles need not meet in one wave.
// ---------------------------------------------------------------------------

typedef const __attribute__((address_space(3))) unsigned char *lds_cptr;  // LDS byte pointer

constexpr int kSWaves = 12;
constexpr int kSThreads = 64 * kSWaves;

// partial accumulators one wave hands to the next (one slot per wave: its
// tile's 32 x 16 fp32 values)
constexpr int kSlotBytes = kRowsMax * 16 * 4;
// LDS bytes of the streaming kernels for reduction length K: the token rows
// of one block for the whole K, then the hand-over slots
__host__ __device__ inline size_t stream_rows_bytes(int K) { return static_cast<size_t>(K) * kRowsMax * 2; }
inline size_t stream_lds_bytes(int K) { return stream_rows_bytes(K) + static_cast<size_t>(kSWaves) * kSlotBytes; }
// upper bound of the static LDS of the streaming and fused kernels
constexpr size_t kStaticLds = 8192;


// Token rows [row0, row0 + rows) of one block, whole K, into LDS chunk tiles.
// G1 copies x into K-slot order; G2 builds act = SwiGLU(g, u) from
// the gate / up pre-activations and permutes it into K-slot order.
// A block of <= 32 rows with K <= 12 * 128 (G1) or 6 * 128 (G2) is one
// batch of loads, all in flight at once.  COH: the gate / up rows were
// written by other workgroups of the same launch, so they are read with
// agent-scope (sc1) loads, which do not hit stale lines of this XCD's L2.
template <bool FIRST, bool COH = false>
__device__ __forceinline__ void stage_block(const MoeArgs &a, int row0, int rows, const int32_t *rtok,
                                            unsigned char *lds) {
  constexpr int kCpol = COH ? kCpolSc1 : 0;
  const int K = FIRST ? a.H : a.I;
  const int nk = K / kKC;
  const int per_row = nk * 16;  // 16-byte pieces (8 values) per row
  const int total = rows * per_row;
  // q / per_row as a multiply-high (exact: q < 2^16, per_row < 2^12)
  const uint32_t magic = 0xFFFFFFFFu / static_cast<uint32_t>(per_row) + 1u;
  // G1: x [T, H] (the host keeps its bytes below 2^31); G2: the block's
  // gate / up rows [rows, 2I]
  const __amdgpu_buffer_rsrc_t src_rsrc =
      FIRST ? make_rsrc(a.x, a.T * a.H * 2)
            : make_rsrc(a.act + static_cast<int64_t>(row0) * (2 * a.I), static_cast<int64_t>(rows) * (2 * a.I) * 2);
  constexpr int kBatch = FIRST ? 12 : 6;
  auto batch = [&](int q0) __attribute__((always_inline)) {
    u32x4 v[kBatch];
    u32x4 vu[FIRST ? 1 : kBatch];
    int dst[kBatch];
    // every load is issued (pieces past the end re-read the last piece), so
    // the batch is in flight at once; only the LDS stores are guarded
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int q0i = q0 + i * kSThreads + static_cast<int>(threadIdx.x);
      const int q = q0i < total ? q0i : total - 1;
      const int r = static_cast<int>(__umulhi(static_cast<uint32_t>(q), magic));
      const int rem = q - r * per_row;
      const int c = rem >> 4, pc = rem & 15;
      const int col = 2 * (c * kKC + pc * 8);  // byte offset within the row
      if constexpr (FIRST) {
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(src_rsrc, rtok[r] * (2 * a.H) + col, 0, 0);
      } else {
        const int off = r * (4 * a.I) + col;
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(src_rsrc, off, 0, kCpol);            // gate, 8 features
        vu[i] = __builtin_amdgcn_raw_buffer_load_b128(src_rsrc, off + 2 * a.I, 0, kCpol);  // up, same features
      }
      dst[i] = q0i < total ? (c * kRowsMax + r) * kRowBytes + 16 * (pc ^ lds_swizzle(r)) : -1;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      u32x4 o = v[i];
      if constexpr (FIRST) {
        const uint4 perm = permute_kslots(make_uint4(o[0], o[1], o[2], o[3]));  // x into K-slot order
        o = u32x4{perm.x, perm.y, perm.z, perm.w};
      } else {
        // gate / up were stored as bf16, so they enter SwiGLU unrounded
        uint32_t p[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t gw = v[i][h], uw = vu[i][h];
          p[h] = swiglu_pk(__uint_as_float(gw << 16), __uint_as_float(gw & 0xFFFF0000u), __uint_as_float(uw << 16),
                           __uint_as_float(uw & 0xFFFF0000u));
        }
        const uint4 perm = permute_kslots(make_uint4(p[0], p[1], p[2], p[3]));
        o = u32x4{perm.x, perm.y, perm.z, perm.w};
      }
      if (dst[i] >= 0) *reinterpret_cast<u32x4 *>(lds + dst[i]) = o;
    }
  };
  for (int q0 = 0; q0 < total; q0 += kBatch * kSThreads) batch(q0);
}

// the steps of one run of KD chunks, unrolled (step(integral_constant<d>))
template <int KD, class Step>
__device__ __forceinline__ void run_steps(Step step) {
  step(std::integral_constant<int, 0>{});
  step(std::integral_constant<int, 1>{});
  if constexpr (KD > 2) {
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
  }
  if constexpr (KD > 4) {
    step(std::integral_constant<int, 4>{});
    step(std::integral_constant<int, 5>{});
    step(std::integral_constant<int, 6>{});
    step(std::integral_constant<int, 7>{});
  }
}

// The units [u_first, u_end) of one CU over its waves: F = nu / W full
// rounds, wave w taking units u_first + w + W i (i < F), then the T = nu % W
// left-over units.  A unit is rpu = nk / KD runs of KD chunks.  When rpu is
// even, each left-over unit t is cut in half so the waves finish together:
// wave t works its head (first rpu / 2 runs) before anything else and hands
// the partial sums over through LDS; wave (T + t) % W continues from them
// after its full rounds -- so every unit still sums its chunks in order, as
// the general kernels do, and the two families agree bit for bit.
// Otherwise wave w takes left-over unit t = w whole.  Per wave that makes up
// to three segments of runs: the head (S1), the full rounds (S2, unit
// stride W) and the left-over unit or tail (S3).
// COH (fused layer kernel): the epilogue stores are agent-scope (sc1), so
// workgroups on other XCDs can read them in the same launch, and G2 stages
// its rows with sc1 loads.  PRE: the wave's first run of codes is issued
// before the staging, then hook() runs (every thread calls it; it may hold
// barriers and the wait for the rows' producers), so the codes stream while
// the workgroup waits.  rwt: routing weight of each row (G2), else
// a.topk_w[rasg[m]].
struct NoHook {
  __device__ void operator()() const {}
};
template <int BITS, bool FOLDED, bool FIRST, int NRT, int KD, bool SQ, bool COH = false, bool PRE = false,
          class Hook = NoHook>
__device__ __forceinline__ void stream_units(const MoeArgs &a, int e, int row0, int rows, const int32_t *rtok,
                                             const int32_t *rasg, int u_first, int u_end, unsigned char *lds,
                                             Hook hook = Hook{}, const float *rwt = nullptr) {
  __shared__ int hand_flag[kSWaves];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lc = lane & 15;
  const int lg = lane >> 4;
  const int K = FIRST ? a.H : a.I;
  const int nk = K / kKC;  // a multiple of KD (host-checked), so a run never crosses a unit
  const int rpu = nk / KD;  // runs per unit
  const int nu = u_end - u_first;
  const int F = nu / kSWaves, T = nu - F * kSWaves;
  const bool split = T > 0 && rpu % 2 == 0;
  const int half = rpu / 2;
  const int ut = u_first + F * kSWaves;  // first left-over unit
  const int t3 = (wave - T + kSWaves) % kSWaves;  // split: the left-over unit whose tail this wave works
  const int n1 = split && wave < T ? half : 0;
  const int n2 = F * rpu;
  const int n3 = split ? (t3 < T ? half : 0) : (wave < T ? rpu : 0);
  const int u3 = split ? ut + t3 : ut + wave;
  const int c3 = split ? half * KD : 0;
  const int nruns = n1 + n2 + n3;
  // Move a cursor (segment index, unit, first chunk, runs left in the
  // segment, unit stride) to the first non-empty segment after `from`
  // (-1: the first one).  Explicit branches with the segments' own values:
  // a select over the segment index would become a table in private memory.
  auto enter = [&](int from, int &sg, int &u, int &c, int &n, int &stride) __attribute__((always_inline)) {
    if (from < 0 && n1 > 0) {
      sg = 0;
      u = ut + wave;
      c = 0;
      n = n1;
      stride = 1;
    } else if (from < 1 && n2 > 0) {
      sg = 1;
      u = u_first + wave;
      c = 0;
      n = n2;
      stride = kSWaves;
    } else {
      sg = 2;
      u = u3;
      c = c3;
      n = n3;
      stride = 1;
    }
  };
  const int rowbytes = BITS == 4 ? (K >> 1) : K;
  const int ng = FIRST ? a.ng1 : a.ng2;
  const int cpg = (FIRST ? a.g1 : a.g2) / kKC;  // chunks per group (group lengths are multiples of 128)
  const int nrows_w = FIRST ? 2 * a.I : a.H;
  constexpr int kLaneBytes = BITS == 4 ? 16 : 32;
  constexpr int kChunkBytes = BITS == 4 ? 64 : 128;
  constexpr int kChunkLds = kRowsMax * kRowBytes;  // one staged chunk of the block's rows
  const __amdgpu_buffer_rsrc_t wrsrc =
      make_rsrc((FIRST ? a.q1 : a.q2) + static_cast<int64_t>(e) * nrows_w * rowbytes,
                static_cast<int64_t>(nrows_w) * rowbytes);
  const __amdgpu_buffer_rsrc_t srsrc = make_rsrc((FIRST ? a.s1 : a.s2) + static_cast<int64_t>(e) * nrows_w * ng,
                                                 static_cast<int64_t>(nrows_w) * ng * 4);
  const __amdgpu_buffer_rsrc_t empty = make_rsrc(a.out, 0);
  const int wvoff = lc * rowbytes + kLaneBytes * lg;  // this lane's codes within a tile chunk
  const int svoff = lc * ng * 4;
  const int sqvoff = lc * ng * 4 + 16 * lg;           // SQ: this lane's 4 scales within a tile
  float *slots = reinterpret_cast<float *>(lds + stream_rows_bytes(K));

  // Load cursor (scalar registers), one run of KD chunks ahead of the
  // compute: the unit lu and first chunk lc0 of the run being loaded, the
  // codes offset wso of its first chunk (chunk d at wso + d * kChunkBytes,
  // an immediate offset), the unit's scale offset suo, the head runs still
  // to load (seg1; then the cursor jumps to uA / cA), and the runs left;
  // after the wave's last run both descriptors become the empty one, so
  // every step issues the same loads and the load counter stays static.
  // SQ (group length 128, at most 16 chunks): instead of one scale load per
  // chunk, lane (r, g) loads the scales of groups 4g .. 4g+3 of its tile row
  // r once per unit (one dwordx4 in the first step of a run that starts a
  // unit or follows a jump, else from the empty descriptor); the scale of
  // chunk c then comes from lane (r, c / 4) by ds_bpermute.  Otherwise every
  // chunk loads its scale (sso, lgrp: the next chunk's scale offset and its
  // position within its group).
  __amdgpu_buffer_rsrc_t rw = nruns > 0 ? wrsrc : empty, rs = nruns > 0 ? srsrc : empty;
  int lseg, lu, lc0, lseg_left, lstride;
  enter(-1, lseg, lu, lc0, lseg_left, lstride);
  int wso = 16 * lu * rowbytes + lc0 * kChunkBytes;
  int suo = 16 * lu * ng * 4;
  int sso = suo + (lc0 / cpg) * 4, lgrp = lc0 % cpg;
  int left = nruns;
  bool sq_force = true;
  u32x4 sq_cur = u32x4{0, 0, 0, 0}, sq_next = u32x4{0, 0, 0, 0};
  auto load_sq = [&](u32x4 &dst) __attribute__((always_inline)) {
    const bool go = lc0 == 0 || sq_force;
    dst = __builtin_amdgcn_raw_buffer_load_b128(go ? rs : empty, sqvoff, go ? suo : 0, 0);
    sq_force = false;
  };
  auto load_w = [&](auto d_tag, WChunk<BITS>(&w)[1], float(&sc)[1]) __attribute__((always_inline)) {
    constexpr int d = decltype(d_tag)::value;
    if constexpr (BITS == 4) {
      w[0].v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wvoff + d * kChunkBytes, wso, 0));
    } else {
      w[0].v0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wvoff + d * kChunkBytes, wso, 0));
      w[0].v1 =
          __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wvoff + d * kChunkBytes + 16, wso, 0));
    }
    if constexpr (!SQ) {
      sc[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, svoff, sso, 0));
      if (++lgrp == cpg) {
        lgrp = 0;
        sso += 4;
      }
    }
  };
  // advance the load cursor past the run just loaded
  auto next_run = [&]() __attribute__((always_inline)) {
    if (--lseg_left == 0 && lseg < 2) {
      enter(lseg, lseg, lu, lc0, lseg_left, lstride);
      wso = 16 * lu * rowbytes + lc0 * kChunkBytes;
      suo = 16 * lu * ng * 4;
      sso = suo + (lc0 / cpg) * 4;
      lgrp = lc0 % cpg;
      sq_force = true;
    } else {
      lc0 += KD;
      wso += KD * kChunkBytes;
      if (lc0 == nk) {
        lc0 = 0;
        lu += lstride;
        wso = 16 * lu * rowbytes;
        suo = 16 * lu * ng * 4;
        sso = suo;
        lgrp = 0;
      }
    }
    if (--left == 0) {
      rw = empty;
      rs = empty;
      wso = 0;
      suo = 0;
      sso = 0;
    }
  };

  floatx4 tot[NRT][1];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) tot[rt][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // epilogue targets of this lane's rows m = rt*16 + 4*lg + j (32-bit
  // element offsets: the host bounds T*k*max(2I, H)*2 below 2^31): G1 writes
  // row row0 + m of the gate / up pre-activations, G2 the slot output of
  // assignment rasg[m] scaled by its routing weight
  const int ld = FIRST ? 2 * a.I : a.H;
  int eoff[NRT][4];
  float ewt[NRT][FIRST ? 1 : 4];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = rt * 16 + 4 * lg + j;
      if constexpr (FIRST) {
        eoff[rt][j] = m < rows ? (row0 + m) * ld + lc : -1;
      } else {
        const int asg = m < rows ? rasg[m] : 0;
        eoff[rt][j] = m < rows ? asg * ld + lc : -1;
        ewt[rt][j] = m < rows ? (rwt ? rwt[m] : a.topk_w[asg]) : 0.0f;
      }
    }
  auto epilogue = [&](int u) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (eoff[rt][j] >= 0) {
          if constexpr (FIRST) {
            // gate (u < I / 16) or up pre-activation, rounded to bf16 (RNE)
            const uint16_t h = static_cast<uint16_t>(cvt2(tot[rt][0][j], 0.0f));
            if constexpr (COH)
              __hip_atomic_store(a.act + eoff[rt][j] + 16 * u, h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
              a.act[eoff[rt][j] + 16 * u] = h;
          } else {
            // slot output y * w, rounded to bf16 (the streaming kernels run MoE layers only)
            const uint16_t y = static_cast<uint16_t>(cvt2(tot[rt][0][j] * ewt[rt][j], 0.0f));
            if constexpr (COH)
              __hip_atomic_store(a.ybf + eoff[rt][j] + 16 * u, y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
              a.ybf[eoff[rt][j] + 16 * u] = y;
          }
        }
      }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) tot[rt][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  };
  // hand the head's partial sums over (slot and flag of this wave)
  auto give = [&]() __attribute__((always_inline)) {
    float *slot = slots + wave * (kSlotBytes / 4);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        slot[(rt * 4 + j) * 64 + lane] = tot[rt][0][j];
        tot[rt][0][j] = 0.0f;
      }
    __hip_atomic_store(&hand_flag[wave], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  // continue from the head wave src handed over (it works that head before
  // anything else, so the wait is short; the cap only bounds the loop, and
  // running out of it marks the call's status: the sums are then wrong)
  auto take = [&](int src) __attribute__((always_inline)) {
    bool got = false;
    for (int spin = 0; spin < (1 << 22); ++spin) {
      // (one wave-uniform decision, so the loop exit is uniform)
      const int f = __hip_atomic_load(&hand_flag[src], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (__builtin_amdgcn_readfirstlane(f) != 0) {
        got = true;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (!got && lane == 0 && a.status) atomicOr(a.status, kStatusHandOver);
    const float *slot = slots + src * (kSlotBytes / 4);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) tot[rt][0][j] = slot[(rt * 4 + j) * 64 + lane];
  };

  // KD chunks of codes in flight; step d of a run consumes slot d and
  // refills it with chunk d of the next run
  WChunk<BITS> wb[KD][1];
  float sb[KD][1];
  auto first_run = [&]() __attribute__((always_inline)) {
    if constexpr (SQ) load_sq(sq_cur);
    run_steps<KD>([&](auto d_tag) __attribute__((always_inline)) {
      constexpr int d = decltype(d_tag)::value;
      load_w(d_tag, wb[d], sb[d]);
      __builtin_amdgcn_sched_barrier(0);
    });
    next_run();
  };
  if constexpr (PRE) {
    // the first run of codes (registers only) goes out first; the hook's
    // barriers also order the previous phase's reads of the LDS rows and
    // hand-over flags before the staging below overwrites them
    if (nruns > 0) first_run();
    hook();
    if (lane == 0) hand_flag[wave] = 0;
    stage_block<FIRST, COH>(a, row0, rows, rtok, lds);
    __syncthreads();
    if (nruns == 0) return;
  } else {
    // the block's token rows, then the first run of codes
    __syncthreads();  // the previous block's rows and hand-over slots are no longer read
    if (lane == 0) hand_flag[wave] = 0;
    stage_block<FIRST, COH>(a, row0, rows, rtok, lds);
    __syncthreads();
    if (nruns == 0) return;
    // The first run's codes go out after the barrier: at the kernel's start
    // every CU asks for a run per wave at once, and a wave waits at the issue
    // of its loads until the memory system takes them -- so each wave starts
    // computing as soon as its own loads are out, instead of all waves
    // waiting for the slowest one's.
    first_run();
  }
  // SQ: whether every scale of the current unit takes the fast dequant
  // (decided per unit, so a run is all fast or all exact-slow); scale slots
  // past the row's last group are not looked at
  auto unit_fast = [&]() __attribute__((always_inline)) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 4; ++i) ok = ok && (4 * lg + i >= ng || dq_fast_ok(__uint_as_float(sq_cur[i])));
    return __all(ok) != 0;
  };
  bool fast_unit = SQ && !FOLDED ? unit_fast() : true;
  // LDS address of this lane's A fragment for K piece 4*lg + s of chunk 0,
  // row lc (the staging's lds_swizzle layout)
  const lds_cptr lbase = (lds_cptr)(lds);
  int aoff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) aoff[s] = lc * kRowBytes + 16 * ((4 * lg + s) ^ lds_swizzle(lc));
  // compute cursor: segment, unit, first chunk of the current run, runs
  // left in the segment, unit stride
  int cseg, cu, cc, cseg_left, cstride;
  enter(-1, cseg, cu, cc, cseg_left, cstride);
  if (split && cseg == 2 && cseg_left > 0) take(t3);
  for (int r = 0; r < nruns; ++r) {
    // the run's A addresses, computed once and kept opaque so every step
    // and row tile reaches its fragment through the instruction's
    // immediate offset (d * kChunkLds + rt * 16 * kRowBytes)
    lds_cptr ab[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      ab[s] = lbase + (aoff[s] + cc * kChunkLds);
      asm volatile("" : "+v"(ab[s]));
    }
    int sqa = (lc + 16 * (cc >> 2)) << 2;  // SQ: source lane of the run's first chunk, in bytes
    asm volatile("" : "+v"(sqa));
    // the fast / exact-slow choice is made per step but from a per-unit
    // flag, so both paths rejoin before the step's loads (one register
    // assignment for the codes in flight)
    run_steps<KD>([&](auto d_tag) __attribute__((always_inline)) {
      constexpr int d = decltype(d_tag)::value;
      auto afrag = [&](int rt, int s) __attribute__((always_inline)) {
        const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(
            ab[s] + (d * kChunkLds + rt * 16 * kRowBytes));
        return make_uint4(v[0], v[1], v[2], v[3]);
      };
      if constexpr (SQ) {
        // chunk cc + d (cc is a multiple of 4): component d % 4 of lane (r, (cc + d) / 4)
        sb[d][0] = __int_as_float(__builtin_amdgcn_ds_bpermute(sqa + 64 * (d >> 2), static_cast<int>(sq_cur[d & 3])));
      }
      // (the registers of the fused layer kernel and of the folded form do
      // not hold the chunk's A fragments ahead)
      if constexpr (FOLDED) {
        chunk_mfma_f<BITS, FOLDED, true, NRT, 1>(wb[d], sb[d], afrag, tot);
      } else {
        if (SQ ? fast_unit : __all(dq_fast_ok(sb[d][0])) != 0)
          chunk_mfma_f<BITS, FOLDED, true, NRT, 1, !COH>(wb[d], sb[d], afrag, tot);
        else
          chunk_mfma_f<BITS, FOLDED, false, NRT, 1, !COH>(wb[d], sb[d], afrag, tot);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (SQ) {
        if (d == 0) load_sq(sq_next);
      }
      load_w(d_tag, wb[d], sb[d]);
      __builtin_amdgcn_sched_barrier(0);
    });
    next_run();
    cc += KD;
    bool moved = false;
    if (cc == nk) {  // (a head never completes its unit)
      epilogue(cu);
      cu += cstride;
      cc = 0;
      moved = true;
    }
    if (--cseg_left == 0 && cseg < 2) {
      if (cseg == 0) give();
      enter(cseg, cseg, cu, cc, cseg_left, cstride);
      if (split && cseg == 2 && cseg_left > 0) take(t3);
      moved = true;
    }
    if constexpr (SQ) {
      if (moved) {
        sq_cur = sq_next;
        if constexpr (!FOLDED) fast_unit = unit_fast();
      }
    }
  }
}

template <int BITS, bool FOLDED, bool FIRST, int KD, bool SQ, bool COH = false, bool PRE = false,
          class Hook = NoHook>
__device__ __forceinline__ void stream_block(const MoeArgs &a, int e, int row0, int rows, const int32_t *rtok,
                                             const int32_t *rasg, int u_first, int u_end, unsigned char *lds,
                                             Hook hook = Hook{}, const float *rwt = nullptr) {
  if (rows <= 16)
    stream_units<BITS, FOLDED, FIRST, 1, KD, SQ, COH, PRE>(a, e, row0, rows, rtok, rasg, u_first, u_end, lds, hook,
                                                            rwt);
  else
    stream_units<BITS, FOLDED, FIRST, 2, KD, SQ, COH, PRE>(a, e, row0, rows, rtok, rasg, u_first, u_end, lds, hook,
                                                            rwt);
}

// Workgroup g of a grid of G runs on XCD g % 8.  Its XCD-major slot
// (g % 8) * (G / 8) + g / 8 numbers the workgroups of one XCD
// consecutively, so the CUs that share a block -- which stage the same
// token rows -- and the blocks of one expert -- which stream the same
// weights at about the same time -- meet in one L2.
__device__ __forceinline__ int xcd_slot(int g, int G) { return G % 8 ? g : (g % 8) * (G / 8) + g / 8; }

// Slot c of G and its share of nb blocks: with nb <= G, slots
// [ceil(b G / nb), ceil((b+1) G / nb)) share block b, slot c taking units
// [i upb / m, (i+1) upb / m) of it; returns false for a slot without a block
// (Wide: 64-bit products, for plan_kernel's tables of any size; the
// in-kernel plan has nb <= G <= 1024 and takes 32-bit arithmetic.)
template <typename Wide = int64_t>
__device__ __forceinline__ bool cu_share(int c, int G, int nb, int upb, int &b, int &ub, int &ue, int *im = nullptr) {
  b = static_cast<int>(static_cast<Wide>(c) * nb / G);
  if (b >= nb) return false;
  const int first = static_cast<int>((static_cast<Wide>(b) * G + nb - 1) / nb);
  const int next = static_cast<int>((static_cast<Wide>(b + 1) * G + nb - 1) / nb);
  const int m = next - first, i = c - first;
  ub = i * upb / m;
  ue = (i + 1) * upb / m;
  if (im) *im = (i << 16) | m;
  return true;
}

constexpr int kPlanMaxN = 2048;  // assignments the fused kernel plans (one workgroup)

// Small layers (T*k <= kPlanMaxN): every workgroup derives the plan of its
// own block from the T*k routed ids instead of reading plan_kernel's
// output -- the same per-expert counts and offsets, the same expert-major
// blocks of <= 32 rows, and the block's assignments in ascending flat index
// (plan_kernel's stable order), so the sorted row numbers G1 writes and G2
// reads agree.  One barrier: after the ids are counted, every wave scans the
// counts in registers, finds its block and compacts the block's assignments
// itself (all waves write the same values into rtok / rasg; the barrier that
// opens the staging orders those writes before any read).  Fills rtok / rasg
// (token and assignment of each row) and returns false when the CU has no
// block.
__device__ __forceinline__ bool block_plan(const MoeArgs &a, int upb, int &e, int &row0, int &rows, int &ub,
                                           int &ue, int &im, int32_t *rtok, int32_t *rasg) {
  __shared__ int cnt[kMaxExperts];
  __shared__ uint16_t ids_l[kPlanMaxN];  // expert of each assignment (0xFFFF: none)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int N = static_cast<int>(a.T * a.k);
  const int E = a.E;
  // the ids are read once, all in one round trip
  constexpr int kIdsPerThread = (kPlanMaxN + kSThreads - 1) / kSThreads;
  int idr[kIdsPerThread];
#pragma unroll
  for (int j = 0; j < kIdsPerThread; ++j) {
    const int i = j * kSThreads + tid;
    idr[j] = i < N ? a.ids[i] : -1;
  }
  for (int i = tid; i < E; i += kSThreads) cnt[i] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kIdsPerThread; ++j) {
    const int i = j * kSThreads + tid;
    const bool ok = idr[j] >= 0 && idr[j] < E;
    if (i < N) ids_l[i] = ok ? static_cast<uint16_t>(idr[j]) : uint16_t{0xFFFF};
    if (ok) atomicAdd(&cnt[idr[j]], 1);
  }
  __syncthreads();
  // lane l: experts 4l .. 4l+3, their rows and row blocks, and the
  // exclusive prefix of both over the lanes
  int c[4], nbk[4], csum = 0, bsum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ex = 4 * lane + i;
    c[i] = ex < E ? cnt[ex] : 0;
    nbk[i] = (c[i] + kRowsMax - 1) / kRowsMax;
    csum += c[i];
    bsum += nbk[i];
  }
  const int cinc = wave_incl_scan(csum), binc = wave_incl_scan(bsum);
  const int nb = __builtin_amdgcn_readlane(binc, 63);
  int b;
  if (!cu_share<uint32_t>(xcd_slot(blockIdx.x, gridDim.x), gridDim.x, nb, upb, b, ub, ue, &im)) return false;
  // the lane whose experts hold block b, then the expert within it
  const int bex = binc - bsum;
  const int owner = static_cast<int>(__builtin_ctzll(__ballot(bex <= b && b < binc)));
  int fe = 0, fblk = 0, foff = 0, fcnt = 0;
  int eb = bex, eo = cinc - csum;
  bool found = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (!found && b < eb + nbk[i]) {
      found = true;
      fe = 4 * lane + i;
      fblk = eb;
      foff = eo;
      fcnt = c[i];
    }
    eb += nbk[i];
    eo += c[i];
  }
  e = __builtin_amdgcn_readlane(fe, owner);
  const int first = (b - __builtin_amdgcn_readlane(fblk, owner)) * kRowsMax;  // rank of the block's first row
  rows = min(kRowsMax, __builtin_amdgcn_readlane(fcnt, owner) - first);
  row0 = __builtin_amdgcn_readlane(foff, owner) + first;
  // stable compaction of expert e's assignments, keeping ranks [first, first + rows)
  const unsigned long long lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int last = first + rows;
  // i / k by multiply-high (exact for i < 2^16; k == 1 would need 2^32)
  const uint32_t kmagic = a.k > 1 ? 0xFFFFFFFFu / static_cast<uint32_t>(a.k) + 1u : 0u;
  int run = 0;
  for (int c0 = 0; c0 < N && run < last; c0 += 256) {
    int idv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = c0 + 64 * j + lane;
      idv[j] = i < N ? ids_l[i] : 0xFFFF;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = c0 + 64 * j + lane;
      const bool hit = idv[j] == e;
      const unsigned long long bal = __ballot(hit);
      const int rank = run + __popcll(bal & lt);
      if (hit && rank >= first && rank < last) {
        rasg[rank - first] = i;
        rtok[rank - first] = a.k > 1 ? static_cast<int>(__umulhi(static_cast<uint32_t>(i), kmagic)) : i;
      }
      run += __popcll(bal);
    }
  }
  return true;
}

// PLAN: kPlanTable -- the blocks come from plan_kernel's table;
// kPlanOwn -- the workgroup plans its own block (block_plan) and records
// it in slot records for the next GEMM; kPlanSlot -- the block comes from
// the slot record the previous GEMM's workgroup of the same slot wrote
// (same grid, same plan: one load instead of a plan).
constexpr int kPlanTable = 0, kPlanOwn = 1, kPlanSlot = 2;

template <int BITS, bool FOLDED, bool FIRST, int KD, bool SQ, int PLAN>
__global__ __launch_bounds__(kSThreads, 1) void moe_stream_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char slds[];
  const int upb = FIRST ? 2 * a.I / 16 : a.H / 16;  // units (16-row tiles) per row block
  if constexpr (PLAN == kPlanOwn) {
    __shared__ int32_t rtok[kRowsMax], rasg[kRowsMax];
    const int slot = xcd_slot(blockIdx.x, gridDim.x);
    int e, row0, rows, ub, ue, im;
    if (!block_plan(a, upb, e, row0, rows, ub, ue, im, rtok, rasg)) {
      if (threadIdx.x == 0) a.slotplan[slot] = make_int4(0, 0, 0, 0);
      return;
    }
    if (threadIdx.x == 0) a.slotplan[slot] = make_int4(e, row0, rows, im);
    if (static_cast<int>(threadIdx.x) < rows) a.slotasg[slot * kRowsMax + threadIdx.x] = rasg[threadIdx.x];
    stream_block<BITS, FOLDED, FIRST, KD, SQ>(a, e, row0, rows, rtok, rasg, ub, ue, slds);
  } else if constexpr (PLAN == kPlanSlot) {
    const int slot = xcd_slot(blockIdx.x, gridDim.x);
    const int4 rec = a.slotplan[slot];
    const int rows = __builtin_amdgcn_readfirstlane(rec.z);
    if (rows == 0) return;
    const int e = __builtin_amdgcn_readfirstlane(rec.x);
    const int row0 = __builtin_amdgcn_readfirstlane(rec.y);
    const int im = __builtin_amdgcn_readfirstlane(rec.w);
    const int i = im >> 16, m = im & 0xFFFF;
    stream_block<BITS, FOLDED, FIRST, KD, SQ>(a, e, row0, rows, nullptr, a.slotasg + slot * kRowsMax,
                                              i * upb / m, (i + 1) * upb / m, slds);
  } else {
    const int nb = __builtin_amdgcn_readfirstlane(a.hdr->n_blk);
    const int G = gridDim.x, c = xcd_slot(blockIdx.x, gridDim.x);
    auto run_block = [&](int b, int ub, int ue) __attribute__((always_inline)) {
      const int4 bi = a.blocks[b];
      const int e = __builtin_amdgcn_readfirstlane(bi.x);
      const int row0 = __builtin_amdgcn_readfirstlane(bi.y);
      const int rows = __builtin_amdgcn_readfirstlane(bi.z);
      stream_block<BITS, FOLDED, FIRST, KD, SQ>(a, e, row0, rows, a.srow + row0, a.sorted + row0, ub, ue, slds);
    };
    if (nb <= G) {
      int b, ub, ue;
      if (!cu_share(c, G, nb, upb, b, ub, ue)) return;
      run_block(b, ub, ue);
    } else {
      const int b0 = static_cast<int>(static_cast<int64_t>(c) * nb / G);
      const int b1 = static_cast<int>(static_cast<int64_t>(c + 1) * nb / G);
      for (int b = b0; b < b1; ++b) run_block(b, 0, upb);
    }
  }
}

// ---------------------------------------------------------------------------
// fused layer kernel (the weight-bandwidth regime: E <= 64, T*k <= kPlanMaxN)
//
// One launch per layer: [route] -> plan -> G1 -> G2 -> combine, one 12-wave
// workgroup per CU.  With logits, workgroup t < T routes token t (the router
// kernel's arithmetic) and publishes its ids and weights; every workgroup then
// derives the whole plan (counts, blocks of <= 32 rows, stable order) in one
// wave, lane e = expert e, and takes a cost-weighted share of one row block in
// each phase (assign_share: blocks of 17..32 rows run two row tiles and get
// more CUs).  Workgroups exchange data three times:
//   routing -> plan: the ids / weights of every token; each routing wave
//     counts once on bar[2] when its stores are complete, and the plan starts
//     when the count reaches T.
//   G1 -> G2: the bf16 gate / up pre-activations of a row block, written by
//     the workgroups whose G1 share is that block and read, all of them, by
//     those whose G2 share is.  Each workgroup adds its G1 tile count to
//     g1_done[b] once its stores are complete; G2 issues its first run of W2
//     codes, then waits (bounded) for its block's count to reach 2I/16 before
//     staging the rows.
//   G2 -> combine: y of each assignment.  After a grid barrier (every
//     workgroup's G2 stores complete), workgroup c sums slice c of the
//     outputs: out[t, h] = bf16(sum_j y[t*k + j, h]) over the valid slots, j
//     ascending -- combine_kernel's arithmetic, spread evenly over the grid.
//     (Letting the last workgroup to finish a token's tiles combine it costs
//     more: a late workgroup is last for all the tokens of its rows and
//     combines them one after another.)
// Visibility across XCDs without writing back or invalidating whole L2s:
// the data goes out with agent-scope (sc1) stores, which write through to the
// point of coherence, and is read with sc1 loads, which do not hit stale L2
// lines.  Each wave waits for its stores (s_waitcnt vmcnt(0)) before the
// workgroup barrier after which one thread adds to a counter; the counters
// are agent-scope atomics.
// The counters are zero on entry and left at zero: the last of a G2 block's
// workgroups to see its G1 count (g1_seen) clears both, and the last
// workgroup to leave the barrier clears its two counts and the routing count.
// The waits need every workgroup resident at once: the grid is one
// workgroup per CU (a second one fits on a CU only for small K, and then the
// grid still fits).  A wait that runs out of its cap sets a status bit and
// goes on (wrong output, no hang).
// ---------------------------------------------------------------------------
constexpr int kFusedRouteMaxT = 64;  // routing in the fused kernel up to this many tokens (E <= 64)
constexpr int kWaitCap = 1 << 20;    // polls of a cross-workgroup wait (~1 s)

// One phase's share of this workgroup in the fused kernel: row block b (its
// index among the layer's blocks), the block's expert e and sorted rows
// [row0, row0 + rows), j the block's place among its expert's blocks, and
// the workgroup's tiles [ub, ue) of the block's upb, being the i-th of the
// block's m workgroups.
struct Share {
  int b, e, j, row0, rows, ub, ue, i, m;
};

// Cost-weighted assignment of CU slot c (of G) to a row block, for E <= 64
// with lane e = expert e holding its count cnt, block count nbk, and the
// exclusive prefixes of both.  A block weighs wlo (<= 16 rows: one row tile
// per weight tile) or whi (17..32 rows: two); the blocks, expert-major, share
// the G slots in proportion to their weights: block [S, S + w) of the total
// W covers slots [ceil(S G / W), ceil((S + w) G / W)).  Every block gets at
// least one slot when W <= wlo G (host-checked through the block count).
__device__ __forceinline__ Share assign_share(int c, int G, int cnt, int nbk, int bexcl, int cexcl, int wlo, int whi,
                                              int upb) {
  auto wrows = [&](int r) { return r > 16 ? whi : wlo; };
  const int w32 = wrows(kRowsMax);
  const int we = nbk > 0 ? (nbk - 1) * w32 + wrows(cnt - kRowsMax * (nbk - 1)) : 0;
  const int pinc = wave_incl_scan(we);
  const int W = __builtin_amdgcn_readlane(pinc, 63);
  const int pex = pinc - we;
  // the expert: the highest one with blocks whose weight starts at or before c W / G
  const uint64_t own = __ballot(nbk > 0 && pex * G <= c * W);
  Share sh;
  sh.e = 63 - __builtin_clzll(own);
  const int pe = __builtin_amdgcn_readlane(pex, sh.e);
  const int ne = __builtin_amdgcn_readlane(nbk, sh.e);
  const int ce = __builtin_amdgcn_readlane(cnt, sh.e);
  sh.j = min((c * W - pe * G) / (w32 * G), ne - 1);
  sh.rows = min(kRowsMax, ce - kRowsMax * sh.j);
  const int S = pe + sh.j * w32, S2 = S + wrows(sh.rows);
  const int first = (S * G + W - 1) / W, next = (S2 * G + W - 1) / W;
  sh.b = __builtin_amdgcn_readlane(bexcl, sh.e) + sh.j;
  sh.row0 = __builtin_amdgcn_readlane(cexcl, sh.e) + kRowsMax * sh.j;
  sh.m = next - first;
  sh.i = c - first;
  sh.ub = sh.i * upb / sh.m;
  sh.ue = (sh.i + 1) * upb / sh.m;
  return sh;
}

// cost weights of a block (<= 16 rows, 17..32 rows) per phase, measured on
// MI355X at C4: GEMM1's two-row-tile blocks take ~1.1x as long, GEMM2's
// ~1.8x (its K is half as long, so the per-row costs of staging the SwiGLU
// rows and of the row tiles' MFMAs weigh more)
constexpr int kW1Lo = 10, kW1Hi = 11, kW2Lo = 5, kW2Hi = 9;

// One wave: the assignments of expert e with ranks [first, first + rows) among
// its assignments in ascending flat index, from ids_l (the expert of each of
// the N assignments, 0xFFFF for none): token -> tok[r], assignment -> asg[r]
// (either may be null).
__device__ __forceinline__ void compact_rows(const uint16_t *ids_l, int N, int k, int e, int first, int rows,
                                             int32_t *tok, int32_t *asg) {
  const int lane = threadIdx.x & 63;
  const unsigned long long lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int last = first + rows;
  int run = 0;
  for (int c0 = 0; c0 < N && run < last; c0 += 64) {
    const int i = c0 + lane;
    const bool hit = i < N && ids_l[i] == e;
    const unsigned long long bal = __ballot(hit);
    const int rank = run + __popcll(bal & lt);
    if (hit && rank >= first && rank < last) {
      if (tok) tok[rank - first] = i / k;
      if (asg) asg[rank - first] = i;
    }
    run += __popcll(bal);
  }
}

// Slice blockIdx.x of the layer's combine: out[t, h..h+4) = bf16(sum_j y[t*k +
// j, h..h+4)) over the slots with a valid id, j ascending, the bf16 slot
// outputs summed in fp32 (combine_kernel's sums), y read with sc1 loads
// (other workgroups wrote it in this launch).  Slots without a valid id were never written and are left out; with routing
// in-kernel every id is valid.
__device__ __forceinline__ void fused_combine(const MoeArgs &a, bool route) {
  const int k = a.k, H = a.H;
  const int64_t nq = a.T * H / 4;  // 4 outputs per task
  const int64_t q0 = nq * blockIdx.x / gridDim.x, q1 = nq * (blockIdx.x + 1) / gridDim.x;
  // (the host bounds T*k*H*2 below 2^31: 32-bit byte offsets); bf16 slot outputs
  const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.ybf, a.T * k * H * 2);
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  for (int64_t q = q0 + threadIdx.x; q < q1; q += kSThreads) {
    const int64_t t = q / (H / 4);
    const int h = static_cast<int>(q - t * (H / 4)) * 4;
    floatx4 s = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < k; j0 += 8) {
      // up to 8 slots' loads in flight at once; slots past k or without a
      // valid id read the token's first slot and are not added
      u32x2 v[8];
      bool ok[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = j0 + jj;
        const int id = j < k ? (route ? 0 : a.ids[t * k + j]) : -1;
        ok[jj] = id >= 0 && id < a.E;
        const int off = static_cast<int>(((t * k + (ok[jj] ? j : 0)) * H + h) * 2);
        v[jj] = __builtin_amdgcn_raw_buffer_load_b64(yr, off, 0, kCpolSc1);
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        if (ok[jj])
          s += floatx4{__uint_as_float(v[jj][0] << 16), __uint_as_float(v[jj][0] & 0xFFFF0000u),
                       __uint_as_float(v[jj][1] << 16), __uint_as_float(v[jj][1] & 0xFFFF0000u)};
    }
    uint2 o;
    o.x = static_cast<uint32_t>(f32_to_bf16_bits(s[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(s[1])) << 16);
    o.y = static_cast<uint32_t>(f32_to_bf16_bits(s[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(s[3])) << 16);
    *reinterpret_cast<uint2 *>(a.out + t * H + h) = o;
  }
}

// the plan's tables fit the smallest rows area (K = 512)
constexpr int kPlanLds = 2 * kPlanMaxN + 64 * 8 + kFusedRouteMaxT * 64 + 64 * 4;
static_assert(kPlanLds <= 512 * kRowsMax * 2, "plan tables exceed the rows area");

// Route token t (logits row t, E <= 64, lane e = expert e) with one wave:
// ids and weights to slots t*k + rank of ids_out / w_out with agent-scope
// stores, then, once they are complete, one count on route_cnt.
__device__ __forceinline__ void fused_route_token(const MoeArgs &a, int t) {
  const int lane = threadIdx.x & 63;
  const int E = a.E, k = a.k;
  const int64_t idx = static_cast<int64_t>(t) * E + min(lane, E - 1);
  float v = a.ldt == LQ_F32 ? load_f32<LQ_F32>(a.logits, idx)
                            : a.ldt == LQ_F16 ? load_f32<LQ_F16>(a.logits, idx) : load_f32<LQ_BF16>(a.logits, idx);
  if (lane >= E) v = -__builtin_inff();
  route_values64(v, E, k, a.renorm, [&](int rank, int e, float w) __attribute__((always_inline)) {
    __hip_atomic_store(a.ids_out + t * k + rank, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.w_out + t * k + rank, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  });
  __builtin_amdgcn_s_waitcnt(0);  // this wave's id / weight stores are complete
  if (lane == 0) __hip_atomic_fetch_add(a.bar + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int BITS, int KD1, int KD2, bool SQ>
__global__ __launch_bounds__(kSThreads, 1) void moe_fused_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char slds[];
  __shared__ int32_t rtok[kRowsMax], rasg[kRowsMax];
  __shared__ float rwt[kRowsMax];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = static_cast<int>(a.T * a.k);
  const int T = static_cast<int>(a.T), k = a.k, H = a.H, E = a.E;
  const int G = gridDim.x, c = xcd_slot(blockIdx.x, gridDim.x);
  const bool route = a.logits != nullptr;
  // plan tables, in the rows area until the G1 staging: the expert of each
  // assignment (ids given), or each expert's token mask and each (token,
  // expert) pair's slot (routing in-kernel); the expert counts
  uint16_t *ids_l = reinterpret_cast<uint16_t *>(slds);
  unsigned long long *mask_l = reinterpret_cast<unsigned long long *>(slds + 2 * kPlanMaxN);
  uint8_t *slot_l = slds + 2 * kPlanMaxN + 64 * 8;
  int *cnt_l = reinterpret_cast<int *>(slds + 2 * kPlanMaxN + 64 * 8 + kFusedRouteMaxT * 64);

  // ---- routing (workgroup t < T routes token t) and the expert counts
  if (tid < 64) {
    cnt_l[tid] = 0;
    mask_l[tid] = 0;
  }
  if (route) {
    if (wave == 0 && static_cast<int>(blockIdx.x) < T) fused_route_token(a, blockIdx.x);
    if (tid == 0) {
      bool ok = false;
      for (int spin = 0; spin < kWaitCap; ++spin) {
        if (__hip_atomic_load(a.bar + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= T) {
          ok = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!ok && a.status) atomicOr(a.status, kStatusRouteWait);
    }
    __syncthreads();
    for (int i = tid; i < N; i += kSThreads) {
      const int id = __hip_atomic_load(a.ids_out + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int t = i / k;
      atomicOr(mask_l + id, 1ull << t);
      slot_l[t * 64 + id] = static_cast<uint8_t>(i - t * k);
    }
  } else {
    __syncthreads();
    for (int i = tid; i < N; i += kSThreads) {
      const int id = a.ids[i];
      const bool ok = id >= 0 && id < E;
      ids_l[i] = ok ? static_cast<uint16_t>(id) : uint16_t{0xFFFF};
      if (ok) atomicAdd(cnt_l + id, 1);
    }
  }
  __syncthreads();
  const unsigned long long mask = route ? mask_l[lane] : 0ull;
  const int cnt = route ? __popcll(mask) : (lane < E ? cnt_l[lane] : 0);

  // ---- the plan: blocks of <= 32 rows, expert-major; this workgroup's share of each phase
  const int nbk = (cnt + kRowsMax - 1) / kRowsMax;
  const int cinc = wave_incl_scan(cnt), binc = wave_incl_scan(nbk);
  if (__builtin_amdgcn_readlane(binc, 63) == 0) {
    // no valid assignment (ids given): every output is zero
    fused_combine(a, route);
    return;
  }
  const int upb1 = 2 * a.I / 16, upb2 = H / 16;
  const Share s1 = assign_share(c, G, cnt, nbk, binc - nbk, cinc - cnt, kW1Lo, kW1Hi, upb1);
  const Share s2 = assign_share(c, G, cnt, nbk, binc - nbk, cinc - cnt, kW2Lo, kW2Hi, upb2);
  // rows: wave 0 the tokens of the G1 block, wave 1 the assignments and routing weights of the G2 block
  if (wave < 2) {
    const Share &sh = wave == 0 ? s1 : s2;
    if (route) {
      const unsigned long long me =
          (static_cast<unsigned long long>(static_cast<uint32_t>(__builtin_amdgcn_readlane(
               static_cast<int>(mask >> 32), sh.e))) << 32) |
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mask & 0xFFFFFFFFu), sh.e));
      const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
      const int r = __popcll(me & below) - kRowsMax * sh.j;
      if (((me >> lane) & 1) && r >= 0 && r < sh.rows) {
        if (wave == 0) {
          rtok[r] = lane;
        } else {
          const int asg = lane * k + slot_l[lane * 64 + sh.e];
          rasg[r] = asg;
          rwt[r] = __hip_atomic_load(a.w_out + asg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    } else {
      compact_rows(ids_l, N, k, sh.e, kRowsMax * sh.j, sh.rows, wave == 0 ? rtok : nullptr,
                   wave == 0 ? nullptr : rasg);
      if (wave == 1 && lane < sh.rows) rwt[lane] = a.topk_w[rasg[lane]];
    }
  }
  __syncthreads();  // rows complete; the plan tables are no longer read (the G1 staging overwrites them)

  // ---- G1: this workgroup's share of its G1 block's W1 tiles
  stream_block<BITS, false, true, KD1, SQ, true>(a, s1.e, s1.row0, s1.rows, rtok, nullptr, s1.ub, s1.ue, slds);
  __builtin_amdgcn_s_waitcnt(0);  // every gate / up store of this wave is complete

  // ---- G2: this workgroup's share of its G2 block's W2 tiles, once that block's G1 is complete
  int seen = 0;
  auto wait_g1 = [&]() __attribute__((always_inline)) {
    __syncthreads();  // every wave's G1 stores are complete
    if (tid == 0) {
      __hip_atomic_fetch_add(a.g1_done + s1.b, s1.ue - s1.ub, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bool ok = false;
      for (int spin = 0; spin < kWaitCap; ++spin) {
        if (__hip_atomic_load(a.g1_done + s2.b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= upb1) {
          ok = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!ok && a.status) atomicOr(a.status, kStatusGemm1Wait);
      seen = __hip_atomic_fetch_add(a.g1_seen + s2.b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
  };
  stream_block<BITS, false, false, KD2, SQ, true, true>(a, s2.e, s2.row0, s2.rows, nullptr, rasg, s2.ub, s2.ue, slds,
                                                         wait_g1, rwt);
  __builtin_amdgcn_s_waitcnt(0);  // every y store of this wave is complete
  __syncthreads();
  int left = 0;
  if (tid == 0) {
    __hip_atomic_fetch_add(a.bar, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool ok = false;
    for (int spin = 0; spin < kWaitCap; ++spin) {
      if (__hip_atomic_load(a.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= static_cast<int>(gridDim.x)) {
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!ok && a.status) atomicOr(a.status, kStatusGridWait);
    left = __hip_atomic_fetch_add(a.bar + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  fused_combine(a, route);
  if (tid == 0 && left == static_cast<int>(gridDim.x) - 1) {
    // every workgroup has passed the barrier (and long since the routing
    // count): clear them for the next call
    __hip_atomic_store(a.bar, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.bar + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.bar + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0 && seen == s2.m - 1) {
    // every workgroup of the G2 block has seen its G1 count: clear it for the next call
    __hip_atomic_store(a.g1_done + s2.b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(a.g1_seen + s2.b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// plan: stable permutation + work list (one workgroup)
// ---------------------------------------------------------------------------

constexpr int kPlanBlock = 1024;
constexpr int kPlanWaves = kPlanBlock / 64;

struct PlanArgs {
  const int32_t *ids;
  int64_t N;
  int E;
  int32_t *counts;
  int32_t *offsets;
  int32_t *sorted;
  int32_t *srow;  // token of each sorted row (nullptr: not written)
  int k;
  // block table (blocks == nullptr: permutation only) of blocks of at most
  // block_rows sorted rows
  int4 *blocks;
  int block_rows;
  PlanHeader *hdr;
};

// Block table from the expert counts cnt[] and their exclusive offsets
// off[] (LDS): blocks of at most p.block_rows sorted rows, expert-major;
// nbs (E + 1 entries) and tmp (E) are LDS scratch.  Every thread of the
// workgroup calls it.
__device__ __forceinline__ void plan_blocks(const PlanArgs &p, const int *cnt, const int *off, int *nbs, int *tmp) {
  const int tid = threadIdx.x;
  const int E = p.E;
  const int br = p.block_rows;
  for (int e = tid; e < E; e += kPlanBlock) tmp[e] = (cnt[e] + br - 1) / br;
  __syncthreads();
  if ((tid >> 6) == 0) wave0_exclusive_scan(tmp, nbs, E, &nbs[E]);
  __syncthreads();
  // block b of expert e covers sorted rows [off[e] + br j, + br) with j = b - nbs[e]
  const int nb_total = nbs[E];
  for (int b = tid; b < nb_total; b += kPlanBlock) {
    int lo = 0, hi = E;  // largest e with nbs[e] <= b
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (nbs[mid] <= b) lo = mid;
      else hi = mid;
    }
    const int e = lo;
    const int r0 = off[e] + (b - nbs[e]) * br;
    p.blocks[b] = make_int4(e, r0, min(br, off[e] + cnt[e] - r0), 0);
  }
  if (tid == 0) p.hdr->n_blk = nb_total;
  __syncthreads();
}

// Stable scatter of assignments [a_begin, a_end): chunks of kPlanBlock
// assignments in order; within a chunk, rank = peers with the same expert
// in lower lanes of this wave + peers in lower waves.  base[e] (LDS) is the
// sorted position of expert e's next assignment and advances; wcnt (LDS,
// zero on entry and on exit) holds per-wave counts.
template <class IdAt>
__device__ __forceinline__ void plan_scatter(const PlanArgs &p, IdAt id_at, int *base, int (*wcnt)[kMaxExperts],
                                             int64_t a_begin, int64_t a_end) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int E = p.E;
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // the next chunk's id is loaded while this chunk is ranked and scattered
  int next = a_begin + tid < a_end ? id_at(a_begin + tid) : -1;
  for (int64_t chunk = a_begin; chunk < a_end; chunk += kPlanBlock) {
    const int64_t a = chunk + tid;
    const int raw = next;
    next = a + kPlanBlock < a_end ? id_at(a + kPlanBlock) : -1;
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
      p.sorted[pos] = static_cast<int32_t>(a);
      if (p.srow) p.srow[pos] = static_cast<int32_t>(a / p.k);
    }
    __syncthreads();
    for (int e = tid; e < E; e += kPlanBlock) {
      int s = 0;
      for (int w = 0; w < kPlanWaves; ++w) {
        s += wcnt[w][e];
        wcnt[w][e] = 0;
      }
      base[e] += s;
    }
    __syncthreads();
  }
}

// the plan for one workgroup of kPlanBlock threads; id_at(a) returns the
// expert of assignment a (read from memory or from LDS)
template <class IdAt>
__device__ __forceinline__ void plan_body(const PlanArgs &p, IdAt id_at) {
  __shared__ int hist[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int nbs[kMaxExperts + 1];  // exclusive scan of row blocks per expert
  __shared__ int wcnt[kPlanWaves][kMaxExperts];
  __shared__ int total;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int E = p.E;
  for (int e = tid; e < kMaxExperts; e += kPlanBlock) hist[e] = 0;
  for (int i = tid; i < kPlanWaves * kMaxExperts; i += kPlanBlock) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  // (8 ids per thread in flight at once: the loop is latency-bound otherwise)
  for (int64_t a0 = 0; a0 < p.N; a0 += 8 * kPlanBlock) {
    int idv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t a = a0 + j * kPlanBlock + tid;
      idv[j] = a < p.N ? id_at(a) : -1;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (idv[j] >= 0 && idv[j] < E) atomicAdd(&hist[idv[j]], 1);
  }
  __syncthreads();
  if (wave == 0) wave0_exclusive_scan(hist, base, E, &total);
  __syncthreads();
  for (int e = tid; e < E; e += kPlanBlock) {
    p.counts[e] = hist[e];
    p.offsets[e] = base[e];
  }
  if (tid == 0) p.offsets[E] = total;
  if (p.blocks != nullptr) plan_blocks(p, hist, base, nbs, wcnt[0]);
  for (int e = tid; e < E; e += kPlanBlock) wcnt[0][e] = 0;
  __syncthreads();
  plan_scatter(p, id_at, base, wcnt, 0, p.N);
}

// Multi-workgroup plan for large layers, two launches with the same result
// as plan_kernel.  Segment s is assignments [s kPlanSeg, (s+1) kPlanSeg).
// plan_count_kernel: workgroup s writes its segment's expert counts to
// seg_cnt[s][E].  plan_scatter_kernel: workgroup s adds up every segment's
// counts (the totals) and those of the segments before it (its prefix),
// scans the totals into offsets, and scatters its own segment stably from
// offsets + prefix; workgroup 0 also writes counts, offsets and the block
// table.
constexpr int kPlanSeg = kPlanBlock;  // one chunk per segment: no chunk loop in the scatter

__global__ __launch_bounds__(kPlanBlock) void plan_count_kernel(PlanArgs p, int32_t *seg_cnt) {
  __shared__ int hist[kMaxExperts];
  const int tid = threadIdx.x;
  const int E = p.E;
  for (int e = tid; e < E; e += kPlanBlock) hist[e] = 0;
  __syncthreads();
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * kPlanSeg;
  constexpr int kPer = kPlanSeg / kPlanBlock;
  int idv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int64_t a = a0 + j * kPlanBlock + tid;
    idv[j] = a < p.N ? p.ids[a] : -1;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (idv[j] >= 0 && idv[j] < E) atomicAdd(&hist[idv[j]], 1);
  __syncthreads();
  for (int e = tid; e < E; e += kPlanBlock) seg_cnt[static_cast<int64_t>(blockIdx.x) * E + e] = hist[e];
}

__global__ __launch_bounds__(kPlanBlock) void plan_scatter_kernel(PlanArgs p, const int32_t *seg_cnt, int nseg) {
  __shared__ int tot[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int pre[kMaxExperts];
  __shared__ int nbs[kMaxExperts + 1];
  __shared__ int wcnt[kPlanWaves][kMaxExperts];
  __shared__ int total;
  const int tid = threadIdx.x;
  const int E = p.E;
  const int seg = blockIdx.x;
  for (int e = tid; e < E; e += kPlanBlock) {
    tot[e] = 0;
    pre[e] = 0;
  }
  for (int i = tid; i < kPlanWaves * kMaxExperts; i += kPlanBlock) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  const int64_t n_cnt = static_cast<int64_t>(nseg) * E;
  for (int64_t i = tid; i < n_cnt; i += kPlanBlock) {
    const int c = seg_cnt[i];
    const int e = static_cast<int>(i % E);
    if (c) {
      atomicAdd(&tot[e], c);
      if (i / E < seg) atomicAdd(&pre[e], c);
    }
  }
  __syncthreads();
  if ((tid >> 6) == 0) wave0_exclusive_scan(tot, base, E, &total);
  __syncthreads();
  if (seg == 0) {
    for (int e = tid; e < E; e += kPlanBlock) {
      p.counts[e] = tot[e];
      p.offsets[e] = base[e];
    }
    if (tid == 0) p.offsets[E] = total;
    if (p.blocks != nullptr) plan_blocks(p, tot, base, nbs, wcnt[0]);
    for (int e = tid; e < E; e += kPlanBlock) wcnt[0][e] = 0;
  }
  for (int e = tid; e < E; e += kPlanBlock) base[e] += pre[e];
  __syncthreads();
  const int64_t a_begin = static_cast<int64_t>(seg) * kPlanSeg;
  plan_scatter(p, [&](int64_t a) { return p.ids[a]; }, base, wcnt, a_begin, min(p.N, a_begin + kPlanSeg));
}

__global__ __launch_bounds__(kPlanBlock) void plan_kernel(PlanArgs p) {
  plan_body(p, [&](int64_t a) { return p.ids[a]; });
}

// x [rows, H] -> xperm, each group of 8 bf16 in K-slot order (8 values per thread)
__global__ __launch_bounds__(256) void permute_rows_kernel(const uint16_t *__restrict__ x, int64_t n8,
                                                          uint16_t *__restrict__ xperm) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n8)
    reinterpret_cast<uint4 *>(xperm)[i] = permute_kslots(reinterpret_cast<const uint4 *>(x)[i]);
}

// QuantLinear set-up: x [M, K] -> act [M, K] in the GEMMs' K-slot order
// (8 values per thread), the nslot routing slots all expert 0 with weight
// 1.0, and the plan of one expert, which is the identity: sorted / srow
// [i] = i, blocks of br rows [b br, b br + br) (the plan kernel's output
// for these ids, without its launch)
__global__ __launch_bounds__(256) void linear_setup_kernel(const uint16_t *__restrict__ x, int64_t n8, int64_t M,
                                                           int64_t nslot, uint16_t *__restrict__ act,
                                                           int32_t *__restrict__ ids, float *__restrict__ weights,
                                                           int32_t *__restrict__ sorted, int32_t *__restrict__ srow,
                                                           int4 *__restrict__ blocks, PlanHeader *hdr, int br) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n8) reinterpret_cast<uint4 *>(act)[i] = permute_kslots(reinterpret_cast<const uint4 *>(x)[i]);
  if (i < nslot) {
    ids[i] = 0;
    weights[i] = 1.0f;
  }
  if (i < M) {
    sorted[i] = static_cast<int32_t>(i);
    srow[i] = static_cast<int32_t>(i);
  }
  const int64_t nb = (M + br - 1) / br;
  if (i < nb) blocks[i] = make_int4(0, static_cast<int>(i * br), static_cast<int>(min<int64_t>(br, M - i * br)), 0);
  if (i == 0) hdr->n_blk = static_cast<int32_t>(nb);
}

// ---------------------------------------------------------------------------
// QuantLinear for a few rows (M <= 32), one launch: out = bf16(x . W^T).
//
// Workgroup b owns output columns [32 b, 32 b + 32) -- two 16-row tiles of
// W -- and has S waves; wave ks sums the chunks of K slice ks (nks whole
// 128-wide chunks), the slices the general GEMM2 + combine path uses for the
// same shape.  Each wave streams its two tiles' codes and scales (kD chunks
// in flight) and reads its A fragments straight from x in natural order (x
// is small and stays in L2; each fragment feeds both tiles), permuting each
// 8-value piece into the K-slot order in registers; the per-chunk arithmetic
// is chunk_mfma_f's.  The S partial tiles meet in LDS and are added in
// ascending slice order from 0.0f, as the combine adds the general path's
// slots, then rounded once to bf16 -- so the two paths agree bit for bit.
// Rows of x past M read zeros (offsets past the buffer's end) and are never
// stored.
// ---------------------------------------------------------------------------
struct LinArgs {
  const uint16_t *x;  // [M, K] bf16
  const int8_t *q;    // [N, K] int8 or [N, K/2] packed
  const float *s;     // [N, ng]
  uint16_t *out;      // [M, N] bf16
  int M, K, N;
  int G, ng;          // group length along K (a multiple of 32) and groups per row
  int nks;            // chunks per K slice (a multiple of the kernel's KD)
};

constexpr int kLinNT = 2;          // 16-row weight tiles per workgroup
constexpr int kLinMaxSlices = 16;  // linear_ksplit's cap

template <int BITS, int NRT, int KD, int MAXS>
__global__ __launch_bounds__(64 * MAXS) void linear_small_kernel(LinArgs a) {
  constexpr int NT = kLinNT;
  constexpr int kElems = NRT * 4 * NT * 64;  // one partial of the workgroup's tiles
  __shared__ float part[MAXS][kElems];
  const int tid = threadIdx.x;
  const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's K slice
  const int S = static_cast<int>(blockDim.x >> 6);
  const int lane = tid & 63;
  const int lc = lane & 15;
  const int lg = lane >> 4;
  const int n0 = 16 * NT * static_cast<int>(blockIdx.x);
  constexpr int kLaneBytes = BITS == 4 ? 16 : 32;  // one lane's 32 codes of a chunk
  constexpr int kChunkBytes = BITS == 4 ? 64 : 128;
  const int rowbytes = BITS == 4 ? (a.K >> 1) : a.K;
  const int c_first = ks * a.nks;
  const __amdgpu_buffer_rsrc_t wrsrc = make_rsrc(a.q + static_cast<int64_t>(n0) * rowbytes, 16ll * NT * rowbytes);
  const __amdgpu_buffer_rsrc_t srsrc = make_rsrc(a.s + static_cast<int64_t>(n0) * a.ng, 16ll * NT * a.ng * 4);
  const int64_t xbytes = static_cast<int64_t>(a.M) * a.K * 2;  // below 2^31 (host-checked)
  const __amdgpu_buffer_rsrc_t xrsrc = make_rsrc(a.x, xbytes);
  const __amdgpu_buffer_rsrc_t empty = make_rsrc(a.out, 0);  // reads zeros, no memory traffic
  const int wvoff = lc * rowbytes + kLaneBytes * lg;  // tile c adds 16 c rows
  const int svoff = lc * a.ng * 4;
  int xoff[NRT];  // row 16 rt + lc, K offset 32 lg of each chunk; rows past M read zeros
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    const int m = 16 * rt + lc;
    xoff[rt] = m < a.M ? m * a.K * 2 + 64 * lg : static_cast<int>(xbytes);
  }

  WChunk<BITS> wb[KD][NT];
  float sb[KD][NT];
  uint4 xb[KD][NRT][4];
  // chunk i of this slice into ring slot d (the loads stay in flight); past
  // the slice's end every load goes through the empty descriptor, so each
  // step issues the same loads and the wait counts stay exact
  auto load = [&](int i, int d) __attribute__((always_inline)) {
    const bool live = i < a.nks;
    const int c = c_first + (live ? i : 0);
    const __amdgpu_buffer_rsrc_t rw = live ? wrsrc : empty, rs = live ? srsrc : empty, rx = live ? xrsrc : empty;
    // the group of this lane's 32 codes (G is a multiple of 32, so they share it)
    const int sidx = (c * kKC + 32 * lg) / a.G;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int vo = wvoff + 16 * t * rowbytes;
      if constexpr (BITS == 4) {
        wb[d][t].v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo, c * kChunkBytes, 0));
      } else {
        wb[d][t].v0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo, c * kChunkBytes, 0));
        wb[d][t].v1 =
            __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo + 16, c * kChunkBytes, 0));
      }
      sb[d][t] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rs, svoff + 16 * t * a.ng * 4 + 4 * sidx, 0, 0));
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
      for (int p = 0; p < 4; ++p)
        xb[d][rt][p] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xoff[rt] + 16 * p, c * kKC * 2, 0));
  };

  floatx4 tot[NRT][NT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int t = 0; t < NT; ++t) tot[rt][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int d = 0; d < KD; ++d) load(d, d);
  for (int i0 = 0; i0 < a.nks; i0 += KD) {
#pragma unroll
    for (int d = 0; d < KD; ++d) {
      // A fragment of step s: K piece 4 lg + s of the chunk, in K-slot order
      auto afrag = [&](int rt, int s) __attribute__((always_inline)) { return permute_kslots(xb[d][rt][s]); };
      if (__all(dq_fast_ok(sb[d][0]) && dq_fast_ok(sb[d][1])))
        chunk_mfma_f<BITS, false, true, NRT, NT>(wb[d], sb[d], afrag, tot);
      else
        chunk_mfma_f<BITS, false, false, NRT, NT>(wb[d], sb[d], afrag, tot);
      load(i0 + d + KD, d);  // the chunk KD ahead
    }
  }
  // partial element ((rt * 4 + j) * NT + t) * 64 + lane
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < NT; ++t) part[ks][((rt * 4 + j) * NT + t) * 64 + lane] = tot[rt][t][j];
  __syncthreads();
  for (int e = tid; e < kElems; e += static_cast<int>(blockDim.x)) {
    float acc = 0.0f;  // the combine's order: 0, then the slots by ascending slice
    for (int u = 0; u < S; ++u) acc += part[u][e];
    const int l = e & 63, t = (e >> 6) % NT, rj = (e >> 6) / NT;  // rj = rt * 4 + j
    const int m = 16 * (rj >> 2) + 4 * (l >> 4) + (rj & 3);
    if (m < a.M) a.out[static_cast<int64_t>(m) * a.N + n0 + 16 * t + (l & 15)] = f32_to_bf16_bits(acc);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

struct WsLayout {
  size_t status, g1_done, g1_seen, bar, sync_end;  // sync region: zero before the first call, left zero
  size_t counts, offsets, sorted, srow, hdr, blocks, slotplan, slotasg, segcnt, ids, weights, xperm, act, ybuf, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// CU slots the streaming GEMMs' slot records cover (one workgroup per CU)
constexpr int kMaxSlots = 1024;

// row blocks of at most kRowsMax sorted rows: one partial block per expert at most
int64_t max_blocks_for(int64_t T, int E, int k) {
  const int64_t N = T * k;
  return std::min<int64_t>(E, N) + N / kRowsMax;
}

// The workspace starts with the sync region -- the status word (at offset
// 0) and the fused kernel's counters (per row block, up to kSyncBlocks of
// them, and its grid barrier) -- which must be zero before the first call on a
// workspace (lq_moe_workspace_init) and which every call leaves zero.  Its
// size and place do not depend on the shape, so one initialisation serves
// every later call.  The rest is scratch each call overwrites.
constexpr int kSyncBlocks = 1024;  // CUs the fused kernel's per-block counters cover
WsLayout ws_layout(int64_t T, int H, int I, int E, int k) {
  const int64_t N = T * k;
  WsLayout w;
  size_t off = 0;
  auto take = [&](size_t &field, size_t bytes) {
    field = off;
    off = align256(off + bytes);
  };
  take(w.status, sizeof(uint32_t));
  take(w.g1_done, sizeof(int32_t) * kSyncBlocks);
  take(w.g1_seen, sizeof(int32_t) * kSyncBlocks);
  take(w.bar, sizeof(int32_t) * 4);
  w.sync_end = off;
  take(w.counts, sizeof(int32_t) * E);
  take(w.offsets, sizeof(int32_t) * (E + 1));
  take(w.sorted, sizeof(int32_t) * N);
  take(w.srow, sizeof(int32_t) * N);
  take(w.hdr, sizeof(PlanHeader));
  take(w.blocks, sizeof(int4) * max_blocks_for(T, E, k));
  take(w.slotplan, sizeof(int4) * kMaxSlots);
  take(w.slotasg, sizeof(int32_t) * kMaxSlots * kRowsMax);
  take(w.segcnt, sizeof(int32_t) * E * ((N + kPlanSeg - 1) / kPlanSeg));  // multi-workgroup plan
  take(w.ids, sizeof(int32_t) * N);
  take(w.weights, sizeof(float) * N);
  take(w.xperm, sizeof(uint16_t) * T * H);
  take(w.act, sizeof(uint16_t) * N * 2 * I);  // act [N, I] (general) or gate/up [N, 2I] (streaming)
  take(w.ybuf, sizeof(uint16_t) * N * H);  // bf16 slot outputs
  w.total = off;
  return w;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// persistent grid: resident workgroups of one GEMM kernel on this device,
// a multiple of 8 (one share per XCD), no more than the items can use
template <int BITS, bool FOLDED, bool FIRST, bool G128>
int gemm_grid(int64_t max_items) {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int g = cached[dev];
  if (g == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, moe_gemm_kernel<BITS, FOLDED, FIRST, G128>, kThreads, 0) !=
            hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    g = cus * per_cu;
    cached[dev] = g;
  }
  const int64_t want = (std::max<int64_t>(max_items, 1) + 7) / 8 * 8;
  return static_cast<int>(std::max<int64_t>(8, std::min<int64_t>(g / 8 * 8, want)));
}

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

// The GEMM family a layer runs on.  Wide: at least kWideMinRows routed rows
// per expert on average (measured on MI355X at E64 H2048 I1024, INT4 and
// INT8: the wide kernels win from 32 rows per expert on, the streaming ones
// at 16); streaming: the weight-bandwidth regime below that; general: every
// other supported shape.
enum class Path { kStream, kGeneral, kWide };
constexpr int kWideMinRows = 32;

// the wide kernels need whole items along N (128 features, 256 output
// rows), whole pairs of 128-wide K chunks, and exact weights (the folded
// form keeps its own kernels)
bool wide_eligible(int H, int I, int flags) {
  return H % kWR2 == 0 && I % kWR2 == 0 && !(flags & LQ_MOE_FOLDED_SCALES);
}

bool stream_eligible(int bits, int H, int I, int64_t g1, int64_t g2);

int validate_layer(const void *x, int64_t T, int H, int I, int E, int k, const int8_t *q1, const float *s1,
                   const int8_t *q2, const float *s2, int bits, int64_t group_w1, int64_t group_w2, int flags,
                   void *workspace, size_t ws_bytes, void *out) {
  if (bits != 4 && bits != 8) return fail(LQ_ERR_VALUE, "bits must be 8 or 4, got " + std::to_string(bits));
  if (T < 0 || H <= 0 || I <= 0 || k <= 0) return fail(LQ_ERR_VALUE, "moe_forward: bad shape");
  if (E < 1 || E > kMaxExperts)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: 1 <= num_experts <= " + std::to_string(kMaxExperts));
  if (k > E) return fail(LQ_ERR_VALUE, "moe_forward: top_k exceeds num_experts");
  if (flags & ~(LQ_MOE_FOLDED_SCALES | LQ_MOE_GENERAL_KERNEL | LQ_MOE_WIDE_KERNEL | LQ_MOE_STREAM_KERNEL |
                LQ_MOE_FUSED_LAYER))
    return fail(LQ_ERR_VALUE, "moe_forward: unknown flags");
  {
    const int forced = flags & (LQ_MOE_GENERAL_KERNEL | LQ_MOE_WIDE_KERNEL | LQ_MOE_STREAM_KERNEL);
    if (forced & (forced - 1))
      return fail(LQ_ERR_VALUE,
                  "moe_forward: LQ_MOE_WIDE_KERNEL, LQ_MOE_STREAM_KERNEL and LQ_MOE_GENERAL_KERNEL exclude each other");
  }
  if ((flags & LQ_MOE_WIDE_KERNEL) && !wide_eligible(H, I, flags))
    return fail(LQ_ERR_UNSUPPORTED,
                "moe_forward: the wide kernels need hidden % 256 == 0, intermediate % 256 == 0 and exact weights "
                "(no LQ_MOE_FOLDED_SCALES)");
  if (H % kR2 != 0 || I % kF1 != 0)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: needs hidden % 128 == 0 and intermediate % 64 == 0");
  const int64_t g1 = effective_group(H, group_w1);
  const int64_t g2 = effective_group(I, group_w2);
  if (g1 % 32 != 0 || g2 % 32 != 0)
    return fail(LQ_ERR_UNSUPPORTED,
                "moe_forward: the group length along K must be a multiple of 32 (got " + std::to_string(g1) +
                    " for w1, " + std::to_string(g2) + " for w2)");
  const int64_t N = T * k;
  // the GEMMs address x, the bf16 gate / up rows [N, 2I] and slot outputs
  // [N, H], one expert's codes and one expert's scales through 32-bit
  // offsets (bytes below kOutOfRange; element offsets into those buffers
  // below 2^30)
  if (T > (int64_t{1} << 18) || N * static_cast<int64_t>(2 * I > H ? 2 * I : H) * 2 > 0x7FFFFFFFll ||
      T * static_cast<int64_t>(H) * 2 >= kOutOfRange)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: too many tokens for one call");
  if (int64_t{2} * I * H >= kOutOfRange)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: one expert's weights exceed 2 GiB");
  if ((flags & LQ_MOE_STREAM_KERNEL) && !stream_eligible(bits, H, I, g1, g2))
    return fail(LQ_ERR_UNSUPPORTED,
                "moe_forward: the streaming kernels need hidden and intermediate in whole 512-wide (INT4) or "
                "256-wide (INT8) steps, group lengths that are multiples of 128, and K <= the LDS capacity");
  if (max_blocks_for(T, E, k) * (I / kF1 + H / kR2) > 0x3FFFFFFF)
    return fail(LQ_ERR_UNSUPPORTED, "moe_forward: work list too long");
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

// G1 -> G2 -> combine, marks[first + 1 ..] after each
// per-device facts the launches need (queried once per device)
struct DeviceInfo {
  int cus = 0;         // compute units
  int max_lds = 0;     // LDS bytes one workgroup may use
};
DeviceInfo device_info() {
  static DeviceInfo cache[64];
  static std::once_flag once[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  std::call_once(once[dev], [dev] {
    DeviceInfo d;
    if (hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || d.cus <= 0)
      d.cus = 256;
    if (hipDeviceGetAttribute(&d.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      d.max_lds = 65536;
    cache[dev] = d;
  });
  return cache[dev];
}

// The streaming kernels cover shapes whose K splits into whole runs of 4
// (INT4) or 2 (INT8) 128-wide chunks -- the chunks of codes kept in flight
// -- with group lengths that are multiples of 128, and whose token rows for
// the whole K fit one workgroup's LDS.
bool stream_eligible(int bits, int H, int I, int64_t g1, int64_t g2) {
  const int step = kKC * (bits == 4 ? 4 : 2);
  const size_t lds = stream_lds_bytes(std::max(H, I));
  // (kStaticLds: what the streaming kernels declare statically)
  return H % step == 0 && I % step == 0 && g1 % kKC == 0 && g2 % kKC == 0 &&
         lds + kStaticLds <= static_cast<size_t>(device_info().max_lds);
}

// let a kernel's dynamic LDS take what its static LDS leaves of the
// workgroup's share (once per kernel and process)
template <class Fn>
int allow_dynamic_lds(Fn *fn, std::once_flag &once, hipError_t &rc) {
  std::call_once(once, [&] {
    hipFuncAttributes fa{};
    rc = hipFuncGetAttributes(&fa, reinterpret_cast<const void *>(fn));
    if (rc == hipSuccess)
      rc = hipFuncSetAttribute(reinterpret_cast<const void *>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                               device_info().max_lds - static_cast<int>(fa.sharedSizeBytes));
  });
  if (rc != hipSuccess) return fail(LQ_ERR_RUNTIME, std::string("hipFuncSetAttribute failed: ") + hipGetErrorString(rc));
  return LQ_OK;
}

template <int BITS, bool FOLDED, bool FIRST, int KD, bool SQ, int PLAN>
int launch_stream_kd(const MoeArgs &a, hipStream_t st) {
  static std::once_flag once;
  static hipError_t attr_rc = hipSuccess;
  const int rc = allow_dynamic_lds(moe_stream_kernel<BITS, FOLDED, FIRST, KD, SQ, PLAN>, once, attr_rc);
  if (rc) return rc;
  const size_t lds = stream_lds_bytes(FIRST ? a.H : a.I);
  moe_stream_kernel<BITS, FOLDED, FIRST, KD, SQ, PLAN><<<device_info().cus, kSThreads, lds, st>>>(a);
  return check_launch(FIRST ? "moe_stream_gemm1" : "moe_stream_gemm2");
}

// inplan: G1 plans its blocks in-kernel and records them per slot, G2
// reads the records; otherwise both read plan_kernel's table
template <int BITS, bool FOLDED, bool FIRST, int KD, bool SQ>
int launch_stream_plan(const MoeArgs &a, hipStream_t st, bool inplan) {
  if (!inplan) return launch_stream_kd<BITS, FOLDED, FIRST, KD, SQ, kPlanTable>(a, st);
  return launch_stream_kd<BITS, FOLDED, FIRST, KD, SQ, FIRST ? kPlanOwn : kPlanSlot>(a, st);
}

// chunks in flight per wave for reduction length nk * 128: 8 KB of codes
// where K allows (INT4: 8 x 1 KB, INT8: 4 x 2 KB), half that otherwise; the
// folded INT4 form keeps 4 (its extra accumulators leave no registers for
// 8).  The exact INT4 form also takes 4 when 8 would leave an odd number of
// runs per unit: left-over units are then split between waves, which gains
// more than the deeper prefetch (a unit of 8 chunks: 23.4 us instead of
// 24.7 us for the C4 down projection).
template <int BITS, bool FOLDED>
int stream_kd(int nk) {
  constexpr int kDeep = BITS == 4 ? (FOLDED ? 4 : 8) : 4;
  return nk % kDeep == 0 && (kDeep < 8 || (nk / kDeep) % 2 == 0) ? kDeep : kDeep / 2;
}

// per-unit scale loads (SQ): group length 128, at most 16 groups, runs of at least 4 chunks
inline bool stream_sq(int group, int nk, int kd) { return group == kKC && nk <= 16 && kd >= 4; }

template <int BITS, bool FOLDED, bool FIRST>
int launch_stream(const MoeArgs &a, hipStream_t st, bool inplan) {
  const int nk = (FIRST ? a.H : a.I) / kKC;
  constexpr int kDeep = BITS == 4 ? (FOLDED ? 4 : 8) : 4;
  const int kd = stream_kd<BITS, FOLDED>(nk);
  const bool sq = stream_sq(FIRST ? a.g1 : a.g2, nk, kd);
  if (kd == kDeep)
    return sq ? launch_stream_plan<BITS, FOLDED, FIRST, kDeep, true>(a, st, inplan)
              : launch_stream_plan<BITS, FOLDED, FIRST, kDeep, false>(a, st, inplan);
  if constexpr (kDeep / 2 >= 4) {
    if (sq) return launch_stream_plan<BITS, FOLDED, FIRST, kDeep / 2, true>(a, st, inplan);
  }
  return launch_stream_plan<BITS, FOLDED, FIRST, kDeep / 2, false>(a, st, inplan);
}

template <int BITS, int KD1, int KD2, bool SQ>
int launch_fused_k(const MoeArgs &a, hipStream_t st) {
  static std::once_flag once;
  static hipError_t attr_rc = hipSuccess;
  const int rc = allow_dynamic_lds(moe_fused_kernel<BITS, KD1, KD2, SQ>, once, attr_rc);
  if (rc) return rc;
  const size_t lds = stream_lds_bytes(std::max(a.H, a.I));
  moe_fused_kernel<BITS, KD1, KD2, SQ><<<device_info().cus, kSThreads, lds, st>>>(a);
  return check_launch("moe_fused_layer");
}

// the fused layer kernel with each GEMM's run depth; per-unit scale loads
// when both GEMMs can take them
template <int BITS>
int launch_fused(const MoeArgs &a, hipStream_t st) {
  constexpr int kHi = BITS == 4 ? 8 : 4, kLo = kHi / 2;
  const int nk1 = a.H / kKC, nk2 = a.I / kKC;
  const int kd1 = stream_kd<BITS, false>(nk1), kd2 = stream_kd<BITS, false>(nk2);
  const bool sq = stream_sq(a.g1, nk1, kd1) && stream_sq(a.g2, nk2, kd2);
  if (kd1 == kHi && kd2 == kHi)
    return sq ? launch_fused_k<BITS, kHi, kHi, true>(a, st) : launch_fused_k<BITS, kHi, kHi, false>(a, st);
  if (kd1 == kHi)
    return sq && kLo >= 4 ? launch_fused_k<BITS, kHi, kLo, kLo >= 4>(a, st) : launch_fused_k<BITS, kHi, kLo, false>(a, st);
  if (kd2 == kHi)
    return sq && kLo >= 4 ? launch_fused_k<BITS, kLo, kHi, kLo >= 4>(a, st) : launch_fused_k<BITS, kLo, kHi, false>(a, st);
  return sq && kLo >= 4 ? launch_fused_k<BITS, kLo, kLo, kLo >= 4>(a, st) : launch_fused_k<BITS, kLo, kLo, false>(a, st);
}

template <int BITS, bool FOLDED>
int launch_general(const MoeArgs &a, int64_t max_g1, int64_t max_g2, hipStream_t st, ProfileMarks &pm, int first) {
  if (a.g1 == kKC)
    moe_gemm_kernel<BITS, FOLDED, true, true><<<gemm_grid<BITS, FOLDED, true, true>(max_g1), kThreads, 0, st>>>(a);
  else
    moe_gemm_kernel<BITS, FOLDED, true, false><<<gemm_grid<BITS, FOLDED, true, false>(max_g1), kThreads, 0, st>>>(a);
  int rc = check_launch("moe_gemm1");
  if (rc) return rc;
  pm.mark(first + 1);
  if (a.g2 == kKC)
    moe_gemm_kernel<BITS, FOLDED, false, true><<<gemm_grid<BITS, FOLDED, false, true>(max_g2), kThreads, 0, st>>>(a);
  else
    moe_gemm_kernel<BITS, FOLDED, false, false><<<gemm_grid<BITS, FOLDED, false, false>(max_g2), kThreads, 0, st>>>(
        a);
  rc = check_launch("moe_gemm2");
  if (rc) return rc;
  pm.mark(first + 2);
  return LQ_OK;
}

// persistent grid of the wide kernels: resident workgroups (a multiple of 8),
// no more than the items can use
template <int BITS, bool FIRST, bool G128>
int wide_grid(int64_t max_items) {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int g = cached[dev];
  if (g == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, moe_wide_kernel<BITS, FIRST, G128>, kWThreads, 0) !=
            hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    g = device_info().cus * per_cu;
    cached[dev] = g;
  }
  const int64_t want = (std::max<int64_t>(max_items, 1) + 7) / 8 * 8;
  return static_cast<int>(std::max<int64_t>(8, std::min<int64_t>(g / 8 * 8, want)));
}

template <int BITS>
int launch_wide(const MoeArgs &a, int64_t max_blocks, hipStream_t st, ProfileMarks &pm, int first) {
  const int64_t max_g1 = max_blocks * (a.I / kWF1), max_g2 = max_blocks * (a.H / kWR2);
  if (a.g1 == kKC)
    moe_wide_kernel<BITS, true, true><<<wide_grid<BITS, true, true>(max_g1), kWThreads, 0, st>>>(a);
  else
    moe_wide_kernel<BITS, true, false><<<wide_grid<BITS, true, false>(max_g1), kWThreads, 0, st>>>(a);
  int rc = check_launch("moe_wide_gemm1");
  if (rc) return rc;
  pm.mark(first + 1);
  if (a.g2 == kKC)
    moe_wide_kernel<BITS, false, true><<<wide_grid<BITS, false, true>(max_g2), kWThreads, 0, st>>>(a);
  else
    moe_wide_kernel<BITS, false, false><<<wide_grid<BITS, false, false>(max_g2), kWThreads, 0, st>>>(a);
  rc = check_launch("moe_wide_gemm2");
  if (rc) return rc;
  pm.mark(first + 2);
  return LQ_OK;
}

template <int BITS, bool FOLDED>
int launch_phases(const MoeArgs &a, int64_t max_g1, int64_t max_g2, hipStream_t st, ProfileMarks &pm, int first,
                  Path path, bool inplan) {
  if (path == Path::kWide) {
    if constexpr (FOLDED) {
      return fail(LQ_ERR_UNSUPPORTED, "moe_forward: the wide kernels take exact weights only");
    } else {
      const int64_t max_blocks = std::min<int64_t>(a.E, a.T * a.k) + a.T * a.k / kWRows;
      int rc = launch_wide<BITS>(a, max_blocks, st, pm, first);
      if (rc) return rc;
    }
  } else if (path == Path::kStream) {
    int rc = launch_stream<BITS, FOLDED, true>(a, st, inplan);
    if (rc) return rc;
    pm.mark(first + 1);
    rc = launch_stream<BITS, FOLDED, false>(a, st, inplan);
    if (rc) return rc;
    pm.mark(first + 2);
  } else {
    int rc = launch_general<BITS, FOLDED>(a, max_g1, max_g2, st, pm, first);
    if (rc) return rc;
  }
  const int64_t n8 = a.T * a.H / 8;  // 8 outputs per thread
  combine_kernel<true><<<static_cast<int>(ceil_div(n8, kCombineBlock)), kCombineBlock, 0, st>>>(a.ybf, a.ids, a.T,
                                                                                                a.H, a.k, a.E, a.out);
  const int rc = check_launch("moe_combine");
  if (rc) return rc;
  pm.mark(first + 3);
  return LQ_OK;
}


// the plan's arguments over the workspace
PlanArgs plan_args(const int32_t *topk_ids, int64_t T, int E, int k, char *ws, const WsLayout &w) {
  PlanArgs p;
  p.ids = topk_ids;
  p.N = T * k;
  p.E = E;
  p.counts = reinterpret_cast<int32_t *>(ws + w.counts);
  p.offsets = reinterpret_cast<int32_t *>(ws + w.offsets);
  p.sorted = reinterpret_cast<int32_t *>(ws + w.sorted);
  p.blocks = reinterpret_cast<int4 *>(ws + w.blocks);
  p.srow = reinterpret_cast<int32_t *>(ws + w.srow);
  p.k = k;
  p.block_rows = kRowsMax;
  p.hdr = reinterpret_cast<PlanHeader *>(ws + w.hdr);
  return p;
}

Path choose_path(int bits, int64_t T, int H, int I, int E, int k, int64_t group_w1, int64_t group_w2, int flags) {
  if (flags & LQ_MOE_WIDE_KERNEL) return Path::kWide;  // (validate_layer checked the forced family)
  if (flags & LQ_MOE_STREAM_KERNEL) return Path::kStream;
  if (flags & LQ_MOE_GENERAL_KERNEL) return Path::kGeneral;
  if (wide_eligible(H, I, flags) && T * k >= static_cast<int64_t>(kWideMinRows) * E) return Path::kWide;
  if (stream_eligible(bits, H, I, effective_group(H, group_w1), effective_group(I, group_w2))) return Path::kStream;
  return Path::kGeneral;
}

// The fused layer kernel takes a streaming-family layer whose assignments one
// workgroup plans (T*k <= kPlanMaxN) and whose row blocks each get a CU of
// their own (at most ceil(T*k / 32) + min(E, T*k) blocks), in the exact
// weight form.
bool fused_eligible(Path path, bool folded, int64_t T, int E, int k, int flags) {
  if (!(flags & LQ_MOE_FUSED_LAYER)) return false;
  const int64_t nb_max = ceil_div(T * k, kRowsMax) + std::min<int64_t>(E, T * k);
  const int64_t cus = device_info().cus;
  // every block gets a CU in both phases' cost-weighted splits
  const bool fits = nb_max * kW1Hi <= kW1Lo * cus && nb_max * kW2Hi <= kW2Lo * cus;
  return path == Path::kStream && !folded && E <= 64 && T * k <= kPlanMaxN && fits && cus <= kSyncBlocks;
}

// Routing inside the fused kernel: workgroup t routes token t (one wave, E <= 64).
bool route_in_kernel(int64_t T, int E) { return T <= kFusedRouteMaxT && T <= device_info().cus && E <= 64; }

// Layer arguments over the workspace and the caller's buffers.
MoeArgs layer_args(const void *x, int64_t T, int H, int I, int E, int k, const int8_t *q1, const float *s1,
                   const int8_t *q2, const float *s2, int64_t g1, int64_t g2, const int32_t *topk_ids,
                   const float *topk_weights, char *ws, const WsLayout &w, const PlanArgs &p, void *out) {
  MoeArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.xperm = reinterpret_cast<uint16_t *>(ws + w.xperm);
  a.q1 = q1;
  a.s1 = s1;
  a.q2 = q2;
  a.s2 = s2;
  a.ids = topk_ids;
  a.topk_w = topk_weights;
  a.offsets = p.offsets;
  a.sorted = p.sorted;
  a.blocks = p.blocks;
  a.srow = p.srow;
  a.hdr = p.hdr;
  a.slotplan = reinterpret_cast<int4 *>(ws + w.slotplan);
  a.slotasg = reinterpret_cast<int32_t *>(ws + w.slotasg);
  a.act = reinterpret_cast<uint16_t *>(ws + w.act);
  a.ybuf = nullptr;  // (QuantLinear's fp32 partial sums)
  a.ybf = reinterpret_cast<uint16_t *>(ws + w.ybuf);
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
  a.ksplit = 1;
  a.g1_done = reinterpret_cast<int32_t *>(ws + w.g1_done);
  a.g1_seen = reinterpret_cast<int32_t *>(ws + w.g1_seen);
  a.bar = reinterpret_cast<int32_t *>(ws + w.bar);
  a.status = reinterpret_cast<uint32_t *>(ws + w.status);
  return a;
}

// [x permute] -> [plan] -> G1 -> G2 -> combine, or the fused layer kernel
// (one launch).  The streaming and fused GEMMs stage x themselves; the
// general and wide ones need its K-slot permuted copy in the workspace
// (x_permuted: already written by the router).  With logits (fused only),
// the fused kernel routes the tokens itself and writes ids / weights to
// ids_out / topk_weights (workspace).
int moe_forward_impl(const void *x, bool x_permuted, int64_t T, int H, int I, int E, int k,
                     const int8_t *q1, const float *s1, const int8_t *q2, const float *s2, int bits,
                     int64_t group_w1, int64_t group_w2, int flags, const int32_t *topk_ids,
                     const float *topk_weights, char *ws, void *out, hipStream_t st, ProfileMarks &pm,
                     int first_mark, const void *logits = nullptr, int ldt = LQ_F32, int renorm = 0,
                     int32_t *ids_out = nullptr) {
  const WsLayout w = ws_layout(T, H, I, E, k);
  const int64_t g1 = effective_group(H, group_w1);
  const int64_t g2 = effective_group(I, group_w2);
  // the folded form applies one scale per 128-wide K chunk
  const bool folded = (flags & LQ_MOE_FOLDED_SCALES) && g1 % kKC == 0 && g2 % kKC == 0;
  const Path path = choose_path(bits, T, H, I, E, k, group_w1, group_w2, flags);
  const bool stream = path == Path::kStream;
  const bool fused = fused_eligible(path, folded, T, E, k, flags);

  PlanArgs p = plan_args(topk_ids, T, E, k, ws, w);
  if (path == Path::kWide) p.block_rows = kWRows;
  MoeArgs a = layer_args(x, T, H, I, E, k, q1, s1, q2, s2, g1, g2, topk_ids, topk_weights, ws, w, p, out);
  if (fused) {
    if (logits) {
      a.logits = logits;
      a.ldt = ldt;
      a.renorm = renorm;
      a.ids_out = ids_out;
      a.w_out = const_cast<float *>(topk_weights);
    }
    pm.mark(first_mark);
    const int rc = bits == 4 ? launch_fused<4>(a, st) : launch_fused<8>(a, st);
    if (rc) return rc;
    for (int i = 1; i <= 3; ++i) pm.mark(first_mark + i);  // one launch: the later stages take no time
    return pm.rc;
  }
  if (logits) return fail(LQ_ERR_RUNTIME, "moe_forward: in-kernel routing needs the fused layer kernel");
  if (!stream && !x_permuted) {
    const int64_t n8 = T * H / 8;
    permute_rows_kernel<<<static_cast<int>(ceil_div(n8, 256)), 256, 0, st>>>(
        static_cast<const uint16_t *>(x), n8, reinterpret_cast<uint16_t *>(ws + w.xperm));
  }
  // small layers on the streaming GEMMs plan their blocks in-kernel
  // (every block of the in-kernel plan needs a CU of its own: there are at
  // most ceil(T*k / 32) + min(E, T*k) blocks)
  const int64_t nb_max = ceil_div(T * k, kRowsMax) + std::min<int64_t>(E, T * k);
  const bool inplan =
      stream && T * k <= kPlanMaxN && nb_max <= device_info().cus && device_info().cus <= kMaxSlots;
  int rc = LQ_OK;
  const int64_t nseg = ceil_div(T * k, kPlanSeg);
  if (inplan) {
    // no plan launch
  } else if (nseg > 1) {  // large layers: one workgroup per segment of assignments
    int32_t *segcnt = reinterpret_cast<int32_t *>(ws + w.segcnt);
    plan_count_kernel<<<static_cast<int>(nseg), kPlanBlock, 0, st>>>(p, segcnt);
    rc = check_launch("moe_plan_count");
    if (rc) return rc;
    plan_scatter_kernel<<<static_cast<int>(nseg), kPlanBlock, 0, st>>>(p, segcnt, static_cast<int>(nseg));
    rc = check_launch("moe_plan_scatter");
  } else {
    plan_kernel<<<1, kPlanBlock, 0, st>>>(p);
    rc = check_launch("moe_plan");
  }
  if (rc) return rc;
  pm.mark(first_mark);
  const int64_t blocks = max_blocks_for(T, E, k);
  const int64_t max_g1 = blocks * (I / kF1), max_g2 = blocks * (H / kR2);
  if (bits == 4)
    rc = folded ? launch_phases<4, true>(a, max_g1, max_g2, st, pm, first_mark, path, inplan)
                : launch_phases<4, false>(a, max_g1, max_g2, st, pm, first_mark, path, inplan);
  else
    rc = folded ? launch_phases<8, true>(a, max_g1, max_g2, st, pm, first_mark, path, inplan)
                : launch_phases<8, false>(a, max_g1, max_g2, st, pm, first_mark, path, inplan);
  if (rc) return rc;
  return pm.rc;
}

ProfileMarks take_profile(hipStream_t st) {
  ProfileMarks pm{t_prof_events, t_prof_n, st};
  t_prof_events = nullptr;
  t_prof_n = 0;
  return pm;
}

}  // namespace

int launch_permute(const int32_t *ids, int64_t N, int E, int32_t *counts, int32_t *offsets, int32_t *sorted,
                   hipStream_t st) {
  PlanArgs p{};
  p.ids = ids;
  p.N = N;
  p.E = E;
  p.counts = counts;
  p.offsets = offsets;
  p.sorted = sorted;
  p.blocks = nullptr;
  p.block_rows = kRowsMax;
  p.srow = nullptr;
  p.k = 1;
  plan_kernel<<<1, kPlanBlock, 0, st>>>(p);
  return check_launch("moe_permute");
}

}  // namespace lq

using namespace lq;

extern "C" size_t lq_moe_workspace_bytes(int64_t T, int H, int I, int E, int k) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 0;
  return ws_layout(T, H, I, E, k).total;
}

extern "C" size_t lq_moe_sync_bytes(void) { return ws_layout(1, 1, 1, 1, 1).sync_end; }

extern "C" int lq_moe_workspace_init(void *workspace, lq_stream_t stream) {
  if (!workspace) return fail(LQ_ERR_VALUE, "moe_workspace_init: null workspace");
  LQ_HIP_CHECK(hipMemsetAsync(workspace, 0, lq_moe_sync_bytes(), as_stream(stream)));
  return LQ_OK;
}

extern "C" int lq_moe_status(const void *workspace, uint32_t *status, int clear, lq_stream_t stream) {
  if (!workspace || !status) return fail(LQ_ERR_VALUE, "moe_status: null pointer");
  const hipStream_t st = as_stream(stream);
  LQ_HIP_CHECK(hipMemcpyAsync(status, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  LQ_HIP_CHECK(hipStreamSynchronize(st));
  if (clear && *status) {
    // the counters of a call whose wait gave up may be left non-zero: clear the whole sync region
    LQ_HIP_CHECK(hipMemsetAsync(const_cast<void *>(workspace), 0, lq_moe_sync_bytes(), st));
  }
  return LQ_OK;
}

extern "C" int lq_moe_profile_events(void *const *events, int n_events) {
  if (n_events < 0) return fail(LQ_ERR_VALUE, "moe_profile_events: negative count");
  t_prof_events = n_events ? events : nullptr;
  t_prof_n = n_events;
  return LQ_OK;
}

extern "C" int lq_moe_forward(const void *x, int64_t T, int H, int I, int E, int k, const int8_t *q1,
                              const float *s1, const int8_t *q2, const float *s2, int bits, int64_t group_w1,
                              int64_t group_w2, int flags, const int32_t *topk_ids, const float *topk_weights,
                              void *workspace, size_t ws_bytes, void *out, lq_stream_t stream) {
  const hipStream_t st = as_stream(stream);
  ProfileMarks pm = take_profile(st);
  int rc = validate_layer(x, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, flags, workspace, ws_bytes,
                          out);
  if (rc || T == 0) return rc;
  if (!topk_ids || !topk_weights) return fail(LQ_ERR_VALUE, "moe_forward: null routing pointer");
  pm.mark(0);
  return moe_forward_impl(x, false, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, flags,
                          topk_ids, topk_weights, static_cast<char *>(workspace), out, st, pm, 1);
}

extern "C" int lq_moe_layer(const void *x, const void *logits, int logits_dtype, int64_t T, int H, int I, int E,
                            int k, int renormalize, const int8_t *q1, const float *s1, const int8_t *q2,
                            const float *s2, int bits, int64_t group_w1, int64_t group_w2, int flags,
                            void *workspace, size_t ws_bytes, void *out, int32_t *topk_ids_out,
                            lq_stream_t stream) {
  const hipStream_t st = as_stream(stream);
  ProfileMarks pm = take_profile(st);
  int rc = validate_layer(x, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, flags, workspace, ws_bytes,
                          out);
  if (rc || T == 0) return rc;
  if (!logits) return fail(LQ_ERR_VALUE, "moe_layer: null logits");
  char *ws = static_cast<char *>(workspace);
  const WsLayout w = ws_layout(T, H, I, E, k);
  int32_t *ids = topk_ids_out ? topk_ids_out : reinterpret_cast<int32_t *>(ws + w.ids);
  float *weights = reinterpret_cast<float *>(ws + w.weights);
  pm.mark(0);
  const Path path = choose_path(bits, T, H, I, E, k, group_w1, group_w2, flags);
  const bool folded = (flags & LQ_MOE_FOLDED_SCALES) && effective_group(H, group_w1) % kKC == 0 &&
                      effective_group(I, group_w2) % kKC == 0;
  if (fused_eligible(path, folded, T, E, k, flags) && route_in_kernel(T, E)) {
    if (logits_dtype != LQ_F32 && logits_dtype != LQ_BF16 && logits_dtype != LQ_F16)
      return fail(LQ_ERR_VALUE, "route_topk: logits must be float32, float16 or bfloat16");
    pm.mark(1);  // no router launch: the fused kernel routes
    return moe_forward_impl(x, true, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, flags, ids, weights,
                            ws, out, st, pm, 2, logits, logits_dtype, renormalize, ids);
  }
  // the general GEMMs stage the K-slot permuted copy of x the router writes
  rc = launch_route_topk(logits, logits_dtype, T, E, k, renormalize, ids, weights, st,
                         static_cast<const uint16_t *>(x), H,
                         path == Path::kStream ? nullptr : reinterpret_cast<uint16_t *>(ws + w.xperm));
  if (rc) return rc;
  pm.mark(1);
  return moe_forward_impl(x, true, T, H, I, E, k, q1, s1, q2, s2, bits, group_w1, group_w2, flags, ids,
                          weights, ws, out, st, pm, 2);
}

// ---------------------------------------------------------------------------
// allocation-free layer: the workspace is a file-scope device array
// ---------------------------------------------------------------------------

namespace lq {

// Each GPU the library runs on holds its own copy of this array from the
// code object's load to the end of the process.  64 MiB covers every layer
// whose per-assignment buffers fit: the gate / up rows (T*k*2I*2 bytes) and
// the bf16 slot outputs (T*k*H*2) are the largest terms, 16 MiB each at
// T*k = 4096 with H = 2048, I = 1024.
constexpr size_t kScratchBytes = size_t{64} << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

// Device addresses of `scratch`, one per device, taken once with that device
// current.  The host-side name `scratch` is not a device address: only these
// pointers reach kernels.
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
char *g_scratch_ptr[kScratchDevices] = {};

int scratch_on_current_device(char **out) {
  int dev = 0;
  LQ_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices)
    return fail(LQ_ERR_UNSUPPORTED, "moe_layer_noalloc: device index " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    LQ_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(LQ_ERR_RUNTIME, "moe_layer_noalloc: hipGetSymbolAddress gave a null address");
    g_scratch_ptr[dev] = static_cast<char *>(p);
  }
  *out = g_scratch_ptr[dev];
  return LQ_OK;
}

// Clears n 32-bit words with vector stores (a kernel rather than a memset
// node, so a captured call replays it as well).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *__restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0u;
}

}  // namespace lq

extern "C" int lq_moe_layer_noalloc(const void *x, const void *logits, int logits_dtype, int64_t T, int H, int I,
                                    int E, int k, int renormalize, const int8_t *q1, const float *s1,
                                    const int8_t *q2, const float *s2, int bits, int64_t group_w1,
                                    int64_t group_w2, int flags, void *out, int32_t *topk_ids_out,
                                    lq_stream_t stream) {
  // shape errors other than the scratch limit are lq_moe_layer's to report
  if (T >= 0 && T <= (int64_t{1} << 18) && H > 0 && I > 0 && E > 0 && E <= kMaxExperts && k > 0 && k <= E) {
    const size_t need = ws_layout(T, H, I, E, k).total;
    if (need > kScratchBytes)
      return fail(LQ_ERR_UNSUPPORTED, "moe_layer_noalloc: this layer needs " + std::to_string(need) +
                                          " bytes of scratch, more than the static array's " +
                                          std::to_string(kScratchBytes) +
                                          "; split the tokens or call lq_moe_layer with a workspace");
  }
  char *ws = nullptr;
  int rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  const hipStream_t st = as_stream(stream);
  // the sync region must start zero; a call whose bounded wait gave up may
  // have left it otherwise, so every call clears it first
  const int words = static_cast<int>(lq_moe_sync_bytes() / sizeof(uint32_t));
  zero_words_kernel<<<1, 256, 0, st>>>(reinterpret_cast<uint32_t *>(ws), words);
  rc = check_launch("moe_layer_noalloc");
  if (rc) return rc;
  return lq_moe_layer(x, logits, logits_dtype, T, H, I, E, k, renormalize, q1, s1, q2, s2, bits, group_w1,
                      group_w2, flags, ws, kScratchBytes, out, topk_ids_out, stream);
}

// K slices of the general GEMM for QuantLinear: with few row blocks the
// items (block, 128-row slice) cannot fill the GPU, so each item also takes
// one of S equal K slices (whole 128-wide chunks) and writes its partial sums
// to slot S * row + slice of the workspace; the combine adds the S slots in
// ascending order (deterministic).  S doubles until about 512 items exist
// (two per CU), capped at 16.  A pure function of the shape, so the
// workspace query and the call agree.
int linear_ksplit(int64_t M, int K, int N) {
  if (K % kKC != 0) return 1;
  const int64_t items = ceil_div(M, kRowsMax) * (N / kR2);
  const int nkc = K / kKC;
  int S = 1;
  while (items * S < 512 && S < 16 && nkc % (2 * S) == 0) S *= 2;
  return S;
}

// the wide kernels take a QuantLinear from 128 rows on (their 128-row
// dequant amortisation; measured on MI355X, 8192 x 8192 INT8: the general
// kernel is ahead at 64 rows), with K slices of whole 256-wide pairs of
// chunks until about 512 items exist (at most 16)
bool linear_wide(int64_t M, int K, int N, int flags) {
  if (flags & LQ_MOE_WIDE_KERNEL) return true;
  if (flags & LQ_MOE_GENERAL_KERNEL) return false;
  return wide_eligible(N, K, 0) && M >= kWRows;
}

// a few rows without a forced family take the one-launch small kernel (its
// waves are the general path's K slices, at most kLinMaxSlices of them; two
// row tiles fit its registers with up to 8 slices)
bool linear_small(int64_t M, int K, int N, int flags) {
  if (flags & (LQ_MOE_WIDE_KERNEL | LQ_MOE_GENERAL_KERNEL)) return false;
  if (M < 1 || K % kKC != 0) return false;
  return M <= 16 || (M <= 32 && linear_ksplit(M, K, N) <= 8);
}

int linear_wide_ksplit(int64_t M, int K, int N) {
  const int64_t items = ceil_div(M, kWRows) * (N / kWR2);
  const int npair = K / (2 * kKC);
  int S = 1;
  while (items * S < 512 && S < 16 && npair % (2 * S) == 0) S *= 2;
  return S;
}

// Workspace of a QuantLinear call: the one-expert plan (offsets, sorted
// rows, row blocks of 32 or 128 rows), the S slots of every row (ids 0,
// weights 1), x in K-slot order [M, K] bf16 and the S partial sums of every
// output [M, S, N] fp32.  S is the larger of the two families' K-slice counts,
// so one size serves either family.
struct LinLayout {
  size_t offsets, sorted, srow, hdr, blocks, ids, weights, act, ybuf, total;
  int S;
};

LinLayout lin_layout(int64_t M, int K, int N) {
  LinLayout w;
  w.S = std::max(linear_ksplit(M, K, N), K % (2 * kKC) == 0 ? linear_wide_ksplit(M, K, N) : 1);
  const int64_t slots = M * w.S;
  size_t off = 0;
  auto take = [&](size_t &field, size_t bytes) {
    field = off;
    off = align256(off + bytes);
  };
  take(w.offsets, sizeof(int32_t) * 2);
  take(w.sorted, sizeof(int32_t) * M);
  take(w.srow, sizeof(int32_t) * M);
  take(w.hdr, sizeof(PlanHeader));
  take(w.blocks, sizeof(int4) * std::max<int64_t>(1, ceil_div(M, kRowsMax)));
  take(w.ids, sizeof(int32_t) * slots);
  take(w.weights, sizeof(float) * slots);
  take(w.act, sizeof(uint16_t) * M * K);
  take(w.ybuf, sizeof(float) * slots * N);
  w.total = off;
  return w;
}

// QuantLinear (runtime/linear.py:127-131): out = bf16(x . dequant(W)^T) with
// fp32 accumulation, W [N, K] packed INT4 / INT8 with fp32 group scales
// along K -- the layer's second GEMM with one expert, top-1, weight 1.0:
// set-up (x into K-slot order, ids 0, weights 1, and the one-expert plan),
// GEMM2 (the wide family from 128 rows on, else the general one; both split
// K into slices until about 512 items exist), combine.
extern "C" size_t lq_linear_workspace_bytes(int64_t M, int K, int N) {
  if (M < 0 || K <= 0 || N <= 0) return 0;
  return lin_layout(M, K, N).total;
}

extern "C" int lq_quant_linear(const void *x, int64_t M, int K, int N, const int8_t *q, const float *s, int bits,
                               int64_t group, int flags, void *workspace, size_t ws_bytes, void *out,
                               lq_stream_t stream) {
  const hipStream_t st = as_stream(stream);
  if (bits != 4 && bits != 8) return fail(LQ_ERR_VALUE, "bits must be 8 or 4, got " + std::to_string(bits));
  if (M < 0 || K <= 0 || N <= 0) return fail(LQ_ERR_VALUE, "quant_linear: bad shape");
  if (flags & ~(LQ_MOE_GENERAL_KERNEL | LQ_MOE_WIDE_KERNEL)) return fail(LQ_ERR_VALUE, "quant_linear: unknown flags");
  if ((flags & LQ_MOE_GENERAL_KERNEL) && (flags & LQ_MOE_WIDE_KERNEL))
    return fail(LQ_ERR_VALUE, "quant_linear: LQ_MOE_WIDE_KERNEL and LQ_MOE_GENERAL_KERNEL exclude each other");
  if (N % kR2 != 0 || K % kF1 != 0)
    return fail(LQ_ERR_UNSUPPORTED, "quant_linear: needs out_features % 128 == 0 and in_features % 64 == 0");
  const int64_t g = effective_group(K, group);
  if (g % 32 != 0)
    return fail(LQ_ERR_UNSUPPORTED, "quant_linear: the group length along K must be a multiple of 32 (got " +
                                        std::to_string(g) + ")");
  const bool wide_ok = wide_eligible(N, K, 0);
  if ((flags & LQ_MOE_WIDE_KERNEL) && !wide_ok)
    return fail(LQ_ERR_UNSUPPORTED, "quant_linear: the wide kernels need out_features % 256 == 0 and "
                                    "in_features % 256 == 0");
  if (M > (int64_t{1} << 18) || M * static_cast<int64_t>(N > K ? N : K) * 4 > 0x7FFFFFFFll ||
      M * static_cast<int64_t>(K) * 2 >= kOutOfRange)
    return fail(LQ_ERR_UNSUPPORTED, "quant_linear: too many rows for one call");
  if (int64_t{1} * N * K >= kOutOfRange) return fail(LQ_ERR_UNSUPPORTED, "quant_linear: weight exceeds 2 GiB");
  if (M == 0) return LQ_OK;
  if (!x || !q || !s || !workspace || !out) return fail(LQ_ERR_VALUE, "quant_linear: null pointer");
  if (!aligned16(x) || !aligned16(q) || !aligned16(workspace) || !aligned16(out))
    return fail(LQ_ERR_VALUE, "quant_linear: x, qweight, workspace and out must be 16-byte aligned");
  const bool wide = linear_wide(M, K, N, flags);
  const int S = wide ? linear_wide_ksplit(M, K, N) : linear_ksplit(M, K, N);
  const LinLayout w = lin_layout(M, K, N);
  if (ws_bytes < w.total)
    return fail(LQ_ERR_VALUE, "quant_linear: workspace too small (" + std::to_string(ws_bytes) + " < " +
                                  std::to_string(w.total) + ")");
  if (linear_small(M, K, N, flags)) {
    // one launch: each workgroup sums the general path's S K slices of two
    // 16-column tiles itself (no set-up, no workspace, no combine)
    LinArgs la;
    la.x = static_cast<const uint16_t *>(x);
    la.q = q;
    la.s = s;
    la.out = static_cast<uint16_t *>(out);
    la.M = static_cast<int>(M);
    la.K = K;
    la.N = N;
    la.G = static_cast<int>(g);
    la.ng = static_cast<int>(K / g);
    la.nks = K / kKC / S;
    const dim3 grid(static_cast<unsigned>(N / (16 * kLinNT))), block(static_cast<unsigned>(64 * S));
    const bool two = M > 16;
    // chunks in flight per wave: 4 for one row tile with up to 8 waves (256
    // registers each), else 2 (two row tiles take linear_small only with up
    // to 8 waves: with 16, 128 registers do not hold them)
    const int kd = S <= 8 && !two ? (la.nks % 4 == 0 ? 4 : la.nks % 2 == 0 ? 2 : 1) : (la.nks % 2 == 0 ? 2 : 1);
#define LQ_LIN_SMALL(B)                                                                        \
  do {                                                                                         \
    if (two) {                                                                                 \
      if (kd == 2) linear_small_kernel<B, 2, 2, 8><<<grid, block, 0, st>>>(la);                \
      else linear_small_kernel<B, 2, 1, 8><<<grid, block, 0, st>>>(la);                        \
    } else if (S <= 8) {                                                                       \
      if (kd == 4) linear_small_kernel<B, 1, 4, 8><<<grid, block, 0, st>>>(la);                \
      else if (kd == 2) linear_small_kernel<B, 1, 2, 8><<<grid, block, 0, st>>>(la);           \
      else linear_small_kernel<B, 1, 1, 8><<<grid, block, 0, st>>>(la);                        \
    } else {                                                                                   \
      if (kd == 2) linear_small_kernel<B, 1, 2, kLinMaxSlices><<<grid, block, 0, st>>>(la);    \
      else linear_small_kernel<B, 1, 1, kLinMaxSlices><<<grid, block, 0, st>>>(la);            \
    }                                                                                          \
  } while (0)
    if (bits == 4)
      LQ_LIN_SMALL(4);
    else
      LQ_LIN_SMALL(8);
#undef LQ_LIN_SMALL
    return check_launch("quant_linear_small");
  }
  char *ws = static_cast<char *>(workspace);
  int32_t *ids = reinterpret_cast<int32_t *>(ws + w.ids);
  float *weights = reinterpret_cast<float *>(ws + w.weights);
  uint16_t *act = reinterpret_cast<uint16_t *>(ws + w.act);
  const int64_t n8 = M * K / 8;
  PlanArgs p;
  p.ids = ids;
  p.N = M;
  p.E = 1;
  p.k = 1;
  p.counts = nullptr;
  p.offsets = reinterpret_cast<int32_t *>(ws + w.offsets);
  p.sorted = reinterpret_cast<int32_t *>(ws + w.sorted);
  p.srow = reinterpret_cast<int32_t *>(ws + w.srow);
  p.blocks = reinterpret_cast<int4 *>(ws + w.blocks);
  p.hdr = reinterpret_cast<PlanHeader *>(ws + w.hdr);
  p.block_rows = wide ? kWRows : kRowsMax;
  linear_setup_kernel<<<static_cast<int>(ceil_div(std::max(n8, M * S), 256)), 256, 0, st>>>(
      static_cast<const uint16_t *>(x), n8, M, M * S, act, ids, weights, p.sorted, p.srow, p.blocks, p.hdr,
      p.block_rows);
  int rc = check_launch("quant_linear_setup");
  if (rc) return rc;
  MoeArgs a{};
  a.q2 = q;
  a.s2 = s;
  a.ids = ids;
  a.topk_w = weights;
  a.offsets = p.offsets;
  a.sorted = p.sorted;
  a.blocks = p.blocks;
  a.srow = p.srow;
  a.hdr = p.hdr;
  a.act = act;
  a.ybuf = reinterpret_cast<float *>(ws + w.ybuf);
  a.out = static_cast<uint16_t *>(out);
  a.T = M;
  a.H = N;
  a.I = K;
  a.E = 1;
  a.k = 1;
  a.g2 = static_cast<int>(g);
  a.ng2 = static_cast<int>(K / g);
  a.ksplit = S;
  const int64_t blocks = max_blocks_for(M, 1, 1);
  if (wide) {
    const int64_t items = (1 + M / kWRows) * (N / kWR2) * S;
    const bool g128 = a.g2 == kKC;
    if (bits == 4 && g128)
      moe_wide_kernel<4, false, true><<<wide_grid<4, false, true>(items), kWThreads, 0, st>>>(a);
    else if (bits == 4)
      moe_wide_kernel<4, false, false><<<wide_grid<4, false, false>(items), kWThreads, 0, st>>>(a);
    else if (g128)
      moe_wide_kernel<8, false, true><<<wide_grid<8, false, true>(items), kWThreads, 0, st>>>(a);
    else
      moe_wide_kernel<8, false, false><<<wide_grid<8, false, false>(items), kWThreads, 0, st>>>(a);
  } else {
    const int64_t items = blocks * (N / kR2) * S;
    const bool g128 = a.g2 == kKC;
    if (bits == 4 && g128)
      moe_gemm_kernel<4, false, false, true><<<gemm_grid<4, false, false, true>(items), kThreads, 0, st>>>(a);
    else if (bits == 4)
      moe_gemm_kernel<4, false, false, false><<<gemm_grid<4, false, false, false>(items), kThreads, 0, st>>>(a);
    else if (g128)
      moe_gemm_kernel<8, false, false, true><<<gemm_grid<8, false, false, true>(items), kThreads, 0, st>>>(a);
    else
      moe_gemm_kernel<8, false, false, false><<<gemm_grid<8, false, false, false>(items), kThreads, 0, st>>>(a);
  }
  rc = check_launch("quant_linear_gemm");
  if (rc) return rc;
  const int64_t n2 = M * N / 2;
  combine_kernel<false><<<static_cast<int>(ceil_div(n2, kCombineBlock)), kCombineBlock, 0, st>>>(a.ybuf, ids, M, N,
                                                                                                 S, 1, a.out);
  return check_launch("quant_linear_combine");
}
