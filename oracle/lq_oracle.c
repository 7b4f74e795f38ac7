/*
 * lq_oracle.c -- CPU restatement of LLaDA_Quant's quantized expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library, and only as the checker the
 * HIP path is compared against (or as the timed CPU baseline).  The product
 * (liblladaq.so and the llada_quant_amd package) never links or calls it.
 *
 * Each function cites the reference code it restates (paths relative to
 * Ahmed-Hedhili-se/LLaDA_Quant v0.2.0).  Arithmetic follows the reference's
 * torch-on-CPU semantics exactly: IEEE binary32 operations in the same order,
 * round-half-to-even for torch.round, and torch's CPU summation order for the
 * per-group squared error of the MSE scale search.
 *
 * Build: see oracle/Makefile (gcc -O2, no fast-math: every float operation
 * must be the correctly rounded IEEE one).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OQ_F32 0
#define OQ_F16 1
#define OQ_BF16 2

/* ---------------------------------------------------------------------- */
/* scalar conversions                                                      */
/* ---------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* torch's float -> bfloat16 (c10::BFloat16 round_to_nearest_even): NaN maps
 * to 0x7FC0, everything else rounds half to even on the dropped 16 bits. */
uint16_t oq_f32_to_bf16(float f) {
  if (isnan(f)) return 0x7FC0;
  uint32_t u = f2u(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oq_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16 -> binary32 (exact). */
float oq_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* IEEE binary32 -> binary16, round half to even (what c10::Half does). */
uint16_t oq_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u); /* NaN */
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
  if (a < 0x38800000u) {                                   /* subnormal half */
    /* value / 2^-24, rounded half-even: exact in double for the range */
    double v = (double)u2f(a) * 16777216.0;
    double r = nearbyint(v);
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t mant_odd = (a >> 13) & 1u;
  a += 0xFFFu + mant_odd;
  a -= 0x38000000u; /* rebias 127 -> 15 */
  return (uint16_t)(sign | (uint16_t)(a >> 13));
}

static float load_as_f32(const void *p, int dtype, int64_t i) {
  switch (dtype) {
    case OQ_F16: return oq_f16_to_f32(((const uint16_t *)p)[i]);
    case OQ_BF16: return oq_bf16_to_f32(((const uint16_t *)p)[i]);
    default: return ((const float *)p)[i];
  }
}

/* Round an fp32 value to `dtype` and back (tensor.to(dtype).float()). */
static float round_through(float v, int dtype) {
  switch (dtype) {
    case OQ_F16: return oq_f16_to_f32(oq_f32_to_f16(v));
    case OQ_BF16: return oq_bf16_to_f32(oq_f32_to_bf16(v));
    default: return v;
  }
}

static void store_from_f32(void *p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case OQ_F16: ((uint16_t *)p)[i] = oq_f32_to_f16(v); break;
    case OQ_BF16: ((uint16_t *)p)[i] = oq_f32_to_bf16(v); break;
    default: ((float *)p)[i] = v; break;
  }
}

/* ---------------------------------------------------------------------- */
/* algorithms/symmetric.py:29-36                                           */
/* ---------------------------------------------------------------------- */

int oq_qmax(int bits) { return (1 << (bits - 1)) - 1; }
int oq_qmin(int bits) { return -(1 << (bits - 1)); }

/* algorithms/symmetric.py:85-90 (_as_groups): G divides K -> K/G groups of
 * G, else (or G == -1) one group spanning the whole last axis. */
int64_t oq_effective_group(int64_t k, int64_t group_size) {
  if (group_size == -1 || group_size <= 0 || k % group_size != 0) return k;
  return group_size;
}

/* ---------------------------------------------------------------------- */
/* torch CPU summation order of x.sum(dim=-1) over a contiguous fp32 row.  */
/*                                                                         */
/* Restates ATen's cascade_sum for a contiguous inner reduction as it runs */
/* on x86 (8-float vectors, 4-way ILP, 4-level cascade):                   */
/*   vectorized_inner_sum: vec_acc = row_sum(vectors); final = 0;          */
/*       final += tail scalars; final += vec_acc lanes 0..7                */
/*   row_sum: multi_row_sum over rows of 4 vectors, tail vectors into      */
/*       partial 0, then partial0 += partial1, += partial2, += partial3    */
/*   multi_row_sum: level_power = max(4, ceil_log2(n)/4) cascade           */
/* The search loss `work.pow_(2).sum(dim=-1)` (symmetric.py:198) is summed */
/* this way; the order decides which candidate wins a near tie.  Checked   */
/* bit-exact against torch for row lengths 1..8192 in                      */
/* tests/test_oracle.py.                                                   */
/* ---------------------------------------------------------------------- */

#define OQ_LANES 8
#define OQ_ILP 4
#define OQ_LEVELS 4

static int64_t ceil_log2_i64(int64_t x) {
  if (x <= 1) return 0;
  int64_t r = 0;
  uint64_t v = (uint64_t)(x - 1);
  while (v) { r++; v >>= 1; }
  return r;
}

/* multi_row_sum over `size` rows; row i supplies OQ_ILP accumulator inputs,
 * each of width `w` floats (w = OQ_LANES for vectors, 1 for scalars).
 * elem(i, k, l) = x[(i*OQ_ILP + k) * w + l]. */
static void multi_row_sum(const float *x, int64_t size, int w, float *out /* [OQ_ILP][OQ_LANES] */) {
  float acc[OQ_LEVELS][OQ_ILP][OQ_LANES];
  memset(acc, 0, sizeof(acc));
  int64_t level_power = ceil_log2_i64(size) / OQ_LEVELS;
  if (level_power < 4) level_power = 4;
  const int64_t level_step = (int64_t)1 << level_power;
  const int64_t level_mask = level_step - 1;
  int64_t i = 0;
  for (; i + level_step <= size;) {
    for (int64_t j = 0; j < level_step; ++j, ++i)
      for (int k = 0; k < OQ_ILP; ++k)
        for (int l = 0; l < w; ++l) acc[0][k][l] += x[(i * OQ_ILP + k) * w + l];
    for (int j = 1; j < OQ_LEVELS; ++j) {
      for (int k = 0; k < OQ_ILP; ++k)
        for (int l = 0; l < w; ++l) {
          acc[j][k][l] += acc[j - 1][k][l];
          acc[j - 1][k][l] = 0.0f;
        }
      const int64_t mask = level_mask << (j * level_power);
      if ((i & mask) != 0) break;
    }
  }
  for (; i < size; ++i)
    for (int k = 0; k < OQ_ILP; ++k)
      for (int l = 0; l < w; ++l) acc[0][k][l] += x[(i * OQ_ILP + k) * w + l];
  for (int j = 1; j < OQ_LEVELS; ++j)
    for (int k = 0; k < OQ_ILP; ++k)
      for (int l = 0; l < w; ++l) acc[0][k][l] += acc[j][k][l];
  for (int k = 0; k < OQ_ILP; ++k)
    for (int l = 0; l < w; ++l) out[k * OQ_LANES + l] = acc[0][k][l];
}

/* row_sum over `size` units of width w (units are vectors or scalars). */
static void row_sum(const float *x, int64_t size, int w, float *res /* [w] */) {
  const int64_t size_ilp = size / OQ_ILP;
  float ps[OQ_ILP][OQ_LANES];
  multi_row_sum(x, size_ilp, w, &ps[0][0]);
  for (int64_t i = size_ilp * OQ_ILP; i < size; ++i)
    for (int l = 0; l < w; ++l) ps[0][l] += x[i * w + l];
  for (int k = 1; k < OQ_ILP; ++k)
    for (int l = 0; l < w; ++l) ps[0][l] += ps[k][l];
  for (int l = 0; l < w; ++l) res[l] = ps[0][l];
}

float oq_torch_cpu_sum(const float *x, int64_t n) {
  float out = 0.0f; /* the output is zero-filled, then accumulated into */
  if (n >= OQ_LANES) {
    const int64_t vec_size = n / OQ_LANES;
    float vacc[OQ_LANES];
    row_sum(x, vec_size, OQ_LANES, vacc);
    float final_acc = 0.0f;
    for (int64_t k = vec_size * OQ_LANES; k < n; ++k) final_acc += x[k];
    for (int l = 0; l < OQ_LANES; ++l) final_acc += vacc[l];
    return out + final_acc;
  }
  float r;
  row_sum(x, n, 1, &r);
  return out + r;
}

/* ---------------------------------------------------------------------- */
/* algorithms/symmetric.py:117-119 (_amax_scale) and :122-204              */
/* (search_group_scale).  `w` holds fp32 values (the exact upcast of the   */
/* input dtype); one group is `glen` consecutive values.                   */
/* ---------------------------------------------------------------------- */

static float amax_scale(const float *w, int64_t glen, int bits) {
  float amax = 0.0f;
  for (int64_t i = 0; i < glen; ++i) {
    float a = fabsf(w[i]);
    if (a > amax || isnan(a)) amax = a;
  }
  return amax / (float)oq_qmax(bits); /* fp32 tensor / python int: IEEE divide */
}

/* candidate ratio as torch uses it: the python double
 * 1.0 - max_shrink * step / grid, converted to fp32 when it multiplies the
 * fp32 base tensor (symmetric.py:189-190). */
static float candidate_ratio(double max_shrink, int step, int grid) {
  double r = 1.0 - max_shrink * (double)step / (double)grid;
  return (float)r;
}

static float search_one_group(const float *w, int64_t glen, int bits, int grid,
                              double max_shrink, float *work) {
  const float qmax = (float)oq_qmax(bits), qmin = (float)oq_qmin(bits);
  const float base = amax_scale(w, glen, bits);
  float best_scale = base;
  float best_err = INFINITY;
  for (int step = 0; step < grid; ++step) {
    const float cand = base * candidate_ratio(max_shrink, step, grid);
    const float safe = cand > 0.0f ? cand : 1.0f;
    for (int64_t i = 0; i < glen; ++i) {
      float v = w[i] / safe;           /* work = wf / safe          */
      v = nearbyintf(v);               /* round_ (half to even)     */
      v = v < qmin ? qmin : v;         /* clamp_(qmin, qmax)        */
      v = v > qmax ? qmax : v;
      v = v * safe;                    /* mul_(safe)                */
      v = v - w[i];                    /* sub_(wf)                  */
      work[i] = v * v;                 /* pow_(2)                   */
    }
    const float err = oq_torch_cpu_sum(work, glen);
    if (err < best_err) { /* strict: the earlier (larger) ratio wins ties */
      best_err = err;
      best_scale = cand;
    }
  }
  return base > 0.0f ? best_scale : 0.0f;
}

/* w: n_groups x glen values in w_dtype; scale out: fp32 [n_groups]. */
int oq_search_group_scale(const void *w, int w_dtype, int64_t n_groups, int64_t glen,
                          int bits, int grid, double max_shrink, float *scale) {
  if (grid < 1 || !(max_shrink >= 0.0 && max_shrink < 1.0)) return 1;
  float *wf = (float *)malloc(sizeof(float) * (size_t)glen * 2);
  if (!wf) return 3;
  float *work = wf + glen;
  for (int64_t g = 0; g < n_groups; ++g) {
    for (int64_t i = 0; i < glen; ++i) wf[i] = load_as_f32(w, w_dtype, g * glen + i);
    scale[g] = search_one_group(wf, glen, bits, grid, max_shrink, work);
  }
  free(wf);
  return 0;
}

/* ---------------------------------------------------------------------- */
/* algorithms/symmetric.py:207-269 (quantize_tensor) + :296-313 (pack_int4)*/
/* w [rows, k] in w_dtype -> q int8 ([rows,k] or packed [rows,k/2]) and    */
/* scale [rows, ng] in scale_dtype.                                        */
/* ---------------------------------------------------------------------- */

int oq_quantize(const void *w, int w_dtype, int64_t rows, int64_t k, int bits,
                int64_t group_size, int mse, int grid, double max_shrink,
                int8_t *q, void *scale, int scale_dtype) {
  if (bits != 4 && bits != 8) return 1;
  if (bits == 4 && k % 2 != 0) return 1;
  const int64_t g = oq_effective_group(k, group_size);
  const int64_t ng = k / g;
  const float qmax = (float)oq_qmax(bits), qmin = (float)oq_qmin(bits);
  float *wf = (float *)malloc(sizeof(float) * (size_t)g * 2);
  int8_t *qrow = (int8_t *)malloc((size_t)k);
  if (!wf || !qrow) { free(wf); free(qrow); return 3; }
  float *work = wf + g;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t gi = 0; gi < ng; ++gi) {
      const int64_t base_idx = r * k + gi * g;
      for (int64_t i = 0; i < g; ++i) wf[i] = load_as_f32(w, w_dtype, base_idx + i);
      float chosen = mse ? search_one_group(wf, g, bits, grid, max_shrink, work)
                         : amax_scale(wf, g, bits);
      /* scale = chosen.to(scale_dtype); safe = where(scale > 0, scale, 1) */
      const float stored = round_through(chosen, scale_dtype);
      store_from_f32(scale, scale_dtype, r * ng + gi, stored);
      const float safe = stored > 0.0f ? stored : 1.0f;
      for (int64_t i = 0; i < g; ++i) {
        float v = nearbyintf(wf[i] / safe);
        v = v < qmin ? qmin : v;
        v = v > qmax ? qmax : v;
        qrow[gi * g + i] = (int8_t)v;
      }
    }
    if (bits == 4) {
      for (int64_t i = 0; i < k / 2; ++i) {
        const int lo = qrow[2 * i] & 0x0F, hi = qrow[2 * i + 1] & 0x0F;
        q[r * (k / 2) + i] = (int8_t)(uint8_t)(lo | (hi << 4));
      }
    } else {
      memcpy(q + r * k, qrow, (size_t)k);
    }
  }
  free(wf);
  free(qrow);
  return 0;
}

/* algorithms/symmetric.py:296-313: returns 1 if a value is outside [-8, 7]. */
int oq_pack_int4(const int8_t *q, int64_t rows, int64_t k, int8_t *packed) {
  if (k % 2 != 0) return 2;
  for (int64_t i = 0; i < rows * k; ++i)
    if (q[i] < -8 || q[i] > 7) return 1;
  for (int64_t i = 0; i < rows * k / 2; ++i) {
    const int lo = q[2 * i] & 0x0F, hi = q[2 * i + 1] & 0x0F;
    packed[i] = (int8_t)(uint8_t)(lo | (hi << 4));
  }
  return 0;
}

/* algorithms/symmetric.py:316-346: low = (b << 4) >> 4, high = b >> 4 with
 * arithmetic shifts on int8. */
void oq_unpack_int4(const int8_t *packed, int64_t n_bytes, int8_t *out) {
  for (int64_t i = 0; i < n_bytes; ++i) {
    const int b = packed[i];
    const int8_t lo = (int8_t)((int8_t)(b << 4) >> 4);
    const int8_t hi = (int8_t)(b >> 4);
    out[2 * i] = lo;
    out[2 * i + 1] = hi;
  }
}

/* algorithms/symmetric.py:272-293: (fp32(q) * fp32(s)).to(out_dtype). */
int oq_dequant(const int8_t *q, const void *scale, int scale_dtype, int64_t rows,
               int64_t k, int bits, int64_t group_size, void *out, int out_dtype) {
  if (bits != 4 && bits != 8) return 1;
  const int64_t g = oq_effective_group(k, group_size);
  const int64_t ng = k / g;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < k; ++i) {
      int v;
      if (bits == 4) {
        const int b = q[r * (k / 2) + i / 2];
        v = (i & 1) ? (int8_t)(b >> 4) : (int8_t)((int8_t)(b << 4) >> 4);
      } else {
        v = q[r * k + i];
      }
      const float s = load_as_f32(scale, scale_dtype, r * ng + i / g);
      store_from_f32(out, out_dtype, r * k + i, (float)v * s);
    }
  }
  return 0;
}

/* ---------------------------------------------------------------------- */
/* Routing: softmax(logits, fp32) then topk(k) (trajectory/llada.py:       */
/* 228-234).  Probabilities are computed in double from the fp32 logits;   */
/* ids are ordered by descending logit (= descending probability, softmax  */
/* being monotone), ties to the lower expert id.                           */
/* ---------------------------------------------------------------------- */

int oq_route_topk(const void *logits, int logits_dtype, int64_t T, int E, int k,
                  int renormalize, int32_t *ids, float *weights) {
  if (k < 1 || k > E) return 1;
  double *p = (double *)malloc(sizeof(double) * (size_t)E);
  float *x = (float *)malloc(sizeof(float) * (size_t)E);
  char *taken = (char *)malloc((size_t)E);
  if (!p || !x || !taken) { free(p); free(x); free(taken); return 3; }
  for (int64_t t = 0; t < T; ++t) {
    float m = -INFINITY;
    for (int e = 0; e < E; ++e) {
      x[e] = load_as_f32(logits, logits_dtype, t * E + e);
      if (x[e] > m) m = x[e];
    }
    double s = 0.0;
    for (int e = 0; e < E; ++e) { p[e] = exp((double)x[e] - (double)m); s += p[e]; }
    for (int e = 0; e < E; ++e) p[e] /= s;
    memset(taken, 0, (size_t)E);
    double wsum = 0.0;
    for (int j = 0; j < k; ++j) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || x[e] > x[best]) best = e;
      }
      taken[best] = 1;
      ids[t * k + j] = best;
      wsum += p[best];
    }
    for (int j = 0; j < k; ++j) {
      const double pj = p[ids[t * k + j]];
      weights[t * k + j] = (float)(renormalize ? pj / wsum : pj);
    }
  }
  free(p); free(x); free(taken);
  return 0;
}

/* Stable counting sort of the flat assignments by expert
 * (analysis/moe_regime.py:197-213 bincount; moe_align_block_size order). */
int oq_moe_permute(const int32_t *ids, int64_t T, int k, int E, int32_t *counts,
                   int32_t *offsets, int32_t *sorted) {
  const int64_t n = T * (int64_t)k;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t a = 0; a < n; ++a) {
    if (ids[a] < 0 || ids[a] >= E) return 1;
    counts[ids[a]]++;
  }
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t *fill = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
  if (!fill) return 3;
  for (int e = 0; e < E; ++e) fill[e] = offsets[e];
  for (int64_t a = 0; a < n; ++a) sorted[fill[ids[a]]++] = (int32_t)a;
  free(fill);
  return 0;
}

/* ---------------------------------------------------------------------- */
/* MoE layer with dequantized BF16 weights (the reference's dequantize-    */
/* then-fused_moe path), fp64 accumulation rounded where the reference     */
/* rounds:                                                                 */
/*   g, u = bf16(x W1[e][:I]^T), bf16(x W1[e][I:]^T)                       */
/*   act  = bf16(bf16(silu(g)) * u)  (INFERENCE_REPO_CHANGES.md:296-309)   */
/*   out[t] = sum_j w[t,j] * (act W2[e]^T)   returned in fp32              */
/* Gate/up split follows tests/unit/conftest.py:37-43 and                  */
/* benchmarks/bench_numerical.py:28-36.                                    */
/*   x [T,H] bf16 bits; w1 [E,2I,H] bf16 bits; w2 [E,H,I] bf16 bits        */
/* ---------------------------------------------------------------------- */

int oq_moe_forward(const uint16_t *x, int64_t T, int H, int I, int E, int k,
                   const uint16_t *w1, const uint16_t *w2, const int32_t *ids,
                   const float *weights, float *out) {
  for (int64_t a = 0; a < T * (int64_t)k; ++a)
    if (ids[a] < 0 || ids[a] >= E) return 1;
  int rc = 0;
#pragma omp parallel
  {
    float *xf = (float *)malloc(sizeof(float) * (size_t)H);
    float *act = (float *)malloc(sizeof(float) * (size_t)I);
    double *acc = (double *)malloc(sizeof(double) * (size_t)H);
    if (!xf || !act || !acc) {
#pragma omp atomic write
      rc = 3;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t t = 0; t < T; ++t) {
        for (int h = 0; h < H; ++h) xf[h] = oq_bf16_to_f32(x[t * H + h]);
        for (int h = 0; h < H; ++h) acc[h] = 0.0;
        for (int j = 0; j < k; ++j) {
          const int e = ids[t * k + j];
          const uint16_t *W1 = w1 + (int64_t)e * 2 * I * H;
          const uint16_t *W2 = w2 + (int64_t)e * H * I;
          for (int n = 0; n < I; ++n) {
            double g = 0.0, u = 0.0;
            const uint16_t *rg = W1 + (int64_t)n * H, *ru = W1 + (int64_t)(I + n) * H;
            for (int h = 0; h < H; ++h) {
              g += (double)xf[h] * (double)oq_bf16_to_f32(rg[h]);
              u += (double)xf[h] * (double)oq_bf16_to_f32(ru[h]);
            }
            const float gb = oq_bf16_to_f32(oq_f32_to_bf16((float)g));
            const float ub = oq_bf16_to_f32(oq_f32_to_bf16((float)u));
            const float silu = (float)((double)gb / (1.0 + exp(-(double)gb)));
            const float sb = oq_bf16_to_f32(oq_f32_to_bf16(silu));
            act[n] = oq_bf16_to_f32(oq_f32_to_bf16(sb * ub));
          }
          const double wj = (double)weights[t * k + j];
          for (int h = 0; h < H; ++h) {
            const uint16_t *r2 = W2 + (int64_t)h * I;
            double y = 0.0;
            for (int n = 0; n < I; ++n) y += (double)act[n] * (double)oq_bf16_to_f32(r2[n]);
            acc[h] += wj * y;
          }
        }
        for (int h = 0; h < H; ++h) out[t * H + h] = (float)acc[h];
      }
    }
    free(xf); free(act); free(acc);
  }
  return rc;
}
