/*
 * lladaq.h -- C ABI of liblladaq.so, the MI355X (gfx950) implementation of
 * LLaDA_Quant's quantized MoE expert path.
 *
 * Conventions
 *   - Every tensor argument is a caller-owned DEVICE pointer to contiguous,
 *     row-major memory on the current HIP device; sizes are element counts.
 *   - `stream` is a hipStream_t passed as an opaque pointer (NULL = the
 *     default stream). Every call is asynchronous with respect to the host
 *     and ordered on that stream.
 *   - Every function returns an LQ_* status. On failure lq_last_error()
 *     returns a thread-local message naming the problem. No C++ exception
 *     crosses this boundary, and no function allocates device memory:
 *     lq_moe_forward takes a caller-supplied workspace sized by
 *     lq_moe_workspace_bytes.
 *   - dtype codes: LQ_F32, LQ_F16, LQ_BF16 (IEEE binary32, binary16, bfloat16).
 *
 * Reference citations are to Ahmed-Hedhili-se/LLaDA_Quant v0.2.0
 * (src/LLaDA_Quant/...) and to the fused_moe interface it calls
 * (INFERENCE_REPO_CHANGES.md).
 */
#ifndef LLADAQ_H
#define LLADAQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LQ_ABI_VERSION 3

/* status codes */
#define LQ_OK 0
#define LQ_ERR_VALUE 1       /* bad argument; the Python layer raises ValueError   */
#define LQ_ERR_UNSUPPORTED 2 /* valid but not implemented on this path             */
#define LQ_ERR_RUNTIME 3     /* a HIP runtime call failed                          */

/* dtype codes */
#define LQ_F32 0
#define LQ_F16 1
#define LQ_BF16 2

/* lq_moe_forward / lq_moe_layer flags */
#define LQ_MOE_FOLDED_SCALES 1 /* exact integer codes in the MFMA, group scale in fp32 */
#define LQ_MOE_GENERAL_KERNEL 2 /* use the general GEMM kernels for every shape (same results) */
#define LQ_MOE_WIDE_KERNEL 4    /* use the wide (matrix-core) GEMM kernels (same results; H % 256, I % 256) */
#define LQ_MOE_STREAM_KERNEL 8  /* use the streaming (bandwidth) GEMM kernels (same results; see lq_moe_forward) */
#define LQ_MOE_FUSED_LAYER 16 /* streaming family, E <= 64, T*k <= 2048: the whole layer as one launch
                                 (moe_fused_kernel; same results) instead of GEMM1, GEMM2, combine */

/* scale search codes (QuantConfig.scale_search) */
#define LQ_SCALE_AMAX 0
#define LQ_SCALE_MSE 1

typedef void *lq_stream_t;

/* Version of this ABI (LQ_ABI_VERSION). */
int lq_abi_version(void);

/* Thread-local message of the last failed call on this thread. */
const char *lq_last_error(void);

/*
 * Pack int4 values (int8 storage, one value per byte) two per byte along the
 * last axis: element 2i in the low nibble, 2i+1 in the high nibble, two's
 * complement.  Replaces algorithms/symmetric.py:296-313 (pack_int4).
 *   q       [rows, k]      int8, values expected in [-8, 7]
 *   packed  [rows, k/2]    int8
 *   range_flag  one device int32 the caller zeroes; the kernel stores 1 into
 *           it if any value lies outside [-8, 7] (the Python layer then
 *           raises the reference's ValueError).
 * k must be even.
 */
int lq_pack_int4(const int8_t *q, int64_t rows, int64_t k, int8_t *packed,
                 int32_t *range_flag, lq_stream_t stream);

/*
 * Inverse of lq_pack_int4 with sign extension of both nibbles.
 * Replaces algorithms/symmetric.py:316-346 (unpack_int4).
 *   packed [rows, k_packed] int8  ->  out [rows, 2*k_packed] int8
 */
int lq_unpack_int4(const int8_t *packed, int64_t rows, int64_t k_packed,
                   int8_t *out, lq_stream_t stream);

/*
 * out = cast(fp32(q) * fp32(scale[row, k / G]), out_dtype), bit-exact to the
 * reference reconstruction.  Replaces algorithms/symmetric.py:272-293
 * (dequantize_tensor) and the PACKED property body runtime/moe.py:199-216.
 *   q      [rows, k] int8 (bits=8) or [rows, k/2] packed int8 (bits=4)
 *   scale  [rows, ng] in scale_dtype; ng = k/G, or 1 when group_size == -1 or
 *          G does not divide k (the reference's per-row fallback)
 *   out    [rows, k] in out_dtype
 */
int lq_dequant(const int8_t *q, const void *scale, int scale_dtype,
               int64_t rows, int64_t k, int bits, int64_t group_size,
               void *out, int out_dtype, lq_stream_t stream);

/*
 * Groupwise symmetric quantization of w [rows, k] along its last axis, with
 * amax or MSE clip-search scales; bits=4 output is packed.
 * Replaces algorithms/symmetric.py:207-269 (quantize_tensor) together with
 * :117-119 (_amax_scale) and :122-204 (search_group_scale).
 *   w       [rows, k] in w_dtype (f32, f16 or bf16)
 *   q       [rows, k] int8 (bits=8, or bits=4 with pack=0: one value per
 *           byte) or [rows, k/2] int8 (bits=4, pack!=0: two per byte)
 *   scale   [rows, ng] in scale_dtype
 * scale_search: LQ_SCALE_AMAX or LQ_SCALE_MSE; grid/max_shrink are the
 * search's candidate count and clip range (ignored for amax).
 */
int lq_quantize(const void *w, int w_dtype, int64_t rows, int64_t k, int bits,
                int pack, int64_t group_size, int scale_search, int grid,
                double max_shrink, int8_t *q, void *scale, int scale_dtype,
                lq_stream_t stream);

/*
 * MSE-optimal per-group scale alone (fp32), for grouped weights viewed as
 * [n_groups, group_len].  Replaces algorithms/symmetric.py:122-204
 * (search_group_scale).
 */
int lq_search_group_scale(const void *w, int w_dtype, int64_t n_groups,
                          int64_t group_len, int bits, int grid,
                          double max_shrink, float *scale, lq_stream_t stream);

/*
 * Router front end: probs = softmax(fp32(logits)), top-k ids ordered by
 * descending probability (ties: lower expert id first), their probabilities
 * as weights, renormalized to sum 1 when `renormalize` != 0.
 * Replaces the routing in TritonFusedMoEBlock.forward, restated at
 * trajectory/llada.py:228-234 (softmax(gate(x), fp32).topk(k)).
 *   logits [T, E] in logits_dtype (f32 or bf16); ids [T, k] int32;
 *   weights [T, k] f32.  1 <= k <= E <= 256.
 */
int lq_route_topk(const void *logits, int logits_dtype, int64_t T, int E,
                  int k, int renormalize, int32_t *topk_ids,
                  float *topk_weights, lq_stream_t stream);

/*
 * weights[t, j] = probs[t, ids[t, j]] (optionally renormalized), for callers
 * that hand fused_moe a gating_output of softmax probabilities plus topk_ids
 * (INFERENCE_REPO_CHANGES.md:110-111).  ids are int32 (ids_int64 == 0) or
 * int64 (ids_int64 != 0); ids32_out receives them as int32.
 */
int lq_gather_topk_weights(const float *probs, const void *ids, int ids_int64,
                           int64_t T, int E, int k, int renormalize,
                           int32_t *ids32_out, float *topk_weights,
                           lq_stream_t stream);

/*
 * Stable expert permutation of the T*k assignments (flat index a = t*k + j):
 *   counts[e]     number of assignments routed to expert e
 *   offsets[e]    exclusive prefix of counts (offsets[E] = T*k)
 *   sorted[p]     assignment ids grouped by expert, ascending a within one
 *                 expert (the bit-identical order of moe_align_block_size,
 *                 INFERENCE_REPO_CHANGES.md:274-278; counts restate
 *                 analysis/moe_regime.py:197-213 expert_token_stats)
 * ids are int32 in [0, E).
 */
int lq_moe_permute(const int32_t *topk_ids, int64_t T, int k, int E,
                   int32_t *counts, int32_t *offsets, int32_t *sorted,
                   lq_stream_t stream);

/*
 * Bytes of workspace lq_moe_forward / lq_moe_layer need for this shape.
 * A workspace starts with a sync region of lq_moe_sync_bytes() bytes (the
 * same size and place for every shape): a status word at offset 0 and the
 * counters through which the workgroups of the fused layer kernel hand data
 * to each other.  It must be zero before the first call on a workspace
 * (lq_moe_workspace_init, or allocate it zeroed), and every call leaves it
 * zero; the rest of the workspace is scratch.  One workspace serves one
 * stream at a time.  (No counterpart in the reference: its dequantize-then-
 * fused_moe path allocates through torch.)
 */
size_t lq_moe_workspace_bytes(int64_t T, int H, int I, int E, int k);

/* Size of the sync region at the start of every MoE workspace. */
size_t lq_moe_sync_bytes(void);

/* Zero the sync region of a workspace (hipMemsetAsync on `stream`).  Call once
 * after allocating it; not under graph capture. */
int lq_moe_workspace_init(void *workspace, lq_stream_t stream);

/*
 * Read the status word of a workspace after the calls on `stream` (this call
 * synchronises the stream).  Bit 1: a wave of a streaming GEMM gave up
 * waiting for another wave's partial sums; bit 2: the fused layer kernel
 * gave up waiting for its row block's GEMM1 tiles; bit 4: ... for the other
 * workgroups before its combine; bit 8: ... for the routing of every token
 * (its workgroups were not all resident at once, e.g. the GPU was shared).
 * Any of them means the output of some call since the last clear is wrong.
 * clear != 0 zeroes the whole sync region when the word is not zero.
 * Debugging aid; no counterpart in the reference.
 */
int lq_moe_status(const void *workspace, uint32_t *status, int clear,
                  lq_stream_t stream);

/*
 * The quantized expert layer (fused_moe with packed weights):
 *   out[t] = bf16(sum_j y[t,j]) (fp32 sum, j ascending),  e = ids[t,j]
 *   y[t,j] = bf16(w[t,j] * W2[e]^T act(W1[e] x[t])) (the slot output, stored
 *   in the compute dtype as the Triton fused_moe stores its GEMM2 tiles)
 *   act(g, u) = bf16(bf16(silu(bf16(g))) * bf16(u)), gate = W1[e][:I],
 *   up = W1[e][I:].
 * Replaces dequantize-then-fused_moe: runtime/moe.py:199-216 feeding
 * fused_moe(x, w1, w2, gating_output, topk_ids) (INFERENCE_REPO_CHANGES.md:
 * 37-63, 110-111, 259-265, 296-309).
 *   x   [T, H] bf16                         out [T, H] bf16
 *   q1  [E, 2I, H] int8 / [E, 2I, H/2] packed, s1 [E, 2I, H/G1] f32
 *   q2  [E, H, I]  int8 / [E, H, I/2]  packed, s2 [E, H, I/G2]  f32
 *   group_w1, group_w2: group lengths G1 (along H) and G2 (along I) as the
 *           quantizer recorded them for each tensor (-1 = one group per row)
 *   flags   0: the matrix cores consume the reference's dequantized weights
 *           bf16(fp32(q) * s) bit for bit (dequantize-then-matmul up to the
 *           fp32 summation order).  LQ_MOE_FOLDED_SCALES: the codes enter as
 *           exact small integers and each group's fp32 scale multiplies the
 *           integer dot product of its 128-wide K chunk -- cheaper, but the
 *           weights are not rounded to bf16 first, which moves the output by
 *           about the reference tolerance (mean-relative ~5e-3); group lengths
 *           that are not multiples of 128 ignore the flag.
 *   topk_ids [T, k] int32, topk_weights [T, k] f32; ids outside [0, E)
 *           contribute nothing
 *   workspace of ws_bytes >= lq_moe_workspace_bytes(T, H, I, E, k)
 * Requires H % 128 == 0, I % 64 == 0, group lengths (after the per-row
 * fallback) that are multiples of 32, T <= 262144 and T*k*max(2I, H)*2 <
 * 2^31 (the bf16 per-assignment buffers; larger inputs go in token chunks,
 * which is exact).  Kernels on `stream`:
 * the expert plan, GEMM1, GEMM2, combine, with an x permute in front for the
 * general and wide GEMMs.  With LQ_MOE_FUSED_LAYER, small layers of the
 * streaming family (E <= 64, T*k <= 2048, exact weights) run as ONE launch
 * instead, the fused layer kernel (plan, GEMM1, GEMM2 and combine, the
 * workgroups handing data to each other through the workspace's sync
 * region).  No host synchronisation.
 */
int lq_moe_forward(const void *x, int64_t T, int H, int I, int E, int k,
                   const int8_t *q1, const float *s1, const int8_t *q2,
                   const float *s2, int bits, int64_t group_w1,
                   int64_t group_w2, int flags, const int32_t *topk_ids,
                   const float *topk_weights, void *workspace,
                   size_t ws_bytes, void *out, lq_stream_t stream);

/*
 * The whole MoE layer from router logits: lq_route_topk into the workspace,
 * then lq_moe_forward (the TritonFusedMoEBlock.forward sequence after the
 * gate: softmax -> topk -> fused_moe; trajectory/llada.py:228-234 and
 * INFERENCE_REPO_CHANGES.md:110-111).  One host call, one stream.  When the
 * fused layer kernel takes the layer and T <= 64, E <= 64, that one launch
 * also routes (every workgroup routes all tokens with lq_route_topk's
 * arithmetic), so the layer is a single kernel.
 *   logits [T, E] in logits_dtype; topk_ids_out (optional, [T, k] int32)
 *   receives the routing; all other arguments as lq_moe_forward.
 */
int lq_moe_layer(const void *x, const void *logits, int logits_dtype,
                 int64_t T, int H, int I, int E, int k, int renormalize,
                 const int8_t *q1, const float *s1, const int8_t *q2,
                 const float *s2, int bits, int64_t group_w1,
                 int64_t group_w2, int flags, void *workspace,
                 size_t ws_bytes, void *out, int32_t *topk_ids_out,
                 lq_stream_t stream);

/*
 * lq_moe_layer without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a 64 MiB device array inside the library (one per GPU, held
 * until the process ends); a layer whose lq_moe_workspace_bytes exceeds it
 * is rejected with LQ_ERR_UNSUPPORTED.  Allocates nothing: no hipMalloc or
 * hipFree.  Each call first clears the array's sync region with a kernel.
 * Every call on one GPU shares that array, so calls that overlap on one GPU
 * (two streams, two threads) race and give wrong results; the bounded-wait
 * status word is not reported.  Arguments and results as lq_moe_layer.
 */
int lq_moe_layer_noalloc(const void *x, const void *logits, int logits_dtype,
                         int64_t T, int H, int I, int E, int k,
                         int renormalize, const int8_t *q1, const float *s1,
                         const int8_t *q2, const float *s2, int bits,
                         int64_t group_w1, int64_t group_w2, int flags,
                         void *out, int32_t *topk_ids_out, lq_stream_t stream);

/*
 * Measurement hook (no counterpart in the reference; its timing is host-side,
 * benchmarks/bench_generation_latency.py:51-72).  Registers caller-owned
 * hipEvent_t handles that the NEXT lq_moe_forward / lq_moe_layer call on
 * this thread records on its stream: events[0] before its first kernel and
 * events[i] after the i-th stage (layer: route, plan, GEMM1, GEMM2, combine;
 * forward: x permute + plan, GEMM1, GEMM2, combine; a stage that launches
 * nothing, such as the plan of a small streaming layer, still records its
 * event).  NULL entries are skipped; the registration is consumed by that
 * one call.  Fence-free events (hipEventDisableSystemFence) keep the markers
 * from adding cache flushes between the stages.
 */
int lq_moe_profile_events(void *const *events, int n_events);

/*
 * QuantLinear forward (replaces runtime/linear.py:127-131, QuantLinear.forward
 * = F.linear(x.to(bf16), dequantize_weight()), with the dequantize of
 * runtime/linear.py:103-111 fused into the GEMM):
 *   out [M, N] bf16 = bf16(x [M, K] bf16 . W^T), fp32 accumulation, where
 *   W = bf16(fp32(q) * s) is the reference's dequantized weight bit for bit;
 *   q [N, K] int8 or [N, K/2] packed INT4, s [N, K/G] f32 (group = -1 or
 *   K % group != 0: one group per row).
 * Requires N % 128 == 0, K % 64 == 0, group length % 32 == 0, M <= 262144.
 * flags: 0, LQ_MOE_WIDE_KERNEL or LQ_MOE_GENERAL_KERNEL (each deterministic;
 * the families may differ in summation order).  The bias of the reference
 * module is added by the caller (a bf16 add after the bf16 product, as the
 * reference does).  Kernels on `stream`: with flags 0 and up to 16 rows (32
 * when K splits into at most 8 slices) one kernel that sums the general
 * family's K slices in its order (the general family's bits; the workspace
 * is not touched); otherwise set-up (which also writes the one-expert plan),
 * GEMM (the wide family from 128 rows on, else the general one; both may
 * split K into slices), combine.  No host synchronisation, no device
 * allocation.
 */
int lq_quant_linear(const void *x, int64_t M, int K, int N, const int8_t *q,
                    const float *s, int bits, int64_t group, int flags,
                    void *workspace, size_t ws_bytes, void *out,
                    lq_stream_t stream);

/*
 * Router GEMM fused with the top-k softmax router (trajectory/llada.py:228-234
 * with the gate in front: router_logits = block.gate(x_flat), a bias-free
 * bf16 nn.Linear, then softmax(dtype=float32).topk(k)):
 *   x [T, H] bf16, gate_weight [E, H] bf16 (E <= 64, H % 32 == 0, both
 *   16-byte aligned); logits = bf16(x . gate_weight^T) with fp32
 *   accumulation; ids / weights as lq_route_topk computes them from those
 *   logits; logits_out [T, E] bf16 receives the logits when not NULL (the
 *   reference's routing hook records them).
 */
int lq_route_gemm_topk(const void *x, const void *gate_weight, int64_t T,
                       int H, int E, int k, int renormalize,
                       int32_t *topk_ids, float *topk_weights,
                       void *logits_out, lq_stream_t stream);

/* Bytes of workspace lq_quant_linear needs for M rows, K in, N out features. */
size_t lq_linear_workspace_bytes(int64_t M, int K, int N);

#ifdef __cplusplus
}
#endif

#endif /* LLADAQ_H */
