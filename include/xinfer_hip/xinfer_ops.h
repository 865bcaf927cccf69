/*
 * xinfer_hip -- C-ABI of the MI355X (gfx950) INT4-G128-SYM projection path.
 *
 * Drop-in replacement for the reference's src/ops linear/sampling entry
 * points. Each function below names the reference declaration it replaces.
 * Differences that every function shares:
 *   - `sycl::queue&`  -> `stream`: a hipStream_t passed as void* (NULL = the
 *     default stream). Work is enqueued asynchronously, like the reference's
 *     returned sycl::event; the caller decides when to synchronise.
 *   - `sycl::event`   -> an int status (XINFER_OK or a negative code below).
 *   - `sycl::half*`   -> void* holding IEEE binary16 values.
 *
 * Data layout (reference tools/convert/qwen3_8_27b/convert.py:93-119 and
 * src/targets/qwen3_8_27b/weights.cpp:261-262), unchanged from `.xinfer`:
 *   W  uint8 [N][K/2]  byte j of a row holds k=2j in bits 0-3 and k=2j+1 in
 *                      bits 4-7, each a two's-complement int4 in [-8, 7]
 *   S  fp16  [N][K/G]  one scale per (output row, group of G consecutive k)
 *   X  [M][K], Y [M][N], row-major, device memory.  bias: optional fp32 [N].
 *
 * Preconditions the reference assumed silently and this library checks:
 * group_size == 128 and K % 128 == 0 (XINFER_ERR_UNSUPPORTED otherwise);
 * W, X 16-byte aligned, S and fp16 Y 2-byte aligned, fp32 buffers 4-byte
 * aligned (XINFER_ERR_MISALIGNED). As in the reference (src/ops/linear.cpp:176,
 * 359, 513) M, N or K <= 0 is a no-op that returns XINFER_OK.
 *
 * No projection entry point allocates device memory or synchronises: the
 * first call of any shape can be captured into a hipGraph.  The small-batch
 * kernel's cross-block split-K partials live in a static device array that
 * the code object loader places with the library's kernels: 32 slots of
 * 4 MiB + 16 KiB (128.5 MiB) on every device the library runs on, one
 * owned by each stream that calls until xinfer_stream_release gives it
 * back; with every slot owned a call plans without the cross-block split
 * (correct, slower).  Calls on different streams may therefore overlap.  A
 * graph holds the slot of the stream it was captured on: replays of graphs
 * captured on one stream must not overlap each other or that stream's work
 * (a decode-step graph replayed in order on its own stream, as the
 * reference's DecodeGraph does, src/targets/qwen3_8/decode_graph.cpp:9-12,
 * never does).  The only allocating calls are xinfer_argmax_f32 and
 * xinfer_lm_head_argmax_int4 given scratch == NULL (a library-owned buffer
 * per device and stream, grown on demand -- growing waits for the stream and
 * frees the old buffer -- as the reference's argmax falls back to its own
 * allocation, src/ops/sampling.cpp:28-31); pass scratch to keep them
 * capturable.
 * The RMSNorm + projection entry points take a caller-owned workspace for
 * the normalised rows (the reference's forward_layer writes them to an
 * arena buffer, src/targets/qwen3_8/forward.cpp:112-125).
 */
#ifndef XINFER_HIP_XINFER_OPS_H
#define XINFER_HIP_XINFER_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XINFER_OK 0
#define XINFER_ERR_INVALID_ARG (-1)  /* null pointer with non-empty shape, bad count */
#define XINFER_ERR_UNSUPPORTED (-2)  /* group_size != 128, K % 128 != 0, too large  */
#define XINFER_ERR_MISALIGNED (-3)   /* pointer alignment below the kernel's needs  */
#define XINFER_ERR_HIP (-4)          /* the HIP runtime reported a launch error     */
#define XINFER_ERR_SCRATCH (-5)      /* scratch too small / could not be obtained  */

/* Human-readable name of a status code (static string). */
const char* xinfer_status_string(int status);

/* No counterpart in the reference (its queues are created once per
 * DeviceContext and never destroyed).  For long-running callers that create
 * and destroy streams: waits for `stream`'s work, then gives back its
 * split-K slot and frees its argmax scratch on the current device, so a
 * later stream can take them.  Call it before hipStreamDestroy; without it a
 * destroyed stream keeps its slot until the process ends. */
int xinfer_stream_release(void* stream);

/* Library version string, e.g. "xinfer_hip 0.1.0 gfx950". */
const char* xinfer_version(void);

/* ---------------------------------------------------------------------------
 * linear_int4: Y[m][n] = sum_g fp32(S[n][g]) * sum_{j<128} X[m][128g+j] *
 *              q[n][128g+j] (+ bias[n]), FP32 accumulation.
 * M <= 16 runs the bandwidth-bound decode kernels (VALU GEMV at M = 1-2,
 * MFMA small-batch kernel at M = 2-16); larger M (chunked prefill) runs the
 * MFMA GEMM, as the reference routes both through this one call
 * (src/targets/qwen3_8/forward.cpp:284-287).  Dequantisation: the decode
 * kernels (M <= 16) and fp32 outputs at any M multiply the exact integer q
 * by the FP32 group scale, as the reference does; the fp16-output prefill
 * GEMM (M > 16) feeds the matrix cores B = fp16(q*s), rounded once per
 * weight (relative error <= 2^-11, inside the fp16 output's rounding).
 * ------------------------------------------------------------------------- */

/* Replaces `sycl::event linear_int4(sycl::queue&, sycl::half* Y,
 * const sycl::half* X, ...)`  -- src/ops/linear.h:30-39. FP16 in, FP16 out. */
int xinfer_linear_int4_f16(void* stream, void* Y, const void* X,
                           const uint8_t* W_int4, const void* scales,
                           const float* bias, int64_t M, int64_t N, int64_t K,
                           int32_t group_size);

/* Replaces `sycl::event linear_int4(sycl::queue&, float* Y,
 * const sycl::half* X, ...)`  -- src/ops/linear.h:42-51 (LM-head logits). */
int xinfer_linear_int4_f16_f32out(void* stream, float* Y, const void* X,
                                  const uint8_t* W_int4, const void* scales,
                                  const float* bias, int64_t M, int64_t N,
                                  int64_t K, int32_t group_size);

/* Replaces `sycl::event linear_int4(sycl::queue&, float* Y, const float* X,
 * ...)`  -- src/ops/linear.h:54-63 (FP32 in/out, oracle-test overload). */
int xinfer_linear_int4_f32(void* stream, float* Y, const float* X,
                           const uint8_t* W_int4, const void* scales,
                           const float* bias, int64_t M, int64_t N, int64_t K,
                           int32_t group_size);

/* Replaces `void linear_int4_naive(sycl::queue&, float* Y, const float* X,
 * ...)`  -- src/ops/linear.h:159-168: one thread per (m, n), byte-wise
 * unpack, kept as an on-device cross-check of the fast kernels. */
int xinfer_linear_int4_naive_f32(void* stream, float* Y, const float* X,
                                 const uint8_t* W_int4, const void* scales,
                                 const float* bias, int64_t M, int64_t N,
                                 int64_t K, int32_t group_size);

/* ---------------------------------------------------------------------------
 * Multi-projection launch over one X (QKV and the linear-attention in_proj).
 * ------------------------------------------------------------------------- */

/* Same fields and meaning as `FusedProjectionDesc` / `FusedProjectionDescFP32`
 * (src/ops/linear.h:66-81).  Y is fp16 for the _f16 entry point and fp32 for
 * the _f32 one. */
typedef struct xinfer_fused_desc {
    void* Y;                /* [M][N] output                          */
    const uint8_t* W_int4;  /* [N][K/2] packed weights                */
    const void* scales;     /* [N][K/G] fp16 scales                   */
    const float* bias;      /* optional [N] fp32                      */
    int64_t N;              /* output features                        */
} xinfer_fused_desc;

/* Replaces `sycl::event linear_int4_fused(sycl::queue&, const sycl::half* X,
 * const FusedProjectionDesc* descs, int num_descs, M, K, group_size)`
 * -- src/ops/linear.h:97-103.  1 <= num_descs <= 4, else
 * XINFER_ERR_INVALID_ARG (the reference returned an empty event,
 * src/ops/linear.cpp:359). */
int xinfer_linear_int4_fused_f16(void* stream, const void* X,
                                 const xinfer_fused_desc* descs,
                                 int32_t num_descs, int64_t M, int64_t K,
                                 int32_t group_size);

/* Replaces the FP32 overload -- src/ops/linear.h:105-111. */
int xinfer_linear_int4_fused_f32(void* stream, const float* X,
                                 const xinfer_fused_desc* descs,
                                 int32_t num_descs, int64_t M, int64_t K,
                                 int32_t group_size);

/* ---------------------------------------------------------------------------
 * Fused MLP gate/up + SiLU: Y[m][n] = silu(G[m][n]) * U[m][n] with
 * silu(g) = g / (1 + exp(-g)) evaluated in FP32 on the FP32 sums.
 * ------------------------------------------------------------------------- */

/* Replaces `sycl::event mlp_gate_up_swiglu_int4(sycl::queue&, sycl::half* Y,
 * const sycl::half* X, W_gate, scales_gate, W_up, scales_up, M, N, K, G)`
 * -- src/ops/linear.h:117-127. */
int xinfer_mlp_gate_up_swiglu_int4_f16(void* stream, void* Y, const void* X,
                                       const uint8_t* W_gate,
                                       const void* scales_gate,
                                       const uint8_t* W_up,
                                       const void* scales_up, int64_t M,
                                       int64_t N, int64_t K,
                                       int32_t group_size);

/* Replaces the FP32 overload -- src/ops/linear.h:129-139. */
int xinfer_mlp_gate_up_swiglu_int4_f32(void* stream, float* Y, const float* X,
                                       const uint8_t* W_gate,
                                       const void* scales_gate,
                                       const uint8_t* W_up,
                                       const void* scales_up, int64_t M,
                                       int64_t N, int64_t K,
                                       int32_t group_size);

/* ---------------------------------------------------------------------------
 * Greedy argmax: the first (lowest-index) maximum, as the reference's strict
 * '>' scan from element 0 (src/ops/sampling.cpp:60, 80).  A NaN at element 0
 * wins (nothing compares greater than it); other NaNs never win.
 * ------------------------------------------------------------------------- */

/* Bytes of scratch xinfer_argmax_f32 needs for `rows` rows of V logits.
 * Replaces `argmax_scratch_size(int64_t vocab_size)` -- src/ops/sampling.h:13-17
 * (which counted elements of two arrays; this returns one byte count). */
size_t xinfer_argmax_scratch_bytes(int64_t V, int64_t rows);

/* Replaces `int64_t argmax(sycl::queue&, const float* logits, int64_t V,
 * float* partial_max, int64_t* partial_idx)` -- src/ops/sampling.h:22-26.
 * Batched over `rows` rows of logits [rows][V]; writes one int64 id per row
 * to device memory `out_ids` asynchronously (the reference blocked and
 * returned the id; the C++ wrapper in xinfer_ops.hpp restores that).
 * V <= 0 or V == 1 writes 0 (src/ops/sampling.cpp:17-18).  scratch may be
 * NULL (library-owned buffer) or >= xinfer_argmax_scratch_bytes(V, rows). */
int xinfer_argmax_f32(void* stream, const float* logits, int64_t V,
                      int64_t rows, int64_t* out_ids, void* scratch,
                      size_t scratch_bytes);

/* ---------------------------------------------------------------------------
 * LM head + argmax in one pass over the INT4 vocab matrix.
 * Replaces the pair `linear_int4(q, float* logits, const half* X, W, S,
 * nullptr, M, vocab, hidden)` + `argmax(q, logits, vocab)` issued by
 * forward_lm_head / decode_step / forward_verify
 * (src/targets/qwen3_8/forward.cpp:304-307, 596, 729-732;
 * src/ops/sampling.cpp:121).  ids: int32 [M] device; logits: optional fp32
 * [M][N] (NULL = do not store).  M <= 8.
 * ------------------------------------------------------------------------- */
size_t xinfer_lm_head_argmax_scratch_bytes(int64_t M, int64_t N, int64_t K);

int xinfer_lm_head_argmax_int4(void* stream, int32_t* ids, float* logits,
                               const void* X, const uint8_t* W_int4,
                               const void* scales, int64_t M, int64_t N,
                               int64_t K, int32_t group_size, void* scratch,
                               size_t scratch_bytes);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under hipGraph capture, serving loops or harnesses that forbid
 * hipMalloc): xinfer_lm_head_argmax_int4 with the per-block argmax
 * candidates in a static device array of the library (128 KiB per device)
 * instead of caller scratch; no allocation on any call.  Shapes that need
 * more candidates than the array holds return XINFER_ERR_SCRATCH (M <= 8
 * at any vocab size fits today).  All calls on one device share the array:
 * calls that overlap on one device (other streams, concurrent graph
 * replays) race. */
int xinfer_lm_head_argmax_int4_noalloc(void* stream, int32_t* ids, float* logits,
                                       const void* X, const uint8_t* W_int4,
                                       const void* scales, int64_t M, int64_t N,
                                       int64_t K, int32_t group_size);

/* ---------------------------------------------------------------------------
 * Dequantise: out[n][k] = fp32(q[n][k]) * fp32(S[n][k/G]) (exact in FP32).
 * Replaces the converter's `dequantize_int4_symmetric` oracle
 * (tools/convert/qwen3_8_27b/convert.py:129-148) on the device.
 * ------------------------------------------------------------------------- */
int xinfer_dequant_int4_f32(void* stream, float* out, const uint8_t* W_int4,
                            const void* scales, int64_t N, int64_t K,
                            int32_t group_size);

/* ---------------------------------------------------------------------------
 * The operations on either side of the projections in forward_layer
 * (src/targets/qwen3_8/forward.cpp:112-125, 229, 270-290), standalone and
 * fused into the projection kernels.
 * ------------------------------------------------------------------------- */

/* Replaces `rmsnorm(q, half* out, const half* in, const float* weight,
 * num_tokens, hidden_size, eps)` -- src/ops/rmsnorm.h:17-23:
 * out = fp16(in * (1 / sqrt(mean(in^2) + eps)) * weight), FP32 math. */
int xinfer_rmsnorm_f16(void* stream, void* out, const void* in, const float* weight,
                       int64_t num_tokens, int64_t hidden_size, float eps);

/* Replaces `add_inplace(q, half* a, const half* b, n)` -- src/ops/elementwise.h:22:
 * a = fp16(fp32(a) + fp32(b)). */
int xinfer_add_inplace_f16(void* stream, void* a, const void* b, int64_t num_elements);

/* Bytes of workspace the two RMSNorm + projection entry points below need
 * for M rows of K: 0 when the norm runs inside the projection kernel (M = 1,
 * K up to ~6k), else M * K * 2 (the normalised fp16 rows). */
size_t xinfer_rmsnorm_projection_workspace_bytes(int64_t M, int64_t K);

/* rmsnorm (rmsnorm.h:17-23) fused with linear_int4_fused (linear.h:97-103):
 * the input-norm + QKV / linear-attention in_proj pair of forward.cpp:112-125
 * and :237-247.  The projections see exactly the fp16 normalised X that
 * xinfer_rmsnorm_f16 would write (up to the order of the sum of squares).
 * Any M: at M = 1 (and at M = 2 / 3 on the dot2 kernel or the GEMV, M = 3 / 4 / 8
 * with K <= 6144 on the small-batch kernel) the norm runs inside the
 * projection kernel; otherwise the normalised rows
 * go to `workspace`.  The workspace is checked at every M >= 2 (16-byte
 * aligned, at least xinfer_rmsnorm_projection_workspace_bytes(M, K) bytes,
 * else XINFER_ERR_SCRATCH; NULL is fine when that is 0). */
int xinfer_rmsnorm_linear_int4_fused_f16(void* stream, const void* X,
                                         const float* norm_weight, float eps,
                                         const xinfer_fused_desc* descs,
                                         int32_t num_descs, int64_t M, int64_t K,
                                         int32_t group_size, void* workspace,
                                         size_t workspace_bytes);

/* rmsnorm fused with mlp_gate_up_swiglu_int4 (linear.h:117-127): the
 * post-attention norm + gate/up pair of forward.cpp:273-281.  Any M; the
 * workspace as xinfer_rmsnorm_linear_int4_fused_f16. */
int xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16(void* stream, void* Y, const void* X,
                                               const float* norm_weight, float eps,
                                               const uint8_t* W_gate, const void* scales_gate,
                                               const uint8_t* W_up, const void* scales_up,
                                               int64_t M, int64_t N, int64_t K,
                                               int32_t group_size, void* workspace,
                                               size_t workspace_bytes);

/* linear_int4 (linear.h:30-39) fused with add_inplace (elementwise.h:22):
 * residual[m][n] = fp16(residual + fp16(linear(X) + bias)), bit-identical to
 * the pair at forward.cpp:229/270 and :284-290.  Any M. */
int xinfer_linear_int4_residual_f16(void* stream, void* residual, const void* X,
                                    const uint8_t* W_int4, const void* scales,
                                    const float* bias, int64_t M, int64_t N,
                                    int64_t K, int32_t group_size);

#ifdef __cplusplus
}
#endif
#endif /* XINFER_HIP_XINFER_OPS_H */
