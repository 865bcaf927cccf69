/*
 * CPU oracle for the INT4-G128-SYM projection path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the reported CPU baseline.
 * The product path (xinfer_amd/, libxinfer_hip.so) never calls it.
 *
 * Every function restates, in plain C, a loop of the reference's own CPU
 * oracle or converter; the reference file:line is given per function.
 * Layout (reference tools/convert/qwen3_8_27b/convert.py:93-119,
 * src/targets/qwen3_8_27b/weights.cpp:261-262):
 *   W  uint8  [N][K/2]   byte j of a row: k=2j in bits 0-3, k=2j+1 in bits 4-7,
 *                        each nibble two's-complement int4 in [-8, 7]
 *   S  fp16   [N][K/G]   one scale per (row, group of G=128 consecutive k)
 *   X  [M][K], Y [M][N], row-major.
 */
#ifndef XINFER_INT4_ORACLE_H
#define XINFER_INT4_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32, round-to-nearest-even (own implementation). */
float oracle_half_to_float(uint16_t h);
uint16_t oracle_float_to_half(float f);
void oracle_half_to_float_n(const uint16_t* h, float* f, int64_t n);
void oracle_float_to_half_n(const float* f, uint16_t* h, int64_t n);

/* Two's-complement nibble decode (linear.cpp:711-715). */
int oracle_nibble(uint8_t byte, int high);

/* out[n][k] = float(q[n][k]) * float(S[n][k/G])  (convert.py:129-148). */
void oracle_dequant_int4(float* out, const uint8_t* W, const uint16_t* S,
                         int64_t N, int64_t K, int64_t G);

/* Symmetric per-group quantiser (convert.py:93-119): w [N][K] fp32 ->
 * W [N][K/2], S [N][K/G] fp16. */
void oracle_quantize_int4(uint8_t* W, uint16_t* S, const float* w,
                          int64_t N, int64_t K, int64_t G);

/* Y[m][n] = float( sum_g sum_j double(x) * (double(q) * double(s)) + bias[n] )
 * (tests/test_ops_oracle.cpp:319-348; bias as linear.cpp:724-728).
 * nthreads <= 1 runs single-threaded; > 1 uses OpenMP over rows n. */
void oracle_linear_int4(float* Y, const float* X, const uint8_t* W,
                        const uint16_t* S, const float* bias,
                        int64_t M, int64_t N, int64_t K, int64_t G,
                        int nthreads);

/* Y[m][n] = silu(float(gate)) * float(up) with silu(g) = g / (1 + exp(-g))
 * in float (tests/test_ops_oracle.cpp:626-669). */
void oracle_swiglu_int4(float* Y, const float* X,
                        const uint8_t* Wg, const uint16_t* Sg,
                        const uint8_t* Wu, const uint16_t* Su,
                        int64_t M, int64_t N, int64_t K, int64_t G,
                        int nthreads);

/* First (lowest-index) maximum with a strict '>' scan starting at logits[0]
 * (tests/test_ops_oracle.cpp:926-933, src/ops/sampling.cpp:75-85).
 * Returns 0 for V <= 1 (sampling.cpp:17-18). */
int64_t oracle_argmax(const float* logits, int64_t V);

/* RMSNorm, fp16 in/out, fp32 weight: src/ops/rmsnorm.cpp:45-78 (sum of squares
 * in FP32 in index order, inv = 1 / sqrt(sum / H + eps), out = fp16(x * inv * w)). */
void oracle_rmsnorm_f16(uint16_t* out, const uint16_t* in, const float* weight,
                        int64_t tokens, int64_t hidden, float eps);

/* add_inplace, fp16: src/ops/elementwise.cpp:213-231, a = fp16(fp32(a) + fp32(b)). */
void oracle_add_inplace_f16(uint16_t* a, const uint16_t* b, int64_t n);

/* CRC-64/ECMA-182, reflected, one byte per step: src/artifact/checksum.cpp:10-54
 * (table generation :15-31, update :42-47, digest :49-51). */
uint64_t oracle_crc64(const uint8_t* data, int64_t n);

/* Second-largest value's gap: top1 - top2 (for reporting argmax margins). */
float oracle_top2_margin(const float* logits, int64_t V);

#ifdef __cplusplus
}
#endif
#endif
