/*
 * CPU oracle for the INT4-G128-SYM projection path -- TEST INFRASTRUCTURE ONLY.
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg. Nothing in the shipped library calls into this file.
 *
 * Each function restates a loop from the reference's CPU oracle
 * (tests/test_ops_oracle.cpp), its naive device reference
 * (src/ops/linear.cpp:681-730), its converter (tools/convert/qwen3_8_27b/
 * convert.py:93-148) or its argmax contract (src/ops/sampling.cpp:12-92).
 * The checks that pin each function (closed forms, exhaustive fp16 tables,
 * an independent numpy formulation, the reference's integer-pattern
 * fixtures) live in tests/test_oracle.py.
 */
#include "int4_oracle.h"

#include <math.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 ---- */

float oracle_half_to_float(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    float f;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        f = (float)m * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oracle_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan (nan keeps a quiet payload) */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7C00u | 0x200u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 */
    if (ax < 0x38800000u) {                                   /* < 2^-14 */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* value in units of 2^-24 is m >> shift */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

void oracle_half_to_float_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; ++i) f[i] = oracle_half_to_float(h[i]);
}

void oracle_float_to_half_n(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = oracle_float_to_half(f[i]);
}

/* -------------------------------------------------------------- nibbles ---- */

/* src/ops/linear.cpp:711-715: v = byte & 0xF (or >> 4); v >= 8 -> v - 16 */
int oracle_nibble(uint8_t byte, int high) {
    int v = high ? ((byte >> 4) & 0x0F) : (byte & 0x0F);
    if (v >= 8) v -= 16;
    return v;
}

/* convert.py:129-148 dequantize_int4_symmetric: unpacked (float) * scale */
void oracle_dequant_int4(float* out, const uint8_t* W, const uint16_t* S,
                         int64_t N, int64_t K, int64_t G) {
    int64_t ng = K / G;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            uint8_t b = W[n * (K / 2) + k / 2];
            float q = (float)oracle_nibble(b, (int)(k & 1));
            float s = oracle_half_to_float(S[n * ng + k / G]);
            out[n * K + k] = q * s;
        }
    }
}

/* convert.py:93-119 quantize_int4_symmetric, in the same fp32 arithmetic:
 *   scale = clamp(amax|x| / 7, min=1e-8); q = clamp(round_half_even(x/scale),
 *   -8, 7); byte = (q_even & 0xF) | (q_odd & 0xF) << 4; S = fp16(scale). */
void oracle_quantize_int4(uint8_t* W, uint16_t* S, const float* w,
                          int64_t N, int64_t K, int64_t G) {
    int64_t ng = K / G;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t g = 0; g < ng; ++g) {
            const float* x = w + n * K + g * G;
            float amax = 0.0f;
            for (int64_t j = 0; j < G; ++j) {
                float a = fabsf(x[j]);
                if (a > amax || a != a) amax = a;
            }
            float scale = amax / 7.0f;
            if (scale < 1e-8f) scale = 1e-8f;
            S[n * ng + g] = oracle_float_to_half(scale);
            for (int64_t j = 0; j < G; j += 2) {
                float r0 = nearbyintf(x[j] / scale);
                float r1 = nearbyintf(x[j + 1] / scale);
                r0 = r0 < -8.0f ? -8.0f : (r0 > 7.0f ? 7.0f : r0);
                r1 = r1 < -8.0f ? -8.0f : (r1 > 7.0f ? 7.0f : r1);
                int q0 = (int)r0, q1 = (int)r1;
                W[n * (K / 2) + (g * G + j) / 2] =
                    (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
            }
        }
    }
}

/* --------------------------------------------------------------- linear ---- */

/* tests/test_ops_oracle.cpp:319-348: double accumulate of x * (q * s) over
 * groups and byte pairs; one float cast at the end. */
static double dot_row(const float* x, const uint8_t* w, const uint16_t* s,
                      int64_t K, int64_t G) {
    double acc = 0.0;
    int64_t ng = K / G;
    for (int64_t g = 0; g < ng; ++g) {
        double scale = (double)oracle_half_to_float(s[g]);
        int64_t base_k = g * G;
        for (int64_t b = 0; b < G / 2; ++b) {
            uint8_t byte = w[base_k / 2 + b];
            double lo = (double)oracle_nibble(byte, 0);
            double hi = (double)oracle_nibble(byte, 1);
            acc += (double)x[base_k + 2 * b] * (lo * scale);
            acc += (double)x[base_k + 2 * b + 1] * (hi * scale);
        }
    }
    return acc;
}

void oracle_linear_int4(float* Y, const float* X, const uint8_t* W,
                        const uint16_t* S, const float* bias,
                        int64_t M, int64_t N, int64_t K, int64_t G,
                        int nthreads) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    int64_t total = M * N;
    int64_t ng = K / G;
#pragma omp parallel for schedule(static) num_threads(nthreads > 1 ? nthreads : 1) if (nthreads > 1)
    for (int64_t i = 0; i < total; ++i) {
        int64_t m = i / N, n = i % N;
        double acc = dot_row(X + m * K, W + n * (K / 2), S + n * ng, K, G);
        if (bias) acc += (double)bias[n];
        Y[i] = (float)acc;
    }
}

void oracle_swiglu_int4(float* Y, const float* X,
                        const uint8_t* Wg, const uint16_t* Sg,
                        const uint8_t* Wu, const uint16_t* Su,
                        int64_t M, int64_t N, int64_t K, int64_t G,
                        int nthreads) {
    if (M <= 0 || N <= 0 || K <= 0) return;
    int64_t total = M * N;
    int64_t ng = K / G;
#pragma omp parallel for schedule(static) num_threads(nthreads > 1 ? nthreads : 1) if (nthreads > 1)
    for (int64_t i = 0; i < total; ++i) {
        int64_t m = i / N, n = i % N;
        float gate = (float)dot_row(X + m * K, Wg + n * (K / 2), Sg + n * ng, K, G);
        float up = (float)dot_row(X + m * K, Wu + n * (K / 2), Su + n * ng, K, G);
        float silu = gate / (1.0f + expf(-gate));
        Y[i] = silu * up;
    }
}

/* --------------------------------------------------------------- argmax ---- */

int64_t oracle_argmax(const float* logits, int64_t V) {
    if (V <= 1 || !logits) return 0;
    int64_t best = 0;
    float best_val = logits[0];
    for (int64_t i = 1; i < V; ++i) {
        if (logits[i] > best_val) {
            best_val = logits[i];
            best = i;
        }
    }
    return best;
}

float oracle_top2_margin(const float* logits, int64_t V) {
    if (V <= 1) return INFINITY;
    int64_t b = oracle_argmax(logits, V);
    float second = -INFINITY;
    for (int64_t i = 0; i < V; ++i)
        if (i != b && logits[i] > second) second = logits[i];
    return logits[b] - second;
}

/* --------------------------------------------------------------- CRC-64 ---- */

/* src/artifact/checksum.cpp:10-54: table of the reflected polynomial, register
 * starts at all ones, c = (c >> 8) ^ T[(c ^ byte) & 0xFF], result XOR all ones. */
uint64_t oracle_crc64(const uint8_t* data, int64_t n) {
    static uint64_t table[256];
    static int ready = 0;
    const uint64_t poly = 0xC96C5795D7870F42ULL;
    if (!ready) {
        for (uint64_t b = 0; b < 256; ++b) {
            uint64_t c = b;
            for (int i = 0; i < 8; ++i) c = (c & 1) ? (c >> 1) ^ poly : c >> 1;
            table[b] = c;
        }
        ready = 1;
    }
    uint64_t c = 0xFFFFFFFFFFFFFFFFULL;
    for (int64_t i = 0; i < n; ++i) c = (c >> 8) ^ table[(c ^ data[i]) & 0xFF];
    return c ^ 0xFFFFFFFFFFFFFFFFULL;
}

/* -------------------------------------------------- RMSNorm, add_inplace ---- */

/* src/ops/rmsnorm.cpp:45-78. */
void oracle_rmsnorm_f16(uint16_t* out, const uint16_t* in, const float* weight,
                        int64_t tokens, int64_t hidden, float eps) {
    for (int64_t t = 0; t < tokens; ++t) {
        const uint16_t* x = in + t * hidden;
        uint16_t* y = out + t * hidden;
        float ss = 0.0f;
        for (int64_t i = 0; i < hidden; ++i) {
            const float v = oracle_half_to_float(x[i]);
            ss += v * v;
        }
        const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
        for (int64_t i = 0; i < hidden; ++i) {
            const float v = oracle_half_to_float(x[i]);
            y[i] = oracle_float_to_half(v * inv * weight[i]);
        }
    }
}

/* src/ops/elementwise.cpp:213-231. */
void oracle_add_inplace_f16(uint16_t* a, const uint16_t* b, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        a[i] = oracle_float_to_half(oracle_half_to_float(a[i]) + oracle_half_to_float(b[i]));
}
