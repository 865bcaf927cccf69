// Shared device helpers for the gfx950 INT4-G128-SYM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <type_traits>

#include "../../include/xinfer_hip/xinfer_ops.h"

namespace xhip {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGroup = 128;  // k values per scale group (the only supported G)

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(f16, h);
}

// Dequantise one dword = 8 packed two's-complement nibbles (k0..k7, k0 in
// bits 0-3) into four fp16 pairs holding exact integers in [-8, 7]:
//   q[0] = (k0, k4), q[1] = (k1, k5), q[2] = (k2, k6), q[3] = (k3, k7).
// Flipping bit 3 of a nibble turns two's complement into offset binary
// u = q + 8; placing u (or 16u) in the mantissa of fp16 1024.0 gives exactly
// 1024 + u (or 1024 + 16u).  Because the masked nibble bits never overlap the
// exponent bits of 0x6400, "mask, flip bit 3, OR 0x6400" is one AND then one
// XOR with 0x6408 (0x6480 for the high nibble): a single v_bitop3_b32.  One
// packed add (or fma by 1/16) then removes the bias; all values are exact.
__device__ __forceinline__ void dequant8(uint32_t w, f16x2 q[4]) {
    const f16x2 kBias = {(f16)-1032.0f, (f16)-1032.0f};  // -(1024 + 8)
    const f16x2 kSixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 kBias16 = {(f16)-72.0f, (f16)-72.0f};    // -(1024/16 + 8)
    const uint32_t w8 = w >> 8;
    q[0] = as_h2((w & 0x000F000Fu) ^ 0x64086408u) + kBias;
    q[1] = as_h2((w & 0x00F000F0u) ^ 0x64806480u) * kSixteenth + kBias16;
    q[2] = as_h2((w8 & 0x000F000Fu) ^ 0x64086408u) + kBias;
    q[3] = as_h2((w8 & 0x00F000F0u) ^ 0x64806480u) * kSixteenth + kBias16;
}

// Rearrange 8 consecutive fp16 activations (x0..x7 held as 4 packed dwords,
// natural order) into the pair order dequant8 produces.
__device__ __forceinline__ void permute_x8(const uint32_t x[4], f16x2 p[4]) {
    p[0] = as_h2(__builtin_amdgcn_perm(x[2], x[0], 0x05040100u));  // (x0, x4)
    p[1] = as_h2(__builtin_amdgcn_perm(x[2], x[0], 0x07060302u));  // (x1, x5)
    p[2] = as_h2(__builtin_amdgcn_perm(x[3], x[1], 0x05040100u));  // (x2, x6)
    p[3] = as_h2(__builtin_amdgcn_perm(x[3], x[1], 0x07060302u));  // (x3, x7)
}

// Biased decode of 16 nibbles (two dwords, natural nibble order) into 8 fp16
// pairs of exact integers 1024 + u or 1024 + 16u (u = q + 8), in the pair
// order permute_x8 gives the activations; the caller removes the bias per
// 32-k chunk (sum x*q = ta + tb/16 - C).
// Two dwords at once: one 64-bit shift provides the ">> 8" of both
// (bits 24-31 of the low result hold bits of the high dword, but only bits
// 0-7 and 16-23 survive the masks).
__device__ __forceinline__ void decode16_biased(uint32_t w0, uint32_t w1, f16x2 h[8]) {
    const uint64_t w8 = (((uint64_t)w1 << 32) | w0) >> 8;
    const uint32_t a8 = (uint32_t)w8, b8 = (uint32_t)(w8 >> 32);
    h[0] = as_h2((w0 & 0x000F000Fu) ^ 0x64086408u);
    h[1] = as_h2((w0 & 0x00F000F0u) ^ 0x64806480u);
    h[2] = as_h2((a8 & 0x000F000Fu) ^ 0x64086408u);
    h[3] = as_h2((a8 & 0x00F000F0u) ^ 0x64806480u);
    h[4] = as_h2((w1 & 0x000F000Fu) ^ 0x64086408u);
    h[5] = as_h2((w1 & 0x00F000F0u) ^ 0x64806480u);
    h[6] = as_h2((b8 & 0x000F000Fu) ^ 0x64086408u);
    h[7] = as_h2((b8 & 0x00F000F0u) ^ 0x64806480u);
}

// Natural nibble order: byte b of w -> (k_2b, k_2b+1) as exact fp16
// integers (byte permute, one v_bitop3_b32, one packed fma), times the
// group scale.
__device__ __forceinline__ void decode8_natural_scaled(uint32_t w, f16x2 s2, uint32_t out[4]) {
    const f16x2 kMul = {(f16)1.0f, (f16)0.0625f};
    const f16x2 kAdd = {(f16)-1032.0f, (f16)-72.0f};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t sel = 0x0C000C00u | ((uint32_t)b << 16) | (uint32_t)b;
        const uint32_t bb = __builtin_amdgcn_perm(w, w, sel);  // [byte b, 0, byte b, 0]
        const f16x2 q = as_h2((bb & 0x00F0000Fu) ^ 0x64806408u) * kMul + kAdd;
        out[b] = as_u32(q * s2);
    }
}

__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}
// dot2 starting a new sum in its own register: the compiler forms the
// two-operand v_dot2c (destination = accumulator) plus a v_mov of the start
// value; the three-operand encoding needs no copy.
__device__ __forceinline__ float dot2_from(f16x2 a, f16x2 b, float c) {
    float d;
    asm("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ float dot2_from0(f16x2 a, f16x2 b) {
    float d;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
    return d;
}

// DPP / swizzle lane exchanges.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of 32 lanes; every lane receives the total.
__device__ __forceinline__ float sum32(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]  (xor 1)
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]  (xor 2)
    v += dpp<0x124>(v);  // row_ror:4
    v += dpp<0x128>(v);  // row_ror:8  -> full 16-lane row sum
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(
        __builtin_bit_cast(int, v), 0x401F));  // xor 16 within 32 lanes
    return v;
}

// Adds lane L and lane L xor 32 (gfx950 v_permlane32_swap on two copies:
// the first ends as [lo, lo], the second as [hi, hi]).  Written as asm:
// the compiler's builtin returns one register for both halves here.
__device__ __forceinline__ float add_xor32(float x) {
    float t = x;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(t));
    return x + t;
}
// Adds lane L and lane L xor 16 (v_permlane16_swap: odd rows of the first
// copy trade places with even rows of the second).
__device__ __forceinline__ float add_xor16(float x) {
    float t = x;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(t));
    return x + t;
}

// Sums NV values (NV = 1, 2, 4 or 8) each over the 64 lanes in one pass.
// Halving steps on lane bits 0, 1, 2 pair value 2j with 2j+1: each lane
// keeps the one its bit selects and adds the one its exchange partner
// kept for it, so after log2(NV) steps lane L holds a partial of value
// L mod NV; row rotations and the two swaps finish the sums without LDS.
// Lane L returns the total of v[L mod NV].
template <int NV>
__device__ __forceinline__ float wave_sum_multi(const float (&v)[NV], int lane) {
    static_assert(NV == 1 || NV == 2 || NV == 4 || NV == 8, "NV must be 1, 2, 4 or 8");
    float a[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) a[j] = v[j];
    auto halve = [&](auto ctrl, int n, bool bit) {
#pragma unroll
        for (int j = 0; j < n / 2; ++j) {
            const float keep = bit ? a[2 * j + 1] : a[2 * j];
            const float send = bit ? a[2 * j] : a[2 * j + 1];
            a[j] = keep + dpp<decltype(ctrl)::value>(send);
        }
    };
    if constexpr (NV >= 2) halve(std::integral_constant<int, 0xB1>{}, NV, (lane & 1) != 0);
    if constexpr (NV >= 4) halve(std::integral_constant<int, 0x4E>{}, NV / 2, (lane & 2) != 0);
    if constexpr (NV >= 8) halve(std::integral_constant<int, 0x124>{}, NV / 4, (lane & 4) != 0);
    float x = a[0];
    if constexpr (NV < 2) x += dpp<0xB1>(x);
    if constexpr (NV < 4) x += dpp<0x4E>(x);
    if constexpr (NV < 8) x += dpp<0x124>(x);
    x += dpp<0x128>(x);
    return add_xor32(add_xor16(x));
}

// Argmax candidate ordering shared by every argmax kernel: larger value
// wins, ties go to the lower index.  NaN handling reproduces a strict '>'
// scan that starts from element 0: a NaN at index 0 is never beaten (mapped
// to +inf, which also wins every tie by index), any other NaN never wins.
struct ArgCand {
    float v;
    int32_t i;
};

__device__ __forceinline__ float argmax_key(float v, int64_t idx) {
    if (v != v) return idx == 0 ? __builtin_inff() : -__builtin_inff();
    return v;
}

__device__ __forceinline__ bool arg_better(float av, int32_t ai, float bv, int32_t bi) {
    return av > bv || (av == bv && ai < bi);
}

// Argmax candidates of 8 rows over the 64 lanes in one pass, the pattern of
// wave_sum_multi with arg_better in place of the sum: three halving steps
// on lane bits 0-2 leave lane L with a partial candidate of row L mod 8,
// then a row rotation by 8 and the 16 / 32 swaps combine lanes of the same
// row.  Lane L returns row L mod 8's candidate (a total order, so the
// result does not depend on the order of the combines).
template <int CTRL>
__device__ __forceinline__ int32_t dpp_i(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ void swap32_pair(float& v, int32_t& i) {
    float tv = v;
    int32_t ti = i;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(v), "+v"(tv));
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(i), "+v"(ti));
    if (arg_better(tv, ti, v, i)) { v = tv; i = ti; }
}
__device__ __forceinline__ void swap16_pair(float& v, int32_t& i) {
    float tv = v;
    int32_t ti = i;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(v), "+v"(tv));
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(i), "+v"(ti));
    if (arg_better(tv, ti, v, i)) { v = tv; i = ti; }
}
// One argmax candidate over the 64 lanes (every lane receives the result):
// quad exchanges, row rotations by 4 and 8, then the 16 / 32 swaps.
__device__ __forceinline__ void wave_argmax1(float& v, int32_t& i) {
    auto step = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        const float ov = dpp<C>(v);
        const int32_t oi = dpp_i<C>(i);
        if (arg_better(ov, oi, v, i)) { v = ov; i = oi; }
    };
    step(std::integral_constant<int, 0xB1>{});
    step(std::integral_constant<int, 0x4E>{});
    step(std::integral_constant<int, 0x124>{});
    step(std::integral_constant<int, 0x128>{});
    swap16_pair(v, i);
    swap32_pair(v, i);
}
__device__ __forceinline__ void wave_argmax_multi8(const float (&bv)[8], const int32_t (&bi)[8], int lane,
                                                   float& rv, int32_t& ri) {
    float a[8];
    int32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = bv[j];
        b[j] = bi[j];
    }
    auto halve = [&](auto ctrl, int n, bool bit) {
        constexpr int C = decltype(ctrl)::value;
#pragma unroll
        for (int j = 0; j < n / 2; ++j) {
            const float kv = bit ? a[2 * j + 1] : a[2 * j];
            const int32_t ki = bit ? b[2 * j + 1] : b[2 * j];
            const float sv = bit ? a[2 * j] : a[2 * j + 1];
            const int32_t si = bit ? b[2 * j] : b[2 * j + 1];
            const float ov = dpp<C>(sv);
            const int32_t oi = dpp_i<C>(si);
            const bool t = arg_better(ov, oi, kv, ki);
            a[j] = t ? ov : kv;
            b[j] = t ? oi : ki;
        }
    };
    halve(std::integral_constant<int, 0xB1>{}, 8, (lane & 1) != 0);
    halve(std::integral_constant<int, 0x4E>{}, 4, (lane & 2) != 0);
    halve(std::integral_constant<int, 0x124>{}, 2, (lane & 4) != 0);
    float v = a[0];
    int32_t i = b[0];
    {
        const float ov = dpp<0x128>(v);
        const int32_t oi = dpp_i<0x128>(i);
        if (arg_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    swap16_pair(v, i);
    swap32_pair(v, i);
    rv = v;
    ri = i;
}
// Per-row RMSNorm factors of X [M][K] (M <= 8, K a multiple of 8) for a
// block of NTHREADS threads: inv[m] = 1 / sqrt(sum_k x^2 / K + eps), the FP32
// sum of src/ops/rmsnorm.cpp:45-71 (summed in a fixed order here, so every
// block and every call get the same bits).  A power-of-two group of threads
// owns each row and keeps up to 8 of its 16-byte loads in flight.
// red: NTHREADS / 32 floats of LDS; inv: M floats of LDS.
template <int NTHREADS>
__device__ inline void rms_inv_rows(const f16* X, int M, int K, float eps, float* red, float* inv) {
    const int tid = threadIdx.x;
    const int mp = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;  // rows rounded up to a power of two
    const int tpr = NTHREADS / mp;                             // threads per row (>= 32)
    const int seg = tpr < 64 ? tpr : 64;                       // lanes reduced by shuffles
    const int m = tid / tpr, r = tid - m * tpr;
    const int c8 = K >> 3;  // 16-byte chunks per row
    float ss = 0.0f;
    if (m < M) {
        const u32x4* row = reinterpret_cast<const u32x4*>(X + (size_t)m * K);
        for (int c0 = r; c0 < c8; c0 += tpr * 8) {
            u32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = c0 + u * tpr;
                v[u] = c < c8 ? row[c] : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f16x2 h = as_h2(w[j]);
                    const float a = (float)h.x, b = (float)h.y;
                    ss += a * a;
                    ss += b * b;
                }
            }
        }
    }
    for (int off = seg >> 1; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((tid & (seg - 1)) == 0) red[tid / seg] = ss;
    __syncthreads();
    if (tid < M) {
        const int nseg = tpr / seg;
        float s = 0.0f;
        for (int j = 0; j < nseg; ++j) s += red[tid * nseg + j];
        inv[tid] = 1.0f / sqrtf(s / (float)K + eps);
    }
    __syncthreads();
}

// Sum of squares of the 32 fp16 values of four 16-byte chunks, in order.
__device__ inline float sumsq32(const u32x4* v) {
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f16x2 h = as_h2(w[j]);
            const float a = (float)h.x, b = (float)h.y;
            ss += a * a;
            ss += b * b;
        }
    }
    return ss;
}

// Finish of the one-pass RMSNorm prologue (the block stages all of K and
// sums the squares of what it loaded): ssm[m] is this thread's partial sum
// of row m (zero for rows it did not load).  Rows are reduced per wave by
// shuffles, then over the waves in order, so the bits are the same on every
// call.  red: NTHREADS / 64 * 8 floats of LDS; inv: M floats of LDS.
template <int NTHREADS>
__device__ inline void rms_finish_rows(const float (&ssm)[8], int M, int K, float eps, float* red, float* inv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m < M) {
            float v = ssm[m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) red[wave * 8 + m] = v;
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < M) {
        float s = 0.0f;
        for (int w = 0; w < NTHREADS / 64; ++w) s += red[w * 8 + threadIdx.x];
        inv[threadIdx.x] = 1.0f / sqrtf(s / (float)K + eps);
    }
    __syncthreads();
}

// Normalise 8 consecutive activations (one 16-byte chunk starting at k):
// x * inv * w[k] rounded to fp16, the expression of rmsnorm.cpp:78.
__device__ inline u32x4 rms_apply8(u32x4 v, const float* w, float inv) {
    uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f16x2 h = as_h2(a[j]);
        f16x2 o;
        o.x = (f16)((float)h.x * inv * w[2 * j]);
        o.y = (f16)((float)h.y * inv * w[2 * j + 1]);
        a[j] = as_u32(o);
    }
    return u32x4{a[0], a[1], a[2], a[3]};
}

// fp32(low / high fp16 half of h) * s, rounded once: v_fma_mix with an
// addend of -0 (x * s + (-0) is x * s for every x, +0 included), one
// instruction instead of a conversion and a multiply.
__device__ __forceinline__ float f16lo_mul(uint32_t h, float s) {
    float d;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(s), "s"(-0.0f));
    return d;
}
__device__ __forceinline__ float f16hi_mul(uint32_t h, float s) {
    float d;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(s), "s"(-0.0f));
    return d;
}

// The same with the chunk's 8 weights already in registers.
__device__ inline u32x4 rms_apply8(u32x4 v, float4 w0, float4 w1, float inv) {
    const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f16x2 o;
        o.x = (f16)(f16lo_mul(a[j], inv) * w[2 * j]);
        o.y = (f16)(f16hi_mul(a[j], inv) * w[2 * j + 1]);
        a[j] = as_u32(o);
    }
    return u32x4{a[0], a[1], a[2], a[3]};
}

}  // namespace xhip

// Host-side helpers shared by the C-ABI translation units.
namespace xhip_host {

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

int num_cus();                 // compute units of the current device (cached)
int launch_status();           // XINFER_OK or XINFER_ERR_HIP after a launch
// Row-pair GEMV for large M = 1 projections (gemv_pair_int4.hip): whether it
// takes a launch, and the launch (returns 1 when the shape is left to the
// GEMV, else 0 with *rc the launch status).
bool pair_takes(int64_t M, int64_t K, int64_t n_total);
int pair_linear(hipStream_t st, const xinfer_fused_desc* descs, int nd, const void* X, bool y_f32,
                int64_t K, bool residual, const float* norm_w, float eps, int* rc);
int pair_swiglu(hipStream_t st, void* Y, const void* X, const uint8_t* Wg, const void* Sg, const uint8_t* Wu,
                const void* Su, int64_t N, int64_t K, const float* norm_w, float eps, int* rc);
// norm_w: RMSNorm of X in the kernel's staging (fp16 outputs, M = 2, 3;
// otherwise the shape is declined)
int pairm_linear(hipStream_t st, const xinfer_fused_desc* descs, int nd, const void* X, bool y_f32, int64_t M,
                 int64_t K, bool residual, int* rc, const float* norm_w = nullptr, float eps = 0.0f);
// whether pairm_linear / pairm_swiglu take M rows of K (before the even-N
// check; rows = output rows over all descriptors, 2 N for the SwiGLU)
bool pairm_takes(int64_t M, int64_t K, int64_t rows, bool swiglu);
int pairm_swiglu(hipStream_t st, void* Y, const void* X, const uint8_t* Wg, const void* Sg, const uint8_t* Wu,
                 const void* Su, int64_t M, int64_t N, int64_t K, int* rc, const float* norm_w = nullptr,
                 float eps = 0.0f);
// XINFER_PAIR_SWIGLU=0 keeps the M = 1 gate/up SwiGLU on the GEMV (tuning)
inline bool swiglu_pair_on() {
    static const bool on = [] {
        const char* v = getenv("XINFER_PAIR_SWIGLU");
        return !(v && *v && atoi(v) == 0);
    }();
    return on;
}

}  // namespace xhip_host
