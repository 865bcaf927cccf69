// FP32-activation projections, the naive cross-check kernel, device
// dequantisation, and status/version strings.
//
// The FP32 overloads (src/ops/linear.h:54-63, 105-111, 129-139) exist in the
// reference for oracle testing only, so these kernels favour plain FP32
// arithmetic over speed: one 32-lane team per output row, nibbles decoded
// with a sign-extending bit-field extract, FP32 fma against FP32 X.

#include <algorithm>

#include "common.h"
#include "../../include/xinfer_hip/xinfer_artifact.h"

namespace xhip {

struct F32Desc {
    const uint8_t* W;
    const uint16_t* S;
    const uint8_t* W2;   // up matrix for SwiGLU
    const uint16_t* S2;
    const float* bias;
    float* Y;
    int32_t N;
    int32_t block_begin;
};

struct F32Params {
    F32Desc d[4];
    const float* X;
    int32_t ndesc;
    int32_t M;
    int32_t K;
};

__device__ __forceinline__ int nib(uint32_t w, int i) {
    return ((int32_t)(w << (28 - 4 * i))) >> 28;  // sign-extended nibble i
}

// Team (32-lane) dot product of one packed row with one FP32 activation row.
__device__ float row_dot_f32(const float* x, const uint8_t* w, const uint16_t* s, int K,
                             int lane) {
    const int cpr = K >> 5;
    float acc = 0.0f;
    for (int c = lane; c < cpr; c += 32) {
        const u32x4 wv = *reinterpret_cast<const u32x4*>(w + (c << 4));
        const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
        const float* xc = x + (c << 5);
        float t = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int i = 0; i < 8; ++i) t = __builtin_fmaf(xc[8 * d + i], (float)nib(wd[d], i), t);
        acc = __builtin_fmaf(t, h2f(s[c >> 2]), acc);
    }
    return sum32(acc);
}

template <bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_int4_f32x_kernel(const F32Params p) {
    const int lane = threadIdx.x & 31;
    const int team = threadIdx.x >> 5;
    int di = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (i < p.ndesc && (int)blockIdx.x >= p.d[i].block_begin) di = i;
    const F32Desc& d = p.d[di];
    const int n = ((int)blockIdx.x - d.block_begin) * 8 + team;
    if (n >= d.N) return;
    const int K = p.K;
    const int ng = K >> 7;
    const uint8_t* w = d.W + (int64_t)n * (K >> 1);
    const uint16_t* s = d.S + (int64_t)n * ng;
    for (int m = 0; m < p.M; ++m) {
        const float* x = p.X + (int64_t)m * K;
        float v = row_dot_f32(x, w, s, K, lane);
        if (SWIGLU) {
            const float u = row_dot_f32(x, d.W2 + (int64_t)n * (K >> 1), d.S2 + (int64_t)n * ng, K, lane);
            v = v / (1.0f + expf(-v)) * u;
        } else if (d.bias) {
            v += d.bias[n];
        }
        if (lane == 0) d.Y[(int64_t)m * d.N + n] = v;
    }
}

// One thread per (m, n), byte-wise unpack, FP32 accumulate: the same loop as
// the reference's naive device kernel (src/ops/linear.cpp:681-730).
__global__ void linear_int4_naive_kernel(float* Y, const float* X, const uint8_t* W,
                                         const uint16_t* S, const float* bias, int64_t M,
                                         int64_t N, int64_t K) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t m = idx / N, n = idx % N;
    const float* x = X + m * K;
    const uint8_t* w = W + n * (K / 2);
    const uint16_t* s = S + n * (K / kGroup);
    float acc = 0.0f;
    for (int64_t g = 0; g < K / kGroup; ++g) {
        const float scale = h2f(s[g]);
        for (int64_t b = 0; b < kGroup / 2; ++b) {
            const uint8_t byte = w[g * (kGroup / 2) + b];
            int lo = byte & 0x0F;
            if (lo >= 8) lo -= 16;
            int hi = (byte >> 4) & 0x0F;
            if (hi >= 8) hi -= 16;
            const int64_t k0 = g * kGroup + 2 * b;
            acc += x[k0] * ((float)lo * scale);
            acc += x[k0 + 1] * ((float)hi * scale);
        }
    }
    if (bias) acc += bias[n];
    Y[idx] = acc;
}

// out[n][k] = float(q) * float(s): one thread per packed byte.
__global__ void dequant_int4_kernel(float* out, const uint8_t* W, const uint16_t* S, int64_t N,
                                    int64_t K) {
    const int64_t total = N * (K / 2);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = i / (K / 2);
        const int64_t k = (i - n * (K / 2)) * 2;
        const uint32_t b = W[i];
        const float s = h2f(S[n * (K / kGroup) + k / kGroup]);
        out[n * K + k] = (float)nib(b, 0) * s;
        out[n * K + k + 1] = (float)nib(b, 1) * s;
    }
}

// RMSNorm of one token per block (src/ops/rmsnorm.cpp:45-78): FP32 sum of
// squares, inv = 1 / sqrt(mean + eps), out = fp16(x * inv * w).
// One pass for rows of up to 8192 (16-byte aligned, H % 8 == 0): each
// thread loads its chunks of x and of the weights at once and keeps them in
// registers, so the row is read once and the weights' latency hides behind
// the reduction (the two-pass kernel below re-reads x after the reduction
// and only then requests the weights).  Same expression per element
// (rmsnorm.cpp:78); the row sum in a fixed order: chunks of a thread, the
// lanes of a wave, the four waves in order.
__global__ __launch_bounds__(256) void rmsnorm_f16_reg_kernel(f16* out, const f16* in, const float* w,
                                                              int32_t H, float eps) {
    constexpr int kCPT = 4;  // chunks per thread
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = H >> 3;
    const u32x4* xr = reinterpret_cast<const u32x4*>(in + (size_t)blockIdx.x * H);
    const float4* wr = reinterpret_cast<const float4*>(w);
    u32x4* yr = reinterpret_cast<u32x4*>(out + (size_t)blockIdx.x * H);
    u32x4 v[kCPT];
    float4 wa[kCPT], wb[kCPT];
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const int c = tid + u * 256;
        v[u] = u32x4{0u, 0u, 0u, 0u};
        if (c < c8) {
            v[u] = xr[c];
            wa[u] = wr[2 * c];
            wb[u] = wr[2 * c + 1];
        }
    }
    float ss[1] = {0.0f};
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const uint32_t a[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f16x2 h = as_h2(a[j]);
            const float x0 = (float)h.x, x1 = (float)h.y;
            ss[0] += x0 * x0;
            ss[0] += x1 * x1;
        }
    }
    const float t = wave_sum_multi<1>(ss, lane);
    if (lane == 0) red[wave] = t;
    __syncthreads();
    const float inv = 1.0f / sqrtf((((red[0] + red[1]) + red[2]) + red[3]) / (float)H + eps);
#pragma unroll
    for (int u = 0; u < kCPT; ++u) {
        const int c = tid + u * 256;
        if (c < c8) yr[c] = rms_apply8(v[u], wa[u], wb[u], inv);
    }
}

__global__ __launch_bounds__(256) void rmsnorm_f16_kernel(f16* out, const f16* in, const float* w,
                                                          int32_t H, float eps) {
    __shared__ float red[8];
    __shared__ float inv_s[1];
    const f16* x = in + (size_t)blockIdx.x * H;
    f16* y = out + (size_t)blockIdx.x * H;
    const int tid = threadIdx.x;
    if ((H & 7) == 0 && ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
        // 16-byte chunks, several loads in flight per thread in both passes
        rms_inv_rows<256>(x, 1, H, eps, red, inv_s);
        const float inv = inv_s[0];
        const int c8 = H >> 3;
        const u32x4* xr = reinterpret_cast<const u32x4*>(x);
        const float4* wr = reinterpret_cast<const float4*>(w);
        u32x4* yr = reinterpret_cast<u32x4*>(y);
        for (int c0 = tid; c0 < c8; c0 += 256 * 4) {
            u32x4 v[4];
            float4 wa[4], wb[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * 256;
                if (c < c8) {
                    v[u] = xr[c];
                    wa[u] = wr[2 * c];
                    wb[u] = wr[2 * c + 1];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = c0 + u * 256;
                if (c < c8) {
                    const float ww[8] = {wa[u].x, wa[u].y, wa[u].z, wa[u].w, wb[u].x, wb[u].y, wb[u].z, wb[u].w};
                    yr[c] = rms_apply8(v[u], ww, inv);
                }
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int i = tid; i < H; i += 256) {
        const float v = (float)x[i];
        ss += v * v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + eps);
    for (int i = tid; i < H; i += 256) y[i] = (f16)((float)x[i] * inv * w[i]);
}

// a = fp16(fp32(a) + fp32(b)) (src/ops/elementwise.cpp:213-231)
__global__ __launch_bounds__(256) void add_inplace_f16_kernel(f16* a, const f16* b, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        a[i] = (f16)((float)a[i] + (float)b[i]);
}

}  // namespace xhip

using namespace xhip;

namespace {

int check_shape(int64_t M, int64_t N, int64_t K, int32_t G) {
    if (G != kGroup || (K % kGroup) != 0) return XINFER_ERR_UNSUPPORTED;
    if (K > (1LL << 30) || N > (1LL << 30) || M > (1LL << 30)) return XINFER_ERR_UNSUPPORTED;
    return XINFER_OK;
}

int launch_f32(hipStream_t st, F32Params& p, bool swiglu) {
    int blocks = 0;
    for (int i = 0; i < p.ndesc; ++i) {
        p.d[i].block_begin = blocks;
        blocks += (p.d[i].N + 7) / 8;
    }
    for (int i = p.ndesc; i < 4; ++i) p.d[i] = p.d[0], p.d[i].block_begin = 0x7FFFFFFF;
    if (blocks == 0) return XINFER_OK;
    if (swiglu)
        hipLaunchKernelGGL(gemv_int4_f32x_kernel<true>, dim3(blocks), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(gemv_int4_f32x_kernel<false>, dim3(blocks), dim3(256), 0, st, p);
    return xhip_host::launch_status();
}

}  // namespace

extern "C" {

const char* xinfer_status_string(int status) {
    switch (status) {
        case XINFER_OK: return "XINFER_OK";
        case XINFER_ERR_INVALID_ARG: return "XINFER_ERR_INVALID_ARG";
        case XINFER_ERR_UNSUPPORTED: return "XINFER_ERR_UNSUPPORTED";
        case XINFER_ERR_MISALIGNED: return "XINFER_ERR_MISALIGNED";
        case XINFER_ERR_HIP: return "XINFER_ERR_HIP";
        case XINFER_ERR_SCRATCH: return "XINFER_ERR_SCRATCH";
        case XINFER_ERR_IO: return "XINFER_ERR_IO";
        case XINFER_ERR_CHECKSUM: return "XINFER_ERR_CHECKSUM";
        default: return "XINFER_ERR_UNKNOWN";
    }
}

const char* xinfer_version(void) { return "xinfer_hip 0.1.0 gfx950"; }

int xinfer_rmsnorm_f16(void* stream, void* out, const void* in, const float* weight,
                       int64_t num_tokens, int64_t hidden_size, float eps) {
    if (num_tokens <= 0 || hidden_size <= 0) return XINFER_OK;
    if (!out || !in || !weight) return XINFER_ERR_INVALID_ARG;
    if (num_tokens > (1LL << 30) || hidden_size > (1LL << 30)) return XINFER_ERR_UNSUPPORTED;
    const bool one_pass = hidden_size % 8 == 0 && hidden_size <= 8192 && xhip_host::aligned(in, 16) &&
                          xhip_host::aligned(out, 16) && xhip_host::aligned(weight, 16);
    hipLaunchKernelGGL(one_pass ? rmsnorm_f16_reg_kernel : rmsnorm_f16_kernel, dim3((unsigned)num_tokens),
                       dim3(256), 0, reinterpret_cast<hipStream_t>(stream), reinterpret_cast<f16*>(out),
                       reinterpret_cast<const f16*>(in), weight, (int32_t)hidden_size, eps);
    return xhip_host::launch_status();
}

int xinfer_add_inplace_f16(void* stream, void* a, const void* b, int64_t num_elements) {
    if (num_elements <= 0) return XINFER_OK;
    if (!a || !b) return XINFER_ERR_INVALID_ARG;
    const int64_t blocks = std::min<int64_t>((num_elements + 255) / 256, 65536);
    hipLaunchKernelGGL(add_inplace_f16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), reinterpret_cast<f16*>(a),
                       reinterpret_cast<const f16*>(b), num_elements);
    return xhip_host::launch_status();
}

int xinfer_linear_int4_f32(void* stream, float* Y, const float* X, const uint8_t* W_int4,
                           const void* scales, const float* bias, int64_t M, int64_t N, int64_t K,
                           int32_t group_size) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_shape(M, N, K, group_size);
    if (rc) return rc;
    if (!Y || !X || !W_int4 || !scales) return XINFER_ERR_INVALID_ARG;
    using xhip_host::aligned;
    if (!aligned(W_int4, 16) || !aligned(X, 16) || !aligned(scales, 2) || !aligned(Y, 4) ||
        !aligned(bias, 4))
        return XINFER_ERR_MISALIGNED;
    F32Params p = {};
    p.ndesc = 1;
    p.X = X;
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    p.d[0] = F32Desc{W_int4, (const uint16_t*)scales, nullptr, nullptr, bias, Y, (int32_t)N, 0};
    return launch_f32(reinterpret_cast<hipStream_t>(stream), p, false);
}

int xinfer_linear_int4_fused_f32(void* stream, const float* X, const xinfer_fused_desc* descs,
                                 int32_t num_descs, int64_t M, int64_t K, int32_t group_size) {
    if (!descs || num_descs <= 0 || num_descs > 4) return XINFER_ERR_INVALID_ARG;
    if (M <= 0 || K <= 0) return XINFER_OK;
    if (!X) return XINFER_ERR_INVALID_ARG;
    using xhip_host::aligned;
    if (!aligned(X, 16)) return XINFER_ERR_MISALIGNED;
    F32Params p = {};
    p.X = X;
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    int nd = 0;
    for (int i = 0; i < num_descs; ++i) {
        const xinfer_fused_desc& q = descs[i];
        if (q.N <= 0) continue;
        int rc = check_shape(M, q.N, K, group_size);
        if (rc) return rc;
        if (!q.Y || !q.W_int4 || !q.scales) return XINFER_ERR_INVALID_ARG;
        if (!aligned(q.W_int4, 16) || !aligned(q.scales, 2) || !aligned(q.Y, 4) || !aligned(q.bias, 4))
            return XINFER_ERR_MISALIGNED;
        p.d[nd++] = F32Desc{q.W_int4, (const uint16_t*)q.scales, nullptr, nullptr, q.bias,
                            (float*)q.Y, (int32_t)q.N, 0};
    }
    if (nd == 0) return XINFER_OK;
    p.ndesc = nd;
    return launch_f32(reinterpret_cast<hipStream_t>(stream), p, false);
}

int xinfer_mlp_gate_up_swiglu_int4_f32(void* stream, float* Y, const float* X,
                                       const uint8_t* W_gate, const void* scales_gate,
                                       const uint8_t* W_up, const void* scales_up, int64_t M,
                                       int64_t N, int64_t K, int32_t group_size) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_shape(M, N, K, group_size);
    if (rc) return rc;
    if (!Y || !X || !W_gate || !scales_gate || !W_up || !scales_up) return XINFER_ERR_INVALID_ARG;
    using xhip_host::aligned;
    if (!aligned(W_gate, 16) || !aligned(W_up, 16) || !aligned(X, 16) || !aligned(Y, 4) ||
        !aligned(scales_gate, 2) || !aligned(scales_up, 2))
        return XINFER_ERR_MISALIGNED;
    F32Params p = {};
    p.ndesc = 1;
    p.X = X;
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    p.d[0] = F32Desc{W_gate, (const uint16_t*)scales_gate, W_up, (const uint16_t*)scales_up,
                     nullptr, Y, (int32_t)N, 0};
    return launch_f32(reinterpret_cast<hipStream_t>(stream), p, true);
}

int xinfer_linear_int4_naive_f32(void* stream, float* Y, const float* X, const uint8_t* W_int4,
                                 const void* scales, const float* bias, int64_t M, int64_t N,
                                 int64_t K, int32_t group_size) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_shape(M, N, K, group_size);
    if (rc) return rc;
    if (!Y || !X || !W_int4 || !scales) return XINFER_ERR_INVALID_ARG;
    using xhip_host::aligned;
    if (!aligned(X, 4) || !aligned(scales, 2) || !aligned(Y, 4) || !aligned(bias, 4))
        return XINFER_ERR_MISALIGNED;
    const int64_t total = M * N;
    hipLaunchKernelGGL(linear_int4_naive_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, reinterpret_cast<hipStream_t>(stream), Y, X, W_int4,
                       (const uint16_t*)scales, bias, M, N, K);
    return xhip_host::launch_status();
}

int xinfer_dequant_int4_f32(void* stream, float* out, const uint8_t* W_int4, const void* scales,
                            int64_t N, int64_t K, int32_t group_size) {
    if (N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_shape(1, N, K, group_size);
    if (rc) return rc;
    if (!out || !W_int4 || !scales) return XINFER_ERR_INVALID_ARG;
    using xhip_host::aligned;
    if (!aligned(out, 4) || !aligned(scales, 2)) return XINFER_ERR_MISALIGNED;
    const int64_t total = N * (K / 2);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequant_int4_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), out, W_int4,
                       (const uint16_t*)scales, N, K);
    return xhip_host::launch_status();
}

}  // extern "C"
