// INT4-G128-SYM GEMV for decode (M <= 8) on gfx950.
//
// Replaces the reference's sub-group GEMV family (src/ops/linear.cpp:33-163
// split-K, 165-305 main, 351-498 fused, 501-617 SwiGLU) with one MI355X
// design:
//   * a "team" is 32 lanes (half a wave64).  A team owns R consecutive output
//     rows at a time and walks K in steps of 1024: lane j reads the 16-byte
//     chunk j of the step from each of its R rows (global_load_dwordx4, every
//     half-wave instruction covers 512 contiguous bytes of one row).
//   * the lane's 32 activations per m are loaded once per step and reused for
//     all R rows; nibbles are dequantised in registers (dequant8) to exact
//     fp16 integers and multiplied with v_dot2_f32_f16 (FP32 accumulate).
//     The group scale is applied once per 32-k chunk in FP32.
//   * the 4 waves (8 teams) of a block either take 8 different row sets or
//     split K between 2/4/8 teams of the same row set (in-block split-K) so
//     small-N shapes still fill 256 CUs; partials meet in LDS and are summed
//     in a fixed order, so results are run-to-run deterministic.
//   * the team's lanes are reduced with DPP row rotations + one ds_swizzle.
// No MFMA: at M <= 8 the work is bound by HBM bandwidth of the weight stream.

#include "common.h"

namespace xhip {

enum Epilogue { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_ARGMAX = 2 };

struct GemvDesc {
    const uint8_t* W;    // [N][K/2]   (gate matrix for EPI_SWIGLU)
    const uint16_t* S;   // [N][K/128]
    const uint8_t* W2;   // up matrix (EPI_SWIGLU only)
    const uint16_t* S2;
    const float* bias;   // optional [N]
    void* Y;             // [M][N] output (EPI_ARGMAX: optional fp32 logits)
    int32_t N;
    int32_t rowsets;     // ceil(N / R)
    int32_t block_begin; // first block of this descriptor
    int32_t pad;
};

struct GemvParams {
    GemvDesc d[4];
    const f16* X;        // [M][K]
    ArgCand* parts;      // EPI_ARGMAX: [M][gridDim.x] block candidates
    int32_t ndesc;
    int32_t M;           // real rows of X (<= MR)
    int32_t K;
    int32_t ks;          // teams sharing one row set (1, 2, 4, 8)
};

constexpr int kTeams = 8;  // 32-lane teams per 256-thread block

template <int MR, int R, int EPI, typename OutT>
__global__ __launch_bounds__(256) void gemv_int4_kernel(const GemvParams p) {
    constexpr int RR = (EPI == EPI_SWIGLU) ? 2 * R : R;  // weight rows per team
    constexpr int NOUT = R * MR;

    const int tid = threadIdx.x;
    const int lane = tid & 31;
    const int team = tid >> 5;
    const int ks = p.ks;
    const int rs_per_block = kTeams / ks;
    const int rs_local = team / ks;
    const int kslot = team - rs_local * ks;

    // descriptor of this block (blocks of one descriptor are contiguous)
    int di = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (i < p.ndesc && (int)blockIdx.x >= p.d[i].block_begin) di = i;
    const GemvDesc& d = p.d[di];
    const int rowset = ((int)blockIdx.x - d.block_begin) * rs_per_block + rs_local;
    const bool active = rowset < d.rowsets;
    const int N = d.N;
    const int K = p.K;
    const int n0 = rowset * R;
    const int64_t row_bytes = K >> 1;
    const int ng = K >> 7;
    const int cpr = K >> 5;               // 16-byte chunks per row
    const int nsteps = (cpr + 31) >> 5;   // 1024-k steps

    const uint8_t* wrow[RR];
    const uint16_t* srow[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        const int rr = (EPI == EPI_SWIGLU) ? (r % R) : r;
        int n = n0 + rr;
        n = n < N ? n : N - 1;  // tail rows re-read the last row; never stored
        const uint8_t* Wb = (EPI == EPI_SWIGLU && r >= R) ? d.W2 : d.W;
        const uint16_t* Sb = (EPI == EPI_SWIGLU && r >= R) ? d.S2 : d.S;
        wrow[r] = Wb + (int64_t)n * row_bytes;
        srow[r] = Sb + (int64_t)n * ng;
    }
    const f16* xrow[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xrow[m] = p.X + (int64_t)(m < p.M ? m : p.M - 1) * K;

    float acc[RR][MR];
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

    if (active) {
        for (int step = kslot; step < nsteps; step += ks) {
            const int c = (step << 5) + lane;
            if (c < cpr) {
                u32x4 wv[RR];
                float sc[RR];
#pragma unroll
                for (int r = 0; r < RR; ++r)
                    wv[r] = *reinterpret_cast<const u32x4*>(wrow[r] + (c << 4));
#pragma unroll
                for (int r = 0; r < RR; ++r) sc[r] = h2f(srow[r][c >> 2]);
                f16x2 xp[MR][16];
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const u32x4* xs = reinterpret_cast<const u32x4*>(xrow[m] + (c << 5));
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        u32x4 xv = xs[v];
                        uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
                        permute_x8(xa, &xp[m][4 * v]);
                    }
                }
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    f16x2 q[16];
                    dequant8(wv[r].x, &q[0]);
                    dequant8(wv[r].y, &q[4]);
                    dequant8(wv[r].z, &q[8]);
                    dequant8(wv[r].w, &q[12]);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float t = 0.0f;
#pragma unroll
                        for (int i = 0; i < 16; ++i) t = dot2(q[i], xp[m][i], t);
                        acc[r][m] = __builtin_fmaf(t, sc[r], acc[r][m]);
                    }
                }
            }
        }
    }

    // reduce the 32 lanes of the team; every lane ends with every total
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = sum32(acc[r][m]);

    // in-block split-K: teams kslot>0 hand their totals to kslot 0 via LDS
    __shared__ float red[kTeams][RR * MR];
    if (ks > 1) {
        if (lane == 0 && kslot > 0) {
#pragma unroll
            for (int r = 0; r < RR; ++r)
#pragma unroll
                for (int m = 0; m < MR; ++m) red[team][r * MR + m] = acc[r][m];
        }
        __syncthreads();
        if (kslot == 0) {
            for (int j = 1; j < ks; ++j) {
#pragma unroll
                for (int r = 0; r < RR; ++r)
#pragma unroll
                    for (int m = 0; m < MR; ++m) acc[r][m] += red[team + j][r * MR + m];
            }
        }
    }

    // lane l < R*MR of the kslot-0 team finalises output (r, m) = (l / MR, l % MR)
    float val = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float v;
            if (EPI == EPI_SWIGLU) {
                const float g = acc[r][m];
                const float u = acc[R + r][m];
                v = g / (1.0f + expf(-g)) * u;
            } else {
                v = acc[r][m];
            }
            if (lane == r * MR + m) val = v;
        }
    }
    const int orow = lane / MR;
    const int om = lane - orow * MR;
    const int n = n0 + orow;
    const bool writer = active && kslot == 0 && lane < NOUT && n < N && om < p.M;

    if (EPI == EPI_ARGMAX) {
        __shared__ ArgCand cand[kTeams * NOUT];
        if (writer && d.bias) val += d.bias[n];
        if (writer && d.Y) reinterpret_cast<float*>(d.Y)[(int64_t)om * N + n] = val;
        if (kslot == 0 && lane < NOUT) {
            ArgCand c;
            c.v = writer ? argmax_key(val, n) : -__builtin_inff();
            c.i = writer ? n : 0x7FFFFFFF;
            cand[rs_local * NOUT + lane] = c;
        }
        __syncthreads();
        if (tid < MR && tid < p.M) {
            float bv = -__builtin_inff();
            int32_t bi = 0x7FFFFFFF;
            for (int t = 0; t < rs_per_block; ++t)
                for (int r = 0; r < R; ++r) {
                    const ArgCand c = cand[t * NOUT + r * MR + tid];
                    if (arg_better(c.v, c.i, bv, bi)) { bv = c.v; bi = c.i; }
                }
            ArgCand o;
            o.v = bv;
            o.i = bi;
            p.parts[(int64_t)tid * gridDim.x + blockIdx.x] = o;
        }
    } else if (writer) {
        if (EPI == EPI_PLAIN && d.bias) val += d.bias[n];
        reinterpret_cast<OutT*>(d.Y)[(int64_t)om * N + n] = (OutT)val;
    }
}

// Second pass of the fused LM-head argmax: one block per row m reduces the
// per-block candidates in index order.
template <typename IdT>
__global__ __launch_bounds__(256) void argmax_finalize_kernel(const ArgCand* parts,
                                                              int32_t nparts,
                                                              IdT* ids) {
    const int m = blockIdx.x;
    const ArgCand* pm = parts + (int64_t)m * nparts;
    float bv = -__builtin_inff();
    int32_t bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < nparts; i += 256) {
        const ArgCand c = pm[i];
        if (arg_better(c.v, c.i, bv, bi)) { bv = c.v; bi = c.i; }
    }
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = sv[threadIdx.x + s];
            const int32_t oi = si[threadIdx.x + s];
            if (arg_better(ov, oi, sv[threadIdx.x], si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) ids[m] = (IdT)(si[0] == 0x7FFFFFFF ? 0 : si[0]);
}

template __global__ void argmax_finalize_kernel<int32_t>(const ArgCand*, int32_t, int32_t*);
template __global__ void argmax_finalize_kernel<int64_t>(const ArgCand*, int32_t, int64_t*);

}  // namespace xhip

// ------------------------------------------------------------------ host ----

using namespace xhip;

namespace {

constexpr int kRowsM12 = 4;   // R for MR <= 2
constexpr int kRowsM48 = 2;   // R for MR >= 4

struct GemvPlan {
    int mr, r, ks, blocks;
};

// Pick the in-block K split so the launch puts >= ~8 waves on every CU
// (enough 16-byte loads in flight to cover HBM latency).
int choose_ks(int64_t rowsets_total, int K) {
    const int nsteps = (K / 32 + 31) / 32;
    const int64_t target_waves = 8LL * xhip_host::num_cus();
    int ks = 1;
    while (ks < 8 && ks * 2 <= nsteps) {
        const int64_t blocks = (rowsets_total + (kTeams / ks) - 1) / (kTeams / ks);
        if (blocks * 4 >= target_waves) break;
        ks *= 2;
    }
    return ks;
}

int mr_for(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

template <int MR, int EPI, typename OutT>
void launch_mr(GemvParams& p, int blocks, hipStream_t st) {
    constexpr int R = MR <= 2 ? kRowsM12 : kRowsM48;
    hipLaunchKernelGGL((gemv_int4_kernel<MR, R, EPI, OutT>), dim3(blocks), dim3(256), 0, st, p);
}

template <int EPI, typename OutT>
void launch_gemv(GemvParams& p, int blocks, int mr, hipStream_t st) {
    switch (mr) {
        case 1: launch_mr<1, EPI, OutT>(p, blocks, st); break;
        case 2: launch_mr<2, EPI, OutT>(p, blocks, st); break;
        case 4: launch_mr<4, EPI, OutT>(p, blocks, st); break;
        default: launch_mr<8, EPI, OutT>(p, blocks, st); break;
    }
}

// Fill block ranges for the descriptors already stored in p.d[0..ndesc).
int plan_blocks(GemvParams& p, int mr) {
    const int R = mr <= 2 ? kRowsM12 : kRowsM48;
    int64_t total_rs = 0;
    for (int i = 0; i < p.ndesc; ++i) {
        p.d[i].rowsets = (int32_t)((p.d[i].N + R - 1) / R);
        total_rs += p.d[i].rowsets;
    }
    p.ks = choose_ks(total_rs, p.K);
    const int rs_per_block = kTeams / p.ks;
    int blocks = 0;
    for (int i = 0; i < p.ndesc; ++i) {
        p.d[i].block_begin = blocks;
        blocks += (p.d[i].rowsets + rs_per_block - 1) / rs_per_block;
    }
    for (int i = p.ndesc; i < 4; ++i) p.d[i] = p.d[0], p.d[i].block_begin = 0x7FFFFFFF;
    return blocks;
}

int check_common(int64_t M, int64_t N, int64_t K, int32_t G) {
    if (G != kGroup || (K % kGroup) != 0) return XINFER_ERR_UNSUPPORTED;
    if (K > (1LL << 30) || N > (1LL << 30) || M > (1LL << 30)) return XINFER_ERR_UNSUPPORTED;
    return XINFER_OK;
}

}  // namespace

namespace xhip_host {

int num_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cached[dev] = v;
    }
    return cached[dev];
}

int launch_status() { return hipGetLastError() == hipSuccess ? XINFER_OK : XINFER_ERR_HIP; }

// Shared by the C-ABI entry points and the MFMA GEMM fallback split:
// runs the GEMV for one slab of at most 8 activation rows.
template <int EPI, typename OutT>
int gemv_f16(hipStream_t st, const GemvParams& base, int64_t M) {
    GemvParams p = base;
    p.M = (int32_t)M;
    const int mr = mr_for(M);
    const int blocks = plan_blocks(p, mr);
    if (blocks <= 0) return XINFER_OK;
    launch_gemv<EPI, OutT>(p, blocks, mr, st);
    return launch_status();
}

}  // namespace xhip_host

// Forward declaration: M > 8 with fp16 activations (chunked prefill).
namespace xhip_host {
int gemm_int4_f16(hipStream_t st, void* Y, bool y_f32, const void* X, const uint8_t* W,
                  const uint16_t* S, const uint8_t* W2, const uint16_t* S2, const float* bias,
                  int64_t M, int64_t N, int64_t K);
}

namespace {

int linear_f16_impl(void* stream, void* Y, bool y_f32, const void* X, const uint8_t* W,
                    const void* S, const float* bias, int64_t M, int64_t N, int64_t K,
                    int32_t G) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_common(M, N, K, G);
    if (rc) return rc;
    if (!Y || !X || !W || !S) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(W, 16) || !aligned(X, 16) || !aligned(S, 2) || !aligned(Y, y_f32 ? 4 : 2) ||
        !aligned(bias, 4))
        return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (M > 8)
        return gemm_int4_f16(st, Y, y_f32, X, W, (const uint16_t*)S, nullptr, nullptr, bias, M, N, K);
    GemvParams p = {};
    p.ndesc = 1;
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    p.d[0].W = W;
    p.d[0].S = reinterpret_cast<const uint16_t*>(S);
    p.d[0].bias = bias;
    p.d[0].Y = Y;
    p.d[0].N = (int32_t)N;
    return y_f32 ? gemv_f16<EPI_PLAIN, float>(st, p, M) : gemv_f16<EPI_PLAIN, f16>(st, p, M);
}

}  // namespace

extern "C" {

int xinfer_linear_int4_f16(void* stream, void* Y, const void* X, const uint8_t* W_int4,
                           const void* scales, const float* bias, int64_t M, int64_t N,
                           int64_t K, int32_t group_size) {
    return linear_f16_impl(stream, Y, false, X, W_int4, scales, bias, M, N, K, group_size);
}

int xinfer_linear_int4_f16_f32out(void* stream, float* Y, const void* X, const uint8_t* W_int4,
                                  const void* scales, const float* bias, int64_t M, int64_t N,
                                  int64_t K, int32_t group_size) {
    return linear_f16_impl(stream, Y, true, X, W_int4, scales, bias, M, N, K, group_size);
}

int xinfer_linear_int4_fused_f16(void* stream, const void* X, const xinfer_fused_desc* descs,
                                 int32_t num_descs, int64_t M, int64_t K, int32_t group_size) {
    if (!descs || num_descs <= 0 || num_descs > 4) return XINFER_ERR_INVALID_ARG;
    if (M <= 0 || K <= 0) return XINFER_OK;
    if (!X) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(X, 16)) return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    GemvParams p = {};
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    int nd = 0;
    for (int i = 0; i < num_descs; ++i) {
        const xinfer_fused_desc& q = descs[i];
        if (q.N <= 0) continue;  // empty projection: nothing to write
        int rc = check_common(M, q.N, K, group_size);
        if (rc) return rc;
        if (!q.Y || !q.W_int4 || !q.scales) return XINFER_ERR_INVALID_ARG;
        if (!aligned(q.W_int4, 16) || !aligned(q.scales, 2) || !aligned(q.Y, 2) || !aligned(q.bias, 4))
            return XINFER_ERR_MISALIGNED;
        if (M > 8) {
            rc = gemm_int4_f16(st, q.Y, false, X, q.W_int4, (const uint16_t*)q.scales, nullptr,
                               nullptr, q.bias, M, q.N, K);
            if (rc) return rc;
            continue;
        }
        GemvDesc& g = p.d[nd++];
        g.W = q.W_int4;
        g.S = reinterpret_cast<const uint16_t*>(q.scales);
        g.bias = q.bias;
        g.Y = q.Y;
        g.N = (int32_t)q.N;
    }
    if (M > 8 || nd == 0) return XINFER_OK;
    p.ndesc = nd;
    return gemv_f16<EPI_PLAIN, f16>(st, p, M);
}

int xinfer_mlp_gate_up_swiglu_int4_f16(void* stream, void* Y, const void* X,
                                       const uint8_t* W_gate, const void* scales_gate,
                                       const uint8_t* W_up, const void* scales_up, int64_t M,
                                       int64_t N, int64_t K, int32_t group_size) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_common(M, N, K, group_size);
    if (rc) return rc;
    if (!Y || !X || !W_gate || !scales_gate || !W_up || !scales_up) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(W_gate, 16) || !aligned(W_up, 16) || !aligned(X, 16) || !aligned(Y, 2) ||
        !aligned(scales_gate, 2) || !aligned(scales_up, 2))
        return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (M > 8)
        return gemm_int4_f16(st, Y, false, X, W_gate, (const uint16_t*)scales_gate, W_up,
                             (const uint16_t*)scales_up, nullptr, M, N, K);
    GemvParams p = {};
    p.ndesc = 1;
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    p.d[0].W = W_gate;
    p.d[0].S = reinterpret_cast<const uint16_t*>(scales_gate);
    p.d[0].W2 = W_up;
    p.d[0].S2 = reinterpret_cast<const uint16_t*>(scales_up);
    p.d[0].Y = Y;
    p.d[0].N = (int32_t)N;
    return gemv_f16<EPI_SWIGLU, f16>(st, p, M);
}

size_t xinfer_lm_head_argmax_scratch_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || M > 8) return 0;
    GemvParams p = {};
    p.ndesc = 1;
    p.K = (int32_t)(K > 0 ? K : 128);
    p.d[0].N = (int32_t)N;
    const int blocks = plan_blocks(p, mr_for(M));
    return (size_t)M * (size_t)blocks * sizeof(ArgCand);
}

}  // extern "C"

namespace xhip_host {
void* library_scratch(size_t bytes);  // argmax.hip
}

extern "C" int xinfer_lm_head_argmax_int4(void* stream, int32_t* ids, float* logits,
                                          const void* X, const uint8_t* W_int4,
                                          const void* scales, int64_t M, int64_t N, int64_t K,
                                          int32_t group_size, void* scratch,
                                          size_t scratch_bytes) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    if (M > 8) return XINFER_ERR_UNSUPPORTED;
    int rc = check_common(M, N, K, group_size);
    if (rc) return rc;
    if (!ids || !X || !W_int4 || !scales) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(W_int4, 16) || !aligned(X, 16) || !aligned(scales, 2) || !aligned(logits, 4) ||
        !aligned(ids, 4))
        return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    GemvParams p = {};
    p.ndesc = 1;
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    p.M = (int32_t)M;
    p.d[0].W = W_int4;
    p.d[0].S = reinterpret_cast<const uint16_t*>(scales);
    p.d[0].Y = logits;
    p.d[0].N = (int32_t)N;
    const int mr = mr_for(M);
    const int blocks = plan_blocks(p, mr);
    const size_t need = (size_t)M * (size_t)blocks * sizeof(ArgCand);
    if (!scratch) {
        scratch = library_scratch(need);
        if (!scratch) return XINFER_ERR_SCRATCH;
    } else if (scratch_bytes < need || !aligned(scratch, 8)) {
        return XINFER_ERR_SCRATCH;
    }
    p.parts = reinterpret_cast<ArgCand*>(scratch);
    launch_gemv<EPI_ARGMAX, float>(p, blocks, mr, st);
    if (launch_status()) return XINFER_ERR_HIP;
    hipLaunchKernelGGL((argmax_finalize_kernel<int32_t>), dim3((unsigned)M), dim3(256), 0, st,
                       p.parts, (int32_t)blocks, ids);
    return launch_status();
}
