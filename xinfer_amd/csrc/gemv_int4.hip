// INT4-G128-SYM GEMV for decode (M <= 8) on gfx950.
//
// Replaces the reference's sub-group GEMV family (src/ops/linear.cpp:33-163
// split-K, 165-305 main, 351-498 fused, 501-617 SwiGLU) with one MI355X
// design:
//   * a fixed grid of one or two blocks per CU (8 waves at M = 1, else 4);
//     each block owns a contiguous range of output rows.  Its work is a list
//     of items (group of 2R rows, 1024-k step) in row-major order, cut into
//     equal contiguous pieces, one per wave.  Small N therefore splits K across
//     waves by itself (the reference's split-K).  Items are wave-uniform, so
//     all item bookkeeping and row addresses live in SGPRs.
//   * in an item, half-wave h covers rows 2R*g + h*R .. + R - 1; lane j of
//     the half reads the 16-byte chunk j of the step from each row
//     (global_load_dwordx4 with an SGPR base; a half-wave covers 512
//     contiguous bytes of a row).  The next PF items are in flight while one
//     is computed.
//   * activations are staged once per block into LDS, permuted into the
//     pair order of the nibble decode and stored piece-major (a half-wave's
//     ds_read_b128 covers 512 contiguous bytes: no bank conflicts).
//   * decode: "mask, flip bit 3, OR 0x6400" (one v_bitop3_b32 per nibble
//     pair) turns nibble pairs into fp16 pairs (1024 + u, 1024 + u) or
//     (1024 + 16u, 1024 + 16u) with u = q + 8, exactly.  These are fed straight
//     to v_dot2_f32_f16 (FP32 accumulate) in two accumulators, and the bias is
//     removed once per 32-k chunk:  sum_k x*q = ta + tb/16 - C, where
//     C = 1032 * sum(x even k) + 72 * sum(x odd k) is precomputed per chunk
//     during staging.  The group scale is applied to that chunk sum in FP32.
//     When X does not fit in LDS the lanes read X from global memory and use
//     the exact per-pair bias subtraction (dequant8) instead.
//   * when a wave leaves a row group each half-wave reduces its 32 lanes (DPP
//     row rotations + one ds_swizzle) and stores the partial in an LDS slot
//     keyed by (row, first step of its run).  After a barrier the slots of
//     each row are summed in step order: results do not depend on timing.
// No MFMA: at M <= 8 the kernel is bound by the HBM weight stream.

#include <stdlib.h>

#include <atomic>
#include <mutex>

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
    int32_t rows_blk;    // rows per block (multiple of 2R)
    int32_t block_begin; // first block of this descriptor
    int32_t residual;    // EPI_PLAIN, fp16 Y: Y = fp16(Y + fp16(result))
};

struct GemvParams {
    GemvDesc d[4];
    const f16* X;        // [M][K]
    ArgCand* parts;      // EPI_ARGMAX: [M][gridDim.x] block candidates
    const float* norm_w; // RMSNorm weight [K] applied to X while staging (XLDS only), or null
    float norm_eps;
    int32_t ndesc;
    int32_t M;           // real rows of X (<= MR)
    int32_t K;
};

// dynamic LDS in front of the X pieces: RMSNorm partial sums (8 per wave,
// up to 8 waves) and the row factors (8), padded to keep the pieces 16-byte
// aligned
constexpr int kGemvLdsHead = 1024;
static_assert((16 * 8 + 8) * 4 <= kGemvLdsHead, "RMSNorm scratch for up to 16 waves");

template <int RR>
struct ItemRegs {
    u32x4 w[RR];
    uint32_t s[RR];  // raw fp16 scale bits: converted at use, so that a load
                     // never forces a wait on the loads issued before it
};

// (1024 + u)-form decode of one dword: four fp16 pairs, u = q + 8.
//   h[0] = (k0, k4) as 1024 + u     h[1] = (k1, k5) as 1024 + 16u
//   h[2] = (k2, k6) as 1024 + u     h[3] = (k3, k7) as 1024 + 16u
__device__ __forceinline__ void decode8_biased(uint32_t w, f16x2 h[4]) {
    const uint32_t w8 = w >> 8;
    h[0] = as_h2((w & 0x000F000Fu) ^ 0x64086408u);
    h[1] = as_h2((w & 0x00F000F0u) ^ 0x64806480u);
    h[2] = as_h2((w8 & 0x000F000Fu) ^ 0x64086408u);
    h[3] = as_h2((w8 & 0x00F000F0u) ^ 0x64806480u);
}

template <int MR, int R, int EPI, typename OutT, bool XLDS, int PF, int NWV>
__global__ __launch_bounds__(64 * NWV) void gemv_int4_kernel(const GemvParams p) {
    constexpr int NTH = 64 * NWV;                        // threads per block
    constexpr int RR = (EPI == EPI_SWIGLU) ? 2 * R : R;  // weight rows per half-wave item
    constexpr int E = (EPI == EPI_SWIGLU) ? 2 : 1;       // sums per output
    constexpr int G2 = 2 * R;                            // output rows per item

    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    int di = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (i < p.ndesc && (int)blockIdx.x >= p.d[i].block_begin) di = i;
    const GemvDesc& d = p.d[di];
    const int N = d.N;
    const int K = p.K;
    const int row_begin = ((int)blockIdx.x - d.block_begin) * d.rows_blk;
    const int rows_here = min(d.rows_blk, N - row_begin);
    const int groups = (rows_here + G2 - 1) / G2;
    const uint32_t row_bytes = (uint32_t)K >> 1;
    const int ng = K >> 7;
    const int cpr = K >> 5;               // 16-byte chunks per row
    const int nsteps = (cpr + 31) >> 5;   // 1024-k steps
    const int ragged = cpr & 31;          // chunks in a partial last step (0 = none)

    // LDS (XLDS): X pieces [step][m][piece v][lane] (u32x4) and the bias terms
    // C [step][m][lane] (f32), padded to whole 1024-k steps; then partials.
    // A half-wave's piece read covers 512 contiguous bytes (no bank conflicts)
    // and the piece / m offsets are instruction immediates.
    // The first kGemvLdsHead bytes hold the RMSNorm prologue's reduction.
    const int cpad = nsteps * 32;
    float* rms_red = reinterpret_cast<float*>(smem);
    float* rms_inv = rms_red + NWV * 8;
    u32x4* xs = reinterpret_cast<u32x4*>(smem + kGemvLdsHead);
    float* xc = reinterpret_cast<float*>(smem + kGemvLdsHead + (size_t)(XLDS ? MR * 4 * cpad : 0) * 16);
    float* part = xc + (XLDS ? MR * cpad : 0);
    const int nslots = d.rows_blk * MR * E * nsteps;

    const int items = groups * nsteps;
    const int it0 = (wave * items) / NWV;
    const int it1 = ((wave + 1) * items) / NWV;

    const uint8_t* Wb0 = d.W;
    const uint16_t* Sb0 = d.S;
    const uint8_t* Wb1 = (EPI == EPI_SWIGLU) ? d.W2 : d.W;
    const uint16_t* Sb1 = (EPI == EPI_SWIGLU) ? d.S2 : d.S;
    const int row_last = row_begin + rows_here - 1;
    // per-lane byte offsets inside an item (constant for the whole kernel)
    const uint32_t w_lane = (uint32_t)(half * R) * row_bytes + (uint32_t)l32 * 16u;
    const uint32_t s_lane = (uint32_t)(half * R * ng + (l32 >> 2)) * 2u;

    // Raw buffer resources sized to the weight and scale matrices.  Every
    // item issues the same loads with no branches (so the compiler keeps
    // exact vmcnt bookkeeping across the prefetch ring): rows past N fall
    // outside the resource and read as zero, and so do the lanes of a
    // partial last k-step, whose offset is pushed out of range.  (Matrix
    // sizes are checked on the host: < 4 GiB.)
    const uint32_t srow_bytes = (uint32_t)ng * 2u;
    const int nrec_w = (int)((uint32_t)N * row_bytes);
    const int nrec_s = (int)((uint32_t)N * srow_bytes);
    const __amdgpu_buffer_rsrc_t rw0 = __builtin_amdgcn_make_buffer_rsrc((void*)Wb0, (short)0, nrec_w, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw1 = __builtin_amdgcn_make_buffer_rsrc((void*)Wb1, (short)0, nrec_w, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc((void*)Sb0, (short)0, nrec_s, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc((void*)Sb1, (short)0, nrec_s, 0x00020000);
    (void)row_last;

    // load cursor (group, step) of the next item to fetch; wave-uniform.
    // Items past the wave's range are fetched from an out-of-range offset:
    // no memory traffic, zeros in the registers, zero contribution.
    int lg = it0 / nsteps;
    int ls = it0 - lg * nsteps;
    int lcount = it1 - it0;

    auto load_next = [&](ItemRegs<RR>& b) {
        const uint32_t row0 = (uint32_t)(row_begin + lg * G2);   // first row of the item
        const bool lane_bad = (ragged && ls == nsteps - 1 && l32 >= ragged) || lcount <= 0;
        --lcount;
        // 0xFFFFF000 lies past every resource (matrices are < 4 GiB - 4096)
        const uint32_t wv = lane_bad ? 0xFFFFF000u : w_lane + row0 * row_bytes + (uint32_t)ls * 512u;
        const uint32_t sv = lane_bad ? 0xFFFFF000u : s_lane + row0 * srow_bytes + (uint32_t)ls * 16u;
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const int rr = (EPI == EPI_SWIGLU) ? (r % R) : r;
            b.w[r] = __builtin_amdgcn_raw_buffer_load_b128(
                (EPI == EPI_SWIGLU && r >= R) ? rw1 : rw0, (int)(wv + (uint32_t)rr * row_bytes), 0, 2 /*nt*/);
        }
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const int rr = (EPI == EPI_SWIGLU) ? (r % R) : r;
            b.s[r] = __builtin_amdgcn_raw_buffer_load_b16(
                (EPI == EPI_SWIGLU && r >= R) ? rs1 : rs0, (int)(sv + (uint32_t)rr * srow_bytes), 0, 0);
        }
        if (++ls == nsteps) { ls = 0; ++lg; }
    };

    // X staging in up to three rounds (every decode shape): its loads are
    // issued before the weight prefetch, so the staging does not wait for
    // the weights (loads complete in issue order).
    const int nst = MR * cpad;  // 64-byte chunks: (m, chunk)
    auto get = [&](int i, u32x4 (&xv)[4]) {
        const int m = i / cpad;
        const int c = i - m * cpad;
        const int mm = m < p.M ? m : p.M - 1;
#pragma unroll
        for (int v = 0; v < 4; ++v)  // padding chunks read as x = 0
            xv[v] = c < cpr ? *reinterpret_cast<const u32x4*>(p.X + (size_t)mm * K + (c << 5) + (v << 3))
                            : u32x4{0u, 0u, 0u, 0u};
    };
    auto put = [&](int i, u32x4 (&xv)[4]) {
        const int m = i / cpad;
        const int c = i - m * cpad;
        const int st = c >> 5, cl = c & 31;
        const int mm = m < p.M ? m : p.M - 1;
        float se = 0.0f, so = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (p.norm_w && c < cpr) xv[v] = rms_apply8(xv[v], p.norm_w + (c << 5) + (v << 3), rms_inv[mm]);
            const uint32_t xa[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
            f16x2 pr[4];
            permute_x8(xa, pr);
            xs[((st * MR + m) * 4 + v) * 32 + cl] =
                u32x4{as_u32(pr[0]), as_u32(pr[1]), as_u32(pr[2]), as_u32(pr[3])};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f16x2 x2 = as_h2(xa[j]);
                se += (float)x2.x;
                so += (float)x2.y;
            }
        }
        // sum_k x*q = ta + tb/16 - C with ta, tb the biased dot products
        xc[(st * MR + m) * 32 + cl] = -(1032.0f * se + 72.0f * so);
    };
    constexpr int kEarly = 3;  // staging rounds held in registers
    const bool early = XLDS && nst <= kEarly * NTH;
    u32x4 xv0[kEarly][4];
    if (early) {
#pragma unroll
        for (int r = 0; r < kEarly; ++r)
            if (r * NTH + tid < nst) get(r * NTH + tid, xv0[r]);
    }

    ItemRegs<RR> buf[PF + 1];
#pragma unroll
    for (int j = 0; j < PF; ++j) load_next(buf[j]);

    // zero the partial slots; stage X (permuted) and the per-chunk bias terms.
    // RMSNorm prologue: with the early staging the row sums come from the
    // loaded registers (X is read once); otherwise from a pass over X first.
    for (int i = tid; i < nslots; i += NTH) part[i] = 0.0f;
    if (early) {
        if (p.norm_w) {
            float ssm[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < kEarly; ++r) {
                const int i = r * NTH + tid;
                const int m = i / cpad;
                if (i < nst && m < p.M && i - m * cpad < cpr) {
                    const float sq = sumsq32(xv0[r]);
#pragma unroll
                    for (int q = 0; q < 8; ++q) ssm[q] += q == m ? sq : 0.0f;
                }
            }
            rms_finish_rows<NTH>(ssm, p.M, K, p.norm_eps, rms_red, rms_inv);
        }
#pragma unroll
        for (int r = 0; r < kEarly; ++r)
            if (r * NTH + tid < nst) put(r * NTH + tid, xv0[r]);
    } else if (XLDS) {
        if (p.norm_w) rms_inv_rows<NTH>(p.X, p.M, K, p.norm_eps, rms_red, rms_inv);
        for (int i = tid; i < nst; i += NTH) {
            u32x4 xv[4];
            get(i, xv);
            put(i, xv);
        }
    }
    __syncthreads();

    float acc[RR][MR];
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

    auto compute_item = [&](int st, const ItemRegs<RR>& b) {
        const int c = min((st << 5) + l32, cpr - 1);
        f16x2 xp[MR][16];
        float cm[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (XLDS) {
                    const u32x4 xv = xs[((st * MR + m) * 4 + v) * 32 + l32];
                    xp[m][4 * v + 0] = as_h2(xv.x);
                    xp[m][4 * v + 1] = as_h2(xv.y);
                    xp[m][4 * v + 2] = as_h2(xv.z);
                    xp[m][4 * v + 3] = as_h2(xv.w);
                } else {
                    const int mm = m < p.M ? m : p.M - 1;
                    const u32x4 xv = *reinterpret_cast<const u32x4*>(
                        p.X + (size_t)mm * K + (c << 5) + (v << 3));
                    const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
                    permute_x8(xa, &xp[m][4 * v]);
                }
            }
            cm[m] = XLDS ? xc[(st * MR + m) * 32 + l32] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            if (XLDS) {
                f16x2 h[16];
                decode16_biased(b.w[r].x, b.w[r].y, &h[0]);
                decode16_biased(b.w[r].z, b.w[r].w, &h[8]);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float ta = cm[m], tb = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; i += 2) {
                        ta = dot2(h[i], xp[m][i], ta);
                        tb = dot2(h[i + 1], xp[m][i + 1], tb);
                    }
                    acc[r][m] = __builtin_fmaf(__builtin_fmaf(tb, 0.0625f, ta), h2f((uint16_t)b.s[r]), acc[r][m]);
                }
            } else {
                f16x2 q[16];
                dequant8(b.w[r].x, &q[0]);
                dequant8(b.w[r].y, &q[4]);
                dequant8(b.w[r].z, &q[8]);
                dequant8(b.w[r].w, &q[12]);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i) t = dot2(q[i], xp[m][i], t);
                    acc[r][m] = __builtin_fmaf(t, h2f((uint16_t)b.s[r]), acc[r][m]);
                }
            }
        }
    };

    // store this wave's run of row group g (first step s0) and reset
    auto flush = [&](int g, int s0) {
#pragma unroll
        for (int r = 0; r < RR; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[r][m] = sum32(acc[r][m]);
        if (l32 == 0) {
#pragma unroll
            for (int r = 0; r < RR; ++r) {
                const int rr = (EPI == EPI_SWIGLU) ? (r % R) : r;
                const int e = (EPI == EPI_SWIGLU && r >= R) ? 1 : 0;
                const int rl = g * G2 + half * R + rr;
                if (rl < rows_here) {
#pragma unroll
                    for (int m = 0; m < MR; ++m)
                        part[((rl * MR + m) * E + e) * nsteps + s0] = acc[r][m];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RR; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;
    };

    // compute cursor (group, step); a run of one group starts at step run0.
    // The ring loop's body has no branch around a load (exact vmcnt
    // tracking); loads it issues for items past the end read zeros and are
    // never waited on.
    int cg = it0 / nsteps;
    int cs = it0 - cg * nsteps;
    int run0 = cs;
    const int nreal = it1 - it0;
    auto retire = [&](int k) {  // item k computed: close its run when the run ends
        if (++cs == nsteps || k + 1 == nreal) {
            flush(cg, run0);
            if (cs == nsteps) { cs = 0; ++cg; }
            run0 = cs;
        }
    };
    int base = 0;
    for (; base + PF + 1 <= nreal; base += PF + 1) {
#pragma unroll
        for (int j = 0; j <= PF; ++j) {
            load_next(buf[(j + PF) % (PF + 1)]);
            compute_item(min(cs, nsteps - 1), buf[j]);
            retire(base + j);
        }
    }
    // the last nreal - base (<= PF) items are already in the ring: compute
    // them without issuing or waiting on loads for items past the end
    // (waiting on such padding loads cost ~1 us at the end of a wave)
#pragma unroll
    for (int j = 0; j < PF; ++j) {
        if (base + j < nreal) {
            compute_item(min(cs, nsteps - 1), buf[j]);
            retire(base + j);
        }
    }
    __syncthreads();

    // epilogue: sum each output's slots in step order
    const int nout = rows_here * MR;
    if (EPI == EPI_ARGMAX) {
        float bv = -__builtin_inff();
        int32_t bi = 0x7FFFFFFF;
        for (int o = tid; o < nout; o += NTH) {
            const int rl = o / MR, m = o - rl * MR;
            float v = 0.0f;
            for (int s = 0; s < nsteps; ++s) v += part[(rl * MR + m) * nsteps + s];
            const int n = row_begin + rl;
            if (d.bias) v += d.bias[n];
            if (m < p.M) {
                if (d.Y) reinterpret_cast<float*>(d.Y)[(size_t)m * N + n] = v;
                const float key = argmax_key(v, n);
                if (arg_better(key, n, bv, bi)) { bv = key; bi = n; }
            }
        }
        // thread t holds outputs with m == t % MR: reduce over lanes of the same
        // m (lane exchanges at distances >= MR keep m), then over the waves
#pragma unroll
        for (int off = 32; off >= MR; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int32_t oi = __shfl_xor(bi, off);
            if (arg_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        __syncthreads();  // partial slots are reused for the candidates below
        float* cv = part;
        int32_t* ci = reinterpret_cast<int32_t*>(part + NWV * MR);
        if (lane < MR) {
            cv[wave * MR + lane] = bv;
            ci[wave * MR + lane] = bi;
        }
        __syncthreads();
        if (tid < MR && tid < p.M) {
            float b = cv[tid];
            int32_t i = ci[tid];
            for (int w = 1; w < NWV; ++w)
                if (arg_better(cv[w * MR + tid], ci[w * MR + tid], b, i)) { b = cv[w * MR + tid]; i = ci[w * MR + tid]; }
            ArgCand o;
            o.v = b;
            o.i = i;
            p.parts[(size_t)tid * gridDim.x + blockIdx.x] = o;
        }
    } else {
        for (int o = tid; o < nout; o += NTH) {
            const int rl = o / MR, m = o - rl * MR;
            if (m >= p.M) continue;
            const int n = row_begin + rl;
            float v = 0.0f;
            for (int s = 0; s < nsteps; ++s) v += part[((rl * MR + m) * E) * nsteps + s];
            if (EPI == EPI_SWIGLU) {
                float u = 0.0f;
                for (int s = 0; s < nsteps; ++s) u += part[((rl * MR + m) * E + 1) * nsteps + s];
                v = v / (1.0f + expf(-v)) * u;
            } else if (d.bias) {
                v += d.bias[n];
            }
            OutT* y = reinterpret_cast<OutT*>(d.Y) + (size_t)m * N + n;
            if (EPI == EPI_PLAIN && d.residual)  // add_inplace after the projection (elementwise.cpp:227)
                *y = (OutT)((float)*y + (float)(OutT)v);
            else
                *y = (OutT)v;
        }
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
    // the wave by lane exchanges, then the 4 waves in order (a total
    // order: the result does not depend on the combine order)
    wave_argmax1(bv, bi);
    __shared__ float sv[4];
    __shared__ int32_t si[4];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (arg_better(sv[w], si[w], sv[0], si[0])) {
                sv[0] = sv[w];
                si[0] = si[w];
            }
    }
    if (threadIdx.x == 0) ids[m] = (IdT)(si[0] == 0x7FFFFFFF ? 0 : si[0]);
}

template __global__ void argmax_finalize_kernel<int32_t>(const ArgCand*, int32_t, int32_t*);
template __global__ void argmax_finalize_kernel<int64_t>(const ArgCand*, int32_t, int64_t*);

}  // namespace xhip

// ------------------------------------------------------------------ host ----

using namespace xhip;

namespace {


struct GemvPlan {
    int mr, r, pf, blocks, nw;
    bool w16;  // M = 1, R = 2: one 16-wave block per CU in place of two 8-wave blocks
    bool xlds;
    size_t lds;
};

typedef void (*GemvKernel)(GemvParams);

template <int MR, int R, int EPI, typename OutT, int PF>
GemvKernel pick_kernel(bool xlds, bool w16) {
    // M <= 2 with R = 2 runs 8-wave blocks (gemv_waves), everything else 4;
    // M = 1 with R = 2 and X in LDS may run 16-wave blocks
    constexpr int NWV = (MR <= 2 && R == 2) ? 8 : 4;
    if constexpr (MR == 1 && R == 2 && PF == 1)
        if (w16 && xlds) return gemv_int4_kernel<MR, R, EPI, OutT, true, PF, 16>;
    return xlds ? gemv_int4_kernel<MR, R, EPI, OutT, true, PF, NWV>
                : gemv_int4_kernel<MR, R, EPI, OutT, false, PF, NWV>;
}

template <int MR, int R, int EPI, typename OutT>
GemvKernel pick_pf(bool xlds, int pf, bool w16) {
    if (MR == 1 && EPI != EPI_ARGMAX) {
        if (pf <= 1) return pick_kernel<MR, R, EPI, OutT, 1>(xlds, w16);
        if (pf == 2) return pick_kernel<MR, R, EPI, OutT, 2>(xlds, w16);
        return pick_kernel<MR, R, EPI, OutT, 3>(xlds, w16);
    }
    return pick_kernel<MR, R, EPI, OutT, 2>(xlds, w16);
}

template <int EPI, typename OutT>
GemvKernel kernel_for(int mr, int r, bool xlds, int pf, bool w16 = false) {
    switch (mr) {
        case 1:
            return r == 1 ? pick_pf<1, 1, EPI, OutT>(xlds, pf, false)
                 : r == 2 ? pick_pf<1, 2, EPI, OutT>(xlds, pf, w16) : pick_pf<1, 4, EPI, OutT>(xlds, pf, false);
        case 2:
            return r == 2 ? pick_pf<2, 2, EPI, OutT>(xlds, pf, false) : pick_pf<2, 4, EPI, OutT>(xlds, pf, false);
        case 4:
            return r == 1 ? pick_pf<4, 1, EPI, OutT>(xlds, pf, false) : pick_pf<4, 2, EPI, OutT>(xlds, pf, false);
        default:
            return r == 1 ? pick_pf<8, 1, EPI, OutT>(xlds, pf, false) : pick_pf<8, 2, EPI, OutT>(xlds, pf, false);
    }
}

// Tuning overrides (read once): XINFER_GEMV_R, XINFER_GEMV_PF, XINFER_GEMV_BPC,
// XINFER_GEMV_W16.
int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}
struct Overrides {
    int r, pf, bpc, w16;
};
const Overrides& overrides() {
    static const Overrides o = {env_int("XINFER_GEMV_R", 0), env_int("XINFER_GEMV_PF", 0),
                                env_int("XINFER_GEMV_BPC", 0), env_int("XINFER_GEMV_W16", -1)};
    return o;
}

// Waves per block: 8 for M <= 2 with two rows per half-wave (X staged once
// for twice the waves), 4 otherwise.  Measured on MI355X, graph-replayed
// (M = 1): config 1 17.97 -> 17.45 us, q-proj 6.00 -> 5.70, down-proj
// (K = 17408) 12.77 -> 11.05, LM head 65.2 -> 64.5, north-star 17.3 -> 17.4.
int gemv_waves(int mr, int r) { return (mr <= 2 && r == 2) ? 8 : 4; }

// 8-wave blocks run one per CU once their staged X passes 12 KB (each block
// stages all of X, which delays its weight stream), else two.  Measured,
// graph-replayed: down-proj K = 17408 M = 1 11.7 -> 11.0 us, o_proj K = 6144
// M = 1 6.5 -> 5.9, q-proj K = 5120 M = 2 8.5 -> 7.6; at K = 5120 M = 1
// (11 KB) two blocks stay better (q-proj 5.7 vs 6.0).
bool gemv_one_block_per_cu(int nw, size_t x_bytes) { return nw == 8 && x_bytes > 12 * 1024; }

// LDS a GEMV block may use: a block alone on its CU may take the CU's
// 160 KB; otherwise 64 KB keeps two or more blocks resident.
size_t gemv_lds_cap(int nw, size_t x_bytes) {
    return gemv_one_block_per_cu(nw, x_bytes) ? 159 * 1024 : 64 * 1024;
}

int mr_for(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

}  // namespace

namespace xhip_host {
// LDS bytes of the staged X (pieces + bias terms) for MR rows and K.
size_t gemv_x_bytes(int mr, int64_t K) { return (size_t)mr * (size_t)((K / 32 + 31) / 32) * 32 * (64 + 4); }
// Whether the GEMV stages all of X in LDS for M rows (what an RMSNorm
// prologue there needs).
bool gemv_stages_x(int64_t M, int64_t K) {
    const int mr = mr_for(M);
    const size_t xb = gemv_x_bytes(mr, K);
    return xb + 4096 <= gemv_lds_cap(gemv_waves(mr, 2), xb);
}
}  // namespace xhip_host

namespace {

// Allow a kernel more than the default 64 KB of dynamic LDS (once per
// kernel; the attribute must be set before such a launch).
bool allow_lds(GemvKernel k, size_t lds) {
    if (lds <= 64 * 1024) return true;
    static std::mutex mu;
    static GemvKernel done[64];
    static int n = 0;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n; ++i)
        if (done[i] == k) return true;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess)
        return false;
    if (n < 64) done[n++] = k;
    return true;
}

// Resident blocks per CU for a kernel at a given dynamic LDS size (cached).
int blocks_per_cu(GemvKernel k, size_t lds, int threads) {
    struct Entry { GemvKernel k; size_t lds; int dev; int v; };
    static Entry cache[256];
    static int n = 0;
    static std::mutex mu;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n; ++i)
        if (cache[i].k == k && cache[i].lds == lds && cache[i].dev == dev) return cache[i].v;
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, reinterpret_cast<const void*>(k), threads, lds) !=
            hipSuccess || v <= 0)
        v = 1;
    if (v > 8) v = 8;
    if (n < 256) cache[n++] = Entry{k, lds, dev, v};
    return v;
}

// Choose rows per item (R), rows per block and the grid.  Measured on
// MI355X (north-star, config-0/1/2/3 shapes, graph-replayed): two resident
// 256-thread blocks per CU, R = 2 and a one-item prefetch ring are best for
// M = 1; larger M keeps a two-item ring.  Each block runs
// (rows_blk / 2R) * nsteps items over its 4 waves.  Plans are cached per
// (epilogue, M, K, N of each descriptor) so repeated calls skip this.
struct PlanKey {
    int epi, mr, K, ndesc;
    int32_t N[4];
    bool operator==(const PlanKey& o) const {
        return epi == o.epi && mr == o.mr && K == o.K && ndesc == o.ndesc && N[0] == o.N[0] &&
               N[1] == o.N[1] && N[2] == o.N[2] && N[3] == o.N[3];
    }
};
struct PlanEntry {
    PlanKey key;
    GemvPlan plan;
    int32_t rows_blk;
    int dev;
};

template <int EPI, typename OutT>
GemvPlan plan_gemv(GemvParams& p, int mr) {
    PlanKey key = {EPI, mr, p.K, p.ndesc, {0, 0, 0, 0}};
    for (int i = 0; i < p.ndesc; ++i) key.N[i] = p.d[i].N;
    int dev = 0;
    (void)hipGetDevice(&dev);
    static PlanEntry cache[64];
    static int ncache = 0;
    static std::mutex mu;
    GemvPlan best = {};
    int32_t rows_blk = 0;
    bool hit = false;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (int i = 0; i < ncache; ++i)
            if (cache[i].dev == dev && cache[i].key == key) {
                best = cache[i].plan;
                rows_blk = cache[i].rows_blk;
                hit = true;
                break;
            }
    }
    if (!hit) {
        const int K = p.K;
        const int cpr = K / 32;
        const int nsteps = (cpr + 31) / 32;
        const int E = EPI == EPI_SWIGLU ? 2 : 1;
        const int cus = xhip_host::num_cus();
        int64_t total_rows = 0;
        for (int i = 0; i < p.ndesc; ++i) total_rows += p.d[i].N;
        const size_t x_bytes = xhip_host::gemv_x_bytes(mr, K);
        const Overrides& ov = overrides();
        const bool xlds_std = x_bytes + 4096 <= 64 * 1024;
        const int r = ov.r > 0 ? ov.r : (mr >= 4 && !xlds_std ? 1 : 2);
        const size_t lds_cap = gemv_lds_cap(gemv_waves(mr, r), x_bytes);
        const bool xlds = x_bytes + 4096 <= lds_cap;
        const int pf = ov.pf > 0 ? ov.pf : (mr == 1 ? 1 : 2);
        // Two 8-wave blocks per CU -> one 16-wave block (same waves per SIMD,
        // X staged once per CU).  A CU's second 8-wave block gets its X
        // after the first block's weight prefetch (a CU's loads return in
        // order) and starts streaming ~5 us late.  Measured, graph-replayed:
        // fused QKV 9.13 -> 8.95 us, LA in_proj 10.13 -> 10.02, decode layer
        // M = 1 45.95 -> 45.4; single projections lose a little (config 1
        // 16.97 -> 17.19, q-proj 5.63 -> 5.67, N = 48 3.53 -> 3.71), so the
        // default is fused launches only (XINFER_GEMV_W16: 0 never, 1 always).
        const bool w16_ok = ov.bpc <= 0 && EPI != EPI_ARGMAX && mr == 1 && r == 2 && pf == 1 && xlds &&
                            !gemv_one_block_per_cu(gemv_waves(mr, r), x_bytes);
        const bool w16 = w16_ok && (ov.w16 > 0 || (ov.w16 < 0 && p.ndesc >= 2));
        const int nw = w16 ? 16 : gemv_waves(mr, r);
        GemvKernel k = kernel_for<EPI, OutT>(mr, r, xlds, pf, w16);
        int64_t rows = 0;
        size_t lds = 0;
        int bpc = ov.bpc > 0 ? ov.bpc : ((xlds && gemv_one_block_per_cu(nw, x_bytes)) || w16) ? 1 : 2;
        for (int pass = 0; pass < 3; ++pass) {
            const int64_t target = (int64_t)cus * bpc;
            rows = (total_rows + target - 1) / target;
            rows = ((rows + 2 * r - 1) / (2 * r)) * (2 * r);
            size_t part = (size_t)rows * mr * E * nsteps * 4;
            if (EPI == EPI_ARGMAX && part < 2048) part = 2048;
            lds = kGemvLdsHead + (xlds ? x_bytes : 0) + part;
            if (lds <= lds_cap) break;
            bpc *= 2;  // smaller row ranges until the partial slots fit
        }
        (void)allow_lds(k, lds);  // before the occupancy query; checked again at launch
        const int occ = blocks_per_cu(k, lds, 64 * nw);
        auto lds_for = [&](int64_t rr) {
            size_t part = (size_t)rr * mr * E * nsteps * 4;
            if (EPI == EPI_ARGMAX && part < 2048) part = 2048;
            return kGemvLdsHead + (xlds ? x_bytes : 0) + part;
        };
        if (ov.bpc <= 0 && occ < bpc) {  // cannot hold the target residency
            const int64_t target = (int64_t)cus * occ;
            int64_t r2 = (total_rows + target - 1) / target;
            r2 = ((r2 + 2 * r - 1) / (2 * r)) * (2 * r);
            if (lds_for(r2) <= lds_cap) rows = r2;
        }
        // Each descriptor rounds its block count up, so several descriptors
        // can overshoot the resident grid by a block or two, which would then
        // run as a second wave on its own (fused QKV at M = 1: 513 blocks for
        // 512 slots).  Grow the rows per block until the grid is resident.
        if (ov.bpc <= 0) {
            // slots at the planned residency: the occupancy query may allow
            // more blocks per CU than the plan wants (fused QKV at M = 2 is
            // planned one block per CU; counting LDS-allowed slots gave 258
            // blocks on 256 CUs and 15.4 us against 10.2 us for the same rows
            // as one descriptor)
            const int64_t slots = (int64_t)cus * (occ < bpc ? occ : bpc);
            for (int it = 0; it < 64; ++it) {
                int64_t nb = 0;
                for (int i = 0; i < p.ndesc; ++i) nb += (p.d[i].N + rows - 1) / rows;
                if (nb <= slots || lds_for(rows + 2 * r) > lds_cap) break;
                rows += 2 * r;
            }
            lds = lds_for(rows);
        }
        best.mr = mr;
        best.r = r;
        best.pf = pf;
        best.nw = nw;
        best.w16 = w16;
        best.xlds = xlds;
        best.lds = lds;
        rows_blk = (int32_t)rows;
        std::lock_guard<std::mutex> lock(mu);
        if (ncache < 64) cache[ncache++] = PlanEntry{key, best, rows_blk, dev};
    }
    int blocks = 0;
    for (int i = 0; i < p.ndesc; ++i) {
        p.d[i].rows_blk = rows_blk;
        p.d[i].block_begin = blocks;
        blocks += (p.d[i].N + rows_blk - 1) / rows_blk;
    }
    for (int i = p.ndesc; i < 4; ++i) p.d[i] = p.d[0], p.d[i].block_begin = 0x7FFFFFFF;
    best.blocks = blocks;
    return best;
}

template <int EPI, typename OutT>
int launch_plan(const GemvParams& p, const GemvPlan& pl, hipStream_t st) {
    GemvKernel k = kernel_for<EPI, OutT>(pl.mr, pl.r, pl.xlds, pl.pf, pl.w16);
    if (!allow_lds(k, pl.lds)) return XINFER_ERR_HIP;
    hipLaunchKernelGGL(k, dim3(pl.blocks), dim3(64 * pl.nw), pl.lds, st, p);
    return XINFER_OK;
}

int check_common(int64_t M, int64_t N, int64_t K, int32_t G) {
    if (G != kGroup || (K % kGroup) != 0) return XINFER_ERR_UNSUPPORTED;
    if (K > (1LL << 24) || N > (1LL << 30) || M > (1LL << 30)) return XINFER_ERR_UNSUPPORTED;
    // the kernels address one weight matrix with 32-bit buffer offsets
    if (N * (K / 2) >= (1LL << 32) - 4096) return XINFER_ERR_UNSUPPORTED;
    return XINFER_OK;
}

}  // namespace

namespace xhip_host {

int num_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (!v) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

int launch_status() { return hipGetLastError() == hipSuccess ? XINFER_OK : XINFER_ERR_HIP; }

// GEMV for one slab of at most 8 activation rows.
template <int EPI, typename OutT>
int gemv_f16(hipStream_t st, const GemvParams& base, int64_t M) {
    GemvParams p = base;
    p.M = (int32_t)M;
    const GemvPlan pl = plan_gemv<EPI, OutT>(p, mr_for(M));
    if (pl.blocks <= 0) return XINFER_OK;
    if (p.norm_w && !pl.xlds) return XINFER_ERR_UNSUPPORTED;  // the prologue runs while staging X
    if (launch_plan<EPI, OutT>(p, pl, st)) return XINFER_ERR_HIP;
    return launch_status();
}

}  // namespace xhip_host

// Forward declarations: M > 8 with fp16 activations (chunked prefill) and
// the MFMA small-batch kernel for 2 <= M <= 8 (gemv_mb_int4.hip; each returns
// 1 when the shape is left to the VALU GEMV here).
namespace xhip_host {
// norm_w: RMSNorm of X inside the kernel (M = 3, 4, 8 with every row whole in
// one block; otherwise the shape is declined)
int mb_linear(hipStream_t st, const xinfer_fused_desc* descs, int nd, const void* X, bool y_f32,
              int64_t M, int64_t K, bool residual, int* rc, const float* norm_w = nullptr, float eps = 0.0f);
int mb_swiglu(hipStream_t st, void* Y, const void* X, const uint8_t* Wg, const void* Sg,
              const uint8_t* Wu, const void* Su, int64_t M, int64_t N, int64_t K,
              int* rc, const float* norm_w = nullptr, float eps = 0.0f);
int mb_argmax_plan(int64_t M, int64_t N, int64_t K, int* nparts);
int mb_max_m();  // largest M the small-batch kernel takes (then the GEMM)
int mb_argmax(hipStream_t st, float* logits, const void* X, const uint8_t* W, const void* S,
              int64_t M, int64_t N, int64_t K, ArgCand* parts, int* nparts, int* rc);
int gemm_int4_f16(hipStream_t st, void* Y, bool y_f32, const void* X, const uint8_t* W,
                  const uint16_t* S, const uint8_t* W2, const uint16_t* S2, const float* bias,
                  int64_t M, int64_t N, int64_t K, bool residual = false);
}

namespace {

int linear_f16_impl(void* stream, void* Y, bool y_f32, const void* X, const uint8_t* W,
                    const void* S, const float* bias, int64_t M, int64_t N, int64_t K,
                    int32_t G, bool residual = false) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_common(M, N, K, G);
    if (rc) return rc;
    if (!Y || !X || !W || !S) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(W, 16) || !aligned(X, 16) || !aligned(S, 2) || !aligned(Y, y_f32 ? 4 : 2) ||
        !aligned(bias, 4))
        return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (M >= 2 && M <= mb_max_m()) {
        const xinfer_fused_desc one = {Y, W, S, bias, N};
        int mrc = XINFER_OK;
        if (!pairm_linear(st, &one, 1, X, y_f32, M, K, residual, &mrc)) return mrc;
        if (!mb_linear(st, &one, 1, X, y_f32, M, K, residual, &mrc)) return mrc;
    }
    if (M > 8)
        return gemm_int4_f16(st, Y, y_f32, X, W, (const uint16_t*)S, nullptr, nullptr, bias, M, N, K,
                             residual);
    if (M == 1) {  // large N: the row-pair kernel (its 4-wave form for long K)
        const xinfer_fused_desc one = {Y, W, S, bias, N};
        int prc = XINFER_OK;
        if (!pair_linear(st, &one, 1, X, y_f32, K, residual, nullptr, 0.0f, &prc)) return prc;
        if (!pairm_linear(st, &one, 1, X, y_f32, 1, K, residual, &prc)) return prc;
    }
    GemvParams p = {};
    p.ndesc = 1;
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    p.d[0].W = W;
    p.d[0].S = reinterpret_cast<const uint16_t*>(S);
    p.d[0].bias = bias;
    p.d[0].Y = Y;
    p.d[0].N = (int32_t)N;
    p.d[0].residual = residual ? 1 : 0;
    return y_f32 ? gemv_f16<EPI_PLAIN, float>(st, p, M) : gemv_f16<EPI_PLAIN, f16>(st, p, M);
}

// RMSNorm before a projection.  M = 1 (X staged whole by the GEMV): inside
// the projection kernel, from the staged registers; the fused entry points
// below also route M = 2 / 3 (dot2 kernel, GEMV) and M = 4 / 8 (small-batch
// kernel, one k-slice) to kernel variants that apply it while staging X.
// Otherwise the standalone rmsnorm kernel writes the normalised rows to the
// caller's workspace (M * K fp16), which the projection then reads.
// norm_input returns the X the projection reads and whether the kernel
// applies the norm (the M = 1 case).
bool norm_in_projection(int64_t M, int64_t K) { return M == 1 && xhip_host::gemv_stages_x(1, K); }

// The caller's workspace for the normalised rows, checked wherever the
// workspace size is non-zero (also when the kernel then applies the norm
// itself, so that a call's errors do not depend on the route it takes).
int check_norm_ws(const float* norm_w, int64_t M, int64_t K, const void* ws, size_t ws_bytes) {
    if (!norm_w || norm_in_projection(M, K)) return XINFER_OK;
    if (!ws || ws_bytes < (size_t)M * (size_t)K * 2) return XINFER_ERR_SCRATCH;
    if (!xhip_host::aligned(ws, 16)) return XINFER_ERR_MISALIGNED;
    return XINFER_OK;
}

int norm_input(hipStream_t st, const void* X, const float* norm_w, float eps, int64_t M, int64_t K,
               void* ws, size_t ws_bytes, const void** Xp, bool* in_kernel) {
    *Xp = X;
    *in_kernel = false;
    if (!norm_w) return XINFER_OK;
    if (norm_in_projection(M, K)) {
        *in_kernel = true;
        return XINFER_OK;
    }
    if (int rc = check_norm_ws(norm_w, M, K, ws, ws_bytes)) return rc;
    *Xp = ws;
    return xinfer_rmsnorm_f16(st, ws, X, norm_w, M, K, eps);
}

// linear_int4_fused with an optional RMSNorm on X first (norm_w != null).
int fused_f16_impl(void* stream, const void* X0, const xinfer_fused_desc* descs, int32_t num_descs,
                   int64_t M, int64_t K, int32_t group_size, const float* norm_w, float eps,
                   void* ws = nullptr, size_t ws_bytes = 0) {
    if (!descs || num_descs <= 0 || num_descs > 4) return XINFER_ERR_INVALID_ARG;
    if (M <= 0 || K <= 0) return XINFER_OK;
    if (!X0) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(X0, 16) || !aligned(norm_w, 4)) return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for (int i = 0; i < num_descs; ++i) {  // shapes first: nothing is launched for a bad call
        const xinfer_fused_desc& q = descs[i];
        if (q.N <= 0) continue;
        int rc = check_common(M, q.N, K, group_size);
        if (rc) return rc;
    }
    GemvParams p = {};
    p.K = (int32_t)K;
    xinfer_fused_desc live[4];
    int nd = 0;
    for (int i = 0; i < num_descs; ++i) {
        const xinfer_fused_desc& q = descs[i];
        if (q.N <= 0) continue;  // empty projection: nothing to write
        int rc = check_common(M, q.N, K, group_size);
        if (rc) return rc;
        if (!q.Y || !q.W_int4 || !q.scales) return XINFER_ERR_INVALID_ARG;
        if (!aligned(q.W_int4, 16) || !aligned(q.scales, 2) || !aligned(q.Y, 2) || !aligned(q.bias, 4))
            return XINFER_ERR_MISALIGNED;
        live[nd] = q;
        GemvDesc& g = p.d[nd++];
        g.W = q.W_int4;
        g.S = reinterpret_cast<const uint16_t*>(q.scales);
        g.bias = q.bias;
        g.Y = q.Y;
        g.N = (int32_t)q.N;
    }
    if (nd == 0) return XINFER_OK;
    if (int rc = check_norm_ws(norm_w, M, K, ws, ws_bytes)) return rc;
    int64_t rows = 0;
    for (int i = 0; i < nd; ++i) rows += live[i].N;
    // M = 2 / 3 on the dot2 kernel, M = 3 / 4 / 8 on the small-batch kernel:
    // the norm in their X staging (no standalone norm launch) when they
    // take the shape whole
    if (norm_w && (M == 2 || M == 3) && M <= mb_max_m() && pairm_takes(M, K, rows, false)) {
        int mrc = XINFER_OK;
        if (!pairm_linear(st, live, nd, X0, false, M, K, false, &mrc, norm_w, eps)) return mrc;
    }
    if (norm_w && M >= 3 && M <= 8 && M <= mb_max_m()) {
        int mrc = XINFER_OK;
        if (!pairm_takes(M, K, rows, false) && !mb_linear(st, live, nd, X0, false, M, K, false, &mrc, norm_w, eps))
            return mrc;
    }
    // M = 2 on the GEMV (X staged in LDS): the norm in its X staging
    if (norm_w && M == 2 && xhip_host::gemv_stages_x(2, K) && !pairm_takes(2, K, rows, false)) {
        p.X = reinterpret_cast<const f16*>(X0);
        p.norm_w = norm_w;
        p.norm_eps = eps;
        p.ndesc = nd;
        return gemv_f16<EPI_PLAIN, f16>(st, p, M);
    }
    const void* X = X0;
    bool norm_in_kernel = false;
    if (int rc = norm_input(st, X0, norm_w, eps, M, K, ws, ws_bytes, &X, &norm_in_kernel)) return rc;
    p.X = reinterpret_cast<const f16*>(X);
    p.norm_w = norm_in_kernel ? norm_w : nullptr;
    p.norm_eps = eps;
    if (M >= 2 && M <= mb_max_m()) {
        int mrc = XINFER_OK;
        if (!pairm_linear(st, live, nd, X, false, M, K, false, &mrc)) return mrc;
        if (!mb_linear(st, live, nd, X, false, M, K, false, &mrc)) return mrc;
    }
    if (M > 8) {  // one GEMM per descriptor
        for (int i = 0; i < nd; ++i) {
            const xinfer_fused_desc& q = live[i];
            const int rc = gemm_int4_f16(st, q.Y, false, X, q.W_int4, (const uint16_t*)q.scales, nullptr,
                                         nullptr, q.bias, M, q.N, K);
            if (rc) return rc;
        }
        return XINFER_OK;
    }
    if (M == 1) {  // large N: the row-pair kernel (the norm, if any, in its X staging)
        int prc = XINFER_OK;
        if (!pair_linear(st, live, nd, X, false, K, false, norm_in_kernel ? norm_w : nullptr, eps, &prc))
            return prc;
        if (!norm_in_kernel && !pairm_linear(st, live, nd, X, false, 1, K, false, &prc)) return prc;
    }
    p.ndesc = nd;
    return gemv_f16<EPI_PLAIN, f16>(st, p, M);
}

int swiglu_f16_impl(void* stream, void* Y, const void* X0, const uint8_t* W_gate, const void* scales_gate,
                    const uint8_t* W_up, const void* scales_up, int64_t M, int64_t N, int64_t K,
                    int32_t group_size, const float* norm_w, float eps, void* ws = nullptr,
                    size_t ws_bytes = 0) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    int rc = check_common(M, N, K, group_size);
    if (rc) return rc;
    if (!Y || !X0 || !W_gate || !scales_gate || !W_up || !scales_up) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(W_gate, 16) || !aligned(W_up, 16) || !aligned(X0, 16) || !aligned(Y, 2) ||
        !aligned(scales_gate, 2) || !aligned(scales_up, 2) || !aligned(norm_w, 4))
        return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if ((rc = check_norm_ws(norm_w, M, K, ws, ws_bytes))) return rc;
    if (norm_w && (M == 2 || M == 3) && M <= mb_max_m() && pairm_takes(M, K, 2 * N, true)) {
        int mrc = XINFER_OK;  // the norm in the dot2 kernel's X staging
        if (!pairm_swiglu(st, Y, X0, W_gate, scales_gate, W_up, scales_up, M, N, K, &mrc, norm_w, eps)) return mrc;
    }
    if (norm_w && M >= 3 && M <= 8 && M <= mb_max_m() && !pairm_takes(M, K, 2 * N, true)) {
        int mrc = XINFER_OK;  // the norm in the small-batch kernel's X staging
        if (!mb_swiglu(st, Y, X0, W_gate, scales_gate, W_up, scales_up, M, N, K, &mrc, norm_w, eps)) return mrc;
    }
    const bool gemv_norm2 = norm_w && M == 2 && gemv_stages_x(2, K) && !pairm_takes(2, K, 2 * N, true);
    const void* X = X0;
    bool norm_in_kernel = gemv_norm2;  // M = 2: the GEMV's X staging applies the norm
    if (!gemv_norm2 && (rc = norm_input(st, X0, norm_w, eps, M, K, ws, ws_bytes, &X, &norm_in_kernel))) return rc;
    if (M >= 2 && M <= mb_max_m() && !gemv_norm2) {
        int mrc = XINFER_OK;
        if (!pairm_swiglu(st, Y, X, W_gate, scales_gate, W_up, scales_up, M, N, K, &mrc)) return mrc;
        if (!mb_swiglu(st, Y, X, W_gate, scales_gate, W_up, scales_up, M, N, K, &mrc))
            return mrc;
    }
    if (M > 8)
        return gemm_int4_f16(st, Y, false, X, W_gate, (const uint16_t*)scales_gate, W_up,
                             (const uint16_t*)scales_up, nullptr, M, N, K);
    if (M == 1 && swiglu_pair_on()) {  // large N: the row-pair kernel (the norm, if any, in its X staging)
        int prc = XINFER_OK;
        if (!pair_swiglu(st, Y, X, W_gate, scales_gate, W_up, scales_up, N, K, norm_in_kernel ? norm_w : nullptr,
                         eps, &prc))
            return prc;
    }
    GemvParams p = {};
    p.ndesc = 1;
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    p.norm_w = norm_in_kernel ? norm_w : nullptr;
    p.norm_eps = eps;
    p.d[0].W = W_gate;
    p.d[0].S = reinterpret_cast<const uint16_t*>(scales_gate);
    p.d[0].W2 = W_up;
    p.d[0].S2 = reinterpret_cast<const uint16_t*>(scales_up);
    p.d[0].Y = Y;
    p.d[0].N = (int32_t)N;
    return gemv_f16<EPI_SWIGLU, f16>(st, p, M);
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
    return fused_f16_impl(stream, X, descs, num_descs, M, K, group_size, nullptr, 0.0f);
}

int xinfer_mlp_gate_up_swiglu_int4_f16(void* stream, void* Y, const void* X,
                                       const uint8_t* W_gate, const void* scales_gate,
                                       const uint8_t* W_up, const void* scales_up, int64_t M,
                                       int64_t N, int64_t K, int32_t group_size) {
    return swiglu_f16_impl(stream, Y, X, W_gate, scales_gate, W_up, scales_up, M, N, K, group_size,
                           nullptr, 0.0f);
}

size_t xinfer_rmsnorm_projection_workspace_bytes(int64_t M, int64_t K) {
    if (M <= 0 || K <= 0 || norm_in_projection(M, K)) return 0;
    return (size_t)M * (size_t)K * 2;
}

int xinfer_rmsnorm_linear_int4_fused_f16(void* stream, const void* X, const float* norm_weight,
                                         float eps, const xinfer_fused_desc* descs, int32_t num_descs,
                                         int64_t M, int64_t K, int32_t group_size, void* workspace,
                                         size_t workspace_bytes) {
    if (!norm_weight) return XINFER_ERR_INVALID_ARG;
    return fused_f16_impl(stream, X, descs, num_descs, M, K, group_size, norm_weight, eps, workspace,
                          workspace_bytes);
}

int xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16(void* stream, void* Y, const void* X,
                                               const float* norm_weight, float eps,
                                               const uint8_t* W_gate, const void* scales_gate,
                                               const uint8_t* W_up, const void* scales_up, int64_t M,
                                               int64_t N, int64_t K, int32_t group_size, void* workspace,
                                               size_t workspace_bytes) {
    if (!norm_weight) return XINFER_ERR_INVALID_ARG;
    return swiglu_f16_impl(stream, Y, X, W_gate, scales_gate, W_up, scales_up, M, N, K, group_size,
                           norm_weight, eps, workspace, workspace_bytes);
}

int xinfer_linear_int4_residual_f16(void* stream, void* residual, const void* X, const uint8_t* W_int4,
                                    const void* scales, const float* bias, int64_t M, int64_t N,
                                    int64_t K, int32_t group_size) {
    return linear_f16_impl(stream, residual, false, X, W_int4, scales, bias, M, N, K, group_size, true);
}

size_t xinfer_lm_head_argmax_scratch_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || M > 8) return 0;
    int nparts = 0;
    if (M >= 2 && K > 0 && !xhip_host::mb_argmax_plan(M, N, K, &nparts))
        return (size_t)M * (size_t)nparts * sizeof(ArgCand);
    GemvParams p = {};
    p.ndesc = 1;
    p.K = (int32_t)(K > 0 ? K : 128);
    p.d[0].N = (int32_t)N;
    const GemvPlan pl = plan_gemv<EPI_ARGMAX, float>(p, mr_for(M));
    return (size_t)M * (size_t)pl.blocks * sizeof(ArgCand);
}

}  // extern "C"

namespace xhip_host {
void* library_scratch(hipStream_t st, size_t bytes);  // argmax.hip
}

namespace xhip_host {

// LM head + argmax on candidate scratch `cand` of `cand_bytes` bytes; with
// cand == NULL and library_ok, the library's per-stream buffer (allocated on
// first use).
int lm_head_argmax_impl(void* stream, int32_t* ids, float* logits, const void* X, const uint8_t* W_int4,
                        const void* scales, int64_t M, int64_t N, int64_t K, int32_t group_size, void* cand,
                        size_t cand_bytes, bool library_ok) {
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
    auto get_parts = [&](size_t need, ArgCand** parts) {
        if (!cand) {
            if (!library_ok) return XINFER_ERR_SCRATCH;
            cand = library_scratch(st, need);
            if (!cand) return XINFER_ERR_SCRATCH;
            cand_bytes = need;
        }
        if (cand_bytes < need || !aligned(cand, 8)) return XINFER_ERR_SCRATCH;
        *parts = reinterpret_cast<ArgCand*>(cand);
        return XINFER_OK;
    };
    int nparts = 0;
    if (M >= 2 && !mb_argmax_plan(M, N, K, &nparts)) {
        ArgCand* parts = nullptr;
        if (int src = get_parts((size_t)M * (size_t)nparts * sizeof(ArgCand), &parts)) return src;
        int mrc = XINFER_OK;
        if (!mb_argmax(st, logits, X, W_int4, scales, M, N, K, parts, &nparts, &mrc)) {
            if (mrc) return mrc;
            hipLaunchKernelGGL((argmax_finalize_kernel<int32_t>), dim3((unsigned)M), dim3(256), 0, st,
                               parts, (int32_t)nparts, ids);
            return launch_status();
        }
    }
    GemvParams p = {};
    p.ndesc = 1;
    p.X = reinterpret_cast<const f16*>(X);
    p.K = (int32_t)K;
    p.M = (int32_t)M;
    p.d[0].W = W_int4;
    p.d[0].S = reinterpret_cast<const uint16_t*>(scales);
    p.d[0].Y = logits;
    p.d[0].N = (int32_t)N;
    const GemvPlan pl = plan_gemv<EPI_ARGMAX, float>(p, mr_for(M));
    const int blocks = pl.blocks;
    if (int src = get_parts((size_t)M * (size_t)blocks * sizeof(ArgCand), &p.parts)) return src;
    if (launch_plan<EPI_ARGMAX, float>(p, pl, st) || launch_status()) return XINFER_ERR_HIP;
    hipLaunchKernelGGL((argmax_finalize_kernel<int32_t>), dim3((unsigned)M), dim3(256), 0, st,
                       p.parts, (int32_t)blocks, ids);
    return launch_status();
}

}  // namespace xhip_host

extern "C" int xinfer_lm_head_argmax_int4(void* stream, int32_t* ids, float* logits,
                                          const void* X, const uint8_t* W_int4,
                                          const void* scales, int64_t M, int64_t N, int64_t K,
                                          int32_t group_size, void* scratch_buf,
                                          size_t scratch_bytes) {
    return xhip_host::lm_head_argmax_impl(stream, ids, logits, X, W_int4, scales, M, N, K, group_size, scratch_buf,
                               scratch_bytes, true);
}

