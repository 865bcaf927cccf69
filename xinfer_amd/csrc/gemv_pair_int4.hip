// M = 1 INT4-G128-SYM GEMV streaming weight rows in pairs (gfx950), and
// its M = 2..4 form (gemv_pairm_int4_kernel, after the M = 1 kernel).
//
// Same contract as the decode GEMV (src/ops/linear.cpp:165-305, and the
// fused descriptors of linear.cpp:351-498) for large decode projections: one
// activation row, K a multiple of 1024 in 4096..6144, N even.  Two adjacent weight rows are K
// contiguous bytes, i.e. P = K / 1024 pieces of 1 KB: a wave reads a row
// pair as P fully coalesced 1 KB loads (lane j takes bytes 16j..16j+15 of
// each piece).  Streaming whole 1 KB pieces reads faster on MI355X than the
// GEMV's 512-byte row pieces (a pure read of the north-star matrix:
// 14.2-14.6 us in pairs against 15.8-17.0 us in the GEMV's pattern).
//
//   * lane j's 16 bytes of piece i are chunk c = 64 i + j of the pair: row
//     c / (K/32) of the pair, k = 32 (c % (K/32)).  That position is the
//     same for every pair, so each lane keeps the activations of its P
//     chunks in registers (permuted to the decode's pair order, with the
//     chunk's bias term), loaded once.  The block stages X once in LDS for
//     that (one thread per 32-k chunk: 64 bytes loaded, permuted, bias term
//     summed), and every lane reads its chunks from there: X is fetched
//     from L2 once per block instead of twice per wave (the two rows of a
//     pair use the same chunks).
//   * decode and arithmetic as the GEMV: one v_bitop3_b32 per nibble pair
//     gives exact biased fp16 integers, v_dot2_f32_f16 into ta / tb, the
//     chunk's dot product is ta + tb/16 with ta started at the bias term,
//     scaled by the fp16 group scale in FP32;
//   * a wave owns a set of pairs (over all descriptors: a contiguous range,
//     or for large launches every nwaves-th pair), so a row's sum never
//     leaves its wave: 64-lane reduction per pair into a small per-wave LDS
//     buffer; the results are stored after the loop.  No
//     global store or load sits inside the streaming loop: on gfx9 the
//     vector-memory counter counts both, and one there made the compiler
//     drain the prefetch ring on every item (measured);
//   * SwiGLU (SWIGLU = true; d[0] = gate, d[1] = up, N rows each): a wave
//     owns the same pairs of both matrices and streams its gate pairs, then
//     its up pairs; the epilogue forms silu(g) * u from its own LDS
//     results, so gate and up rows never cross waves;
//   * every load is a buffer load with a constant per-lane offset and a
//     wave-uniform pair offset; one item (the P pieces of one pair) in flight
//     while the previous one is computed.  The ring runs whole passes; the
//     last item is computed after it, so no wave waits on a load issued past
//     its end.

#include <stdlib.h>

#include "common.h"

namespace xhip {

struct PairDesc {
    const uint8_t* W;   // [N][K/2]
    const uint16_t* S;  // [N][K/128]
    const float* bias;  // optional [N]
    void* Y;            // [N] fp16 / fp32
    int32_t N;          // even
    int32_t pair_begin; // first pair of this descriptor in the pair space
    int32_t residual;   // fp16 Y: Y = fp16(Y + fp16(result))
};

struct PairParams {
    PairDesc d[4];
    int32_t ndesc;
    int32_t npairs;     // pairs over all descriptors
    int32_t strided;    // 1: wave w takes pairs w, w + waves, ...; 0: a contiguous range
    const f16* X;       // [K]
    // The launch's G pair owners (waves, or pair groups) split the pairs
    // without a division in the kernel: npairs = wq G + wr, and
    // n / G = (n wm) >> (32 + ws) for n < 2^31 (host-computed; G^2 < 2^31).
    int32_t wq, wr, ws;
    uint64_t wm;
    int32_t G;          // = gridDim.x times owners per block (gridDim is an argument load of its own)
    const float* norm_w; // M = 1 kernel: RMSNorm weight [K] applied to X while staging, or null
    float norm_eps;
    // SwiGLU, strided, 0 < wr <= 2 blocks: every wave takes wq gate and wq
    // up pairs, and leftover pair wq G + e goes to block e / 2, its gate rows
    // to wave 2 (e % 2) and its up rows to wave 2 (e % 2) + 1
    int32_t xsplit;
};

// The kernel arguments used before and in the streaming loop, read
// together at the kernel's start: the empty asm needs them all in SGPRs, so
// the compiler issues every load first and waits once (it otherwise chained
// three dependent load/wait rounds ahead of the first weight load).
struct PairArgs {
    const f16* X;
    const uint8_t* w0;
    const uint8_t* w1;
    const uint8_t* w2;
    const uint8_t* w3;
    const uint16_t* s0;
    const uint16_t* s1;
    const uint16_t* s2;
    const uint16_t* s3;
    int pb1, pb2, pb3;  // first pair of descriptors 1-3 (INT_MAX past ndesc)
    bool strided;
    int32_t wq, wr, ws;
    uint64_t wm;
    int32_t G;
    const float* norm_w;
    bool xsplit;
};
__device__ __forceinline__ PairArgs pair_args(const PairParams& p) {
    PairArgs a;
    a.X = p.X;
    a.w0 = p.d[0].W;
    a.w1 = p.d[1].W;
    a.w2 = p.d[2].W;
    a.w3 = p.d[3].W;
    a.s0 = p.d[0].S;
    a.s1 = p.d[1].S;
    a.s2 = p.d[2].S;
    a.s3 = p.d[3].S;
    const int nd = p.ndesc, r1 = p.d[1].pair_begin, r2 = p.d[2].pair_begin, r3 = p.d[3].pair_begin;
    const int st = p.strided;
    a.wq = p.wq;
    a.wr = p.wr;
    a.ws = p.ws;
    a.wm = p.wm;
    a.G = p.G;
    a.norm_w = p.norm_w;
    const int xsp = p.xsplit;
    asm volatile("" ::"s"(a.X), "s"(a.w0), "s"(a.w1), "s"(a.w2), "s"(a.w3), "s"(a.s0), "s"(a.s1), "s"(a.s2),
                 "s"(a.s3), "s"(nd), "s"(r1), "s"(r2), "s"(r3), "s"(st), "s"(a.wq), "s"(a.wr), "s"(a.ws),
                 "s"(a.wm), "s"(a.G), "s"(a.norm_w), "s"(xsp));
    a.xsplit = xsp != 0;
    a.pb1 = nd > 1 ? r1 : 0x7FFFFFFF;
    a.pb2 = nd > 2 ? r2 : 0x7FFFFFFF;
    a.pb3 = nd > 3 ? r3 : 0x7FFFFFFF;
    a.strided = st != 0;
    return a;
}

// Pair range [q0, q0 + nh) of owner g (step qs = 1), or for strided
// launches pairs g, g + G, ... (nh of them).  A 64-bit division here took
// ~0.5 us of the kernel's start before the first load could issue.
__host__ __device__ __forceinline__ void pair_range(const PairArgs& a, uint32_t g, int& q0, int& nh) {
    const uint32_t wq = (uint32_t)a.wq, wr = (uint32_t)a.wr;
    if (a.strided) {
        q0 = (int)g;
        nh = (int)(wq + (g < wr ? 1u : 0u));
    } else {
        auto div = [&](uint32_t n) { return (uint32_t)(((uint64_t)n * a.wm) >> (32 + a.ws)); };
        const uint32_t b = g * wq + div(g * wr), e = (g + 1) * wq + div((g + 1) * wr);
        q0 = (int)b;
        nh = (int)(e - b);
    }
}

// A 32-k chunk's bias term -(1032 sum x_even + 72 sum x_odd) (the biased
// decode's 1024 + u and 1024 + 16u forms, u = q + 8) as dot2 of the natural
// (x_2j, x_2j+1) pairs with this constant: products exact in FP32.
__device__ constexpr f16x2 kBiasPair = {(f16)-1032.0f, (f16)-72.0f};

constexpr int kPairMaxPerWave = 128;  // pairs per wave (LDS results: 1 KB per wave)
constexpr int kPairPF = 1;            // items in flight while one is computed

template <int P, typename OutT, bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_pair_int4_kernel(const PairParams p) {
    constexpr int PF = kPairPF;
    constexpr int K = 1024 * P;
    constexpr int CPR = K / 32;       // 16-byte chunks per row
    static_assert(CPR <= 256, "one staging thread per chunk");
    constexpr int NG = K / 128;       // scale groups per row
    constexpr uint32_t kRowBytes = K / 2;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool hi = lane >= 32;
    const PairArgs a = pair_args(p);

    // --- X staged in LDS once per block: chunk c (32 k, c < K/32) as 64
    // bytes in the decode's pair order plus its bias term.  The global loads
    // go out first, before the weight prefetch (loads complete in issue order, so
    // the staging then waits for X alone).
    __shared__ __align__(16) unsigned char xst[CPR * 64];
    __shared__ float xcb[CPR];
    u32x4 xr[4];
    float4 nwr[8];  // RMSNorm weights of the chunk (norm_w set)
    const bool norm = a.norm_w != nullptr;
    if (tid < CPR) {
        const u32x4* src = reinterpret_cast<const u32x4*>(a.X + tid * 32);
#pragma unroll
        for (int v = 0; v < 4; ++v) xr[v] = src[v];
        if (norm) {
            const float4* nsrc = reinterpret_cast<const float4*>(a.norm_w + tid * 32);
#pragma unroll
            for (int v = 0; v < 8; ++v) nwr[v] = nsrc[v];
        }
    }

    // this wave's pairs
    const int nwaves = a.G;  // gridDim.x * 4
    const int gw = (int)blockIdx.x * 4 + wave;
    // Strided (large launches): the pairs of every wave are spread over the
    // whole matrix, so the XCDs' uneven memory rates average out instead of
    // some XCDs' waves finishing their contiguous ranges ~0.8 us after
    // others (north star 16.2-16.3 -> 16.0 us, config 1 16.0 -> 15.8 us;
    // with 2-3 pairs per wave, as at o_proj, contiguous ranges measured
    // faster).  q0 = first pair, qs = step, nh = pairs of the wave.
    const bool strided = a.strided;
    const int qs = strided ? nwaves : 1;
    int q0, nh;  // nh = pairs of the wave (per matrix for SwiGLU)
    pair_range(a, (uint32_t)gw, q0, nh);
    // leftover split (SwiGLU): nh = wq for every wave, plus one item of the
    // block's leftover pairs: pair px of matrix wave % 2
    int has_x = 0, px = 0;
    if (SWIGLU && a.xsplit) {
        nh = a.wq;
        const int e = 2 * (int)blockIdx.x + (wave >> 1);
        has_x = e < a.wr ? 1 : 0;
        px = a.wq * a.G + e;
    }
    const int q1 = q0 + nh;  // contiguous ranges: one past the last pair

    f16x2 xp[P][16];  // the chunks' activations in the decode's pair order
    float cb[P];      // chunk bias terms -(1032 sum x_even + 72 sum x_odd)

    // per-lane byte offsets of the scales of piece i (within a pair's scales)
    uint32_t soff[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = 64 * i + lane;
        const int row = c < CPR ? 0 : 1;
        const int cr = c - row * CPR;
        soff[i] = (uint32_t)(row * NG + (cr >> 2)) * 2u;
    }

    // --- items (pairs).  The descriptors' fields are read once and selected
    // by wave-uniform compares (no kernel-argument load per item).
    const int pb1 = a.pb1, pb2 = a.pb2, pb3 = a.pb3;
    auto sel = [](int di, auto a0, auto a1, auto a2, auto a3) { return di == 0 ? a0 : di == 1 ? a1 : di == 2 ? a2 : a3; };
    struct Item {
        u32x4 w[P];
        uint32_t s[P];
    };
    const int nitems = SWIGLU ? 2 * nh + has_x : nh;
    // a wave without pairs issues its prefetch against empty resources
    const int live = nitems > 0 ? 1 : 0;
    int lit = 0;  // load cursor (item index within the wave)
    auto load_next = [&](Item& b) {
        const int it = lit < nitems ? lit : (nitems > 0 ? nitems - 1 : 0);  // past the end: repeat
        ++lit;
        int di, qq;  // descriptor, pair within it
        if (SWIGLU) {
            if (it >= 2 * nh) {  // the leftover item
                di = wave & 1;
                qq = px;
            } else {
                di = it >= nh ? 1 : 0;
                qq = live ? q0 + (it - di * nh) * qs : 0;
            }
        } else {
            const int q = live ? q0 + it * qs : 0;
            di = (q >= pb1) + (q >= pb2) + (q >= pb3);
            qq = q - sel(di, 0, pb1, pb2, pb3);
        }
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(sel(di, a.w0, a.w1, a.w2, a.w3) + (size_t)qq * 2 * kRowBytes), (short)0, (int)(2 * kRowBytes) * live, 0x00020000);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(sel(di, a.s0, a.s1, a.s2, a.s3) + (size_t)qq * 2 * NG), (short)0, (int)(2 * NG * 2) * live, 0x00020000);
#pragma unroll
        for (int i = 0; i < P; ++i) {
            b.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(i * 1024 + lane * 16), 0, 2);
            b.s[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)soff[i], 0, 0);
        }
    };

    // --- per pair: the two rows' sums
    float acc[2] = {0.0f, 0.0f};
    auto compute_item = [&](const Item& b) {
#pragma unroll
        for (int i = 0; i < P; ++i) {
            f16x2 h[16];
            decode16_biased(b.w[i].x, b.w[i].y, &h[0]);
            decode16_biased(b.w[i].z, b.w[i].w, &h[8]);
            float ta = cb[i], tb = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; k += 2) {
                ta = dot2(h[k], xp[i][k], ta);
                tb = dot2(h[k + 1], xp[i][k + 1], tb);
            }
            const float v = __builtin_fmaf(tb, 0.0625f, ta) * h2f((uint16_t)b.s[i]);
            // piece i lies in row 0, row 1, or (P odd, i = P/2) splits at lane 32
            if (64 * i + 63 < CPR) {
                acc[0] += v;
            } else if (64 * i >= CPR) {
                acc[1] += v;
            } else {
                acc[0] += hi ? 0.0f : v;
                acc[1] += hi ? v : 0.0f;
            }
        }
    };

    // the pair's two row sums into this wave's LDS buffer
    __shared__ float res[4][2 * kPairMaxPerWave];
    auto finish_pair = [&](int q) {
        const float r = wave_sum_multi<2>(acc, lane);  // lane 0: row 0, lane 1: row 1
        acc[0] = acc[1] = 0.0f;
        if (lane < 2) res[wave][2 * (q - q0) + lane] = r;
    };

    Item buf[PF + 1];
#pragma unroll
    for (int j = 0; j < PF; ++j) load_next(buf[j]);
    __builtin_amdgcn_sched_barrier(0);

    // RMSNorm prologue (fused norm + projection entry points): the row's sum
    // of squares from the staging registers (one chunk per thread, chunk
    // order within a wave, then the waves in order: the same bits on every
    // call), x * inv * w rounded to fp16 as the standalone norm does
    // (src/ops/rmsnorm.cpp:45-78), then staged like a plain X.
    if (norm) {
        __shared__ float rms_red[4];
        // sum of squares: dot2 of each fp16 pair with itself (exact
        // products, FP32 sums), two chains
        float s0 = 0.0f, s1 = 0.0f;
        if (tid < CPR) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                s0 = dot2(as_h2(xr[v].x), as_h2(xr[v].x), s0);
                s1 = dot2(as_h2(xr[v].y), as_h2(xr[v].y), s1);
                s0 = dot2(as_h2(xr[v].z), as_h2(xr[v].z), s0);
                s1 = dot2(as_h2(xr[v].w), as_h2(xr[v].w), s1);
            }
        }
        float ss[1] = {s0 + s1};
        const float t = wave_sum_multi<1>(ss, lane);
        if (lane == 0) rms_red[wave] = t;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const float inv = 1.0f / sqrtf((((rms_red[0] + rms_red[1]) + rms_red[2]) + rms_red[3]) / (float)K + p.norm_eps);
        if (tid < CPR) {
#pragma unroll
            for (int v = 0; v < 4; ++v) xr[v] = rms_apply8(xr[v], nwr[2 * v], nwr[2 * v + 1], inv);
        }
    }
    if (tid < CPR) {
        float c0 = 0.0f, c1 = 0.0f;  // the bias term as dot2 of (x_even, x_odd) with (-1032, -72)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t xa[4] = {xr[v].x, xr[v].y, xr[v].z, xr[v].w};
            f16x2 pr[4];
            permute_x8(xa, pr);
            *reinterpret_cast<u32x4*>(xst + tid * 64 + v * 16) =
                u32x4{as_u32(pr[0]), as_u32(pr[1]), as_u32(pr[2]), as_u32(pr[3])};
            c0 = dot2(as_h2(xa[0]), kBiasPair, c0);
            c1 = dot2(as_h2(xa[1]), kBiasPair, c1);
            c0 = dot2(as_h2(xa[2]), kBiasPair, c0);
            c1 = dot2(as_h2(xa[3]), kBiasPair, c1);
        }
        xcb[tid] = c0 + c1;
    }
    // LDS writes done, then the barrier; no vmcnt wait (a __syncthreads
    // release fence would also wait for the weight prefetch in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int c = 64 * i + lane;
        const int cr = c < CPR ? c : c - CPR;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const u32x4 t = *reinterpret_cast<const u32x4*>(xst + cr * 64 + v * 16);
            xp[i][4 * v] = as_h2(t.x);
            xp[i][4 * v + 1] = as_h2(t.y);
            xp[i][4 * v + 2] = as_h2(t.z);
            xp[i][4 * v + 3] = as_h2(t.w);
        }
        cb[i] = xcb[cr];
    }

    // The ring's body has no branch around a load and no global memory
    // access besides the weight loads (exact vmcnt bookkeeping).  It runs
    // whole passes; the loads it issues past the wave's end are never
    // waited on, and the last items (already in registers) follow it.
    int cit = 0;  // compute cursor
    int base = 0;
    for (; base + PF + 1 <= nitems; base += PF + 1) {
#pragma unroll
        for (int j = 0; j <= PF; ++j) {
            load_next(buf[(j + PF) % (PF + 1)]);
            __builtin_amdgcn_sched_barrier(0);  // the next item's loads go out before this compute
            compute_item(buf[j]);
            finish_pair(q0 + cit++);
        }
    }
#pragma unroll
    for (int j = 0; j < PF; ++j) {
        if (base + j < nitems) {
            compute_item(buf[j]);
            finish_pair(q0 + cit++);
        }
    }

    // results of this wave's rows, per descriptor (wave-uniform), one lane
    // per row: contiguous stores
    if (SWIGLU) {  // rows 2 q0 .. 2 q1 - 1: gate results at [0, 2 nh), up at [2 nh, 4 nh)
        for (int i = lane; i < 2 * nh; i += 64) {
            const float g = res[wave][i], u = res[wave][2 * nh + i];
            reinterpret_cast<OutT*>(p.d[0].Y)[2 * (q0 + (i >> 1) * qs) + (i & 1)] = (OutT)(g / (1.0f + expf(-g)) * u);
        }
        // the leftover pairs: the up wave's two sums through LDS (the
        // condition is uniform over the block: every wave reaches the barrier)
        if (a.xsplit && 2 * (int)blockIdx.x < a.wr) {
            __syncthreads();
            if ((wave & 1) == 0 && has_x && lane < 2) {
                const float g = res[wave][4 * nh + lane], u = res[wave + 1][4 * nh + lane];
                reinterpret_cast<OutT*>(p.d[0].Y)[2 * px + lane] = (OutT)(g / (1.0f + expf(-g)) * u);
            }
        }
        return;
    }
    if (strided) {  // one lane per result
        for (int i = lane; i < 2 * nh; i += 64) {
            const int q = q0 + (i >> 1) * qs;
            const int di = (q >= pb1) + (q >= pb2) + (q >= pb3);
            const PairDesc& d = p.d[di];
            const int n = 2 * (q - sel(di, 0, pb1, pb2, pb3)) + (i & 1);
            float v = res[wave][i];
            if (d.bias) v += d.bias[n];
            OutT* y = reinterpret_cast<OutT*>(d.Y) + n;
            if (d.residual)
                *y = (OutT)((float)*y + (float)(OutT)v);
            else
                *y = (OutT)v;
        }
        return;
    }
    for (int di = 0; di < p.ndesc; ++di) {
        const PairDesc& d = p.d[di];
        const int qb = q0 > d.pair_begin ? q0 : d.pair_begin;
        const int qe = q1 < d.pair_begin + d.N / 2 ? q1 : d.pair_begin + d.N / 2;
        for (int i = 2 * (qb - q0) + lane; i < 2 * (qe - q0); i += 64) {
            const int n = 2 * (q0 - d.pair_begin) + i;
            float v = res[wave][i];
            if (d.bias) v += d.bias[n];
            OutT* y = reinterpret_cast<OutT*>(d.Y) + n;
            if (d.residual)  // add_inplace after the projection (elementwise.cpp:227)
                *y = (OutT)((float)*y + (float)(OutT)v);
            else
                *y = (OutT)v;
        }
    }
}


// M = 2..4 activation rows, and M = 1 with K past the M = 1 kernel's 6144,
// on the row-pair pattern (dot2 per row, no MFMA): the pieces of a pair are
// split over WPP waves so that a lane's
// activations (16 fp16 pairs per piece and row) stay in registers; the
// waves of a pair meet in LDS after the loop.  Same decode, bias terms and
// per-piece arithmetic as the M = 1 kernel; items, strides and the ring
// as there, per pair group (WPP waves).  A wave's part H of the pieces is a
// compile-time constant (one copy of the loop per part, chosen by a
// wave-uniform branch), so the pieces' rows and the split piece's lane
// select are known to the compiler as in the M = 1 kernel.
// waves per pair: as few as keep a wave's activations (16 VGPRs per piece
// and row) within about 160 VGPRs (MR = 1, long K: at most 6 pieces a wave)
constexpr int pairm_wpp(int P, int MR) {
    return MR == 1 ? (P <= 6 ? 1 : (P + 1) / 2 <= 6 ? 2 : 4)
                   : (MR * P <= 10) ? 1 : (MR * ((P + 1) / 2) <= 12) ? 2 : 4;
}
template <int P, int MR>
struct PairmShape {
    static constexpr int WPP = pairm_wpp(P, MR);
    static constexpr int GPB = 4 / WPP;  // pair groups per block
    // part H of a pair's pieces: [H P / WPP, (H + 1) P / WPP) (sizes differ by at most one)
    static constexpr int start(int H) { return H * P / WPP; }
};
constexpr int kPairmMaxItems = 64;  // items per pair group (LDS results)
constexpr int kPairmPF = 1;         // items in flight while one is computed

template <int P, int MR, typename OutT, bool SWIGLU, bool NORM = false>
__global__ __launch_bounds__(256) void gemv_pairm_int4_kernel(const PairParams p) {
    constexpr int K = 1024 * P;
    constexpr int CPR = K / 32;
    constexpr int NG = K / 128;
    constexpr uint32_t kRowBytes = K / 2;
    constexpr int WPP = PairmShape<P, MR>::WPP;
    constexpr int GPB = PairmShape<P, MR>::GPB;
    constexpr int NV = 2 * MR <= 2 ? 2 : 2 * MR <= 4 ? 4 : 8;  // sums per item, padded to a power of two

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool hi = lane >= 32;
    const int pg = wave / WPP;               // pair group of the block
    // part of the pair's pieces; rotated by the block index, so that with
    // two blocks on a CU the larger parts land on different SIMDs
    const int hw = (wave + (int)blockIdx.x) % WPP;
    const int rslot = pg * WPP + hw;         // this wave's LDS results (by part)
    const PairArgs a = pair_args(p);

    const int ngroups = a.G;  // gridDim.x * GPB
    const int gw = (int)blockIdx.x * GPB + pg;
    const bool strided = a.strided;
    const int qs = strided ? ngroups : 1;
    int q0, nh;
    pair_range(a, (uint32_t)gw, q0, nh);
    const int nitems = SWIGLU ? 2 * nh : nh;

    // X staged once per block: chunk c of row m (32 k) as 64 bytes in the
    // decode's pair order plus its bias term
    __shared__ __align__(16) unsigned char xst[MR][CPR * 64];
    __shared__ float xcb[MR][CPR];
    // per item: 2 rows x MR sums of each wave (index (2 it + row) MR + m)
    __shared__ float res[4][kPairmMaxItems * 2 * MR];
    __shared__ float rms_red[NORM ? 4 : 1][MR];  // RMSNorm: the waves' row sums

    const int pb1 = a.pb1, pb2 = a.pb2, pb3 = a.pb3;
    // selects by value (an indexed local array would live in scratch)
    auto sel = [](int di, auto a0, auto a1, auto a2, auto a3) { return di == 0 ? a0 : di == 1 ? a1 : di == 2 ? a2 : a3; };

    auto body = [&](auto part) {
        constexpr int H = decltype(part)::value;
        constexpr int PS = PairmShape<P, MR>::start(H);              // first piece of this part
        constexpr int NPC = PairmShape<P, MR>::start(H + 1) - PS;  // pieces of this part
        static_assert(NPC >= 1, "every part has a piece");

        constexpr int kXR = (MR * CPR + 255) / 256;  // staged chunks per thread
        u32x4 xr[kXR][4];
#pragma unroll
        for (int r = 0; r < kXR; ++r) {
            const int c = tid + 256 * r;
            if (c < MR * CPR) {
                const u32x4* src = reinterpret_cast<const u32x4*>(a.X + (size_t)(c / CPR) * K + (c % CPR) * 32);
#pragma unroll
                for (int v = 0; v < 4; ++v) xr[r][v] = src[v];
            }
        }
        f16x2 xp[NPC][MR][16];
        float cb[NPC][MR];
        uint32_t soff[NPC];
#pragma unroll
        for (int i = 0; i < NPC; ++i) {
            const int c = 64 * (PS + i) + lane;
            const int row = c < CPR ? 0 : 1;
            const int cr = c - row * CPR;
            soff[i] = (uint32_t)(row * NG + (cr >> 2)) * 2u;
        }

        struct Item {
            u32x4 w[NPC];
            uint32_t s[NPC];
        };
        const int live = nitems > 0 ? 1 : 0;
        int lit = 0;
        auto load_next = [&](Item& b) {
            const int it = lit < nitems ? lit : (nitems > 0 ? nitems - 1 : 0);
            ++lit;
            int di, qq;
            if (SWIGLU) {
                di = it >= nh ? 1 : 0;
                qq = live ? q0 + (it - di * nh) * qs : 0;
            } else {
                const int q = live ? q0 + it * qs : 0;
                di = (q >= pb1) + (q >= pb2) + (q >= pb3);
                qq = q - sel(di, 0, pb1, pb2, pb3);
            }
            const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(sel(di, a.w0, a.w1, a.w2, a.w3) + (size_t)qq * 2 * kRowBytes), (short)0,
                (int)(2 * kRowBytes) * live, 0x00020000);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(sel(di, a.s0, a.s1, a.s2, a.s3) + (size_t)qq * 2 * NG), (short)0,
                (int)(2 * NG * 2) * live, 0x00020000);
#pragma unroll
            for (int i = 0; i < NPC; ++i) {
                b.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, (PS + i) * 1024 + lane * 16, 0, 2);
                b.s[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)soff[i], 0, 0);
            }
        };

        // sums of the pair's row 0 / row 1 per activation row; a piece that
        // straddles the rows (P odd, the middle one) splits at lane 32
        float acc[2][MR];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[rr][m] = 0.0f;
        auto compute_item = [&](const Item& b) {
#pragma unroll
            for (int i = 0; i < NPC; ++i) {
                f16x2 hv[16];
                decode16_biased(b.w[i].x, b.w[i].y, &hv[0]);
                decode16_biased(b.w[i].z, b.w[i].w, &hv[8]);
                const float sc = h2f((uint16_t)b.s[i]);
                const int pc = PS + i;  // constant after unrolling
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float ta = dot2_from(hv[0], xp[i][m][0], cb[i][m]);
                    float tb = dot2_from0(hv[1], xp[i][m][1]);
#pragma unroll
                    for (int k = 2; k < 16; k += 2) {
                        ta = dot2(hv[k], xp[i][m][k], ta);
                        tb = dot2(hv[k + 1], xp[i][m][k + 1], tb);
                    }
                    const float v = __builtin_fmaf(tb, 0.0625f, ta) * sc;
                    if (64 * pc + 63 < CPR) {
                        acc[0][m] += v;
                    } else if (64 * pc >= CPR) {
                        acc[1][m] += v;
                    } else {
                        acc[0][m] += hi ? 0.0f : v;
                        acc[1][m] += hi ? v : 0.0f;
                    }
                }
            }
        };

        auto finish_item = [&](int it) {
            float v[NV];
#pragma unroll
            for (int j = 0; j < NV; ++j) v[j] = j < 2 * MR ? acc[j / MR][j % MR] : 0.0f;
            const float r = wave_sum_multi<NV>(v, lane);  // lane j: sum j (pair row j / MR, batch row j % MR)
#pragma unroll
            for (int rr = 0; rr < 2; ++rr)
#pragma unroll
                for (int m = 0; m < MR; ++m) acc[rr][m] = 0.0f;
            if (lane < 2 * MR) res[rslot][it * 2 * MR + lane] = r;
        };

        constexpr int PF = kPairmPF;
        Item buf[PF + 1];
#pragma unroll
        for (int j = 0; j < PF; ++j) load_next(buf[j]);
        __builtin_amdgcn_sched_barrier(0);

        // RMSNorm prologue (NORM, fused norm + projection entry points): the
        // rows' sums of squares from the staging registers (a thread's
        // chunks, the lanes, the four waves in order: the same bits on every
        // call), then x * inv * w rounded to fp16 per element as the
        // standalone norm does (src/ops/rmsnorm.cpp:45-78).  The norm
        // weights are read while staging, after the weight prefetch.
        float inv_m[MR];
        if constexpr (NORM) {
            float ssr[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) ssr[m] = 0.0f;
#pragma unroll
            for (int r = 0; r < kXR; ++r) {
                const int c = tid + 256 * r;
                if (c < MR * CPR) {
                    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        s0 = dot2(as_h2(xr[r][v].x), as_h2(xr[r][v].x), s0);
                        s1 = dot2(as_h2(xr[r][v].y), as_h2(xr[r][v].y), s1);
                        s0 = dot2(as_h2(xr[r][v].z), as_h2(xr[r][v].z), s0);
                        s1 = dot2(as_h2(xr[r][v].w), as_h2(xr[r][v].w), s1);
                    }
                    const int row = c / CPR;
#pragma unroll
                    for (int m = 0; m < MR; ++m) ssr[m] += row == m ? s0 + s1 : 0.0f;
                }
            }
            constexpr int NVN = MR <= 2 ? 2 : 4;
            float sv[NVN];
#pragma unroll
            for (int j = 0; j < NVN; ++j) sv[j] = j < MR ? ssr[j] : 0.0f;
            const float t = wave_sum_multi<NVN>(sv, lane);  // lane j: row j
            if (lane < MR) rms_red[tid >> 6][lane] = t;
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
            for (int m = 0; m < MR; ++m)
                inv_m[m] = 1.0f / sqrtf((((rms_red[0][m] + rms_red[1][m]) + rms_red[2][m]) + rms_red[3][m]) / (float)K +
                                        p.norm_eps);
        }

#pragma unroll
        for (int r = 0; r < kXR; ++r) {
            const int c = tid + 256 * r;
            if (c < MR * CPR) {
                if constexpr (NORM) {
                    const int row = c / CPR;
                    float inv = inv_m[0];
#pragma unroll
                    for (int m = 1; m < MR; ++m) inv = row == m ? inv_m[m] : inv;
                    const float4* wsrc = reinterpret_cast<const float4*>(a.norm_w + (c % CPR) * 32);
                    float4 nw[8];
#pragma unroll
                    for (int v = 0; v < 8; ++v) nw[v] = wsrc[v];
#pragma unroll
                    for (int v = 0; v < 4; ++v) xr[r][v] = rms_apply8(xr[r][v], nw[2 * v], nw[2 * v + 1], inv);
                }
                float c0 = 0.0f, c1 = 0.0f;
                unsigned char* dst = &xst[c / CPR][(c % CPR) * 64];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t xa[4] = {xr[r][v].x, xr[r][v].y, xr[r][v].z, xr[r][v].w};
                    f16x2 pr[4];
                    permute_x8(xa, pr);
                    *reinterpret_cast<u32x4*>(dst + v * 16) =
                        u32x4{as_u32(pr[0]), as_u32(pr[1]), as_u32(pr[2]), as_u32(pr[3])};
                    c0 = dot2(as_h2(xa[0]), kBiasPair, c0);
                    c1 = dot2(as_h2(xa[1]), kBiasPair, c1);
                    c0 = dot2(as_h2(xa[2]), kBiasPair, c0);
                    c1 = dot2(as_h2(xa[3]), kBiasPair, c1);
                }
                xcb[c / CPR][c % CPR] = c0 + c1;
            }
        }
        // LDS writes done, then the barrier (no vmcnt wait: the weight
        // prefetch stays in flight)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int i = 0; i < NPC; ++i) {
            const int c = 64 * (PS + i) + lane;
            const int cr = c < CPR ? c : c - CPR;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const u32x4 t = *reinterpret_cast<const u32x4*>(&xst[m][cr * 64 + v * 16]);
                    xp[i][m][4 * v] = as_h2(t.x);
                    xp[i][m][4 * v + 1] = as_h2(t.y);
                    xp[i][m][4 * v + 2] = as_h2(t.z);
                    xp[i][m][4 * v + 3] = as_h2(t.w);
                }
                cb[i][m] = xcb[m][cr];
            }
        }

        // the ring as in the M = 1 kernel: whole passes, then the items
        // already in registers
        int cit = 0;
        int base = 0;
        for (; base + PF + 1 <= nitems; base += PF + 1) {
#pragma unroll
            for (int j = 0; j <= PF; ++j) {
                load_next(buf[(j + PF) % (PF + 1)]);
                __builtin_amdgcn_sched_barrier(0);
                compute_item(buf[j]);
                finish_item(cit++);
            }
        }
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            if (base + j < nitems) {
                compute_item(buf[j]);
                finish_item(cit++);
            }
        }
    };
    if (hw == 0) {
        body(std::integral_constant<int, 0>{});
    } else if constexpr (WPP >= 2) {
        if (hw == 1) {
            body(std::integral_constant<int, 1>{});
        } else if constexpr (WPP >= 4) {
            if (hw == 2)
                body(std::integral_constant<int, 2>{});
            else
                body(std::integral_constant<int, 3>{});
        }
    }

    // the waves of a pair group add their parts (in wave order) and store
    __syncthreads();
    if (hw != 0) return;
    for (int i = lane; i < 2 * MR * nh; i += 64) {
        const int q = q0 + (i / (2 * MR)) * qs;           // pair (of the gate matrix for SwiGLU)
        const int rr = (i / MR) & 1, m = i % MR;
        const int it = i / (2 * MR);
        float v = 0.0f, u = 0.0f;
#pragma unroll
        for (int w = 0; w < WPP; ++w) {
            v += res[rslot + w][(it * 2 + rr) * MR + m];
            if (SWIGLU) u += res[rslot + w][((nh + it) * 2 + rr) * MR + m];
        }
        if (SWIGLU) {
            const int n = 2 * q + rr;
            reinterpret_cast<OutT*>(p.d[0].Y)[(size_t)m * p.d[0].N + n] = (OutT)(v / (1.0f + expf(-v)) * u);
        } else {
            const int di = (q >= pb1) + (q >= pb2) + (q >= pb3);
            const PairDesc& d = p.d[di];
            const int n = 2 * (q - sel(di, 0, pb1, pb2, pb3)) + rr;
            if (d.bias) v += d.bias[n];
            OutT* y = reinterpret_cast<OutT*>(d.Y) + (size_t)m * d.N + n;
            if (d.residual)
                *y = (OutT)((float)*y + (float)(OutT)v);
            else
                *y = (OutT)v;
        }
    }
}

}  // namespace xhip

using namespace xhip;

namespace xhip_host {

namespace {

typedef void (*PairKernel)(PairParams);

// The split of p.npairs over G owners (see PairParams); false when G is too
// large for the kernel's 32-bit products (G^2 >= 2^31).
bool pair_split(PairParams& p, int64_t G) {
    if (G < 1 || G * G >= (1LL << 31)) return false;
    p.wq = (int32_t)(p.npairs / G);
    p.wr = (int32_t)(p.npairs % G);
    int sh = 0;
    while ((1LL << sh) < G) ++sh;
    p.ws = sh;
    const uint64_t num = 1ULL << (32 + sh);
    p.wm = (num + (uint64_t)G - 1) / (uint64_t)G;
    p.G = (int32_t)G;
    return true;
}

template <typename OutT, bool SWIGLU = false>
PairKernel pair_kernel_for(int P) {
    switch (P) {
        case 4: return gemv_pair_int4_kernel<4, OutT, SWIGLU>;
        case 5: return gemv_pair_int4_kernel<5, OutT, SWIGLU>;
        case 6: return gemv_pair_int4_kernel<6, OutT, SWIGLU>;
        default: return nullptr;
    }
}

}  // namespace

// Whether the pair kernel takes an M = 1 launch of n_total rows: K a
// multiple of 1024 in 4096..6144 (every descriptor's N even, checked by the
// callers).  Measured against the GEMV on MI355X (graph-replayed, rotated
// weights), it is faster at every size: N = 48 / 1024 / 4096 at K = 5120
// 3.34 / 3.57 / 5.01 -> 3.05 / 3.35 / 4.35 us (K = 4096: 3.36 / 3.57 / 4.51
// -> 2.57 / 2.91 / 3.73), config 0 (N = 6144) 5.61 -> 5.15 us, fused QKV
// 8.94 -> 8.66 us, the north star 16.9 -> 15.7 us.
bool pair_takes(int64_t M, int64_t K, int64_t n_total) {
    static const int64_t min_rows = [] {  // XINFER_PAIR_MIN_ROWS: fewest rows (tuning override)
        const char* v = getenv("XINFER_PAIR_MIN_ROWS");
        return (v && *v) ? (int64_t)atoll(v) : (int64_t)2;
    }();
    return M == 1 && K % 1024 == 0 && K >= 4096 && K <= 6144 && n_total >= min_rows;
}

// Returns 1 when the launch is left to the GEMV (odd N, shape not taken),
// else 0 with *rc the launch status.  One 4-wave block per CU (two per CU
// measured 8-10 % slower), more when a wave would exceed kPairMaxPerWave
// pairs.
int pair_linear(hipStream_t st, const xinfer_fused_desc* descs, int nd, const void* X, bool y_f32,
                int64_t K, bool residual, const float* norm_w, float eps, int* rc) {
    if (nd < 1 || nd > 4) return 1;
    int64_t rows = 0;
    for (int i = 0; i < nd; ++i) {
        if (descs[i].N % 2) return 1;
        rows += descs[i].N;
    }
    if (!pair_takes(1, K, rows)) return 1;
    PairParams p = {};
    int pairs = 0;
    for (int i = 0; i < nd; ++i) {
        p.d[i] = PairDesc{descs[i].W_int4, reinterpret_cast<const uint16_t*>(descs[i].scales), descs[i].bias,
                          descs[i].Y, (int32_t)descs[i].N, pairs, residual ? 1 : 0};
        pairs += (int)(descs[i].N / 2);
    }
    p.ndesc = nd;
    p.npairs = pairs;
    p.X = reinterpret_cast<const f16*>(X);
    p.norm_w = norm_w;
    p.norm_eps = eps;
    p.strided = pairs >= 4 * 4 * num_cus() ? 1 : 0;  // >= 4 pairs a wave (fused QKV, 7 a wave: 8.62 -> 8.43 us)
    PairKernel k = y_f32 ? pair_kernel_for<float>((int)(K / 1024)) : pair_kernel_for<f16>((int)(K / 1024));
    if (!k) return 1;
    int64_t blocks = num_cus();
    const int64_t need = (p.npairs + 4LL * kPairMaxPerWave - 1) / (4LL * kPairMaxPerWave);
    if (blocks < need) blocks = need;
    if (blocks > 65535 || !pair_split(p, 4 * blocks)) return 1;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(256), 0, st, p);
    *rc = launch_status();
    return 0;
}

// M = 1 gate/up SwiGLU (fp16 Y[N] = silu(gate) * up) on the pair kernel.
// Returns 1 when left to the GEMV (odd N, shape not taken).
int pair_swiglu(hipStream_t st, void* Y, const void* X, const uint8_t* Wg, const void* Sg, const uint8_t* Wu,
                const void* Su, int64_t N, int64_t K, const float* norm_w, float eps, int* rc) {
    if (N % 2 || !pair_takes(1, K, 2 * N)) return 1;
    PairParams p = {};
    p.d[0] = PairDesc{Wg, reinterpret_cast<const uint16_t*>(Sg), nullptr, Y, (int32_t)N, 0, 0};
    p.d[1] = PairDesc{Wu, reinterpret_cast<const uint16_t*>(Su), nullptr, nullptr, (int32_t)N, 0, 0};
    p.ndesc = 2;
    p.npairs = (int32_t)(N / 2);
    p.X = reinterpret_cast<const f16*>(X);
    p.norm_w = norm_w;
    p.norm_eps = eps;
    p.strided = p.npairs >= 4 * 4 * num_cus() ? 1 : 0;
    PairKernel k = pair_kernel_for<f16, true>((int)(K / 1024));
    if (!k) return 1;
    int64_t blocks = num_cus();
    const int64_t need = (p.npairs + 4LL * (kPairMaxPerWave / 2) - 1) / (4LL * (kPairMaxPerWave / 2));
    if (blocks < need) blocks = need;
    if (blocks > 65535 || !pair_split(p, 4 * blocks)) return 1;
    // leftover pairs split by matrix over the blocks' waves: every wave then
    // streams the same number of items (XINFER_PAIR_XSPLIT=0: off)
    static const int xsplit_env = [] {
        const char* v = getenv("XINFER_PAIR_XSPLIT");
        return (v && *v) ? atoi(v) : 1;
    }();
    p.xsplit = (xsplit_env != 0 && p.strided && p.wr > 0 && p.wr <= 2 * blocks) ? 1 : 0;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(256), 0, st, p);
    *rc = launch_status();
    return 0;
}


namespace {
template <typename OutT, bool SW, int MR, bool NORM = false>
PairKernel pairm_for_p(int P) {
    switch (P) {
        case 4: return gemv_pairm_int4_kernel<4, MR, OutT, SW, NORM>;
        case 5: return gemv_pairm_int4_kernel<5, MR, OutT, SW, NORM>;
        case 6: return gemv_pairm_int4_kernel<6, MR, OutT, SW, NORM>;
        default: return nullptr;
    }
}
// M = 1 with K beyond the row-pair kernel's 6144: a pair's pieces over 4
// waves (K = 7168 .. 24576)
template <typename OutT, int P>
PairKernel pairm_long(int p) {
    if constexpr (P > 24) {
        return nullptr;
    } else {
        return p == P ? gemv_pairm_int4_kernel<P, 1, OutT, false> : pairm_long<OutT, P + 1>(p);
    }
}
template <typename OutT, bool SW>
PairKernel pairm_kernel_for(int P, int64_t M) {
    if (M == 1) {
        if constexpr (SW) return nullptr;
        else return pairm_long<OutT, 7>(P);
    }
    return M == 2 ? pairm_for_p<OutT, SW, 2>(P) : M == 3 ? pairm_for_p<OutT, SW, 3>(P)
         : M == 4 ? pairm_for_p<OutT, SW, 4>(P) : nullptr;
}
// the RMSNorm prologue variants: fp16 outputs at M = 2, 3
template <bool SW>
PairKernel pairm_norm_kernel_for(int P, int64_t M) {
    return M == 2 ? pairm_for_p<f16, SW, 2, true>(P) : M == 3 ? pairm_for_p<f16, SW, 3, true>(P) : nullptr;
}
// launch: one block per CU (more when a pair group would exceed its LDS
// results), strided pairs when every group has at least 4
int pairm_launch(hipStream_t st, PairKernel k, PairParams& p, int P, int64_t M, bool swiglu, int bpc, int* rc) {
    if (!k) return 1;
    const int gpb = 4 / xhip::pairm_wpp(P, (int)M);
    const int64_t cap = swiglu ? kPairmMaxItems / 2 : kPairmMaxItems;  // pairs per group
    int64_t blocks = (int64_t)num_cus() * bpc;
    const int64_t need = (p.npairs + gpb * cap - 1) / (gpb * cap);
    if (blocks < need) blocks = need;
    if (blocks > 65535 || !pair_split(p, gpb * blocks)) return 1;
    p.strided = p.npairs >= 4 * gpb * blocks ? 1 : 0;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(256), 0, st, p);
    *rc = launch_status();
    return 0;
}
// Blocks per CU for an M = 2..4 launch on the row-pair kernel, 0 where the
// small-batch MFMA kernel is faster.  Measured on MI355X (graph-replayed,
// rotated weight copies; pair kernel vs MFMA kernel):
//   gate/up SwiGLU K = 5120, N = 17408: M = 2 18.4 vs 20.2 us (1 block per
//     CU), M = 3 21.8 vs 26.4 us (2 per CU), M = 4 29.3 vs 27.0 us;
//   o_proj K = 6144, N = 5120 (residual): M = 2 7.5 vs 6.6, M = 3 8.8 vs
//     9.6, M = 4 9.9 vs 10.1 us;
//   fused QKV K = 5120, N = 14336: M = 2 10.2 vs 10.0, M = 3 12.0 vs 11.3,
//     M = 4 16.6 vs 11.7 us;
//   one projection, K = 5120, N = 48 / 1024 / 4096 / 6144 / 8192: M = 3
//     4.3 / 4.8 / 7.0 / 8.3 / 9.9 vs 7.8 / 8.1 / 8.8 / 8.8 / 9.1 us, M = 4
//     5.1 / 5.7 / 8.3 / 9.9 / 11.5 vs 7.6 / 8.0 / 8.8 / 8.8 / 9.2 us (M = 2:
//     within a few percent of the GEMV either way).
// The dot2 work grows with M (VALU-bound from M = 2) while the MFMA
// kernel's barely does.  M = 1 with K = 7168 .. 24576 (past the row-pair
// kernel's K) runs here with a pair's pieces over 4 waves: config 2's down
// projection (N = 5120, K = 17408) 10.9 us on the GEMV -> 10.4 us at one
// block per CU, 10.1-10.2 us at two (three: 11.1 us).  XINFER_PAIRM=0 keeps every M >= 2 shape on the
// MFMA kernel, XINFER_PAIRM=<n> (n > 0) sends every shape it can take here
// with n blocks per CU (tuning).
int pairm_bpc(int64_t M, int64_t K, int64_t rows, bool swiglu) {
    static const int mode = [] {  // -1: measured routing
        const char* v = getenv("XINFER_PAIRM");
        return (v && *v) ? atoi(v) : -1;
    }();
    if (mode == 0 || K % 1024) return 0;
    // long K at M = 1 (the row-pair kernel takes K <= 6144), two blocks per
    // CU, from 3072 rows (K = 8192 / 17408: N = 1024 3.6 / 5.4 us on the
    // GEMV vs 4.2 / 5.7 here, N = 4096 5.8 / 9.4 vs 5.3 / 9.2)
    if (M == 1) return (!swiglu && K > 6144 && K <= 24576 && rows >= 3072) ? (mode > 0 ? mode : 2) : 0;
    if (K < 4096 || K > 6144) return 0;
    if (mode > 0) return (M >= 2 && M <= 4) ? mode : 0;
    // short launches at M = 3-4: the MFMA kernel's fixed costs (X slice
    // staging, planner minimum of one tile range per CU) dominate there
    if (M == 3 && rows <= 6144) return 1;
    // M = 2, fused QKV-size launches (the GEMV stages X for all of its
    // blocks' row groups; here a block stages it once for 4 waves): norm +
    // QKV (14336 rows) 12.5 -> 11.5 us with the norm in either kernel
    if (M == 2 && !swiglu && rows >= 12288) return 1;
    if (M == 4 && rows <= (K >= 6144 ? 5120 : 4096)) return 1;
    if (swiglu) return rows < 32768 ? 0 : M == 2 ? 1 : M == 3 ? 2 : 0;
    return 0;
}
}  // namespace

bool pairm_takes(int64_t M, int64_t K, int64_t rows, bool swiglu) { return pairm_bpc(M, K, rows, swiglu) > 0; }

// M = 2..4 on the row-pair pattern (dot2 per row); returns 1 when the
// shape is left to the other kernels.
int pairm_linear(hipStream_t st, const xinfer_fused_desc* descs, int nd, const void* X, bool y_f32, int64_t M,
                 int64_t K, bool residual, int* rc, const float* norm_w, float eps) {
    if (norm_w && (y_f32 || M < 2 || M > 3)) return 1;
    if (nd < 1 || nd > 4) return 1;
    int64_t rows = 0;
    for (int i = 0; i < nd; ++i) {
        if (descs[i].N % 2) return 1;
        rows += descs[i].N;
    }
    const int bpc = pairm_bpc(M, K, rows, false);
    if (!bpc) return 1;
    PairParams p = {};
    int pairs = 0;
    for (int i = 0; i < nd; ++i) {
        p.d[i] = PairDesc{descs[i].W_int4, reinterpret_cast<const uint16_t*>(descs[i].scales), descs[i].bias,
                          descs[i].Y, (int32_t)descs[i].N, pairs, residual ? 1 : 0};
        pairs += (int)(descs[i].N / 2);
    }
    p.ndesc = nd;
    p.npairs = pairs;
    p.X = reinterpret_cast<const f16*>(X);
    const int P = (int)(K / 1024);
    p.norm_w = norm_w;
    p.norm_eps = eps;
    PairKernel k = norm_w ? pairm_norm_kernel_for<false>(P, M)
                 : y_f32  ? pairm_kernel_for<float, false>(P, M) : pairm_kernel_for<f16, false>(P, M);
    return pairm_launch(st, k, p, P, M, false, bpc, rc);
}

int pairm_swiglu(hipStream_t st, void* Y, const void* X, const uint8_t* Wg, const void* Sg, const uint8_t* Wu,
                 const void* Su, int64_t M, int64_t N, int64_t K, int* rc, const float* norm_w, float eps) {
    if (norm_w && (M < 2 || M > 3)) return 1;
    const int bpc = pairm_bpc(M, K, 2 * N, true);
    if (N % 2 || !bpc) return 1;
    PairParams p = {};
    p.d[0] = PairDesc{Wg, reinterpret_cast<const uint16_t*>(Sg), nullptr, Y, (int32_t)N, 0, 0};
    p.d[1] = PairDesc{Wu, reinterpret_cast<const uint16_t*>(Su), nullptr, nullptr, (int32_t)N, 0, 0};
    p.ndesc = 2;
    p.npairs = (int32_t)(N / 2);
    p.X = reinterpret_cast<const f16*>(X);
    const int P = (int)(K / 1024);
    p.norm_w = norm_w;
    p.norm_eps = eps;
    return pairm_launch(st, norm_w ? pairm_norm_kernel_for<true>(P, M) : pairm_kernel_for<f16, true>(P, M), p, P, M,
                        true, bpc, rc);
}

}  // namespace xhip_host
