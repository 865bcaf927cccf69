// INT4-G128-SYM prefill GEMM (M > 16, fp16 output) with producer and
// consumer waves, gfx950.
//
// Same contract as the reference's linear_int4 at M > 8
// (src/ops/linear.h:30-39; chunked prefill calls it with M = chunk,
// src/targets/qwen3_8/forward.cpp:284-287): Y = X * dequant(W)^T (+ bias),
// FP32 accumulation, fp16 output.
//
// The cost of this GEMM beyond its MFMAs is the nibble decode (VALU), and on
// a gfx950 SIMD VALU and MFMA instructions do not overlap, whichever waves
// issue them (measured).  So the tile is chosen to use every decoded weight
// as often as possible, and the decode runs in waves of its own, which keeps
// the MFMA waves' instruction streams free of it:
//
//   * block = 256 rows (M) x 136 weight rows (N), 8 waves: waves 0-3 are
//     consumers (MFMA), waves 4-7 producers (copies + decode); wave w and
//     w + 4 share a SIMD.  Each decoded weight feeds 256 rows (twice the
//     reuse of a 128-row tile, half the decode per FLOP).  N = 17408 =
//     128 * 136 and M = 512 give exactly 256 blocks.
//   * K advances in steps of 64.  Per step the producers copy X (32 KB) and
//     the packed weights (4.25 KB) global -> LDS with buffer_load ... lds
//     (X two steps ahead, weights three), decode the next step's weights to
//     fp16 (exact integer times the fp16 group scale) into one of two B
//     buffers, and the consumers run this step's MFMAs from LDS.  One
//     s_barrier per step; the consumers reach it right after issuing their
//     last MFMAs of the step and read the next step's first operands while
//     those MFMAs run.
//   * consumer c owns rows 64c .. 64c+63 and the first 128 columns: 2 x 4
//     tiles of v_mfma_f32_32x32x16_f16 (128 accumulators), plus the last 8
//     columns as a third 32-column tile whose B operand has 8 live columns
//     (it reuses the A operands already in registers: as four 16x16x32
//     tiles it needed A reads of its own, measured 1.7 % slower).
//   * LDS layouts are chosen per 16-byte chunk (a copy places any global
//     16 bytes at any lane slot): each quad of lanes of an X copy reads 64
//     contiguous bytes of one row, into an XOR-swizzled layout; B is stored
//     in the MFMA operand layouts; every operand read is free of LDS bank
//     conflicts.
//   * the output tile is staged in LDS as fp16 and written with 16-byte
//     stores along its rows.
//
// B = fp16(q * s): q (an integer in [-8, 7]) is exact in fp16 and the
// product is rounded once (relative error <= 2^-11), well inside the fp16
// output's own rounding and the BASELINE bound; fp32 outputs take the exact
// kernel in gemm_int4.hip.

#include <stdlib.h>

#include <mutex>

#include "common.h"

namespace xhip {

struct GemmWsParams {
    const f16* X;       // [M][K]
    const uint8_t* W;   // [N][K/2]
    const uint16_t* S;  // [N][K/128]
    const float* bias;  // optional [N]
    f16* Y;             // [M][N]
    int32_t M, N, K;
    int32_t mblocks;
    int32_t xcd_map;    // 1: the blocks of one XCD share an M block
    int32_t residual;   // Y = fp16(Y + fp16(result))
};

namespace ws {
constexpr int kBM = 256;            // block rows
constexpr int kBN = 136;            // block weight rows: 128 + 8
constexpr int kStepK = 64;          // k per step
constexpr int kXStages = 3;
constexpr int kWStages = 4;
constexpr int kXBytes = kBM * kStepK * 2;     // 32 KB: blocks of 8 rows x 64 k (1 KB)
constexpr int kWBytes = kBN * kStepK / 2;     // 4352 B
constexpr int kBMain = 128 * kStepK * 2;      // 16 KB: [32-col tile][substep] blocks of 1 KB
constexpr int kBBytes = kBMain + 4 * 1024;    // + the last 8 columns: [substep] blocks of 1 KB
constexpr int kSChunk = kBN * 16;             // 8 groups of scales per row: 2176 B
constexpr int kOffX = 0;
constexpr int kOffW = kOffX + kXStages * kXBytes;   // 98304
constexpr int kOffB = kOffW + kWStages * kWBytes;   // 115712
constexpr int kOffS = kOffB + 2 * kBBytes;          // 156672
constexpr int kLds = kOffS + 2 * kSChunk;           // 161024
static_assert(kLds <= 160 * 1024, "LDS of one CU");
constexpr int kXPL = kXBytes / 16 / 256;            // X copies per producer lane per step: 8
}  // namespace ws

typedef float f32x16 __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void* ws_lds_ptr_t;
// 16 bytes per lane, buffer (rsrc) + per-lane byte offset + wave-uniform
// byte offset -> LDS wave base + lane * 16 (no VALU address arithmetic).
__device__ __forceinline__ void ws_copy16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          unsigned char* lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (ws_lds_ptr_t)lds_wave_base, 16, (int)voff, (int)soff, 0, 0);
}
#define XHIP_WS_VMCNT(n) \
    __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

__global__ __launch_bounds__(512) void gemm_ws_int4_kernel(const GemmWsParams p) {
    using namespace ws;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool producer = wave >= 4;
    const int pw = wave & 3;  // index among the producers / consumers

    int mb, nr;
    {
        const int b = blockIdx.x;
        if (p.xcd_map) {
            const int per = 8 / p.mblocks;
            const int xcd = b & 7, s = b >> 3;
            mb = xcd % p.mblocks;
            nr = s * per + xcd / p.mblocks;
        } else {
            mb = b % p.mblocks;
            nr = b / p.mblocks;
        }
    }
    const int M = p.M, N = p.N, K = p.K;
    const int m0 = mb * kBM, n0 = nr * kBN;
    const int nsteps = K / kStepK;
    const int ng = K >> 7;
    const uint32_t row_bytes = (uint32_t)(K >> 1);

    if (producer) {
        // ---------------- producers: copies and decode ----------------
        // (byte offsets within the buffers: the host keeps M*K*2 and N*K/2
        // below 2^31)
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.X, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), 0x00020000);
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.W, (short)0, (int)((uint32_t)N * row_bytes), 0x00020000);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.S, (short)0, (int)((uint32_t)N * (uint32_t)ng * 2u), 0x00020000);
        // X copy j: 1 KB block i = 8 pw + j holds rows 8i .. 8i+7 of the
        // step's 64 k (whole 128-byte rows).  Each quad of lanes reads one
        // aligned 64 bytes of one row (the memory pipeline merges a quad's
        // accesses to one line; lanes of a quad in different rows measured
        // 3x slower): lane l = 4 q + p, quad q = 8 h + r8 -> row 8i + r8,
        // 8-k chunk 4 h + (p ^ x), x = ((r8 >> 2) & 1) | ((i & 1) << 1).  The
        // XOR spreads 16 consecutive rows of one chunk over the 16 bank
        // groups of 16 bytes (conflict-free operand reads).
        uint32_t xoff[kXPL];
#pragma unroll
        for (int j = 0; j < kXPL; ++j) {
            const int i = kXPL * pw + j;
            const int q = lane >> 2, pp = lane & 3, r8 = q & 7, h = q >> 3;
            const int row = min(m0 + 8 * i + r8, M - 1);
            const int chunk = 4 * h + (pp ^ (((r8 >> 2) & 1) | ((i & 1) << 1)));
            xoff[j] = ((uint32_t)row * (uint32_t)K + 8u * chunk) * 2u;
        }
        // Weight pieces (16 bytes = 32 k of one row): main piece u < 256 =
        // row u % 128, k-half u / 128, at u*16 of a weight stage (producer pw
        // copies pieces 64 pw .. +63); the last 8 rows' 16 pieces (k-half
        // l/8, row 128 + l%8) at 4096 + l*16, copied by producer 0 lanes 0-15.
        const int un = 64 * pw + lane;
        const int mn = un & 127, mh = un >> 7;
        const uint32_t woff = (uint32_t)min(n0 + mn, N - 1) * row_bytes + 16u * mh;
        const uint32_t woffl = (uint32_t)min(n0 + 128 + (lane & 7), N - 1) * row_bytes + 16u * ((lane >> 3) & 1);
        // Decode, main piece: its 4 dwords (8-k chunks c = 4 mh + j) -> 16
        // fp16 bytes each at B block (mn/32, c/2), slot (mn%32) + 32 (c%2)
        // (the 32x32x16 B layout; for a fixed j, 16 consecutive lanes write
        // consecutive slots).  The last 8 rows: dword d = 16 pw + lane
        // (lanes < 16) = chunk c = d / 8, row 128 + d % 8 -> block c / 2 of
        // the last-8 part, slot (row - 128) + 32 (c % 2) (the 32x32x16 B
        // layout; slots of columns 8-31 are never written: their outputs are
        // dropped).
        int bdst[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * mh + j;
            bdst[j] = ((mn >> 5) * 4 + (c >> 1)) * 1024 + ((mn & 31) + 32 * (c & 1)) * 16;
        }
        const int ld = 16 * pw + (lane & 15);
        const int lhj = ld >> 3, lrow = 128 + (ld & 7);
        const int lsrc = 4096 + ((lhj >> 2) * 8 + (ld & 7)) * 16 + (lhj & 3) * 4;
        const int ldst = kBMain + (lhj >> 1) * 1024 + ((ld & 7) + 32 * (lhj & 1)) * 16;
        // scales: row r = 64 pw + lane < 136 copies S[r][8c .. 8c+7]
        // (producers 0-2; producer 2 only lanes 0-7)
        const uint32_t soff = (uint32_t)min(n0 + min(64 * pw + lane, kBN - 1), N - 1) * (uint32_t)ng * 2u;

        auto copy_x = [&](int s) {
            const int ss = s < nsteps ? s : nsteps - 1;
            unsigned char* st = smem + kOffX + (s % kXStages) * kXBytes;
#pragma unroll
            for (int j = 0; j < kXPL; ++j)
                ws_copy16(rx, xoff[j], (uint32_t)ss * (kStepK * 2), st + (kXPL * pw + j) * 1024);
        };
        auto copy_w = [&](int s) {
            const int ss = s < nsteps ? s : nsteps - 1;
            unsigned char* st = smem + kOffW + (s % kWStages) * kWBytes;
            ws_copy16(rw, woff, (uint32_t)ss * 32u, st + pw * 1024);
            if (pw == 0) {
                if (lane < 16) ws_copy16(rw, woffl, (uint32_t)ss * 32u, st + 4096);
            }
        };
        auto copy_s = [&](int c) {
            const int cc = c * 8 < ng ? c : (ng >> 3) - 1;
            unsigned char* st = smem + kOffS + (c & 1) * kSChunk;
            if (pw < 3) {
                if (64 * pw + lane < kBN) ws_copy16(rs, soff, (uint32_t)cc * 16u, st + pw * 1024);
            }
        };
        // weights of step s (s % 4 == sm4, a constant after unrolling, so the
        // LDS offsets fold into the instructions) -> B buffer s % 2
        auto decode = [&](int s, const int sm4) {
            const unsigned char* wst = smem + kOffW + sm4 * kWBytes;
            unsigned char* bst = smem + kOffB + (sm4 & 1) * kBBytes;
            const int g = s >> 1;
            const unsigned char* sc = smem + kOffS + ((g >> 3) & 1) * kSChunk + (g & 7) * 2;
            const u32x4 w = *reinterpret_cast<const u32x4*>(wst + un * 16);
            const f16 sh = *reinterpret_cast<const f16*>(sc + mn * 16);
            const uint32_t wl = *reinterpret_cast<const uint32_t*>(wst + lsrc);  // lanes >= 16: unused
            const f16 shl = *reinterpret_cast<const f16*>(sc + lrow * 16);
            __builtin_amdgcn_sched_barrier(0);
            uint32_t o[5][4];
            const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) decode8_natural_scaled(wd[j], f16x2{sh, sh}, o[j]);
            decode8_natural_scaled(wl, f16x2{shl, shl}, o[4]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<u32x4*>(bst + bdst[j]) = u32x4{o[j][0], o[j][1], o[j][2], o[j][3]};
            if (lane < 16) *reinterpret_cast<u32x4*>(bst + ldst) = u32x4{o[4][0], o[4][1], o[4][2], o[4][3]};
        };
        // vmcnt: everything but the newest copies of the current step (the
        // copy counts differ by producer: wave-uniform branches)
        auto wait_all_but_step = [&](bool with_scales) {
            if (pw == 0) {
                if (with_scales) XHIP_WS_VMCNT(kXPL + 2 + 1); else XHIP_WS_VMCNT(kXPL + 2);
            } else if (pw == 3) {
                XHIP_WS_VMCNT(kXPL + 1);
            } else {
                if (with_scales) XHIP_WS_VMCNT(kXPL + 1 + 1); else XHIP_WS_VMCNT(kXPL + 1);
            }
        };
        // prologue: scales of chunk 0, weights of steps 0-2, X of steps 0-1
        copy_s(0);
        copy_w(0);
        copy_w(1);
        copy_x(0);
        copy_w(2);
        copy_x(1);
        wait_all_but_step(false);      // scales, W0, W1, X0 landed (W2, X1 may fly)
        __builtin_amdgcn_s_barrier();  // every producer's copies
        decode(0, 0);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();  // B0 ready: step 0 may start
        // steps in fours (nsteps = K / 64 is a multiple of 16), so that the
        // weight stage and B buffer of each step are constants
        auto step = [&](int s, const int sm4) {
            // consumers: X(s), B(s).  Here: copy W(s+3), X(s+2), then decode
            // W(s+1) (copies first: their issue overlaps the consumers' MFMAs
            // instead of following the decode; 99.0 -> 98.0 us at config 4)
            copy_w(s + 3);
            copy_x(s + 2);
            const bool sc = (s & 15) == 1;  // chunk c+1 of the scales at step 16c+1
            if (sc) copy_s((s >> 4) + 1);
            if (s + 1 < nsteps) decode(s + 1, (sm4 + 1) & 3);
            wait_all_but_step(sc);          // X(s+1), W(s+2) landed
            __builtin_amdgcn_s_waitcnt(0xC07F);  // decoded chunks written
            __builtin_amdgcn_s_barrier();
        };
        for (int s = 0; s < nsteps; s += 4) {
            step(s, 0);
            step(s + 1, 1);
            step(s + 2, 2);
            step(s + 3, 3);
        }
        XHIP_WS_VMCNT(0);
        __builtin_amdgcn_s_barrier();  // E1
    } else {
        // ---------------- consumers: MFMAs ----------------
        const int c = pw;
        f32x16 acc[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[mt][j][e] = 0.0f;
        f32x16 lac[2];  // the last 8 columns as a 32-column tile (columns 8-31 dead)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) lac[mt][e] = 0.0f;
        // X operands (see the copy layout): row r, chunk c sits in block
        // r/8 at slot 4 (8 (c/4) + r%8) + ((c%4) ^ x(r)).  32x32x16 A of
        // 32-row tile mt, substep kk: lane l = row 32 mt + l%32, chunk
        // 2 kk + l/32 -> xa[mt][kk]; the last 8 columns use the same A.
        auto xslot = [](int r, int ch) {
            const int x = ((r >> 2) & 1) | (((r >> 3) & 1) << 1);
            return (r >> 3) * 1024 + 16 * (4 * (8 * (ch >> 2) + (r & 7)) + ((ch & 3) ^ x));
        };
        int xa[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) xa[mt][kk] = xslot(32 * (2 * c + mt) + (lane & 31), 2 * kk + (lane >> 5));
        f16x8 a[2][2], b[2][4], bl[2];
        // operands of substep kk of step s into register set `set`
        auto load = [&](int s, int kk, int set) {
            const unsigned char* xs = smem + kOffX + (s % kXStages) * kXBytes;
            const unsigned char* bs = smem + kOffB + (s & 1) * kBBytes;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
                a[set][mt] = *reinterpret_cast<const f16x8*>(xs + xa[mt][kk]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                b[set][j] = *reinterpret_cast<const f16x8*>(bs + (j * 4 + kk) * 1024 + lane * 16);
            bl[set] = *reinterpret_cast<const f16x8*>(bs + kBMain + kk * 1024 + lane * 16);
        };
        auto mfma_main = [&](int set) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[set][mt], b[set][j], acc[mt][j], 0, 0, 0);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
                lac[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[set][mt], bl[set], lac[mt], 0, 0, 0);
        };
        __builtin_amdgcn_s_barrier();  // prologue copies landed
        __builtin_amdgcn_s_barrier();  // B0 ready
        load(0, 0, 0);
        // Per step: substeps 0-3 (operands of kk+1 read while the MFMAs of kk
        // run), 10 MFMAs per substep (8 + the last 8 columns' 2).  The
        // barrier follows the issue of the step's last MFMAs: every operand
        // of the step is then in registers, and the first operands of the
        // next step are read while those MFMAs run.
        for (int s = 0; s < nsteps; ++s) {
            load(s, 1, 1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_main(0);
            __builtin_amdgcn_sched_barrier(0);
            load(s, 2, 0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_main(1);
            __builtin_amdgcn_sched_barrier(0);
            load(s, 3, 1);
            __builtin_amdgcn_sched_barrier(0);
            mfma_main(0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_main(1);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            if (s + 1 < nsteps) {
                load(s + 1, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- epilogue: the block's output tile [256][136] is staged in LDS
        // as fp16.  D layout of the 32x32x16 MFMA: lane l, register e:
        // column l%32, row 8(e/4) + 4(l/32) + e%4.
        __builtin_amdgcn_s_barrier();  // E1: the producers' copies have landed, stages free
        f16* T = reinterpret_cast<f16*>(smem);
        {
            const int li = lane & 31, lj = lane >> 5;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int col = 32 * j + li;
                const float bn = (p.bias && n0 + col < N) ? p.bias[n0 + col] : 0.0f;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int row = 64 * c + 32 * mt + 8 * (e >> 2) + 4 * lj + (e & 3);
                        T[row * kBN + col] = (f16)(acc[mt][j][e] + bn);
                    }
            }
        }
        if ((lane & 31) < 8) {
            const int col = 128 + (lane & 31);
            const float bn = (p.bias && n0 + col < N) ? p.bias[n0 + col] : 0.0f;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    T[(64 * c + 32 * mt + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * kBN + col] = (f16)(lac[mt][e] + bn);
        }
    }
    __syncthreads();
    f16* T = reinterpret_cast<f16*>(smem);
    // global stores: 16 bytes per thread along the rows (N % 8 == 0), else
    // one element at a time; the residual form adds the stored fp16 result
    // to Y in FP32 and rounds once (linear_int4 then add_inplace)
    if ((N & 7) == 0) {
        constexpr int kC = kBN / 8;  // 17 chunks of 8 columns per row
        for (int q = tid; q < kBM * kC; q += 512) {
            const int row = q / kC, ch = q - row * kC;
            const int m = m0 + row, n = n0 + 8 * ch;
            if (m < M && n < N) {
                u32x4 v = *reinterpret_cast<const u32x4*>(T + row * kBN + 8 * ch);
                u32x4* y = reinterpret_cast<u32x4*>(p.Y + (size_t)m * N + n);
                if (p.residual) {
                    const u32x4 r = *y;
                    const uint32_t rv[4] = {r.x, r.y, r.z, r.w};
                    uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const f16x2 a = as_h2(rv[i]), b2 = as_h2(vv[i]);
                        f16x2 o;
                        o.x = (f16)((float)a.x + (float)b2.x);
                        o.y = (f16)((float)a.y + (float)b2.y);
                        vv[i] = as_u32(o);
                    }
                    v = u32x4{vv[0], vv[1], vv[2], vv[3]};
                }
                *y = v;
            }
        }
    } else {
        for (int q = tid; q < kBM * kBN; q += 512) {
            const int row = q / kBN, col = q - row * kBN;
            const int m = m0 + row, n = n0 + col;
            if (m < M && n < N) {
                f16* y = p.Y + (size_t)m * N + n;
                const f16 v = T[q];
                *y = p.residual ? (f16)((float)*y + (float)v) : v;
            }
        }
    }
}

}  // namespace xhip

// ------------------------------------------------------------------ host ----

namespace xhip_host {
int num_cus();
int launch_status();

// Plain fp16-output prefill projection on the producer/consumer kernel.
// Returns 1 when the shape is left to the other GEMM (K not a multiple of
// 1024, M too small, 32-bit offsets exceeded, or a grid that would leave
// a partial last round of blocks).
int gemm_ws_linear(hipStream_t st, void* Y, const void* X, const uint8_t* W, const uint16_t* S,
                   const float* bias, int64_t M, int64_t N, int64_t K, bool residual, int* rc) {
    using namespace xhip;
    static const int mode = [] {  // XINFER_GEMM_WS: 0 never, 1 whenever the shape fits (tuning)
        const char* v = getenv("XINFER_GEMM_WS");
        return (v && *v) ? atoi(v) : -1;
    }();
    if (mode == 0 || K % 1024 != 0 || M <= 16) return 1;
    if (M * K * 2 >= (1LL << 31) || N * K / 2 >= (1LL << 31)) return 1;  // 32-bit buffer offsets
    GemmWsParams p = {};
    p.X = reinterpret_cast<const f16*>(X);
    p.W = W;
    p.S = S;
    p.bias = bias;
    p.Y = reinterpret_cast<f16*>(Y);
    p.M = (int32_t)M;
    p.N = (int32_t)N;
    p.K = (int32_t)K;
    p.residual = residual ? 1 : 0;
    p.mblocks = (int32_t)((M + ws::kBM - 1) / ws::kBM);
    const int64_t nranges = (N + ws::kBN - 1) / ws::kBN;
    const int64_t blocks = p.mblocks * nranges;
    const int cus = num_cus();
    // whole rounds of one block per CU (a partial last round idles CUs for
    // a full block time): at least 90 % of the last round filled, and the
    // rows mostly live (M at least 3/4 of the row blocks)
    if (mode < 0) {
        if (blocks % cus != 0 && (blocks % cus) * 10 < (int64_t)cus * 9) return 1;
        if (M * 4 < (int64_t)p.mblocks * ws::kBM * 3) return 1;
    }
    p.xcd_map = (8 % p.mblocks == 0) && (blocks % 8 == 0) ? 1 : 0;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_ws_int4_kernel),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, ws::kLds);
    });
    if (attr != hipSuccess) {
        *rc = XINFER_ERR_HIP;
        return 0;
    }
    hipLaunchKernelGGL(gemm_ws_int4_kernel, dim3((unsigned)blocks), dim3(512), ws::kLds, st, p);
    *rc = launch_status();
    return 0;
}

}  // namespace xhip_host
