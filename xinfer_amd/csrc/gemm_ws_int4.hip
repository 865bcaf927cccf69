// INT4-G128-SYM prefill GEMM (M > 16, fp16 output) with producer and
// consumer waves, gfx950.
//
// Same contract as the reference's linear_int4 at M > 8
// (src/ops/linear.h:30-39; chunked prefill calls it with M = chunk,
// src/targets/qwen3_8/forward.cpp:284-287): Y = X * dequant(W)^T (+ bias),
// FP32 accumulation, fp16 output.
//
// Block = 256 rows (M) x 136 weight rows (N); N = 17408 = 128 * 136 and
// M = 512 give exactly 256 blocks, one per CU, so each decoded weight feeds
// 256 rows.  The wave roles, pipeline and LDS layouts are described at the
// kernel below.
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
    int32_t y16;        // Y 16-byte aligned and N % 8 == 0: 16-byte stores
};

// Store a block's output tile, staged in LDS as fp16 T[BM][BN], to Y: 16
// bytes per thread along the rows when Y allows it (y16), else one element
// at a time; the residual form adds the stored fp16 result to Y in FP32 and
// rounds once (linear_int4 then add_inplace).
__device__ __forceinline__ void gemm_tile_store(const GemmWsParams& p, const f16* T, int m0, int n0,
                                                int BM, int BN, int tid, int nthr) {
    const int M = p.M, N = p.N;
    if (p.y16) {
        const int nc = BN / 8;
        for (int q = tid; q < BM * nc; q += nthr) {
            const int row = q / nc, ch = q - row * nc;
            const int m = m0 + row, n = n0 + 8 * ch;
            if (m < M && n < N) {
                u32x4 v = *reinterpret_cast<const u32x4*>(T + row * BN + 8 * ch);
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
        for (int q = tid; q < BM * BN; q += nthr) {
            const int row = q / BN, col = q - row * BN;
            const int m = m0 + row, n = n0 + col;
            if (m < M && n < N) {
                f16* y = p.Y + (size_t)m * N + n;
                const f16 v = T[q];
                *y = p.residual ? (f16)((float)*y + (float)v) : v;
            }
        }
    }
}

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

// byte b of w -> (k_2b, k_2b+1) as fp16(q * s)
__device__ __forceinline__ uint32_t il_dq_byte(uint32_t w, int b, f16x2 s2) {
    const f16x2 kMul = {(f16)1.0f, (f16)0.0625f};
    const f16x2 kAdd = {(f16)-1032.0f, (f16)-72.0f};
    const uint32_t sel = 0x0C000C00u | ((uint32_t)b << 16) | (uint32_t)b;
    const uint32_t bb = __builtin_amdgcn_perm(w, w, sel);
    const f16x2 q = as_h2((bb & 0x00F0000Fu) ^ 0x64806408u) * kMul + kAdd;
    return as_u32(q * s2);
}

// ---------------------------------------------------------------------------
// Prefill GEMM, producer/consumer waves, 8 waves = two per SIMD:
//   * consumers (waves 0-3): consumer c owns rows 64c .. 64c+63 x all 136
//     columns; per 64-k step it copies its own 64 rows of the next-but-one
//     step's X into LDS (LDS-DMA, coalesced 64-byte quads; no other wave
//     reads them, so only its own vmcnt orders them) and issues 40 MFMAs:
//     per 16-k substep 8 v_mfma_f32_32x32x16_f16 (2 row tiles x 4 column
//     tiles) and 2 v_mfma_f32_16x16x32_f16 for the last 8 columns (below),
//     with the next substep's 7 operand reads in between.
//   * producers (waves 4-7): copy the packed weights (five steps ahead) and
//     scales, read a step's packed weights one step before decoding them,
//     and decode (q * s as fp16, one rounding) into the MFMA B layouts.
//   * one s_barrier per step publishes the decoded weights; consumers reach
//     it before their last substep's MFMAs (whose operands are already in
//     registers) and read the next step's first operands while they run.
// Every VALU instruction of the decode sits in the producers' instruction
// stream and every MFMA in the consumers': a gfx950 SIMD issues both
// streams' instructions side by side, while one wave alone could not issue
// its decode and LDS stores between its own MFMAs without stalling them
// (measured).
// Last 8 columns: lanes 0-15 / 32-47 of a 32x32x16 A operand hold rows 0-15
// and lanes 16-31 / 48-63 rows 16-31 of the tile; a 16x16x32 B operand that
// is zero outside (k-block parity == column / 8) gives columns 0-7 the rows
// 0-15 and columns 8-15 the rows 16-31 of the same 8 weight columns: 32 rows
// x 8 columns x 16 k in one 16-cycle MFMA (a 32x32x16 one would take 32
// cycles for the same, 24 of its 32 columns dead).
namespace ws {
constexpr int kBM = 256;
constexpr int kBN = 136;
constexpr int kStepK = 64;
constexpr int kXStages = 3;
constexpr int kWStages = 5;
constexpr int kWAhead = 5;                    // W(s + 5) copied during step s
constexpr int kXBytes = kBM * kStepK * 2;     // 32 KB
constexpr int kWBytes = kBN * kStepK / 2;     // 4352 B
constexpr int kBMain = 128 * kStepK * 2;      // 16 KB: [32-col tile][substep] blocks of 1 KB
constexpr int kBLeft = 4 * 256;               // last 8 columns: [substep][chunk][row] x 16 B
constexpr int kBBytes = kBMain + kBLeft;
constexpr int kSChunk = kBN * 16;
constexpr int kOffX = 0;
constexpr int kOffW = kOffX + kXStages * kXBytes;   // 98304
constexpr int kOffB = kOffW + kWStages * kWBytes;   // 120064
constexpr int kOffZ = kOffB + 2 * kBBytes;          // 154880: zeros read by dead leftover lanes
constexpr int kOffD = kOffZ + kBLeft;               // 155904: sink of lanes 16-63's leftover stores
constexpr int kOffS = kOffD + 768;                  // 156672
constexpr int kLds = kOffS + 2 * kSChunk;           // 161024
static_assert(kLds <= 160 * 1024, "LDS of one CU");
static_assert(kBM * kBN * 2 <= kOffW, "output staging inside the X stages");
}  // namespace ws

__global__ __launch_bounds__(512) void gemm_ws_int4_kernel(const GemmWsParams p) {
    using namespace ws;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = wave & 3;  // consumer / producer index

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

    if (wave >= 4) {
        // ------------------------- producers -------------------------
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.W, (short)0, (int)((uint32_t)N * row_bytes), 0x00020000);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.S, (short)0, (int)((uint32_t)N * (uint32_t)ng * 2u), 0x00020000);
        // weight pieces: main piece u = 64 c + lane (row u % 128, k-half
        // u / 128) at u*16 of a stage; the last 8 rows' 16 pieces (row
        // 128 + l%8, k-half l/8) at 4096 + l*16, copied by producer 0 lanes 0-15
        const int un = 64 * c + lane;
        const int mn = un & 127, mh = un >> 7;
        const uint32_t woff = (uint32_t)min(n0 + mn, N - 1) * row_bytes + 16u * mh;
        const uint32_t woffl = (uint32_t)min(n0 + 128 + (lane & 7), N - 1) * row_bytes + 16u * ((lane >> 3) & 1);
        // decoded main piece: dword j (8-k chunk ch = 4 mh + j) -> B block
        // (mn/32, ch/2), slot (mn%32) + 32 (ch%2): the 32x32x16 B layout
        int bdst[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ch = 4 * mh + j;
            bdst[j] = kOffB + ((mn >> 5) * 4 + (ch >> 1)) * 1024 + ((mn & 31) + 32 * (ch & 1)) * 16;
        }
        // last 8 rows: dword ld = 16 c + l (lanes 0-15) = chunk lhj = ld/8 of
        // row 128 + ld%8 -> slot [substep lhj/2][chunk lhj%2][row] of the
        // leftover operand; lanes 16-63 decode a copy into the sink
        const int ld = 16 * c + (lane & 15);
        const int lhj = ld >> 3, lr = ld & 7;
        const int lsrc = 4096 + ((lhj >> 2) * 8 + lr) * 16 + (lhj & 3) * 4;
        const int ldst = lane < 16 ? kOffB + kBMain + (lhj >> 1) * 256 + ((lhj & 1) * 8 + lr) * 16
                                   : kOffD + (lane - 16) * 16;
        const int ldst_buf = lane < 16 ? kBBytes : 0;
        // scales: row r = 64 c + lane < 136 copies S[r][8k .. 8k+7] (producers 0-2)
        const uint32_t soff = (uint32_t)min(n0 + min(64 * c + lane, kBN - 1), N - 1) * (uint32_t)ng * 2u;

        auto copy_w = [&](int s) {
            const int ss = s < nsteps ? s : nsteps - 1;
            unsigned char* st = smem + kOffW + (s % kWStages) * kWBytes;
            ws_copy16(rw, woff, (uint32_t)ss * 32u, st + c * 1024);
            if (c == 0) {
                if (lane < 16) ws_copy16(rw, woffl, (uint32_t)ss * 32u, st + 4096);
            }
        };
        auto copy_s = [&](int k) {
            const int kk = k * 8 < ng ? k : (ng >> 3) - 1;
            unsigned char* st = smem + kOffS + (k & 1) * kSChunk;
            if (c < 3) {
                if (64 * c + lane < kBN) ws_copy16(rs, soff, (uint32_t)kk * 16u, st + c * 1024);
            }
        };
        // vmcnt before step s's barrier: every copy but those of steps s-1
        // and s has landed (W(s+3) is read after the next barrier).  Per step
        // a producer copies its weight piece (producer 0 also the last 8
        // rows'); a scale copy in between only makes the wait stricter.
        auto wait_all_but_two_steps = [&]() {
            if (c == 0) XHIP_WS_VMCNT(4); else XHIP_WS_VMCNT(2);
        };
        // packed weights + scales of step s, two register sets
        uint32_t pw[2][5];
        f16 psh[2], pshl[2];
        auto pread = [&](int s, int set) {
            const unsigned char* wst = smem + kOffW + (s % kWStages) * kWBytes;
            const int g = s >> 1;
            const unsigned char* sc = smem + kOffS + ((g >> 3) & 1) * kSChunk + (g & 7) * 2;
            const u32x4 v = *reinterpret_cast<const u32x4*>(wst + un * 16);
            pw[set][0] = v.x; pw[set][1] = v.y; pw[set][2] = v.z; pw[set][3] = v.w;
            pw[set][4] = *reinterpret_cast<const uint32_t*>(wst + lsrc);
            psh[set] = *reinterpret_cast<const f16*>(sc + mn * 16);
            pshl[set] = *reinterpret_cast<const f16*>(sc + (128 + lr) * 16);
        };
        auto decode = [&](int set, int bf) {
            uint32_t o[5][4];
#pragma unroll
            for (int d = 0; d < 5; ++d) {
                const f16 sh = d < 4 ? psh[set] : pshl[set];
#pragma unroll
                for (int b = 0; b < 4; ++b) o[d][b] = il_dq_byte(pw[set][d], b, f16x2{sh, sh});
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<u32x4*>(smem + bdst[j] + bf * kBBytes) = u32x4{o[j][0], o[j][1], o[j][2], o[j][3]};
            *reinterpret_cast<u32x4*>(smem + ldst + bf * ldst_buf) = u32x4{o[4][0], o[4][1], o[4][2], o[4][3]};
        };
        // prologue: scales of chunk 0, weights of steps 0 .. kWAhead-1
        // (zero area and X: the consumers)
        copy_s(0);
#pragma unroll
        for (int i = 0; i < kWAhead; ++i) copy_w(i);
        XHIP_WS_VMCNT(0);
        __builtin_amdgcn_s_barrier();  // P1: weights, scales, zero area, X of step 0
        pread(0, 0);
        pread(1, 1);
        decode(0, 0);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();  // P2: B(0) ready
        // step s: read W(s+2), copy W(s+5) (+ scales), decode W(s+1) (read
        // during step s-1), wait for this step's stores and for W(s+3)
        auto step = [&](int s, const int sm2) {
            pread(s + 2, sm2);  // set sm2 held W(s) (decoded in step s-1)
            copy_w(s + kWAhead);
            const bool sc = (s & 15) == 1;
            if (sc) copy_s((s >> 4) + 1);
            decode(sm2 ^ 1, sm2 ^ 1);
            wait_all_but_two_steps();
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
        };
        for (int s = 0; s < nsteps; s += 2) {
            step(s, 0);
            step(s + 1, 1);
        }
        XHIP_WS_VMCNT(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();  // E1
        __syncthreads();               // E2: output tile staged
    } else {
        // ------------------------- consumers -------------------------
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.X, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), 0x00020000);
        // X copy j: 1 KB block i = 8 c + j holds rows 8i .. 8i+7 of the
        // step's 64 k; each quad of lanes reads 64 contiguous bytes of one row
        // into an XOR-swizzled slot order (conflict-free operand reads)
        uint32_t xoff[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = 8 * c + j;
            const int q = lane >> 2, pp = lane & 3, r8 = q & 7, h = q >> 3;
            const int row = min(m0 + 8 * i + r8, M - 1);
            const int chunk = 4 * h + (pp ^ (((r8 >> 2) & 1) | ((i & 1) << 1)));
            xoff[j] = ((uint32_t)row * (uint32_t)K + 8u * chunk) * 2u;
        }
        auto copy_x = [&](int s, int j) {
            const int ss = s < nsteps ? s : nsteps - 1;
            unsigned char* st = smem + kOffX + (s % kXStages) * kXBytes;
            ws_copy16(rx, xoff[j], (uint32_t)ss * (kStepK * 2), st + (8 * c + j) * 1024);
        };
        // operand addresses: row r, chunk ch sits in block r/8 at slot
        // 4 (8 (ch/4) + r%8) + ((ch%4) ^ x(r)); 32x32x16 A of row tile mt,
        // substep kk: lane l = row 32 mt + l%32, chunk 2 kk + l/32
        auto xslot = [](int r, int ch) {
            const int x = ((r >> 2) & 1) | (((r >> 3) & 1) << 1);
            return (r >> 3) * 1024 + 16 * (4 * (8 * (ch >> 2) + (r & 7)) + ((ch & 3) ^ x));
        };
        int xa[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) xa[mt][kk] = xslot(32 * (2 * c + mt) + (lane & 31), 2 * kk + (lane >> 5));
        // leftover B operand (16x16x32): lane l = column j = l%16, k-block
        // kb = l/16; live when kb%2 == j/8 (weight column 128 + j%8, chunk
        // kb/2 of the substep); dead lanes read zeros
        int blo[2];
        {
            const int j16 = lane & 15, kb = lane >> 4;
            const bool live = (kb & 1) == (j16 >> 3);
#pragma unroll
            for (int bf = 0; bf < 2; ++bf)
                blo[bf] = live ? kOffB + bf * kBBytes + kBMain + ((kb >> 1) * 8 + (j16 & 7)) * 16 : kOffZ;
        }
        f32x16 acc[2][4];
        f32x4 lac[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[mt][j][e] = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) lac[mt][e] = 0.0f;
        }
        f16x8 a[2][2], b[2][4], bl[2];
        auto opread = [&](int r, int set, uint32_t xs, int bf, int kk) {
            if (r < 2) {
                a[set][r] = *reinterpret_cast<const f16x8*>(smem + xs + xa[r][kk]);
            } else if (r < 6) {
                const int j = r - 2;
                b[set][j] = *reinterpret_cast<const f16x8*>(smem + kOffB + bf * kBBytes + (j * 4 + kk) * 1024 + lane * 16);
            } else {
                bl[set] = *reinterpret_cast<const f16x8*>(smem + blo[bf] + kk * 256);
            }
        };
        auto mfma = [&](int i, int set) {
            if (i < 8) {
                const int mt = i >> 2, j = i & 3;
                acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[set][mt], b[set][j], acc[mt][j], 0, 0, 0);
            } else {
                const int mt = i - 8;
                lac[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[set][mt], bl[set], lac[mt], 0, 0, 0);
            }
        };
        // prologue: zero area, X of steps 0-1
        reinterpret_cast<uint32_t*>(smem + kOffZ)[tid] = 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) copy_x(0, j);
#pragma unroll
        for (int j = 0; j < 8; ++j) copy_x(1, j);
        XHIP_WS_VMCNT(8);              // X(0) landed
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();  // P1
        __builtin_amdgcn_s_barrier();  // P2: B(0) ready
#pragma unroll
        for (int r = 0; r < 7; ++r) opread(r, 0, kOffX, 0, 0);
#define WS_FENCE __builtin_amdgcn_sched_barrier(0)
        // step s: substeps 0-2 (reads of the next substep between the
        // MFMAs; X copies of step s+2 every 5 MFMAs), wait + barrier,
        // substep 3 (reads of step s+1's substep 0)
        auto step = [&](int s, const int sm2) {
            const int bc = sm2, bn = sm2 ^ 1;
            const uint32_t xs = kOffX + (uint32_t)(s % kXStages) * kXBytes;
            const uint32_t xsn = kOffX + (uint32_t)((s + 1) % kXStages) * kXBytes;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int set = kk & 1;
                if (kk == 3) {
                    XHIP_WS_VMCNT(6);                    // own X(s+1) landed
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // operand reads done
                    __builtin_amdgcn_s_barrier();        // B(s+1) ready, B(s-1) free
                }
#pragma unroll
                for (int i = 0; i < 10; ++i) {
                    WS_FENCE;
                    mfma(i, set);
                    WS_FENCE;
                    if (i < 7) {
                        if (kk < 3) opread(i, set ^ 1, xs, bc, kk + 1);
                        else opread(i, set ^ 1, xsn, bn, 0);
                    }
                    const int slot = 10 * kk + i;
                    if (slot % 5 == 1) copy_x(s + 2, slot / 5);
                }
            }
            WS_FENCE;
        };
        for (int s = 0; s < nsteps; s += 2) {
            step(s, 0);
            step(s + 1, 1);
        }
#undef WS_FENCE
        XHIP_WS_VMCNT(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();  // E1: every stage free
        // ---- stage the [256][136] tile in LDS as fp16.  32x32x16 D: lane
        // l, register e: column l%32, row 8(e/4) + 4(l/32) + e%4.  16x16x32
        // D of the last 8 columns: lane l, register e: column j = l%16, row
        // 4(l/16) + e + 16 (j/8) of the 32-row tile, weight column 128 + j%8.
        f16* T = reinterpret_cast<f16*>(smem);
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
        const int j16 = lane & 15;
        const int col = 128 + (j16 & 7);
        const float bn = (p.bias && n0 + col < N) ? p.bias[n0 + col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = 64 * c + 32 * mt + 4 * (lane >> 4) + e + 16 * (j16 >> 3);
                T[row * kBN + col] = (f16)(lac[mt][e] + bn);
            }
        __syncthreads();  // E2
    }
    gemm_tile_store(p, reinterpret_cast<const f16*>(smem), m0, n0, kBM, kBN, tid, 512);
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
    p.y16 = ((N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) ? 1 : 0;
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
