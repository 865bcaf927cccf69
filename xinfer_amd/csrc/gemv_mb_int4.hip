// INT4-G128-SYM small-batch decode projection (2 <= M <= 8) on gfx950.
//
// Same contract as the reference's sub-group GEMV at M > 1 (the batched rows
// of src/ops/linear.cpp:165-305, the fused variants 351-498 and 501-617, and
// the LM-head linear + argmax of src/targets/qwen3_8/forward.cpp:304-307):
// every output is sum_k x[m][k] * q[n][k] * s[n][k/128] with FP32
// accumulation.  At M = 8 a dot-product GEMV spends 4 * M v_dot2 per packed
// dword on top of its decode: more VALU time than the HBM stream it rides
// on.  This kernel decodes each nibble once and lets the matrix cores apply
// it to all M rows:
//
//   * output tile = 16 weight rows (n) x 16 activation rows (m, the first M
//     real).  Per 128-k group a lane loads one 16-byte chunk of packed
//     weights: lane l holds row n = l % 16 and k-quarter l / 16 of the group,
//     which is exactly the B-operand layout of v_mfma_f32_16x16x32_f16.  The
//     nibbles are decoded to exact fp16 integers (dequant8: one v_bitop3_b32
//     and one packed add/fma per pair) and fed to four MFMAs (one per dword)
//     that sum the whole group in FP32; the group's fp16 scale is then applied
//     to the group sum in FP32 (acc += s * sum), as in the reference.
//   * the A operand (activations) comes from LDS: the block stages its k-slice
//     of X once, permuted into the pair order of the decode, so that lane l
//     (row m = l % 16, k-quarter l / 16) reads one ds_read_b128 per MFMA.
//     Rows m >= M read row M - 1: they only feed output rows that are dropped.
//   * a block owns a contiguous range of 16-row tiles and one k-slice; its
//     waves take contiguous runs of tiles, T at a time, and stream every
//     group of the slice with the next PF items in flight (raw buffer loads,
//     branch-free: rows past N and padding items read zeros without memory
//     traffic).  Results go through LDS to a coalesced epilogue.
//   * when K is long and N short (the down projection) the planner splits K
//     over ks blocks per tile range.  Each writes its FP32 partial sums to
//     the calling stream's split-K slot (a static device array, scratch.hip);
//     the last block of a range (device-scope counter) adds the
//     slices in slice order, so results do not depend on timing, and resets
//     the counter for the next call.
// Epilogues: bias + fp16/fp32 store, SiLU(gate) * up (paired tiles), and the
// LM-head argmax (per-block candidates, reduced by argmax_finalize_kernel).

#include <stdlib.h>

#include <algorithm>
#include <cstdint>
#include <mutex>

#include "common.h"

namespace xhip {

enum MbEpilogue { MB_PLAIN = 0, MB_SWIGLU = 1, MB_ARGMAX = 2 };

struct MbDesc {
    const uint8_t* W;    // [N][K/2]   (gate matrix for MB_SWIGLU)
    const uint16_t* S;   // [N][K/128]
    const uint8_t* W2;   // up matrix (MB_SWIGLU only)
    const uint16_t* S2;
    const float* bias;   // optional [N]
    void* Y;             // [M][N] output (MB_ARGMAX: optional fp32 logits)
    int32_t N;
    int32_t block_begin; // first block of this descriptor
    int32_t range_begin; // first tile range of this descriptor (counters, parts)
    int32_t residual;    // MB_PLAIN, fp16 Y: Y = fp16(Y + fp16(result))
    int32_t nr;          // tile ranges of this descriptor (its tiles split evenly over them)
};

struct MbParams {
    MbDesc d[4];
    const f16* X;        // [M][K]
    ArgCand* parts;      // MB_ARGMAX: [M][nranges] block candidates
    float* ws;           // ks > 1: [ks][E][M][N] partial sums, slices ws_slice floats apart
    uint32_t* cnt;       // ks > 1: one arrival counter per tile range (zero between calls)
    int64_t ws_desc[4];  // float offset of each descriptor's partials in ws
    int32_t ws_slice[4]; // floats per k-slice of each descriptor (multiple of 64: 256-byte aligned)
    int32_t ndesc;
    int32_t M;           // 2..8 (argmax), 2..64 otherwise
    int32_t K;
    int32_t ks;          // k-slices per tile range
    int32_t gps;         // groups per k-slice (the last slice may be shorter)
    int32_t tiles_blk;   // 16-row tiles of the largest range
    int32_t nranges;     // tile ranges over all descriptors
    int32_t lkw;         // log2 of the waves that share a run of tiles, splitting its groups
    const float* norm_w; // RMSNorm weight [K] applied to X while staging (M == MR, one k-slice), or null
    float norm_eps;
};

constexpr uint32_t kOutOfRange = 0xFFFFF000u;  // >= every buffer resource size used here

// Two groups per item: a lane's two 16-byte loads of an item fall in the same
// 128-byte line of its row.  Weights are loaded with the default cache policy
// (measured faster here than the streaming hint: the other half of each line
// is read by the same wave a few instructions later).
#ifndef XHIP_MB_PF
#define XHIP_MB_PF 3
#endif
#ifndef XHIP_MB_GP
#define XHIP_MB_GP 2
#endif
#ifndef XHIP_MB_AUX
#define XHIP_MB_AUX 0
#endif
constexpr int kGP = XHIP_MB_GP;  // 128-k groups per item (the plain and SwiGLU forms)
// Cache-policy bit for device-scope coherence (sc1): stores write through and
// loads do not hit stale lines of another XCD's L2.
constexpr int kDeviceCoherent = 16;

static_assert(kGP == 2, "an item's two group scales are one dword");
// The LM head's items: 4 groups (16 rows x 256 bytes, its scales one
// 2-byte load per group), 3 in flight: M = 8, N = 151936 84.8 -> 83.8 us
// (five interleaved runs) against 2 groups and 4 in flight; 4 groups with
// 2 or 4 in flight measured between the two.
#ifndef XHIP_MB_GPA
#define XHIP_MB_GPA 4
#endif
#ifndef XHIP_MB_PFA
#define XHIP_MB_PFA 3
#endif
template <int E, int GP = kGP>
struct MbItem {
    u32x4 w[E * GP];
    uint32_t s[E * GP];  // fp16 group scales: s[x] holds both of matrix x's (the LM head: one per s[gi])
    uint32_t sh[E];       // s[x]'s first scale at bit sh[x] (0, or 16 for the array's last scale)
};

__device__ __forceinline__ f16x8 pack_q8(const f16x2 q[4]) {
    f16x8 r;
    r[0] = q[0].x; r[1] = q[0].y; r[2] = q[1].x; r[3] = q[1].y;
    r[4] = q[2].x; r[5] = q[2].y; r[6] = q[3].x; r[7] = q[3].y;
    return r;
}

template <int MR, int EPI, typename OutT, int NW, int NORM = 0>
__global__ __launch_bounds__(64 * NW) void gemv_mb_int4_kernel(const MbParams p) {
    constexpr int E = (EPI == MB_SWIGLU) ? 2 : 1;  // sums per output (weight tiles per item)
    constexpr int GP = EPI == MB_ARGMAX ? XHIP_MB_GPA : kGP;  // groups per item
    constexpr int NT = 64 * NW;

    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int l16 = lane & 15;
    const int kq = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    int di = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (i < p.ndesc && (int)blockIdx.x >= p.d[i].block_begin) di = i;
    const MbDesc& d = p.d[di];
    const int N = d.N;
    const int K = p.K;
    const int M = p.M;
    const int ks = p.ks;
    const int local = (int)blockIdx.x - d.block_begin;
    const int range = local / ks;
    const int slice = local - range * ks;
    const int grange = d.range_begin + range;
    // tiles split evenly over the descriptor's ranges (counts differ by at most one)
    const int ntiles = (N + 15) >> 4;
    const int tb = range * ntiles / d.nr, te = (range + 1) * ntiles / d.nr;
    const int n0 = tb * 16;
    const int rows_here = min(te * 16, N) - n0;
    const int tiles_here = (rows_here + 15) >> 4;
    const int ng = K >> 7;
    const int g0 = slice * p.gps;
    const int ngs = min(p.gps, ng - g0);
    const uint32_t row_bytes = (uint32_t)K >> 1;

    // LDS: X slice as MFMA A operands [group][k-quarter][dword t][m < MR] (16 B
    // each), then the block's results [wave of the run][row][m][e] (fp32:
    // one slice per wave sharing a run, summed in order), then the argmax
    // candidates of the waves (NW values, NW indices) and one flag word.
    f16x8* xs = reinterpret_cast<f16x8*>(smem);
    // Slot of piece r (r = (group * 4 + k-quarter) * 4 + dword of the slice)
    // of row m: row blocks of MR slots, the row XOR-swizzled by the
    // k-quarter, so that the staging stores of consecutive pieces of one row
    // spread over the 16-byte bank groups (conflict-free at MR = 4, 2-way at
    // 8, 4-way at 16; 4 / 8 / 16-way unswizzled), while the A-operand reads
    // of one piece by the MR rows stay one contiguous block and a lane's
    // four dwords stay immediate offsets from one address.
    auto xslot = [](int r, int m) { return r * MR + (m ^ ((r >> 2) & 3)); };
    float* outl = reinterpret_cast<float*>(smem + (size_t)p.gps * 16 * MR * 16);
    // (argmax: 8 candidates per wave, one per activation row)
    constexpr int kCand = EPI == MB_ARGMAX ? 8 : 1;
    float* candv = outl + ((size_t)p.tiles_blk * 16 * M * E << p.lkw);
    int32_t* candi = reinterpret_cast<int32_t*>(candv + NW * kCand);
    int32_t* flag = candi + NW * kCand;
    // RMSNorm (norm_w set): the weights [K] and the waves' row sums [NW][MR]
    float* nws = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(candv) + 2 * NW * kCand * 4 + 16);
    float* rsum = nws + K;

    // Waves come in runs of kw = 2^lkw: the waves of a run share its tiles
    // and split the slice's groups evenly (every wave gets at least one
    // group: the host keeps kw <= groups per slice).  A wave walks its
    // tiles one at a time, all of its groups per tile.
    const int lkw = p.lkw;
    const int kp = wave & ((1 << lkw) - 1);  // this wave's part of the groups
    const int nr = NW >> lkw;                // runs per block
    const int wr = wave >> lkw;
    const int t0 = (wr * tiles_here) / nr;
    const int t1 = ((wr + 1) * tiles_here) / nr;
    const int gb = (kp * ngs) >> lkw;                   // first group of this wave
    const int ngw = (((kp + 1) * ngs) >> lkw) - gb;     // groups of this wave (>= 1)
    const int nig = (ngw + GP - 1) / GP;  // items per tile
    const int nreal = (t1 - t0) * nig;

    const int nrec_w = (int)((uint32_t)N * row_bytes);
    // Scales: one 4-byte load per item and lane holds both groups' fp16
    // scales (a dword load at any 2-byte offset; two 2-byte loads per item,
    // scattered over the 16 rows, cost a pure read of this weight pattern
    // ~25 % of its rate, the dword ~6 %).  No load reaches past the scale
    // array: the one dword that would (the array's last scale, in an item
    // whose second group is padding) is read 2 bytes lower and its upper
    // half used.
    const int nrec_s = (int)((uint32_t)N * (uint32_t)ng * 2u);
    const uint32_t slast = (uint32_t)nrec_s - 4u;  // the host keeps N K / 128 >= 2
    const __amdgpu_buffer_rsrc_t rw0 = __builtin_amdgcn_make_buffer_rsrc((void*)d.W, (short)0, nrec_w, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc((void*)d.S, (short)0, nrec_s, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw1 = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(EPI == MB_SWIGLU ? d.W2 : d.W), (short)0, nrec_w, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(EPI == MB_SWIGLU ? d.S2 : d.S), (short)0, nrec_s, 0x00020000);

    // Every load is in bounds, so the addressing needs no per-lane checks:
    // a lane's row offset is set once per tile (rows past N read row N - 1
    // and are never stored), the group offset is wave-uniform (the buffer
    // instruction's scalar offset), and a padding group past the wave's
    // last reloads that last group and gets a zero scale in the compute.
    uint32_t vwt = 0, vst = 0;  // lane offsets (bytes) of the load tile's row at the wave's first group
    auto set_tile = [&](int tile) {
        const uint32_t n = (uint32_t)min(n0 + tile * 16 + l16, N - 1);
        vwt = n * row_bytes + (uint32_t)(g0 + gb) * 64u + (uint32_t)kq * 16u;
        vst = (n * (uint32_t)ng + (uint32_t)(g0 + gb)) * 2u;
    };
    set_tile(t0);
    int lt = t0, lg = 0, lrem = nreal;  // load cursor (wave-uniform): tile, item, items left
    // the item's two group scales; sh = 16 where the dword was read 2 bytes
    // lower (its upper half is the first group's scale)
    auto load_scales = [&](const __amdgpu_buffer_rsrc_t& rs, uint32_t vs, uint32_t& sh) -> uint32_t {
        const uint32_t o = vs + (uint32_t)(lg * (2 * GP));
        const uint32_t oc = o < slast ? o : slast;
        sh = (o - oc) << 3;
        return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)oc, 0, 0);
    };
    auto load_next = [&](MbItem<E, GP>& b) {
        // argmax: past the wave's last item, out-of-range offsets (zeros
        // without memory traffic, nothing for the epilogue's waits to wait
        // on; the other epilogues measured faster repeating the last item)
        const bool oor = EPI == MB_ARGMAX && lrem <= 0;
        const uint32_t vw = oor ? kOutOfRange : vwt;
        const uint32_t vs = oor ? kOutOfRange : vst;
        if constexpr (E == 2) {
            // SwiGLU: a matrix's two groups (the two halves of each row's
            // 128-byte line) back to back, then the other matrix's (gate/up
            // M = 4 / 8 28.1 / 30.3 -> 26.75 / 29.2 us against alternating
            // matrices); the plain form keeps each group's scale next to it
#pragma unroll
            for (int e = 0; e < E; ++e) {
#pragma unroll
                for (int gi = 0; gi < GP; ++gi) {
                    const int g = __builtin_amdgcn_readfirstlane(min(lg * GP + gi, ngw - 1));  // wave-uniform: a scalar offset
                    b.w[e * GP + gi] =
                        __builtin_amdgcn_raw_buffer_load_b128(e ? rw1 : rw0, (int)vw, g * 64, XHIP_MB_AUX);
                }
                b.s[e] = load_scales(e ? rs1 : rs0, vs, b.sh[e]);
            }
        } else {
#pragma unroll
            for (int gi = 0; gi < GP; ++gi) {
                // wave-uniform (a scalar offset; without the explicit form
                // the compiler waterfalled some plain instantiations)
                const int g = EPI == MB_ARGMAX ? min(lg * GP + gi, ngw - 1)
                                               : __builtin_amdgcn_readfirstlane(min(lg * GP + gi, ngw - 1));
                b.w[gi] = __builtin_amdgcn_raw_buffer_load_b128(rw0, (int)vw, g * 64, XHIP_MB_AUX);
                if constexpr (EPI == MB_ARGMAX)  // the LM head measured faster with a 2-byte load per group
                    b.s[gi] = __builtin_amdgcn_raw_buffer_load_b16(rs0, (int)vs, g * 2, 0);
            }
            if constexpr (EPI != MB_ARGMAX) b.s[0] = load_scales(rs0, vs, b.sh[0]);
        }
        // past the last item the cursor stays: the extra loads repeat it
        if (--lrem > 0 && ++lg == nig) {
            lg = 0;
            set_tile(++lt);
        }
    };

    // Stage X[:, slice] (permuted to the decode's pair order).  The loads of
    // the first round (up to kStageUnroll chunks per thread) are issued
    // before the weight prefetch: loads complete in issue order, so the
    // staging then waits for X alone while the weight items stay in flight.
    // A later round would wait behind the prefetch: 4-wave blocks (one per
    // SIMD, registers to spare) take 8 chunks per thread, so an X slice of up
    // to 128 KB is one round (K = 17408, M = 8: 92 KB, 5.75 chunks a thread).
    constexpr int kStageUnroll = NW == 4 ? 8 : 4;
    const int chunks = ngs * 4 * M;  // 64-byte chunks: (group, k-quarter, m)
    // chunk i -> (m, q): a shift and a mask when M is the power-of-two row
    // stride MR (the decode shapes M = 4, 8, 16), else a division by M
    static_assert((MR & (MR - 1)) == 0, "MR is a power of two");
    constexpr int kLogMR = MR == 4 ? 2 : MR == 8 ? 3 : 4;
    const bool m_full = M == MR;
    auto chunk_m = [&](int i) { return m_full ? (i & (MR - 1)) : i % M; };
    auto chunk_q = [&](int i) { return m_full ? (i >> kLogMR) : i / M; };
    auto get = [&](int i, u32x4 (&xv)[4]) {
        const int m = chunk_m(i);
        const int q = chunk_q(i);
        const u32x4* src = reinterpret_cast<const u32x4*>(
            p.X + (size_t)m * K + (size_t)(g0 + (q >> 2)) * 128 + (q & 3) * 32);
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[v] = src[v];
    };
    auto put = [&](int i, const u32x4 (&xv)[4]) {
        const int m = chunk_m(i);
        const int q = chunk_q(i);
        const int cq = q & 3, gl = q >> 2;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t xa[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
            f16x2 pr[4];
            permute_x8(xa, pr);
            xs[xslot((gl * 4 + cq) * 4 + t, m)] = pack_q8(pr);
        }
    };
    // Without the norm the slice is staged by 16-byte pieces in row order:
    // thread tid takes pieces tid + u NT, so consecutive lanes read
    // consecutive 16 bytes of a row (whole 1 KB runs per load instruction;
    // the chunk order below, rows fastest, put the lanes of a quad in
    // different rows: measured ~3.5x slower per byte).  Piece r of row m
    // (slice order) is dword t = r % 4 of k-quarter (r / 4) % 4 of group
    // r / 16.  The norm form keeps the chunk order: a thread's chunks are
    // then all of one row, which its row sums use.
    constexpr bool norm = NORM != 0;  // p.norm_w set; NORM = 1: M == MR, 2: M < MR
    const int ppr = ngs * 16;  // pieces per row of the slice
    const int pieces = ppr * M;
    const int dm = NT / ppr, dr = NT - dm * ppr;
    struct PieceCursor { int m, r; };  // piece tid + u NT as (row, piece of the row)
    auto advance = [&](PieceCursor& c) {
        c.r += dr;
        c.m += dm;
        if (c.r >= ppr) {
            c.r -= ppr;
            ++c.m;
        }
    };
    auto pput = [&](const PieceCursor& c, const u32x4 v) {
        const uint32_t xa[4] = {v.x, v.y, v.z, v.w};
        f16x2 pq[4];
        permute_x8(xa, pq);
        xs[xslot(c.r, c.m)] = pack_q8(pq);  // r = (gl * 4 + cq) * 4 + t
    };
    // X through a buffer resource: 32-bit offsets, and a piece past the
    // slice reads zeros without a branch around its load
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.X, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), 0x00020000);
    auto poff = [&](const PieceCursor& c) -> uint32_t {
        return ((uint32_t)c.m * (uint32_t)K + (uint32_t)g0 * 128u + (uint32_t)c.r * 8u) * 2u;
    };
    // the slice is all of X (one k-slice): piece i is bytes 16 i .. 16 i + 15
    // (the LM head; the other epilogues measured no faster with this form)
    const bool whole = EPI == MB_ARGMAX && ngs * 128 == K;
    const int nround = __builtin_amdgcn_readfirstlane((pieces + NT - 1) / NT);
    constexpr int kPU = 4 * kStageUnroll;  // pieces per thread and round (the chunks' registers)
    u32x4 xv0[kStageUnroll][4];
    PieceCursor cl = {tid / ppr, tid - (tid / ppr) * ppr};  // load cursor
    PieceCursor cs = cl;                                     // store cursor
    if constexpr (!norm) {
        if (whole) {
#pragma unroll
            for (int u = 0; u < kPU; ++u)
                if (u < nround)
                    xv0[u >> 2][u & 3] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(tid * 16), u * NT * 16, 0);
        } else {
#pragma unroll
            for (int u = 0; u < kPU; ++u) {
                if (tid + u * NT < pieces)
                    xv0[u >> 2][u & 3] = *reinterpret_cast<const u32x4*>(
                        p.X + (size_t)cl.m * K + (size_t)g0 * 128 + cl.r * 8);
                advance(cl);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u)
            if (tid + u * NT < chunks) get(tid + u * NT, xv0[u]);
    }
    // RMSNorm weights: requested with X, stored to LDS once they land (the
    // host keeps K <= 6144: K / 4 <= kNormPT * NT)
    constexpr int kNormPT = 1536 / NT;
    float4 nwv[kNormPT];
#pragma unroll
    for (int u = 0; u < kNormPT; ++u) nwv[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (norm) {
#pragma unroll
        for (int u = 0; u < kNormPT; ++u)
            nwv[u] = reinterpret_cast<const float4*>(p.norm_w)[min(tid + u * NT, (K >> 2) - 1)];
    }

    // items in flight per wave: a SwiGLU item carries both matrices' groups
    // (twice the bytes), and one item less measured faster there (gate/up
    // M = 4 / 8 28.9 / 31.4 -> 28.2 / 30.3 us) while the plain form lost
    // 1.5-4.6 % with it, and also with one more; the LM head's 4-group
    // items: XHIP_MB_PFA
    constexpr int PF = EPI == MB_SWIGLU ? XHIP_MB_PF - 1 : EPI == MB_ARGMAX ? XHIP_MB_PFA : XHIP_MB_PF;
    MbItem<E, GP> buf[PF + 1];
#pragma unroll
    for (int j = 0; j < PF; ++j) load_next(buf[j]);

    // RMSNorm prologue (fused norm + projection entry points; the host
    // plans one k-slice and one staging round, so the block holds every row
    // whole): the rows' sums of squares in a fixed order, then x * inv * w
    // rounded to fp16 per element as the standalone norm does
    // (src/ops/rmsnorm.cpp:45-78).  M == MR: a thread's chunks are all of
    // row tid % MR (its chunks, the row's lanes in xor order, the waves in
    // order).  Otherwise each chunk's sum goes to LDS and one wave per row
    // adds the row's chunks (lanes over the chunks in order, then the
    // 64-lane reduction), leaving 1/rms per row in LDS.
    float inv = 0.0f;
    float* css = rsum + 256;  // M != MR: per-chunk sums of squares
    if constexpr (norm) {
#pragma unroll
        for (int u = 0; u < kNormPT; ++u)
            if (tid + u * NT < (K >> 2)) reinterpret_cast<float4*>(nws)[tid + u * NT] = nwv[u];
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u)
            if (tid + u * NT < chunks) {
                float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    c0 = dot2(as_h2(xv0[u][t].x), as_h2(xv0[u][t].x), c0);
                    c1 = dot2(as_h2(xv0[u][t].y), as_h2(xv0[u][t].y), c1);
                    c0 = dot2(as_h2(xv0[u][t].z), as_h2(xv0[u][t].z), c0);
                    c1 = dot2(as_h2(xv0[u][t].w), as_h2(xv0[u][t].w), c1);
                }
                if constexpr (NORM == 1) {
                    s0 += c0;
                    s1 += c1;
                } else {
                    css[tid + u * NT] = c0 + c1;
                }
            }
        if constexpr (NORM == 1) {
            float sr = s0 + s1;
#pragma unroll
            for (int off = MR; off < 64; off <<= 1) sr += __shfl_xor(sr, off);
            if (lane < MR) rsum[wave * MR + lane] = sr;
            __syncthreads();
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) tot += rsum[w * MR + (tid & (MR - 1))];
            inv = 1.0f / sqrtf(tot / (float)K + p.norm_eps);
        } else {
            __syncthreads();
            const int nq = chunks / M;  // chunks per row
            for (int m = wave; m < M; m += NW) {
                float sv[1] = {0.0f};
                for (int q = lane; q < nq; q += 64) sv[0] += css[q * M + m];
                const float t = wave_sum_multi<1>(sv, lane);
                if (lane == 0) rsum[m] = 1.0f / sqrtf(t / (float)K + p.norm_eps);
            }
            __syncthreads();
        }
    }

    if constexpr (!norm) {
#pragma unroll
        for (int u = 0; u < kPU; ++u) {
            if (tid + u * NT < pieces) pput(cs, xv0[u >> 2][u & 3]);
            advance(cs);
        }
        cl = cs;  // piece tid + kPU NT
        for (int i0 = tid + NT * kPU; i0 < pieces; i0 += NT * kPU) {  // further rounds
            u32x4 xv[kPU];
#pragma unroll
            for (int u = 0; u < kPU; ++u) {
                xv[u] = __builtin_amdgcn_raw_buffer_load_b128(
                    rx, (int)(i0 + u * NT < pieces ? poff(cl) : kOutOfRange), 0, 0);
                advance(cl);
            }
#pragma unroll
            for (int u = 0; u < kPU; ++u) {
                if (i0 + u * NT < pieces) pput(cs, xv[u]);
                advance(cs);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u)
            if (tid + u * NT < chunks) {
                const int q = chunk_q(tid + u * NT);
                float iv = inv;
                if constexpr (NORM == 2) iv = rsum[chunk_m(tid + u * NT)];
                const float4* wk = reinterpret_cast<const float4*>(nws + (g0 + (q >> 2)) * 128 + (q & 3) * 32);
#pragma unroll
                for (int t = 0; t < 4; ++t) xv0[u][t] = rms_apply8(xv0[u][t], wk[2 * t], wk[2 * t + 1], iv);
                put(tid + u * NT, xv0[u]);
            }
        for (int i0 = tid + NT * kStageUnroll; i0 < chunks; i0 += NT * kStageUnroll) {  // further rounds
            u32x4 xv[kStageUnroll][4];
#pragma unroll
            for (int u = 0; u < kStageUnroll; ++u)
                if (i0 + u * NT < chunks) get(i0 + u * NT, xv[u]);
#pragma unroll
            for (int u = 0; u < kStageUnroll; ++u)
                if (i0 + u * NT < chunks) put(i0 + u * NT, xv[u]);
        }
    }
    __syncthreads();  // X staged

    f32x4 acc[E];
#pragma unroll
    for (int x = 0; x < E; ++x) acc[x] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // A operands: lane l reads row m = l % 16 (rows past M repeat row M - 1;
    // their results are never stored) of k-quarter l / 16; the stride of m
    // is the compile-time MR, so the four dwords of a group are immediate
    // offsets from one address.
    const f16x8* xl = xs + xslot(kq * 4, l16 < M ? l16 : M - 1);
    auto compute_item = [&](int it, const MbItem<E, GP>& b) {
        f16x8 xa[GP][4];
        int gl[GP];
#pragma unroll
        for (int gi = 0; gi < GP; ++gi) {
            gl[gi] = it * GP + gi;
            const f16x8* xg = xl + (gb + min(gl[gi], ngw - 1)) * (16 * MR);
#pragma unroll
            for (int t = 0; t < 4; ++t) xa[gi][t] = xg[t * MR];
        }
#pragma unroll
        for (int x = 0; x < E; ++x) {
            // the groups' MFMA chains are independent: interleaved
            f32x4 c[GP];
#pragma unroll
            for (int gi = 0; gi < GP; ++gi) c[gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int gi = 0; gi < GP; ++gi) {
                    const u32x4 wv = b.w[x * GP + gi];
                    const uint32_t wd = t == 0 ? wv.x : t == 1 ? wv.y : t == 2 ? wv.z : wv.w;
                    f16x2 q[4];
                    dequant8(wd, q);
                    c[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[gi][t], pack_q8(q), c[gi], 0, 0, 0);
                }
            }
#pragma unroll
            for (int gi = 0; gi < GP; ++gi) {
                const uint16_t sb = EPI == MB_ARGMAX ? (uint16_t)b.s[gi] : (uint16_t)((b.s[x] >> b.sh[x]) >> (16 * gi));
                const float s = gl[gi] < ngw ? h2f(sb) : 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[x][e] = __builtin_fmaf(s, c[gi][e], acc[x][e]);
            }
        }
    };

    // D layout of the 16x16 MFMA: lane l holds rows m = 4 * (l / 16) + e
    // (e = 0..3) of column n = l % 16.
    auto flush = [&](int tile) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = 4 * kq + e;
            if (m < M) {
#pragma unroll
                for (int x = 0; x < E; ++x)
                    outl[((((kp * p.tiles_blk) + tile) * 16 + l16) * M + m) * E + x] = acc[x][e];
            }
        }
#pragma unroll
        for (int x = 0; x < E; ++x) acc[x] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };

    int ct = t0, cgl = 0;  // compute cursor: tile, item
    for (int base = 0; base < nreal; base += PF + 1) {
#pragma unroll
        for (int j = 0; j <= PF; ++j) {
            load_next(buf[(j + PF) % (PF + 1)]);
            compute_item(cgl, buf[j]);
            if (base + j < nreal && ++cgl == nig) {
                flush(ct);
                cgl = 0;
                ++ct;
            }
        }
    }
    __syncthreads();

    // ---- epilogue over the block's rows x M (n fastest: coalesced stores)
    const int nout = rows_here * M;
    if (lkw > 0) {  // sum the run's slices in slice order
        const int sl = p.tiles_blk * 16 * M * E;
        for (int o = tid; o < nout * E; o += NT) {
            float v = outl[o];
            for (int q = 1; q < (1 << lkw); ++q) v += outl[q * sl + o];
            outl[o] = v;
        }
        __syncthreads();
    }
    if (ks > 1) {
        // partials [slice][e][m][n] of this descriptor (< 2 GiB: checked on the host)
        const uint32_t sst = (uint32_t)p.ws_slice[di];
        const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc(
            p.ws + p.ws_desc[di], (short)0, (int)((uint32_t)ks * sst * 4u), 0x00020000);
        for (int o = tid; o < nout; o += NT) {
            const int m = o / rows_here, rl = o - m * rows_here;
#pragma unroll
            for (int x = 0; x < E; ++x)
                __builtin_amdgcn_raw_buffer_store_b32(
                    __builtin_bit_cast(uint32_t, outl[(rl * M + m) * E + x]), rws,
                    (int)(((uint32_t)slice * sst + ((uint32_t)x * M + m) * (uint32_t)N + n0 + rl) * 4u), 0,
                    kDeviceCoherent);
        }
        // Arrival protocol on the memory model: the block's partial stores
        // happen before thread 0's arrival (workgroup barrier); the arrival
        // is an agent-scope release fetch_add, and the last arriver (the one
        // that counts ks - 1) issues an agent-scope acquire fence, so every
        // arriver's partials happen before the last arriver's loads (for its
        // other threads through the workgroup barrier after the fence).  The
        // partials also move with device-coherent (sc1) accesses, so the
        // release / acquire find no dirty or stale lines of theirs in the
        // XCDs' L2s.
        __syncthreads();
        if (tid == 0) {
            const uint32_t old = __hip_atomic_fetch_add(&p.cnt[grange], 1u, __ATOMIC_RELEASE,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            const bool last = old == (uint32_t)(ks - 1);
            if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            flag[0] = last ? 1 : 0;
        }
        __syncthreads();
        if (flag[0] == 0) return;  // another slice of this range finishes it
        for (int o = tid; o < nout; o += NT) {
            const int m = o / rows_here, rl = o - m * rows_here;
#pragma unroll
            for (int x = 0; x < E; ++x) {
                // slices in order, the loads of 8 slices in flight at a time
                const uint32_t off = (((uint32_t)x * M + m) * (uint32_t)N + n0 + rl) * 4u;
                float v = 0.0f;
                for (int s0 = 0; s0 < ks; s0 += 8) {
                    float pv[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        pv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                            rws, (int)(s0 + u < ks ? (uint32_t)(s0 + u) * sst * 4u + off : kOutOfRange), 0,
                            kDeviceCoherent));
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (s0 + u < ks) v += pv[u];
                }
                outl[(rl * M + m) * E + x] = v;
            }
        }
        __syncthreads();
        if (tid == 0) __hip_atomic_store(&p.cnt[grange], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    if constexpr (EPI == MB_ARGMAX) {
        // Every activation row at once: a thread's rows, then the wave in
        // one multi-row pass (DPP halving steps and lane swaps: lane L ends
        // with row L mod 8), then the waves for row m by thread m.
        // arg_better is a total order (value, then the lower index), so the
        // candidate does not depend on the order of the comparisons.  (One
        // row at a time, with shuffles and two barriers per row, this
        // epilogue cost ~5 us of the M = 8 LM head.)
        float bv[kCand];
        int32_t bi[kCand];
#pragma unroll
        for (int m = 0; m < kCand; ++m) {
            bv[m] = -__builtin_inff();
            bi[m] = 0x7FFFFFFF;
        }
        // the descriptor's pointers once (a store through Y could otherwise
        // make the compiler reload them from the kernel arguments)
        const float* const biasp = d.bias;
        float* const logits = reinterpret_cast<float*>(d.Y);
        for (int rl = tid; rl < rows_here; rl += NT) {
            const int n = n0 + rl;
            const float bn = biasp ? biasp[n] : 0.0f;
            float v[kCand];
            if (M == 8) {  // the row's M results: two 16-byte LDS reads
                const float4 a = reinterpret_cast<const float4*>(outl + rl * 8)[0];
                const float4 b2 = reinterpret_cast<const float4*>(outl + rl * 8)[1];
                v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
                v[4] = b2.x; v[5] = b2.y; v[6] = b2.z; v[7] = b2.w;
            } else {
#pragma unroll
                for (int m = 0; m < kCand; ++m) v[m] = m < M ? outl[rl * M + m] : 0.0f;
            }
#pragma unroll
            for (int m = 0; m < kCand; ++m) {
                if (m < M) {
                    const float vm = biasp ? v[m] + bn : v[m];
                    if (logits) logits[(size_t)m * N + n] = vm;
                    const float key = argmax_key(vm, n);
                    if (arg_better(key, n, bv[m], bi[m])) { bv[m] = key; bi[m] = n; }
                }
            }
        }
        // lane L: the wave's candidate of row L mod 8
        float rv;
        int32_t ri;
        wave_argmax_multi8(bv, bi, lane, rv, ri);
        if (lane < kCand) {
            candv[wave * kCand + lane] = rv;
            candi[wave * kCand + lane] = ri;
        }
        __syncthreads();
        if (tid < M) {
            float b = candv[tid];
            int32_t i = candi[tid];
            for (int w = 1; w < NW; ++w)
                if (arg_better(candv[w * kCand + tid], candi[w * kCand + tid], b, i)) {
                    b = candv[w * kCand + tid];
                    i = candi[w * kCand + tid];
                }
            ArgCand c;
            c.v = b;
            c.i = i;
            p.parts[(size_t)tid * p.nranges + grange] = c;
        }
    } else {
        for (int o = tid; o < nout; o += NT) {
            const int m = o / rows_here, rl = o - m * rows_here;
            const int n = n0 + rl;
            float v = outl[(rl * M + m) * E];
            if (EPI == MB_SWIGLU) {
                const float u = outl[(rl * M + m) * E + 1];
                v = v / (1.0f + expf(-v)) * u;
            } else if (d.bias) {
                v += d.bias[n];
            }
            OutT* y = reinterpret_cast<OutT*>(d.Y) + (size_t)m * N + n;
            if (EPI == MB_PLAIN && d.residual)  // add_inplace after the projection (elementwise.cpp:227)
                *y = (OutT)((float)*y + (float)(OutT)v);
            else
                *y = (OutT)v;
        }
    }
}

}  // namespace xhip

// ------------------------------------------------------------------ host ----

using namespace xhip;

namespace {

typedef void (*MbKernel)(MbParams);

template <int MR, int EPI, typename OutT>
MbKernel mb_pick_nw(int nw) {
    return nw >= 16 ? gemv_mb_int4_kernel<MR, EPI, OutT, 16>
         : nw >= 8  ? gemv_mb_int4_kernel<MR, EPI, OutT, 8>
                    : gemv_mb_int4_kernel<MR, EPI, OutT, 4>;
}

template <int EPI, typename OutT>
MbKernel mb_kernel_for(int mr, int nw, int norm = 0) {
    if constexpr ((EPI == MB_PLAIN || EPI == MB_SWIGLU) && std::is_same<OutT, f16>::value) {
        if (norm == 1) {  // M == MR (4 or 8) at 4 or 8 waves
            if (mr == 4) return nw >= 8 ? gemv_mb_int4_kernel<4, EPI, f16, 8, 1> : gemv_mb_int4_kernel<4, EPI, f16, 4, 1>;
            return nw >= 8 ? gemv_mb_int4_kernel<8, EPI, f16, 8, 1> : gemv_mb_int4_kernel<8, EPI, f16, 4, 1>;
        }
        if (norm == 2 && mr == 4)  // M = 3
            return nw >= 8 ? gemv_mb_int4_kernel<4, EPI, f16, 8, 2> : gemv_mb_int4_kernel<4, EPI, f16, 4, 2>;
    }
    if (norm) return nullptr;
    if (mr <= 4) return mb_pick_nw<4, EPI, OutT>(nw);
    if (mr <= 8 || EPI == MB_ARGMAX) return mb_pick_nw<8, EPI, OutT>(nw);  // the LM head: M <= 8
    if constexpr (EPI != MB_ARGMAX) return mb_pick_nw<16, EPI, OutT>(nw);
    return nullptr;
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

struct MbOverrides {
    int nw, ks, bpc, min_m, raise, kw, balance;
};
const MbOverrides& mb_overrides() {
    static const MbOverrides o = {env_int("XINFER_MB_NW", 0),
                                  env_int("XINFER_MB_KS", 0), env_int("XINFER_MB_BPC", 0),
                                  env_int("XINFER_MB_MIN_M", 0), env_int("XINFER_MB_RAISE", -1),
                                  env_int("XINFER_MB_KW", 0), env_int("XINFER_MB_BALANCE", 1)};
    return o;
}

// Prologue of a wave (X staging share, ring fill, epilogue) in units of one
// group of one tile, for the planner's cost model.
constexpr int64_t kMbWaveSetup = 8;

constexpr size_t kMaxLds = 160 * 1024;
// Chunked-prefill rows 9..16 fill the 16-row MFMA tile (N = 17408,
// K = 5120: 21.6 / 25.1 us at M = 9 / 16 against 47 / 48 us for the GEMM,
// whose 128-row tiles are mostly padding there).  Two to four M-tiles per
// weight tile (M = 17..64) measured slower than the GEMM: the X slice of
// 32-64 rows forces 5-10 k-slices and a large split-K combine.
constexpr int kMaxMbM = 16;

}  // namespace

namespace xhip_host {

struct MbPlan {
    int mr, nw, ks, gps, tiles_blk, blocks, nranges, kw;
    size_t lds, ws_floats;
    MbKernel k;
};

// Plan a small-batch launch.  Returns false when the shape does not fit the
// kernel (X slice of one group per block beyond LDS) or M is outside 2..8.
//   ks:  the smallest number of k-slices whose X slice fits the LDS budget,
//        raised while the tile ranges alone cannot give every CU `bpc`
//        blocks (short N, long K); argmax keeps ks = 1.
//   tiles per block: the tiles spread evenly over cus * bpc / ks ranges.
//   kw:  waves per run of tiles, splitting the slice's groups (every wave
//        has a tile of its run): the smallest power of two that gives at
//        least half as many blocks as CUs, at most the waves of a block and
//        the groups of the shortest slice.  This adds blocks to short-N
//        shapes without a cross-block combine; more waves per tile than
//        that measured slower (each wave then decodes fewer groups per
//        fixed prologue).
//   MR:  the m stride of the staged X (4, 8 or 16: M rounded up).
bool gemv_stages_x(int64_t M, int64_t K);  // gemv_int4.hip

// ws_cap / cnt_cap: the split-K slot available to this call (floats of
// partials, tile-range counters); a plan that splits K beyond it is rejected.
// raise_ok = false keeps ks at what the X slice needs (no extra slices for
// short N), the retry when the raised plan does not fit the slot.
bool splitk_slot(hipStream_t st, float** partials, size_t* partial_floats, uint32_t** counters,
                 int* ncounters);  // scratch.hip

template <int EPI, typename OutT>
bool plan_mb(MbParams& p, MbPlan& pl, size_t ws_cap, int64_t cnt_cap, bool raise_ok) {
    const MbOverrides& ov = mb_overrides();
    const int M = p.M;
    // M = 2: the VALU GEMV measured faster while it stages all of X in LDS
    // (K = 5120: 8.1 vs 8.2 us, N = 34816: 19.3 vs 27.3 us); beyond that its
    // global-X path is slower than this kernel (K = 17408: 20.3 vs 14.5 us)
    const int min_m = ov.min_m > 0 ? ov.min_m : gemv_stages_x(2, p.K) ? 3 : 2;
    if (M < min_m || M < 2 || M > (EPI == MB_ARGMAX ? 8 : kMaxMbM)) return false;
    for (int i = 0; i < p.ndesc; ++i)  // the kernel's 4-byte scale loads need two scales
        if ((int64_t)p.d[i].N * (p.K / 128) < 2) return false;
    const int E = EPI == MB_SWIGLU ? 2 : 1;
    const int ng = p.K / 128;
    const int cus = num_cus();
    // RMSNorm in the staging: every row whole in the block (one k-slice and
    // one staging round, checked below)
    const bool norm = p.norm_w != nullptr;
    // (M = 4 / 8: a thread's chunks are all of one row; M = 3: per-chunk
    // sums through LDS; at M = 5-7 that form measured no faster than the
    // norm kernel first)
    if (norm && (EPI == MB_ARGMAX || (M != 3 && M != 4 && M != 8))) return false;
    int64_t tiles_total = 0;
    for (int i = 0; i < p.ndesc; ++i) tiles_total += (p.d[i].N + 15) / 16;
    const int mr = M <= 4 ? 4 : M <= 8 ? 8 : 16;
    const size_t xg = (size_t)mr * 256;  // LDS bytes of X per group
    size_t x_budget = EPI == MB_ARGMAX ? 96 * 1024 : mr >= 16 ? 64 * 1024 : 48 * 1024;
    // Long K at an 8-row stride (X over four 48 KB slices): 96 KB slices,
    // still 4 waves.  Measured at K = 17408, N = 5120: M = 5 20.1 -> 16.3 us,
    // M = 8 21.6 -> 18.0 (3 slices instead of 6).  At K <= 6144 the larger
    // slices leave one block per CU and lose (gate/up M = 8 42.1 -> 45.7 us).
    const bool long_k8 = EPI != MB_ARGMAX && mr == 8 && (size_t)ng * xg > 4 * 48 * 1024;
    if (long_k8) x_budget = 96 * 1024;
    // All of X within 80 KB at the 8-row stride (K <= 5120): one slice, no
    // split-K combine, 4 waves at one block per CU (with the balanced plan
    // below).  Measured at M = 8: gate/up SwiGLU 37.1 -> 29.5 us, fused QKV
    // 15.9 -> 13.3 us; o_proj (K = 6144, 96 KB) lost (11.1 -> 11.6), so the
    // limit stays at 80 KB.
    const bool whole8 = EPI != MB_ARGMAX && mr == 8 && (size_t)ng * xg <= 80 * 1024;
    if (whole8) x_budget = 80 * 1024;
    // 9-16 rows (16-row stride) with X within two 80 KB slices (K <= 5120):
    // two slices and 8-wave blocks instead of three 53 KB slices of 4 waves.
    // Measured at N = 17408, K = 5120, M = 9 / 12 / 16: linear 22.3 / 24.4 /
    // 27.4 -> 20.0 / 21.2 / 22.5 us, SwiGLU 40.9 / 44.4 / 49.3 -> 38.3 /
    // 40.4 / 42.8 us.
    const bool two16 = EPI != MB_ARGMAX && mr == 16 && (size_t)ng * xg <= 160 * 1024;
    if (two16) x_budget = 80 * 1024;
    int ks = ov.ks > 0 ? ov.ks : (int)((ng * xg + x_budget - 1) / x_budget);
    if (EPI == MB_ARGMAX) ks = 1;
    if (ks > ng) ks = ng;
    const size_t slice = (size_t)ng * xg / ks;
    // X slice beyond nw_at: 8 waves.  The LM head keeps 4 waves at one block
    // per CU (M = 8, N = 151936: 94.0 -> 89.5 us against 8 waves).  Long K at
    // the 8-row stride (config 2 at M = 5-8) takes 8 waves for its 92 KB
    // slices (M = 8 19.3 -> 18.4 us).
    const size_t nw_at = long_k8 ? 64 * 1024 : whole8 ? 96 * 1024 : 64 * 1024;
    int nw = ov.nw > 0 ? ov.nw : (EPI != MB_ARGMAX && slice > nw_at) ? 8 : 4;
    nw = nw >= 16 ? 16 : nw >= 8 ? 8 : 4;
    int bpc = ov.bpc > 0 ? ov.bpc : (nw >= 8 ? 1 : 2);
    // LDS of the norm: its weights and the waves' row sums
    const size_t norm_lds = norm ? (size_t)p.K * 4 + 256 * 4 + (size_t)ng * 4 * M * 4 : 0;
    // never plan more blocks per CU than their X slices leave resident
    if (ov.bpc <= 0) {
        const int fit = (int)(kMaxLds / (slice + 4096 + norm_lds));
        if (fit < bpc) bpc = fit < 1 ? 1 : fit;
    }
    const int64_t target = (int64_t)cus * bpc;
    int64_t tiles_blk = 0, ranges = 0;
    for (int pass = 0; pass < 2; ++pass) {
        int64_t rt = target / ks;
        if (rt < 1) rt = 1;
        tiles_blk = (tiles_total + rt - 1) / rt;
        ranges = 0;
        for (int i = 0; i < p.ndesc; ++i) ranges += ((p.d[i].N + 15) / 16 + tiles_blk - 1) / tiles_blk;
        if (pass == 0 && ov.ks <= 0 && ov.raise != 0 && raise_ok && EPI != MB_ARGMAX && ranges * ks < target) {
            int ks2 = (int)(target / ranges);
            if (ks2 > ng) ks2 = ng;
            if (ks2 > ks) { ks = ks2; continue; }
        }
        break;
    }
    const int gps = (ng + ks - 1) / ks;
    ks = (ng + gps - 1) / gps;
    const int last = ng - (ks - 1) * gps;  // groups of the shortest slice
    int kw_cap = 1;
    while (kw_cap * 2 <= nw && kw_cap * 2 <= last) kw_cap *= 2;
    const int64_t tiles_want = tiles_blk;
    int kw = 1;
    for (;; kw *= 2) {
        if (ov.kw > 0 && kw * 2 <= ov.kw && kw < kw_cap) continue;
        tiles_blk = tiles_want < nw / kw ? nw / kw : tiles_want;  // every run of waves has a tile
        ranges = 0;
        for (int i = 0; i < p.ndesc; ++i) ranges += ((p.d[i].N + 15) / 16 + tiles_blk - 1) / tiles_blk;
        if (ov.kw > 0 || kw >= kw_cap || ranges * ks * 2 >= cus) break;
    }
    // Ranges per descriptor: ceil(tiles / tiles_blk), tiles split evenly.
    int nrd[4] = {1, 1, 1, 1};
    for (int i = 0; i < p.ndesc; ++i) nrd[i] = (int)(((p.d[i].N + 15) / 16 + tiles_blk - 1) / tiles_blk);
    // Balance.  A wave's time is its tiles times its groups, and a CU's waves
    // share its SIMDs, so a launch takes about (blocks per CU) x (tiles per
    // wave) x (groups per wave) units plus a prologue per wave.  The plan
    // above rounds tiles per block up and may leave CUs with two blocks
    // while others have one (gate/up SwiGLU, M = 4: 272 blocks of 4 tiles on
    // 256 CUs).  Candidates with exactly c blocks per CU (c <= bpc), tiles
    // spread over the ranges in proportion, and kw waves per tile (every run
    // of waves with a tile) are scored the same way; the lowest wins, the
    // plan above on ties.
    auto cost = [&](int64_t nblocks, int64_t tmax, int kwc) {
        const int64_t per_cu = (nblocks + cus - 1) / cus;
        const int64_t runs = nw / kwc;
        return per_cu * (((tmax + runs - 1) / runs) * ((gps + kwc - 1) / kwc) + kMbWaveSetup);
    };
    if (ov.balance && ov.kw <= 0) {
        int64_t best = cost(ranges * ks, tiles_blk, kw);
        for (int c = 1; c <= bpc; ++c) {
            int64_t R = (int64_t)cus * c / ks;
            if (R > tiles_total) R = tiles_total;
            if (R < p.ndesc) continue;
            int nr[4] = {1, 1, 1, 1};
            int64_t used = 0;
            for (int i = 0; i < p.ndesc; ++i) {
                const int64_t t = (p.d[i].N + 15) / 16;
                nr[i] = (int)std::max<int64_t>(1, std::min<int64_t>(t, t * R / tiles_total));
                used += nr[i];
            }
            while (used < R) {  // leftover ranges to the descriptor with the most tiles per range
                int bi = -1;
                int64_t bt = 0;
                for (int i = 0; i < p.ndesc; ++i) {
                    const int64_t t = (p.d[i].N + 15) / 16;
                    if (nr[i] < t && (t + nr[i] - 1) / nr[i] > bt) { bt = (t + nr[i] - 1) / nr[i]; bi = i; }
                }
                if (bi < 0) break;
                ++nr[bi];
                ++used;
            }
            int64_t tmax = 0, tmin = INT64_MAX;
            for (int i = 0; i < p.ndesc; ++i) {
                const int64_t t = (p.d[i].N + 15) / 16;
                tmax = std::max<int64_t>(tmax, (t + nr[i] - 1) / nr[i]);
                tmin = std::min<int64_t>(tmin, t / nr[i]);
            }
            for (int kwc = 1; kwc <= kw_cap; kwc *= 2) {
                if (tmin < nw / kwc) continue;  // a run of waves without a tile
                const size_t l = (size_t)gps * xg + (size_t)tmax * 16 * M * E * 4 * kwc + 2 * nw * 4 * (EPI == MB_ARGMAX ? 8 : 1) + 16 + norm_lds;
                if (l * c > kMaxLds) continue;
                const int64_t cc = cost(used * ks, tmax, kwc);
                if (cc < best) {
                    best = cc;
                    kw = kwc;
                    tiles_blk = tmax;
                    ranges = used;
                    for (int i = 0; i < 4; ++i) nrd[i] = nr[i];
                }
            }
        }
    }
    int lkw = 0;
    while ((1 << lkw) < kw) ++lkw;
    const size_t lds = (size_t)gps * xg + (size_t)tiles_blk * 16 * M * E * 4 * kw + 2 * nw * 4 * (EPI == MB_ARGMAX ? 8 : 1) + 16 + norm_lds;
    if (lds > kMaxLds) return false;
    // the norm's single staging round: chunks and weights per thread within
    // the kernel's unrolls (8 / 4 chunks at 4 / 8 waves, 1536 float4 of
    // weights per block)
    if (norm && (ks != 1 || nw > 8 || (int64_t)ng * 4 * M > (nw == 4 ? 8 : 4) * 64 * nw || p.K > 6144))
        return false;
    if (ks > 1 && ranges > cnt_cap) return false;
    for (int i = 0; ks > 1 && i < p.ndesc; ++i)  // 32-bit buffer offsets into the partials
        if ((int64_t)ks * (E * M * p.d[i].N + 64) * 4 >= (1LL << 31)) return false;
    pl.mr = mr;
    pl.nw = nw;
    pl.ks = ks;
    pl.gps = gps;
    pl.tiles_blk = (int)tiles_blk;
    pl.nranges = (int)ranges;
    pl.kw = kw;
    pl.lds = lds;
    pl.k = mb_kernel_for<EPI, OutT>(mr, nw, !norm ? 0 : M == mr ? 1 : 2);
    if (!pl.k) return false;
    int blocks = 0, rbeg = 0;
    int64_t wsoff = 0;
    for (int i = 0; i < p.ndesc; ++i) {
        const int r = nrd[i];
        p.d[i].nr = r;
        p.d[i].block_begin = blocks;
        p.d[i].range_begin = rbeg;
        p.ws_desc[i] = wsoff;
        p.ws_slice[i] = (int32_t)(((int64_t)E * M * p.d[i].N + 63) / 64 * 64);
        blocks += r * ks;
        rbeg += r;
        wsoff += (int64_t)ks * p.ws_slice[i];
    }
    for (int i = p.ndesc; i < 4; ++i) {
        p.d[i] = p.d[0];
        p.d[i].block_begin = 0x7FFFFFFF;
        p.ws_desc[i] = 0;
        p.ws_slice[i] = 0;
    }
    if (ks > 1 && (size_t)wsoff > ws_cap) return false;
    pl.blocks = blocks;
    pl.ws_floats = ks > 1 ? (size_t)wsoff : 0;
    p.ks = ks;
    p.gps = gps;
    p.tiles_blk = (int)tiles_blk;
    p.nranges = (int)ranges;
    p.lkw = lkw;
    return true;
}

// Plan against the calling stream's split-K slot: the raised plan first,
// then the plan with the fewest slices; with no slot (every slot owned by
// another stream) only plans without a cross-block split are accepted.
template <int EPI, typename OutT>
bool plan_mb_stream(hipStream_t st, MbParams& p, MbPlan& pl) {
    float* ws = nullptr;
    uint32_t* cnt = nullptr;
    size_t ws_cap = 0;
    int ncnt = 0;
    if (!splitk_slot(st, &ws, &ws_cap, &cnt, &ncnt)) {
        ws = nullptr;
        cnt = nullptr;
        ws_cap = 0;
        ncnt = 0;
    }
    p.ws = ws;
    p.cnt = cnt;
    return plan_mb<EPI, OutT>(p, pl, ws_cap, ncnt, true) || plan_mb<EPI, OutT>(p, pl, ws_cap, ncnt, false);
}

template <int EPI, typename OutT>
int launch_mb(const MbParams& p0, const MbPlan& pl, hipStream_t st) {
    MbParams p = p0;
    if (pl.lds > 64 * 1024) {
        static std::mutex mu;
        static const void* done[256];
        static int ndone = 0;
        std::lock_guard<std::mutex> lock(mu);
        bool seen = false;
        for (int i = 0; i < ndone; ++i) seen |= done[i] == reinterpret_cast<const void*>(pl.k);
        if (!seen) {
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(pl.k),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds) != hipSuccess)
                return XINFER_ERR_HIP;
            if (ndone < 256) done[ndone++] = reinterpret_cast<const void*>(pl.k);
        }
    }
    hipLaunchKernelGGL(pl.k, dim3((unsigned)pl.blocks), dim3(64 * pl.nw), pl.lds, st, p);
    return launch_status();
}

// Entry points used by the GEMV front end (gemv_int4.hip).  Return 1 when the
// shape is not handled here (the caller then runs the VALU GEMV).
int mb_linear(hipStream_t st, const xinfer_fused_desc* descs, int nd, const void* X, bool y_f32,
              int64_t M, int64_t K, bool residual, int* rc, const float* norm_w, float eps) {
    MbParams p = {};
    p.X = reinterpret_cast<const f16*>(X);
    p.norm_w = norm_w;
    p.norm_eps = eps;
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    p.ndesc = nd;
    for (int i = 0; i < nd; ++i) {
        p.d[i].residual = residual ? 1 : 0;
        p.d[i].W = descs[i].W_int4;
        p.d[i].S = reinterpret_cast<const uint16_t*>(descs[i].scales);
        p.d[i].bias = descs[i].bias;
        p.d[i].Y = descs[i].Y;
        p.d[i].N = (int32_t)descs[i].N;
    }
    MbPlan pl;
    const bool ok = y_f32 ? plan_mb_stream<MB_PLAIN, float>(st, p, pl) : plan_mb_stream<MB_PLAIN, f16>(st, p, pl);
    if (!ok) return 1;
    *rc = y_f32 ? launch_mb<MB_PLAIN, float>(p, pl, st) : launch_mb<MB_PLAIN, f16>(p, pl, st);
    return 0;
}

int mb_swiglu(hipStream_t st, void* Y, const void* X, const uint8_t* Wg, const void* Sg,
              const uint8_t* Wu, const void* Su, int64_t M, int64_t N, int64_t K,
              int* rc, const float* norm_w, float eps) {
    MbParams p = {};
    p.X = reinterpret_cast<const f16*>(X);
    p.norm_w = norm_w;
    p.norm_eps = eps;
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    p.ndesc = 1;
    p.d[0].W = Wg;
    p.d[0].S = reinterpret_cast<const uint16_t*>(Sg);
    p.d[0].W2 = Wu;
    p.d[0].S2 = reinterpret_cast<const uint16_t*>(Su);
    p.d[0].Y = Y;
    p.d[0].N = (int32_t)N;
    MbPlan pl;
    if (!plan_mb_stream<MB_SWIGLU, f16>(st, p, pl)) return 1;
    *rc = launch_mb<MB_SWIGLU, f16>(p, pl, st);
    return 0;
}

// LM head: plan only (nranges = candidate count per row), or plan + launch.
int mb_argmax_plan(int64_t M, int64_t N, int64_t K, int* nparts) {
    MbParams p = {};
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    p.ndesc = 1;
    p.d[0].N = (int32_t)N;
    MbPlan pl;
    if (!plan_mb<MB_ARGMAX, float>(p, pl, 0, 0, false)) return 1;
    *nparts = pl.nranges;
    return 0;
}

int mb_max_m() {
    static const int v = [] {
        const int o = env_int("XINFER_MB_MAX_M", 0);
        return o > 0 ? (o < kMaxMbM ? o : kMaxMbM) : kMaxMbM;
    }();
    return v;
}

int mb_argmax(hipStream_t st, float* logits, const void* X, const uint8_t* W, const void* S,
              int64_t M, int64_t N, int64_t K, ArgCand* parts, int* nparts, int* rc) {
    MbParams p = {};
    p.X = reinterpret_cast<const f16*>(X);
    p.M = (int32_t)M;
    p.K = (int32_t)K;
    p.ndesc = 1;
    p.parts = parts;
    p.d[0].W = W;
    p.d[0].S = reinterpret_cast<const uint16_t*>(S);
    p.d[0].Y = logits;
    p.d[0].N = (int32_t)N;
    MbPlan pl;
    if (!plan_mb<MB_ARGMAX, float>(p, pl, 0, 0, false)) return 1;
    *nparts = pl.nranges;
    *rc = launch_mb<MB_ARGMAX, float>(p, pl, st);
    return 0;
}

}  // namespace xhip_host
