// Greedy argmax over FP32 logits on gfx950 (batched rows).
//
// Replaces src/ops/sampling.cpp:12-92, whose stage 2 ran on the host after a
// blocking wait.  Here both stages run on the device and the id stays in
// device memory, so a decode step can be captured without a host sync:
//   stage 1: grid (blocks, rows); each 256-thread block scans 4096 logits
//            (16 coalesced loads per thread) and writes one (value, index).
//   stage 2: one block per row reduces the block candidates.
// Ordering: larger value wins, ties go to the lower index (the reference's
// strict '>' from element 0, sampling.cpp:60, 80).

#include <mutex>

#include "common.h"

namespace xhip {

constexpr int kArgBlock = 256;
constexpr int kArgPerThread = 16;
constexpr int kArgSpan = kArgBlock * kArgPerThread;

__device__ __forceinline__ void block_reduce_cand(float& bv, int32_t& bi) {
    // wave64 DPP-free reduction through LDS (runs once per block)
    __shared__ float sv[kArgBlock];
    __shared__ int32_t si[kArgBlock];
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = kArgBlock / 2; s > 0; s >>= 1) {
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
    bv = sv[0];
    bi = si[0];
}

__global__ __launch_bounds__(kArgBlock) void argmax_stage1_kernel(const float* logits, int64_t V,
                                                                  ArgCand* parts) {
    const int64_t row = blockIdx.y;
    const float* x = logits + row * V;
    const int64_t base = (int64_t)blockIdx.x * kArgSpan;
    float bv = -__builtin_inff();
    int32_t bi = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < kArgPerThread; ++i) {
        const int64_t idx = base + (int64_t)i * kArgBlock + threadIdx.x;
        if (idx < V) {
            const float v = argmax_key(x[idx], idx);
            if (arg_better(v, (int32_t)idx, bv, bi)) { bv = v; bi = (int32_t)idx; }
        }
    }
    block_reduce_cand(bv, bi);
    if (threadIdx.x == 0) {
        ArgCand c;
        c.v = bv;
        c.i = bi;
        parts[row * gridDim.x + blockIdx.x] = c;
    }
}

__global__ __launch_bounds__(kArgBlock) void argmax_stage2_kernel(const ArgCand* parts,
                                                                  int32_t nparts, int64_t* ids) {
    const int64_t row = blockIdx.x;
    float bv = -__builtin_inff();
    int32_t bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < nparts; i += kArgBlock) {
        const ArgCand c = parts[row * nparts + i];
        if (arg_better(c.v, c.i, bv, bi)) { bv = c.v; bi = c.i; }
    }
    block_reduce_cand(bv, bi);
    if (threadIdx.x == 0) ids[row] = bi == 0x7FFFFFFF ? 0 : bi;
}

__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace xhip

using namespace xhip;

namespace xhip_host {

// Library-owned scratch for callers that pass scratch == NULL: one buffer
// per device and stream (so calls on different streams never share it),
// grown on demand.  Growing waits for the stream's queued work (which may
// still read the old buffer) and frees the old buffer before allocating the
// new one; xinfer_stream_release frees a stream's buffer.  Returns nullptr
// when the allocation fails or more than kStreams streams of a device hold
// one.
namespace {
constexpr int kScratchStreams = 16;
struct ScratchEntry { hipStream_t st; void* buf; size_t cap; };
std::mutex g_scratch_mu;
ScratchEntry g_scratch[64][kScratchStreams];
int g_nscratch[64] = {0};
}  // namespace

void* library_scratch(hipStream_t st, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchEntry* e = nullptr;
    for (int i = 0; i < g_nscratch[dev]; ++i)
        if (g_scratch[dev][i].st == st && g_scratch[dev][i].buf) e = &g_scratch[dev][i];
    if (!e) {
        for (int i = 0; i < g_nscratch[dev] && !e; ++i)
            if (!g_scratch[dev][i].buf) e = &g_scratch[dev][i];  // a released entry
        if (!e) {
            if (g_nscratch[dev] == kScratchStreams) return nullptr;
            e = &g_scratch[dev][g_nscratch[dev]++];
        }
        *e = ScratchEntry{st, nullptr, 0};
    }
    if (e->cap < bytes) {
        if (e->buf) {
            if (hipStreamSynchronize(st) != hipSuccess) return nullptr;
            (void)hipFree(e->buf);
            e->buf = nullptr;
            e->cap = 0;
        }
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes * 2;
        void* p = nullptr;
        if (hipMalloc(&p, want) != hipSuccess) return nullptr;
        e->buf = p;
        e->cap = want;
    }
    return e->buf;
}

// Frees the library scratch of `st` on the current device (after its work).
void library_scratch_release(hipStream_t st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    for (int i = 0; i < g_nscratch[dev]; ++i) {
        ScratchEntry& e = g_scratch[dev][i];
        if (e.st == st && e.buf) {
            (void)hipFree(e.buf);
            e = ScratchEntry{nullptr, nullptr, 0};
        }
    }
}

void splitk_release(hipStream_t st);  // scratch.hip

}  // namespace xhip_host

extern "C" {

int xinfer_stream_release(void* stream) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (hipStreamSynchronize(st) != hipSuccess) return XINFER_ERR_HIP;
    xhip_host::splitk_release(st);
    xhip_host::library_scratch_release(st);
    return XINFER_OK;
}

size_t xinfer_argmax_scratch_bytes(int64_t V, int64_t rows) {
    if (V <= 1 || rows <= 0) return 0;
    const int64_t nblk = (V + kArgSpan - 1) / kArgSpan;
    return (size_t)(nblk * rows) * sizeof(ArgCand);
}

int xinfer_argmax_f32(void* stream, const float* logits, int64_t V, int64_t rows,
                      int64_t* out_ids, void* scratch, size_t scratch_bytes) {
    if (rows <= 0) return XINFER_OK;
    if (!out_ids) return XINFER_ERR_INVALID_ARG;
    using namespace xhip_host;
    if (!aligned(out_ids, 8) || !aligned(logits, 4)) return XINFER_ERR_MISALIGNED;
    if (V >= 0x7FFFFFFFLL || rows > 65535) return XINFER_ERR_UNSUPPORTED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (V <= 1 || !logits) {
        // the reference returns token 0 for an empty or single-entry vocab
        hipLaunchKernelGGL(fill_i64_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st,
                           out_ids, rows, (int64_t)0);
        return launch_status();
    }
    const int64_t nblk = (V + kArgSpan - 1) / kArgSpan;
    const size_t need = (size_t)(nblk * rows) * sizeof(ArgCand);
    if (!scratch) {
        scratch = library_scratch(st, need);
        if (!scratch) return XINFER_ERR_SCRATCH;
    } else if (scratch_bytes < need || !aligned(scratch, 8)) {
        return XINFER_ERR_SCRATCH;
    }
    ArgCand* parts = reinterpret_cast<ArgCand*>(scratch);
    hipLaunchKernelGGL(argmax_stage1_kernel, dim3((unsigned)nblk, (unsigned)rows), dim3(kArgBlock),
                       0, st, logits, V, parts);
    if (launch_status()) return XINFER_ERR_HIP;
    hipLaunchKernelGGL(argmax_stage2_kernel, dim3((unsigned)rows), dim3(kArgBlock), 0, st, parts,
                       (int32_t)nblk, out_ids);
    return launch_status();
}

}  // extern "C"
