// LM head + argmax for callers that cannot allocate device memory (code
// under hipGraph capture, serving loops that forbid allocation): the variant
// of xinfer_lm_head_argmax_int4 whose per-block argmax candidates go to a
// file-scope device array instead of caller scratch or a library allocation.
// Every block writes its candidate before the finalize kernel reads it, so
// nothing in the array needs to start at zero.  One array per device, shared
// by every call on that device: calls that overlap on one device (other
// streams, concurrent graph replays) race.

#include <mutex>

#include "common.h"

namespace {
constexpr size_t kNoAllocScratchBytes = 128 * 1024;  // 16384 candidates of 8 bytes
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace xhip_host {
int lm_head_argmax_impl(void* stream, int32_t* ids, float* logits, const void* X, const uint8_t* W_int4,
                        const void* scales, int64_t M, int64_t N, int64_t K, int32_t group_size, void* cand,
                        size_t cand_bytes, bool library_ok);  // gemv_int4.hip
}

namespace {
// Device address of `scratch` on the current device, looked up once per
// device with that device current (each device holds its own copy; the
// host-side name is only a stand-in for the symbol, never a device address).
void* noalloc_scratch_ptr() {
    static std::mutex mu;
    static void* ptr[64] = {nullptr};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        ptr[dev] = p;
    }
    return ptr[dev];
}
}  // namespace

extern "C" int xinfer_lm_head_argmax_int4_noalloc(void* stream, int32_t* ids, float* logits,
                                                  const void* X, const uint8_t* W_int4,
                                                  const void* scales, int64_t M, int64_t N, int64_t K,
                                                  int32_t group_size) {
    if (M <= 0 || N <= 0 || K <= 0) return XINFER_OK;
    if (M <= 8 && xinfer_lm_head_argmax_scratch_bytes(M, N, K) > kNoAllocScratchBytes)
        return XINFER_ERR_SCRATCH;  // more candidates than the static array holds
    void* p = noalloc_scratch_ptr();
    if (!p) return XINFER_ERR_HIP;
    return xhip_host::lm_head_argmax_impl(stream, ids, logits, X, W_int4, scales, M, N, K, group_size, p,
                                          kNoAllocScratchBytes, false);
}
