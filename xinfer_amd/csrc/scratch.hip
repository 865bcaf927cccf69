// Split-K workspace of the small-batch kernel without run-time allocation.
//
// The reference's projections allocate nothing per call: its split-K
// partials live in SLM (src/ops/linear.cpp:25-27) and every buffer a call
// touches is the caller's.  The small-batch MFMA kernel splits long K over
// several blocks, so its partial sums cross blocks and need device memory.
// That memory is a file-scope __device__ array here: the code object loader
// places it when the library's kernels are first loaded on a device, so no
// projection call runs hipMalloc, hipMemset or a device synchronisation, and
// the first call of a shape can be captured into a hipGraph.
//
// The array holds kSplitSlots independent slots (partials + arrival
// counters), 32 x (4 MiB + 16 KiB) = 128.5 MiB on every device the library
// runs on.  A slot belongs to one stream of a device until
// xinfer_stream_release gives it back: calls on one stream run in order, so
// they never share a slot concurrently, and calls on different streams use
// different slots.  Every counter is zero at load time and is returned to
// zero by the block that finishes its tile range, so a slot needs no
// clearing between calls.  When every slot of a device is taken (more live
// streams than slots) the caller plans without a cross-block split instead.

#include <mutex>

#include "common.h"

namespace xhip {
constexpr int kSplitSlots = 32;  // torch's stream pool alone hands out 32 streams per device
constexpr size_t kSplitPartialFloats = (size_t)1 << 20;  // 4 MiB of FP32 partials per slot
constexpr int kSplitCounters = 4096;                       // tile ranges per slot

__device__ __align__(256) float g_splitk_partials[kSplitSlots][kSplitPartialFloats];
__device__ __align__(256) uint32_t g_splitk_counters[kSplitSlots][kSplitCounters];
}  // namespace xhip

namespace xhip_host {

namespace {
constexpr int kMaxDev = 64;
struct DevSlots {
    bool resolved = false;
    float* partials = nullptr;    // device address of g_splitk_partials on this device
    uint32_t* counters = nullptr; // device address of g_splitk_counters on this device
    int nused = 0;
    hipStream_t owner[xhip::kSplitSlots] = {};
    bool released[xhip::kSplitSlots] = {};
};
std::mutex g_mu;
DevSlots g_devs[kMaxDev];
}  // namespace

// The split-K slot of `st` on the current device: its partials (capacity in
// floats) and counters (count).  Returns false when the device's slots are
// all owned by other streams or the symbol lookup failed.
bool splitk_slot(hipStream_t st, float** partials, size_t* partial_floats, uint32_t** counters,
                 int* ncounters) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
    std::lock_guard<std::mutex> lock(g_mu);
    DevSlots& d = g_devs[dev];
    if (!d.resolved) {
        void* pa = nullptr;
        void* ca = nullptr;
        if (hipGetSymbolAddress(&pa, HIP_SYMBOL(xhip::g_splitk_partials)) != hipSuccess ||
            hipGetSymbolAddress(&ca, HIP_SYMBOL(xhip::g_splitk_counters)) != hipSuccess || !pa || !ca) {
            (void)hipGetLastError();
            return false;
        }
        d.partials = reinterpret_cast<float*>(pa);
        d.counters = reinterpret_cast<uint32_t*>(ca);
        d.resolved = true;
    }
    int slot = -1, freed = -1;
    for (int i = 0; i < d.nused; ++i) {
        if (d.owner[i] == st && !d.released[i]) slot = i;
        if (d.released[i] && freed < 0) freed = i;
    }
    if (slot < 0) {
        if (freed >= 0) {
            slot = freed;
        } else {
            if (d.nused == xhip::kSplitSlots) return false;
            slot = d.nused++;
        }
        d.owner[slot] = st;
        d.released[slot] = false;
    }
    *partials = d.partials + (size_t)slot * xhip::kSplitPartialFloats;
    *partial_floats = xhip::kSplitPartialFloats;
    *counters = d.counters + (size_t)slot * xhip::kSplitCounters;
    *ncounters = xhip::kSplitCounters;
    return true;
}


// Gives the split-K slot of `st` on the current device back (its counters
// are zero once the stream's work has finished).
void splitk_release(hipStream_t st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return;
    std::lock_guard<std::mutex> lock(g_mu);
    DevSlots& d = g_devs[dev];
    for (int i = 0; i < d.nused; ++i)
        if (d.owner[i] == st && !d.released[i]) {
            d.released[i] = true;
            d.owner[i] = nullptr;
        }
}

}  // namespace xhip_host
