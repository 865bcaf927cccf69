// CRC-64/ECMA-182 (reflected; init and final XOR all ones) on the host and on
// gfx950.  Same checksum as src/artifact/checksum.cpp:10-54.
//
// Both sides split the data into pieces, compute each piece's CRC register
// from zero, and join the pieces with the GF(2) combine of zlib's
// crc32_combine (Mark Adler): for register values (no init, no final XOR)
//     reg(A || B) = reg(A) * x^(8|B|) mod P  XOR  reg(B),
// where the product is a carry-less multiply modulo the CRC polynomial
// (multmodp) and x^(8n) mod P comes from repeated squaring (x2nmodp).
// A register run from init I over M equals x^(8|M|) * I XOR reg_0(M), so the
// standard CRC is  (x^(8N) * ~0  XOR  reg_0(data))  XOR  ~0.
//
// Device layout (verification of uploaded weight sections):
//   * the data (16-byte aligned) is split into a 16-byte-multiple head and a
//     < 16-byte tail.  The head is padded at the front with virtual zero bytes
//     to whole blocks of 128 KB: leading zeros leave a zero register
//     unchanged, so every unit and block has the same length and every
//     combine uses one precomputed constant per tree level.
//   * kernel 1: one 256-thread block per 128 KB; each thread runs
//     slicing-by-8 (8 tables of 256 entries in LDS) over 512 contiguous bytes,
//     then the block joins its 256 registers in an 8-level tree.
//   * kernel 2: one block of 1024 threads folds runs of block registers,
//     joins them in a 10-level tree, appends the tail bytes and applies the
//     init / final XOR terms.

#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <fcntl.h>
#include <sys/stat.h>

#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#include "common.h"
#include "../../include/xinfer_hip/xinfer_artifact.h"

namespace xcrc {

constexpr uint64_t kPoly = 0xC96C5795D7870F42ULL;  // reflected ECMA-182
constexpr int kUnit = 512;                         // bytes per thread
constexpr int kBlockThreads = 256;
constexpr int64_t kBlock = (int64_t)kUnit * kBlockThreads;  // 128 KB
constexpr int kFinalThreads = 1024;

// a * b mod P, reflected representation (bit 63 = x^0); 64 fixed steps.
__host__ __device__ inline uint64_t multmodp(uint64_t a, uint64_t b) {
    uint64_t p = 0;
    for (int i = 63; i >= 0; --i) {
        p ^= b & (0ULL - ((a >> i) & 1ULL));
        b = (b >> 1) ^ (kPoly & (0ULL - (b & 1ULL)));
    }
    return p;
}

// x^(2^k) mod P for k = 0..63
struct X2n {
    uint64_t t[64];
    X2n() {
        uint64_t p = 1ULL << 62;  // x^1
        t[0] = p;
        for (int k = 1; k < 64; ++k) t[k] = p = multmodp(p, p);
    }
};
inline const X2n& x2n() {
    static const X2n v;
    return v;
}

// x^(n * 2^k) mod P
inline uint64_t x2nmodp(uint64_t n, unsigned k) {
    uint64_t p = 1ULL << 63;  // x^0
    while (n) {
        if (n & 1) p = multmodp(x2n().t[k & 63], p);
        n >>= 1;
        ++k;
    }
    return p;
}

// register after processing n zero bytes from r
inline uint64_t shift_bytes(uint64_t r, uint64_t n) { return multmodp(x2nmodp(n, 3), r); }

struct Tables {
    uint64_t t[8][256];
    Tables() {
        for (int b = 0; b < 256; ++b) {
            uint64_t c = (uint64_t)b;
            for (int i = 0; i < 8; ++i) c = (c >> 1) ^ (kPoly & (0ULL - (c & 1ULL)));
            t[0][b] = c;
        }
        for (int k = 1; k < 8; ++k)
            for (int b = 0; b < 256; ++b) t[k][b] = (t[k - 1][b] >> 8) ^ t[0][t[k - 1][b] & 0xFF];
    }
};
inline const Tables& tables() {
    static const Tables v;
    return v;
}

// register update over n bytes (slicing-by-8 on 8-byte words)
uint64_t reg_update(uint64_t c, const uint8_t* p, size_t n) {
    const Tables& T = tables();
    while (n && ((uintptr_t)p & 7)) {
        c = (c >> 8) ^ T.t[0][(c ^ *p++) & 0xFF];
        --n;
    }
    while (n >= 8) {
        uint64_t w;
        memcpy(&w, p, 8);
        c ^= w;
        c = T.t[7][c & 0xFF] ^ T.t[6][(c >> 8) & 0xFF] ^ T.t[5][(c >> 16) & 0xFF] ^
            T.t[4][(c >> 24) & 0xFF] ^ T.t[3][(c >> 32) & 0xFF] ^ T.t[2][(c >> 40) & 0xFF] ^
            T.t[1][(c >> 48) & 0xFF] ^ T.t[0][c >> 56];
        p += 8;
        n -= 8;
    }
    while (n--) c = (c >> 8) ^ T.t[0][(c ^ *p++) & 0xFF];
    return c;
}

int host_threads() {
    unsigned n = std::thread::hardware_concurrency();
    if (n == 0) n = 1;
    return (int)std::min(16u, n);
}

// standard CRC of a host buffer; pieces of >= 8 MB run on host threads
uint64_t crc_buffer(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    const size_t min_piece = 8u << 20;
    int parts = (int)std::min<size_t>((size_t)host_threads(), n / min_piece);
    uint64_t reg0;
    if (parts <= 1) {
        reg0 = reg_update(0, p, n);
    } else {
        std::vector<uint64_t> r(parts);
        std::vector<size_t> b(parts + 1);
        for (int i = 0; i <= parts; ++i) b[i] = n * (size_t)i / (size_t)parts;
        std::vector<std::thread> th;
        for (int i = 0; i < parts; ++i)
            th.emplace_back([&, i] { r[i] = reg_update(0, p + b[i], b[i + 1] - b[i]); });
        for (auto& t : th) t.join();
        reg0 = r[0];
        for (int i = 1; i < parts; ++i) reg0 = shift_bytes(reg0, b[i + 1] - b[i]) ^ r[i];
    }
    return (shift_bytes(~0ULL, n) ^ reg0) ^ ~0ULL;
}

// standard CRC of bytes [0, n) of an open file; false on a short read
bool crc_fd(int fd, uint64_t n, uint64_t* out) {
    const uint64_t min_piece = 16u << 20;
    int parts = (int)std::max<uint64_t>(1, std::min<uint64_t>((uint64_t)host_threads(), n / min_piece));
    std::vector<uint64_t> r(parts, 0);
    std::vector<uint64_t> b(parts + 1);
    for (int i = 0; i <= parts; ++i) b[i] = n * (uint64_t)i / (uint64_t)parts;
    std::vector<int> ok(parts, 1);
    auto work = [&](int i) {
        const size_t chunk = 4u << 20;
        std::vector<uint8_t> buf(chunk);
        uint64_t c = 0, off = b[i];
        while (off < b[i + 1]) {
            const size_t len = (size_t)std::min<uint64_t>(chunk, b[i + 1] - off);
            const ssize_t got = pread(fd, buf.data(), len, (off_t)off);
            if (got != (ssize_t)len) {
                ok[i] = 0;
                return;
            }
            c = reg_update(c, buf.data(), len);
            off += len;
        }
        r[i] = c;
    };
    if (parts == 1) {
        work(0);
    } else {
        std::vector<std::thread> th;
        for (int i = 0; i < parts; ++i) th.emplace_back(work, i);
        for (auto& t : th) t.join();
    }
    uint64_t reg0 = 0;
    for (int i = 0; i < parts; ++i) {
        if (!ok[i]) return false;
        reg0 = shift_bytes(reg0, b[i + 1] - b[i]) ^ r[i];
    }
    *out = (shift_bytes(~0ULL, n) ^ reg0) ^ ~0ULL;
    return true;
}

// ------------------------------------------------------------- device ----

struct BlockParams {
    const uint8_t* data;  // 16-byte aligned
    int64_t head;         // bytes covered by the blocks (multiple of 16)
    int64_t pad;          // virtual zero bytes in front (multiple of 16)
    uint64_t* reg;        // [nblk] block registers
    uint64_t k_unit[8];   // x^(8 * kUnit * 2^l) mod P
};

struct FinalParams {
    const uint64_t* reg;
    const uint8_t* tail;  // last tail_len (< 16) bytes
    uint64_t* out;
    int32_t nblk;
    int32_t q;            // block registers per thread (after front padding)
    int32_t tail_len;
    int32_t pad;
    uint64_t k_blk;       // x^(8 * kBlock) mod P
    uint64_t k_tail;      // x^(8 * tail_len) mod P
    uint64_t init_term;   // x^(8N) * ~0 mod P
    uint64_t k_run[10];   // x^(8 * q * kBlock * 2^l) mod P
};

__device__ inline void build_tables(uint64_t (*T)[256]) {
    const int t = threadIdx.x;
    for (int b = t; b < 256; b += blockDim.x) {
        uint64_t c = (uint64_t)b;
        for (int i = 0; i < 8; ++i) c = (c >> 1) ^ (kPoly & (0ULL - (c & 1ULL)));
        T[0][b] = c;
    }
    __syncthreads();
    for (int k = 1; k < 8; ++k) {
        for (int b = t; b < 256; b += blockDim.x) T[k][b] = (T[k - 1][b] >> 8) ^ T[0][T[k - 1][b] & 0xFF];
        __syncthreads();
    }
}

__device__ inline uint64_t slice8(const uint64_t (*T)[256], uint64_t c, uint64_t w) {
    c ^= w;
    return T[7][c & 0xFF] ^ T[6][(c >> 8) & 0xFF] ^ T[5][(c >> 16) & 0xFF] ^ T[4][(c >> 24) & 0xFF] ^
           T[3][(c >> 32) & 0xFF] ^ T[2][(c >> 40) & 0xFF] ^ T[1][(c >> 48) & 0xFF] ^ T[0][c >> 56];
}

__global__ __launch_bounds__(kBlockThreads) void crc64_blocks_kernel(const BlockParams p) {
    __shared__ uint64_t T[8][256];
    __shared__ uint64_t red[kBlockThreads];
    build_tables(T);
    const int tid = threadIdx.x;
    const int64_t start = ((int64_t)blockIdx.x * kBlockThreads + tid) * kUnit - p.pad;
    uint64_t c = 0;
    if (start >= 0) {
        const xhip::u32x4* src = reinterpret_cast<const xhip::u32x4*>(p.data + start);
#pragma unroll 4
        for (int i = 0; i < kUnit / 16; ++i) {
            const xhip::u32x4 v = __builtin_nontemporal_load(src + i);
            c = slice8(T, c, ((uint64_t)v.y << 32) | v.x);
            c = slice8(T, c, ((uint64_t)v.w << 32) | v.z);
        }
    } else if (start + kUnit > 0) {  // the unit that straddles the front padding
        const int skip = (int)(-start) / 16;
        const xhip::u32x4* src = reinterpret_cast<const xhip::u32x4*>(p.data);
        for (int i = 0; i < kUnit / 16 - skip; ++i) {
            const xhip::u32x4 v = src[i];
            c = slice8(T, c, ((uint64_t)v.y << 32) | v.x);
            c = slice8(T, c, ((uint64_t)v.w << 32) | v.z);
        }
    }
    red[tid] = c;
    __syncthreads();
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        const int s = 1 << l;
        if ((tid & (2 * s - 1)) == 0) red[tid] = multmodp(p.k_unit[l], red[tid]) ^ red[tid + s];
        __syncthreads();
    }
    if (tid == 0) p.reg[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(kFinalThreads) void crc64_final_kernel(const FinalParams p) {
    __shared__ uint64_t red[kFinalThreads];
    const int tid = threadIdx.x;
    const int lead = kFinalThreads * p.q - p.nblk;  // virtual zero blocks in front
    uint64_t c = 0;
    for (int i = 0; i < p.q; ++i) {
        const int v = tid * p.q + i - lead;
        const uint64_t r = v >= 0 ? p.reg[v] : 0ULL;
        c = multmodp(p.k_blk, c) ^ r;
    }
    red[tid] = c;
    __syncthreads();
#pragma unroll
    for (int l = 0; l < 10; ++l) {
        const int s = 1 << l;
        if ((tid & (2 * s - 1)) == 0) red[tid] = multmodp(p.k_run[l], red[tid]) ^ red[tid + s];
        __syncthreads();
    }
    if (tid == 0) {
        uint64_t r = multmodp(p.k_tail, red[0]);
        uint64_t t = 0;
        for (int i = 0; i < p.tail_len; ++i) {
            t ^= p.tail[i];
            for (int j = 0; j < 8; ++j) t = (t >> 1) ^ (kPoly & (0ULL - (t & 1ULL)));
        }
        r ^= t;
        p.out[0] = (r ^ p.init_term) ^ ~0ULL;
    }
}

int64_t device_blocks(size_t length) {
    const int64_t head = (int64_t)(length & ~(size_t)15);
    return (head + kBlock - 1) / kBlock;
}

std::mutex g_scratch_mu;
void* g_scratch[64] = {nullptr};
size_t g_scratch_cap[64] = {0};

void* library_scratch(size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_cap[dev] < bytes) {
        const size_t want = std::max<size_t>(bytes, 64 * 1024);
        void* ptr = nullptr;
        if (hipMalloc(&ptr, want) != hipSuccess) return nullptr;
        g_scratch[dev] = ptr;  // an older buffer may still be read by queued work: kept
        g_scratch_cap[dev] = want;
    }
    return g_scratch[dev];
}

}  // namespace xcrc

namespace xhip_host {
uint64_t crc64_host_buffer(const void* data, size_t n) { return xcrc::crc_buffer(data, n); }
bool crc64_host_fd(int fd, uint64_t n, uint64_t* out) { return xcrc::crc_fd(fd, n, out); }
}  // namespace xhip_host

extern "C" {

uint64_t xinfer_crc64(const void* data, size_t length) {
    if (!data || length == 0) return 0ULL;
    return xcrc::crc_buffer(data, length);
}

uint64_t xinfer_crc64_file(const char* filepath, uint64_t max_bytes) {
    if (!filepath) return 0ULL;
    const int fd = open(filepath, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return 0ULL;
    struct stat st;
    uint64_t out = 0;
    if (fstat(fd, &st) == 0) {
        const uint64_t len = (uint64_t)st.st_size;
        const uint64_t n = (max_bytes > 0 && max_bytes < len) ? max_bytes : len;
        if (!xcrc::crc_fd(fd, n, &out)) out = 0;
    }
    close(fd);
    return out;
}

size_t xinfer_crc64_device_scratch_bytes(size_t length) {
    const int64_t nblk = xcrc::device_blocks(length);
    return (size_t)std::max<int64_t>(nblk, 1) * sizeof(uint64_t);
}

int xinfer_crc64_device(void* stream, const void* d_data, size_t length, uint64_t* d_crc,
                        void* scratch, size_t scratch_bytes) {
    using namespace xcrc;
    if (!d_crc || (length > 0 && !d_data)) return XINFER_ERR_INVALID_ARG;
    if (!xhip_host::aligned(d_data, 16) || !xhip_host::aligned(d_crc, 8)) return XINFER_ERR_MISALIGNED;
    const int64_t nblk = device_blocks(length);
    const size_t need = xinfer_crc64_device_scratch_bytes(length);
    if (!scratch) {
        scratch = library_scratch(need);
        if (!scratch) return XINFER_ERR_SCRATCH;
    } else if (scratch_bytes < need || !xhip_host::aligned(scratch, 8)) {
        return XINFER_ERR_SCRATCH;
    }
    if (nblk > (int64_t)kFinalThreads * (1 << 20)) return XINFER_ERR_UNSUPPORTED;  // > 128 TiB
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t head = (int64_t)(length & ~(size_t)15);
    BlockParams bp = {};
    bp.data = static_cast<const uint8_t*>(d_data);
    bp.head = head;
    bp.pad = nblk * kBlock - head;
    bp.reg = static_cast<uint64_t*>(scratch);
    for (int l = 0; l < 8; ++l) bp.k_unit[l] = x2nmodp((uint64_t)kUnit << l, 3);
    if (nblk > 0) {
        hipLaunchKernelGGL(crc64_blocks_kernel, dim3((unsigned)nblk), dim3(kBlockThreads), 0, st, bp);
        if (xhip_host::launch_status()) return XINFER_ERR_HIP;
    }
    FinalParams fp = {};
    fp.reg = bp.reg;
    fp.tail = static_cast<const uint8_t*>(d_data) + head;
    fp.out = d_crc;
    fp.nblk = (int32_t)nblk;
    fp.q = (int32_t)std::max<int64_t>(1, (nblk + kFinalThreads - 1) / kFinalThreads);
    fp.tail_len = (int32_t)(length - (size_t)head);
    fp.k_blk = x2nmodp((uint64_t)kBlock, 3);
    fp.k_tail = x2nmodp((uint64_t)fp.tail_len, 3);
    fp.init_term = multmodp(x2nmodp((uint64_t)length, 3), ~0ULL);
    for (int l = 0; l < 10; ++l) fp.k_run[l] = x2nmodp((uint64_t)fp.q * (uint64_t)kBlock << l, 3);
    hipLaunchKernelGGL(crc64_final_kernel, dim3(1), dim3(kFinalThreads), 0, st, fp);
    return xhip_host::launch_status();
}

}  // extern "C"
