// .xinfer container reader with device upload and GPU-side CRC-64 checks.
//
// Follows the reference reader (src/artifact/reader.cpp:56-318) check for
// check: header magic, format version, header size, total file size, footer
// magic, metadata bounds, section-table size and bounds, per-section bounds;
// section payloads carry a CRC-64 in the section table and the file carries
// one over every byte before the footer (container.h:35-63).  Host reads use
// pread on one descriptor (no shared stream position, so distinct sections
// can be read from several threads).  A device upload streams the section
// through two pinned staging buffers (read of chunk i+1 overlaps the copy of
// chunk i) and then checks the CRC-64 of the device copy with
// xinfer_crc64_device, so the weights are verified where they will be used.

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "../../include/xinfer_hip/xinfer_artifact.h"

namespace xhip_host {
uint64_t crc64_host_buffer(const void* data, size_t n);  // crc64.hip
bool crc64_host_fd(int fd, uint64_t n, uint64_t* out);
}  // namespace xhip_host

namespace {

const uint8_t kMagic[8] = {'X', 'I', 'N', 'F', 'E', 'R', 0, 0};        // container.h:11
const uint8_t kFooterMagic[8] = {'X', 'I', 'N', 'F', 'F', 'O', 'O', 'T'};  // container.h:14
constexpr uint32_t kFormatVersion = 1;                                    // container.h:16
constexpr size_t kHeaderBytes = 64;
constexpr size_t kEntryBytes = 128;
constexpr size_t kFooterBytes = 16;
constexpr size_t kStageBytes = 32u << 20;  // pinned staging buffer (x2)

static_assert(sizeof(xinfer_file_header) == kHeaderBytes, "header layout");
static_assert(sizeof(xinfer_section_info) == kEntryBytes, "section entry layout");

void set_err(char* err, size_t len, const std::string& msg) {
    if (!err || len == 0) return;
    const size_t n = msg.size() < len - 1 ? msg.size() : len - 1;
    memcpy(err, msg.data(), n);
    err[n] = 0;
}

bool pread_all(int fd, void* dst, size_t n, uint64_t off) {
    uint8_t* p = static_cast<uint8_t*>(dst);
    while (n > 0) {
        const ssize_t got = pread(fd, p, n, (off_t)off);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return false;
        p += got;
        n -= (size_t)got;
        off += (uint64_t)got;
    }
    return true;
}

}  // namespace

struct xinfer_artifact {
    int fd = -1;
    uint64_t file_size = 0;
    xinfer_file_header hdr{};
    uint64_t footer_crc = 0;
    std::string meta;
    std::vector<xinfer_section_info> secs;
    std::unordered_map<std::string, size_t> index;
    // device upload state (created on first upload)
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t stage_done[2] = {nullptr, nullptr};
    uint64_t* crc_host = nullptr;  // pinned
    void* d_scratch = nullptr;     // CRC scratch + result slot
    size_t d_scratch_bytes = 0;
    int d_scratch_dev = -1;

    ~xinfer_artifact() {
        for (int i = 0; i < 2; ++i) {
            if (stage_done[i]) (void)hipEventDestroy(stage_done[i]);
            if (stage[i]) (void)hipHostFree(stage[i]);
        }
        if (crc_host) (void)hipHostFree(crc_host);
        if (d_scratch) {
            int cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(d_scratch_dev);
            (void)hipFree(d_scratch);
            (void)hipSetDevice(cur);
        }
        if (fd >= 0) close(fd);
    }

    const xinfer_section_info* find(const char* name) const {
        if (!name) return nullptr;
        auto it = index.find(name);
        return it == index.end() ? nullptr : &secs[it->second];
    }
};

namespace {

int fail(xinfer_artifact* a, char* err, size_t len, const std::string& msg) {
    delete a;
    set_err(err, len, msg);
    return XINFER_ERR_IO;
}

std::string hex64(uint64_t v) {
    char b[32];
    snprintf(b, sizeof(b), "0x%016llx", (unsigned long long)v);
    return b;
}

}  // namespace

extern "C" {

static int artifact_open_impl(const char* filepath, xinfer_artifact** out, char* err, size_t err_len) {
    *out = nullptr;
    xinfer_artifact* a = new xinfer_artifact();
    a->fd = open(filepath, O_RDONLY | O_CLOEXEC);
    if (a->fd < 0) return fail(a, err, err_len, std::string("Could not open file: ") + filepath);
    struct stat st;
    if (fstat(a->fd, &st) != 0) return fail(a, err, err_len, std::string("Could not stat file: ") + filepath);
    a->file_size = (uint64_t)st.st_size;
    const uint64_t fsize = a->file_size;
    if (fsize < kHeaderBytes + kFooterBytes)
        return fail(a, err, err_len, "File is smaller than minimum required header and footer size.");
    // 1. header (reader.cpp:79-113)
    if (!pread_all(a->fd, &a->hdr, kHeaderBytes, 0)) return fail(a, err, err_len, "Failed to read container header.");
    if (memcmp(a->hdr.magic, kMagic, 8) != 0)
        return fail(a, err, err_len, "Invalid file magic; not a .xinfer artifact.");
    if (a->hdr.format_version != kFormatVersion)
        return fail(a, err, err_len,
                    "Unsupported .xinfer format version: " + std::to_string(a->hdr.format_version));
    if (a->hdr.header_size != kHeaderBytes)
        return fail(a, err, err_len, "Corrupted header size field: " + std::to_string(a->hdr.header_size));
    if (a->hdr.total_file_size != fsize)
        return fail(a, err, err_len,
                    "File size mismatch: header expects " + std::to_string(a->hdr.total_file_size) +
                        " bytes, actual on disk is " + std::to_string(fsize) + " bytes.");
    // 2. footer (reader.cpp:115-128)
    uint8_t foot[kFooterBytes];
    if (!pread_all(a->fd, foot, kFooterBytes, fsize - kFooterBytes))
        return fail(a, err, err_len, "Failed to read container footer.");
    if (memcmp(foot + 8, kFooterMagic, 8) != 0)
        return fail(a, err, err_len, "Invalid footer magic; file may be corrupted or truncated.");
    memcpy(&a->footer_crc, foot, 8);
    // 3. metadata (reader.cpp:130-151)
    if (a->hdr.metadata_size > 0) {
        if (a->hdr.metadata_offset + a->hdr.metadata_size > fsize ||
            a->hdr.metadata_offset + a->hdr.metadata_size < a->hdr.metadata_offset)
            return fail(a, err, err_len, "Metadata offset/size points out of bounds.");
        a->meta.resize(a->hdr.metadata_size);
        if (!pread_all(a->fd, &a->meta[0], a->hdr.metadata_size, a->hdr.metadata_offset))
            return fail(a, err, err_len, "Failed reading metadata block.");
    }
    // 4. section table (reader.cpp:153-190)
    if (a->hdr.section_count > 0) {
        const uint64_t expect = (uint64_t)a->hdr.section_count * kEntryBytes;
        if (a->hdr.section_table_size != expect)
            return fail(a, err, err_len, "Section table size does not match section count.");
        if (a->hdr.section_table_offset + a->hdr.section_table_size > fsize ||
            a->hdr.section_table_offset + a->hdr.section_table_size < a->hdr.section_table_offset)
            return fail(a, err, err_len, "Section table points out of bounds.");
        a->secs.resize(a->hdr.section_count);
        if (!pread_all(a->fd, a->secs.data(), expect, a->hdr.section_table_offset))
            return fail(a, err, err_len, "Failed reading section table.");
        for (size_t i = 0; i < a->secs.size(); ++i) {
            xinfer_section_info& e = a->secs[i];
            e.name[sizeof(e.name) - 1] = 0;  // names are NUL-terminated within 96 bytes
            const std::string name(e.name);
            if (e.offset + e.size > fsize || e.offset + e.size < e.offset)
                return fail(a, err, err_len, "Section '" + name + "' offset + size points out of bounds.");
            a->index[name] = i;  // a repeated name maps to its last entry, as reader.cpp:189
        }
    }
    *out = a;
    return XINFER_OK;
}

// No C++ exception leaves the C ABI: a failed allocation while reading a
// (possibly crafted) header becomes an I/O error.
int xinfer_artifact_open(const char* filepath, xinfer_artifact** out, char* err, size_t err_len) {
    if (!filepath || !out) return XINFER_ERR_INVALID_ARG;
    *out = nullptr;
    try {
        return artifact_open_impl(filepath, out, err, err_len);
    } catch (...) {
        if (err && err_len) snprintf(err, err_len, "%s", "Out of memory while reading the container.");
        return XINFER_ERR_IO;
    }
}

void xinfer_artifact_close(xinfer_artifact* a) { delete a; }

int xinfer_artifact_header(const xinfer_artifact* a, xinfer_file_header* out) {
    if (!a || !out) return XINFER_ERR_INVALID_ARG;
    *out = a->hdr;
    return XINFER_OK;
}

int xinfer_artifact_footer(const xinfer_artifact* a, uint64_t* file_checksum) {
    if (!a || !file_checksum) return XINFER_ERR_INVALID_ARG;
    *file_checksum = a->footer_crc;
    return XINFER_OK;
}

const char* xinfer_artifact_metadata_json(const xinfer_artifact* a, size_t* length) {
    if (!a) {
        if (length) *length = 0;
        return nullptr;
    }
    if (length) *length = a->meta.size();
    return a->meta.data();
}

int32_t xinfer_artifact_section_count(const xinfer_artifact* a) { return a ? (int32_t)a->secs.size() : 0; }

int xinfer_artifact_section_at(const xinfer_artifact* a, int32_t index, xinfer_section_info* out) {
    if (!a || !out || index < 0 || (size_t)index >= a->secs.size()) return XINFER_ERR_INVALID_ARG;
    *out = a->secs[(size_t)index];
    return XINFER_OK;
}

int xinfer_artifact_section_by_name(const xinfer_artifact* a, const char* name, xinfer_section_info* out) {
    if (!a || !out) return XINFER_ERR_INVALID_ARG;
    const xinfer_section_info* e = a->find(name);
    if (!e) return XINFER_ERR_INVALID_ARG;
    *out = *e;
    return XINFER_OK;
}

int xinfer_artifact_read_section(xinfer_artifact* a, const char* name, void* dst, size_t dst_bytes,
                                 char* err, size_t err_len) {
    if (!a) return XINFER_ERR_INVALID_ARG;
    const xinfer_section_info* e = a->find(name);
    if (!e) {
        set_err(err, err_len, std::string("Section not found: ") + (name ? name : "(null)"));
        return XINFER_ERR_INVALID_ARG;
    }
    if (dst_bytes < e->size) {
        set_err(err, err_len, std::string("Destination buffer too small for section: ") + name);
        return XINFER_ERR_INVALID_ARG;
    }
    if (e->size == 0) return XINFER_OK;
    if (!dst) return XINFER_ERR_INVALID_ARG;
    if (!pread_all(a->fd, dst, e->size, e->offset)) {
        set_err(err, err_len, std::string("I/O error while reading section: ") + name);
        return XINFER_ERR_IO;
    }
    const uint64_t crc = xhip_host::crc64_host_buffer(dst, e->size);
    if (crc != e->checksum) {
        set_err(err, err_len, std::string("Checksum mismatch for section: ") + name + " (expected: " +
                                  std::to_string(e->checksum) + ", got: " + std::to_string(crc) + ")");
        return XINFER_ERR_CHECKSUM;
    }
    return XINFER_OK;
}

int xinfer_artifact_validate_checksum(xinfer_artifact* a, char* err, size_t err_len) {
    if (!a) return XINFER_ERR_INVALID_ARG;
    uint64_t crc = 0;
    if (!xhip_host::crc64_host_fd(a->fd, a->hdr.total_file_size - kFooterBytes, &crc)) {
        set_err(err, err_len, "Premature EOF while validating file checksum.");
        return XINFER_ERR_IO;
    }
    if (crc != a->footer_crc) {
        set_err(err, err_len, "File trailing checksum mismatch! (expected: " + hex64(a->footer_crc) +
                                  ", got: " + hex64(crc) + ")");
        return XINFER_ERR_CHECKSUM;
    }
    return XINFER_OK;
}

int xinfer_artifact_upload_section(xinfer_artifact* a, const char* name, void* stream, void* d_dst,
                                   size_t dst_bytes, int verify, char* err, size_t err_len) {
    if (!a) return XINFER_ERR_INVALID_ARG;
    const xinfer_section_info* e = a->find(name);
    if (!e) {
        set_err(err, err_len, std::string("Section not found: ") + (name ? name : "(null)"));
        return XINFER_ERR_INVALID_ARG;
    }
    if (dst_bytes < e->size) {
        set_err(err, err_len, std::string("Destination buffer too small for section: ") + name);
        return XINFER_ERR_INVALID_ARG;
    }
    if (e->size == 0) return e->checksum == 0 ? XINFER_OK : XINFER_ERR_CHECKSUM;
    if (!d_dst) return XINFER_ERR_INVALID_ARG;
    if (verify && !xhip_host::aligned(d_dst, 16)) return XINFER_ERR_MISALIGNED;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (!a->stage[0]) {
        for (int i = 0; i < 2; ++i) {
            if (hipHostMalloc(&a->stage[i], kStageBytes, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&a->stage_done[i], hipEventDisableTiming) != hipSuccess) {
                set_err(err, err_len, "Could not allocate pinned staging buffers.");
                return XINFER_ERR_HIP;
            }
        }
        if (hipHostMalloc((void**)&a->crc_host, sizeof(uint64_t), hipHostMallocDefault) != hipSuccess)
            return XINFER_ERR_HIP;
    }
    // stream the payload through the two staging buffers
    uint64_t pos = 0;
    for (int i = 0; pos < e->size; ++i) {
        const int b = i & 1;
        const size_t len = (size_t)std::min<uint64_t>(kStageBytes, e->size - pos);
        if (i >= 2 && hipEventSynchronize(a->stage_done[b]) != hipSuccess) return XINFER_ERR_HIP;
        if (!pread_all(a->fd, a->stage[b], len, e->offset + pos)) {
            (void)hipStreamSynchronize(st);
            set_err(err, err_len, std::string("I/O error while reading section: ") + name);
            return XINFER_ERR_IO;
        }
        if (hipMemcpyAsync(static_cast<uint8_t*>(d_dst) + pos, a->stage[b], len, hipMemcpyHostToDevice, st) !=
                hipSuccess ||
            hipEventRecord(a->stage_done[b], st) != hipSuccess)
            return XINFER_ERR_HIP;
        pos += len;
    }
    if (verify) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        const size_t need = xinfer_crc64_device_scratch_bytes(e->size) + 256;
        if (a->d_scratch_bytes < need || a->d_scratch_dev != dev) {
            if (hipStreamSynchronize(st) != hipSuccess) return XINFER_ERR_HIP;
            if (a->d_scratch) (void)hipFree(a->d_scratch);
            a->d_scratch = nullptr;
            a->d_scratch_bytes = 0;
            if (hipMalloc(&a->d_scratch, need) != hipSuccess) return XINFER_ERR_HIP;
            a->d_scratch_bytes = need;
            a->d_scratch_dev = dev;
        }
        uint64_t* d_crc = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(a->d_scratch) + need - 256);
        const int rc = xinfer_crc64_device(stream, d_dst, e->size, d_crc, a->d_scratch, need - 256);
        if (rc) return rc;
        if (hipMemcpyAsync(a->crc_host, d_crc, sizeof(uint64_t), hipMemcpyDeviceToHost, st) != hipSuccess)
            return XINFER_ERR_HIP;
    }
    if (hipStreamSynchronize(st) != hipSuccess) return XINFER_ERR_HIP;
    if (verify && *a->crc_host != e->checksum) {
        set_err(err, err_len, std::string("Checksum mismatch for section: ") + name + " (expected: " +
                                  std::to_string(e->checksum) + ", got: " + std::to_string(*a->crc_host) + ")");
        return XINFER_ERR_CHECKSUM;
    }
    return XINFER_OK;
}

int xinfer_artifact_load_linear(xinfer_artifact* a, const char* weight_name, int64_t out_features,
                                int64_t in_features, int32_t group_size, void* stream,
                                xinfer_linear_weight_view* out, char* err, size_t err_len) {
    if (!a || !weight_name || !out) return XINFER_ERR_INVALID_ARG;
    if (group_size <= 0 || out_features <= 0 || in_features <= 0) return XINFER_ERR_INVALID_ARG;
    memset(out, 0, sizeof(*out));
    out->in_features = in_features;
    out->out_features = out_features;
    out->group_size = group_size;
    // expected sizes, weights.cpp:260-261
    const uint64_t w_bytes = (uint64_t)out_features * (uint64_t)(in_features / 2);
    const uint64_t s_bytes = (uint64_t)out_features * (uint64_t)(in_features / group_size) * 2u;
    const std::string wn(weight_name), sn = wn + ".scales";
    const xinfer_section_info* we = a->find(wn.c_str());
    const xinfer_section_info* se = a->find(sn.c_str());
    if (!we) {
        set_err(err, err_len, "Section not found: " + wn);
        return XINFER_ERR_INVALID_ARG;
    }
    if (we->size != w_bytes) {
        set_err(err, err_len, "Weight size mismatch for " + wn + ": expected " + std::to_string(w_bytes) +
                                  ", got " + std::to_string(we->size));
        return XINFER_ERR_IO;
    }
    if (!se) {
        set_err(err, err_len, "Section not found: " + sn);
        return XINFER_ERR_INVALID_ARG;
    }
    if (se->size != s_bytes) {
        set_err(err, err_len, "Scales size mismatch for " + sn + ": expected " + std::to_string(s_bytes) +
                                  ", got " + std::to_string(se->size));
        return XINFER_ERR_IO;
    }
    void* dw = nullptr;
    void* ds = nullptr;
    if (hipMalloc(&dw, w_bytes ? w_bytes : 1) != hipSuccess) return XINFER_ERR_HIP;
    if (hipMalloc(&ds, s_bytes ? s_bytes : 1) != hipSuccess) {
        (void)hipFree(dw);
        return XINFER_ERR_HIP;
    }
    int rc = xinfer_artifact_upload_section(a, wn.c_str(), stream, dw, w_bytes, 1, err, err_len);
    if (!rc) rc = xinfer_artifact_upload_section(a, sn.c_str(), stream, ds, s_bytes, 1, err, err_len);
    if (rc) {
        (void)hipFree(dw);
        (void)hipFree(ds);
        return rc;
    }
    out->d_weights_int4 = dw;
    out->d_scales = ds;
    return XINFER_OK;
}

}  // extern "C"
