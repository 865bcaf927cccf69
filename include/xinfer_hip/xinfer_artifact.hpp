// C++ mirror of the reference's artifact reader over the C-ABI of
// xinfer_artifact.h: same namespace, class and method names as
// src/artifact/reader.h:12-61 and src/artifact/checksum.h:9-21, so runtime
// code written against them compiles unchanged, plus upload_section and
// load_linear for device residency (weights.cpp:252-303).
#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "xinfer_artifact.h"
#include "xinfer_ops.hpp"

namespace xinfer::artifact {

using FileHeader = xinfer_file_header;     // container.h:35-47
using SectionEntry = xinfer_section_info;  // container.h:50-58

// checksum.h:9-21 (one-shot form; the streaming form is not needed here)
struct Crc64 {
    static uint64_t calculate(const void* data, size_t length) { return xinfer_crc64(data, length); }
};

class ArtifactReader {
public:
    ArtifactReader() = default;
    ~ArtifactReader() { close(); }
    ArtifactReader(const ArtifactReader&) = delete;
    ArtifactReader& operator=(const ArtifactReader&) = delete;
    ArtifactReader(ArtifactReader&& o) noexcept : a_(o.a_) { o.a_ = nullptr; }
    ArtifactReader& operator=(ArtifactReader&& o) noexcept {
        if (this != &o) {
            close();
            a_ = o.a_;
            o.a_ = nullptr;
        }
        return *this;
    }

    bool open(const std::string& filepath, std::string* error_msg = nullptr) {
        close();
        char err[1024] = {0};
        const int rc = xinfer_artifact_open(filepath.c_str(), &a_, err, sizeof(err));
        if (rc && error_msg) *error_msg = err;
        return rc == XINFER_OK;
    }
    void close() {
        xinfer_artifact_close(a_);
        a_ = nullptr;
    }
    bool is_open() const { return a_ != nullptr; }

    FileHeader header() const {
        FileHeader h{};
        xinfer_artifact_header(a_, &h);
        return h;
    }
    uint64_t footer_checksum() const {
        uint64_t v = 0;
        xinfer_artifact_footer(a_, &v);
        return v;
    }
    std::string raw_metadata_json() const {
        size_t n = 0;
        const char* p = xinfer_artifact_metadata_json(a_, &n);
        return p ? std::string(p, n) : std::string();
    }

    std::vector<std::string> list_sections() const {
        std::vector<std::string> v;
        for (int32_t i = 0; i < xinfer_artifact_section_count(a_); ++i) {
            SectionEntry e{};
            if (xinfer_artifact_section_at(a_, i, &e) == XINFER_OK) v.emplace_back(e.name);
        }
        return v;
    }
    bool has_section(const std::string& name) const { return get_section_info(name).has_value(); }
    std::optional<SectionEntry> get_section_info(const std::string& name) const {
        SectionEntry e{};
        if (xinfer_artifact_section_by_name(a_, name.c_str(), &e) != XINFER_OK) return std::nullopt;
        return e;
    }

    bool read_section(const std::string& name, std::vector<uint8_t>& out_data, std::string* error_msg = nullptr) {
        auto info = get_section_info(name);
        if (!info) {
            if (error_msg) *error_msg = "Section not found: " + name;
            return false;
        }
        out_data.resize(info->size);
        return read_section(name, out_data.data(), out_data.size(), error_msg);
    }
    bool read_section(const std::string& name, void* dst_buffer, size_t buffer_size,
                      std::string* error_msg = nullptr) {
        char err[1024] = {0};
        const int rc = xinfer_artifact_read_section(a_, name.c_str(), dst_buffer, buffer_size, err, sizeof(err));
        if (rc && error_msg) *error_msg = err;
        return rc == XINFER_OK;
    }
    bool validate_checksum(std::string* error_msg = nullptr) {
        char err[1024] = {0};
        const int rc = xinfer_artifact_validate_checksum(a_, err, sizeof(err));
        if (rc && error_msg) *error_msg = err;
        return rc == XINFER_OK;
    }

    // Section straight into device memory, CRC-64 checked on the GPU.
    bool upload_section(const std::string& name, hipStream_t stream, void* d_dst, size_t dst_bytes,
                        bool verify = true, std::string* error_msg = nullptr) {
        char err[1024] = {0};
        const int rc = xinfer_artifact_upload_section(a_, name.c_str(), stream, d_dst, dst_bytes, verify ? 1 : 0,
                                                      err, sizeof(err));
        if (rc && error_msg) *error_msg = err;
        return rc == XINFER_OK;
    }

    // weights.cpp:252-303: `<name>` and `<name>.scales` into new device
    // allocations (release with hipFree); an invalid view on failure.
    ops::LinearWeightView load_linear(const std::string& weight_name, int64_t out_f, int64_t in_f,
                                      int group_size = 128, hipStream_t stream = nullptr,
                                      std::string* error_msg = nullptr) {
        xinfer_linear_weight_view v{};
        char err[1024] = {0};
        ops::LinearWeightView out;
        out.in_features = in_f;
        out.out_features = out_f;
        out.group_size = group_size;
        const int rc = xinfer_artifact_load_linear(a_, weight_name.c_str(), out_f, in_f, group_size, stream, &v,
                                                   err, sizeof(err));
        if (rc) {
            if (error_msg) *error_msg = err;
            return out;
        }
        out.d_weights_int4 = v.d_weights_int4;
        out.d_scales = v.d_scales;
        return out;
    }

    xinfer_artifact* handle() const { return a_; }

private:
    xinfer_artifact* a_ = nullptr;
};

}  // namespace xinfer::artifact
