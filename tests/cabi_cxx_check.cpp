// Compile/link check of the C++ interface (no GPU calls): exercises the
// argument-validation paths, which return before any device work.
#include <cstdio>

#include "xinfer_hip/xinfer_artifact.hpp"
#include "xinfer_hip/xinfer_ops.hpp"

int main(int argc, char** argv) {
    using namespace xinfer::ops;
    int failures = 0;
    // empty shape: silent no-op, as src/ops/linear.cpp:176
    linear_int4(nullptr, (xinfer::half*)nullptr, (const xinfer::half*)nullptr, nullptr, nullptr,
                nullptr, 0, 16, 128);
    try {  // unsupported group size
        linear_int4(nullptr, (float*)0x1000, (const xinfer::half*)0x1000, (const uint8_t*)0x1000,
                    (const xinfer::half*)0x1000, nullptr, 1, 16, 128, 64);
        ++failures;
    } catch (const Error& e) {
        if (e.status != XINFER_ERR_UNSUPPORTED) ++failures;
    }
    try {  // too many fused descriptors
        FusedProjectionDesc d[5];
        linear_int4_fused(nullptr, (const xinfer::half*)0x1000, d, 5, 1, 128);
        ++failures;
    } catch (const Error& e) {
        if (e.status != XINFER_ERR_INVALID_ARG) ++failures;
    }
    // the fused neighbours of the projections: empty shapes are no-ops, bad
    // arguments are rejected before any device work
    rmsnorm(nullptr, nullptr, nullptr, nullptr, 0, 5120, 1e-6f);
    add_inplace(nullptr, nullptr, nullptr, 0);
    linear_int4_residual(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 16, 128);
    try {  // rmsnorm + projection without a norm weight
        FusedProjectionDesc d[1];
        rmsnorm_linear_int4_fused(nullptr, (const xinfer::half*)0x1000, nullptr, 1e-6f, d, 1, 1, 128);
        ++failures;
    } catch (const Error& e) {
        if (e.status != XINFER_ERR_INVALID_ARG) ++failures;
    }
    try {  // unsupported group size
        rmsnorm_mlp_gate_up_swiglu_int4(nullptr, (xinfer::half*)0x1000, (const xinfer::half*)0x1000,
                                        (const float*)0x1000, 1e-6f, (const uint8_t*)0x1000,
                                        (const xinfer::half*)0x1000, (const uint8_t*)0x1000,
                                        (const xinfer::half*)0x1000, 1, 16, 128, 64);
        ++failures;
    } catch (const Error& e) {
        if (e.status != XINFER_ERR_UNSUPPORTED) ++failures;
    }
    if (argmax_scratch_size(4097, 1) != 16) ++failures;
    LinearWeightView v;  // weights.h:13-23 defaults
    if (v.is_valid() || v.group_size != 128) ++failures;
    v.d_weights_int4 = (void*)0x1000;
    v.d_scales = (void*)0x2000;
    if (!v.is_valid()) ++failures;
    // artifact reader mirror (reader.h names) on a reference-written file
    if (xinfer::artifact::Crc64::calculate("123456789", 9) != 0x995DC9BBDF1939FAULL) ++failures;
    if (argc > 1) {
        xinfer::artifact::ArtifactReader r;
        std::string err;
        if (!r.open(argv[1], &err) || !r.validate_checksum(&err)) ++failures;
        const auto names = r.list_sections();
        if (names.empty() || !r.has_section(names[0]) || r.has_section("no.such")) ++failures;
        std::vector<uint8_t> data;
        if (!r.read_section(names[0], data, &err) || data.size() != r.get_section_info(names[0])->size)
            ++failures;
        if (r.header().section_count != names.size()) ++failures;
        xinfer::artifact::ArtifactReader bad;
        if (bad.open("/nonexistent.xinfer", &err) || err.find("Could not open file") != 0) ++failures;
    }
    std::printf("%s\n", failures ? "FAIL" : "OK");
    return failures;
}
