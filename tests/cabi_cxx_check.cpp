// Compile/link check of the C++ interface (no GPU calls): exercises the
// argument-validation paths, which return before any device work.
#include <cstdio>

#include "xinfer_hip/xinfer_ops.hpp"

int main() {
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
    if (argmax_scratch_size(4097, 1) != 16) ++failures;
    LinearWeightView v;  // weights.h:13-23 defaults
    if (v.is_valid() || v.group_size != 128) ++failures;
    v.d_weights_int4 = (void*)0x1000;
    v.d_scales = (void*)0x2000;
    if (!v.is_valid()) ++failures;
    std::printf("%s\n", failures ? "FAIL" : "OK");
    return failures;
}
