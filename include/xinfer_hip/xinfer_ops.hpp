// xinfer_hip C++ host interface: the reference's `xinfer::ops` projection
// entry points (src/ops/linear.h, src/ops/sampling.h) with the same names,
// overload set, argument order and meaning, implemented on the C-ABI of
// xinfer_ops.h.  Differences from the reference signatures:
//   * `sycl::queue&` -> `hipStream_t` (any pointer-sized stream handle works);
//   * `sycl::half`   -> `xinfer::half` (a 16-bit IEEE binary16 storage type);
//   * return type    -> `void`; failures throw `xinfer::ops::Error` carrying
//     the status code (the reference returned an empty sycl::event for
//     M, N, K <= 0 -- still a silent no-op here -- and had no error reporting).
// Everything is asynchronous on the stream except argmax(), which, like the
// reference (src/ops/sampling.cpp:17-92), blocks and returns the token id.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "xinfer_ops.h"

typedef struct ihipStream_t* hipStream_t;

namespace xinfer {

struct half {
    uint16_t bits;
};

namespace ops {

struct Error : std::runtime_error {
    int status;
    Error(const char* fn, int st)
        : std::runtime_error(std::string(fn) + ": " + xinfer_status_string(st)), status(st) {}
};

namespace detail {
inline void check(const char* fn, int st) {
    if (st != XINFER_OK) throw Error(fn, st);
}
inline void* q(hipStream_t s) { return reinterpret_cast<void*>(s); }
}  // namespace detail

// src/ops/linear.h:30-39  FP16 in -> FP16 out
inline void linear_int4(hipStream_t s, half* Y, const half* X, const uint8_t* W_int4,
                        const half* scales, const float* bias, int64_t M, int64_t N, int64_t K,
                        int group_size = 128) {
    detail::check("linear_int4", xinfer_linear_int4_f16(detail::q(s), Y, X, W_int4, scales, bias,
                                                        M, N, K, group_size));
}

// src/ops/linear.h:42-51  FP16 in -> FP32 out (LM-head logits)
inline void linear_int4(hipStream_t s, float* Y, const half* X, const uint8_t* W_int4,
                        const half* scales, const float* bias, int64_t M, int64_t N, int64_t K,
                        int group_size = 128) {
    detail::check("linear_int4", xinfer_linear_int4_f16_f32out(detail::q(s), Y, X, W_int4, scales,
                                                               bias, M, N, K, group_size));
}

// src/ops/linear.h:54-63  FP32 in -> FP32 out (oracle testing)
inline void linear_int4(hipStream_t s, float* Y, const float* X, const uint8_t* W_int4,
                        const half* scales, const float* bias, int64_t M, int64_t N, int64_t K,
                        int group_size = 128) {
    detail::check("linear_int4", xinfer_linear_int4_f32(detail::q(s), Y, X, W_int4, scales, bias,
                                                        M, N, K, group_size));
}

// src/targets/qwen3_8_27b/weights.h:13-23: what the runtime hands to the
// projections (device pointers of a `.xinfer` weight and its scales).
struct LinearWeightView {
    void* d_weights_int4{nullptr};  // packed INT4 [out_features][in_features / 2]
    void* d_scales{nullptr};        // fp16 [out_features][in_features / group_size]
    int64_t in_features{0};
    int64_t out_features{0};
    int group_size{128};

    bool is_valid() const noexcept { return d_weights_int4 != nullptr && d_scales != nullptr; }
};

// src/ops/linear.h:66-81
struct FusedProjectionDesc {
    half* Y{nullptr};
    const uint8_t* W_int4{nullptr};
    const half* scales{nullptr};
    const float* bias{nullptr};
    int64_t N{0};
};
struct FusedProjectionDescFP32 {
    float* Y{nullptr};
    const uint8_t* W_int4{nullptr};
    const half* scales{nullptr};
    const float* bias{nullptr};
    int64_t N{0};
};

namespace detail {
template <typename D>
inline std::vector<xinfer_fused_desc> to_c(const D* descs, int n) {
    std::vector<xinfer_fused_desc> v;
    for (int i = 0; descs && i < n && i < 4; ++i)
        v.push_back(xinfer_fused_desc{descs[i].Y, descs[i].W_int4, descs[i].scales, descs[i].bias,
                                      descs[i].N});
    return v;
}
}  // namespace detail

// src/ops/linear.h:97-103
inline void linear_int4_fused(hipStream_t s, const half* X, const FusedProjectionDesc* descs,
                              int num_descs, int64_t M, int64_t K, int group_size = 128) {
    auto v = detail::to_c(descs, num_descs);
    detail::check("linear_int4_fused",
                  xinfer_linear_int4_fused_f16(detail::q(s), X, descs ? v.data() : nullptr,
                                               num_descs, M, K, group_size));
}

// src/ops/linear.h:105-111
inline void linear_int4_fused(hipStream_t s, const float* X, const FusedProjectionDescFP32* descs,
                              int num_descs, int64_t M, int64_t K, int group_size = 128) {
    auto v = detail::to_c(descs, num_descs);
    detail::check("linear_int4_fused",
                  xinfer_linear_int4_fused_f32(detail::q(s), X, descs ? v.data() : nullptr,
                                               num_descs, M, K, group_size));
}

// src/ops/linear.h:117-127
inline void mlp_gate_up_swiglu_int4(hipStream_t s, half* Y, const half* X, const uint8_t* W_gate,
                                    const half* scales_gate, const uint8_t* W_up,
                                    const half* scales_up, int64_t M, int64_t N, int64_t K,
                                    int group_size = 128) {
    detail::check("mlp_gate_up_swiglu_int4",
                  xinfer_mlp_gate_up_swiglu_int4_f16(detail::q(s), Y, X, W_gate, scales_gate, W_up,
                                                     scales_up, M, N, K, group_size));
}

// src/ops/linear.h:129-139
inline void mlp_gate_up_swiglu_int4(hipStream_t s, float* Y, const float* X, const uint8_t* W_gate,
                                    const half* scales_gate, const uint8_t* W_up,
                                    const half* scales_up, int64_t M, int64_t N, int64_t K,
                                    int group_size = 128) {
    detail::check("mlp_gate_up_swiglu_int4",
                  xinfer_mlp_gate_up_swiglu_int4_f32(detail::q(s), Y, X, W_gate, scales_gate, W_up,
                                                     scales_up, M, N, K, group_size));
}

// src/ops/linear.h:159-168
inline void linear_int4_naive(hipStream_t s, float* Y, const float* X, const uint8_t* W_int4,
                              const half* scales, const float* bias, int64_t M, int64_t N,
                              int64_t K, int group_size = 128) {
    detail::check("linear_int4_naive", xinfer_linear_int4_naive_f32(detail::q(s), Y, X, W_int4,
                                                                    scales, bias, M, N, K,
                                                                    group_size));
}

// src/ops/rmsnorm.h:17-23 (fp16 activations, fp32 weight)
inline void rmsnorm(hipStream_t s, half* out, const half* in, const float* weight, int64_t num_tokens,
                    int64_t hidden_size, float eps) {
    detail::check("rmsnorm", xinfer_rmsnorm_f16(detail::q(s), out, in, weight, num_tokens, hidden_size, eps));
}

// src/ops/elementwise.h:22 (fp16)
inline void add_inplace(hipStream_t s, half* a, const half* b, int64_t num_elements) {
    detail::check("add_inplace", xinfer_add_inplace_f16(detail::q(s), a, b, num_elements));
}

// Workspace bytes of the two rmsnorm + projection calls below (0 at M = 1).
inline size_t rmsnorm_projection_workspace_size(int64_t M, int64_t K) {
    return xinfer_rmsnorm_projection_workspace_bytes(M, K);
}

// rmsnorm + linear_int4_fused in one call (forward.cpp:112-125, 237-247);
// workspace: caller-owned, rmsnorm_projection_workspace_size(M, K) bytes
inline void rmsnorm_linear_int4_fused(hipStream_t s, const half* X, const float* norm_weight, float eps,
                                      const FusedProjectionDesc* descs, int num_descs, int64_t M,
                                      int64_t K, int group_size = 128, void* workspace = nullptr,
                                      size_t workspace_bytes = 0) {
    auto v = detail::to_c(descs, num_descs);
    detail::check("rmsnorm_linear_int4_fused",
                  xinfer_rmsnorm_linear_int4_fused_f16(detail::q(s), X, norm_weight, eps,
                                                       descs ? v.data() : nullptr, num_descs, M, K,
                                                       group_size, workspace, workspace_bytes));
}

// rmsnorm + mlp_gate_up_swiglu_int4 in one call (forward.cpp:273-281)
inline void rmsnorm_mlp_gate_up_swiglu_int4(hipStream_t s, half* Y, const half* X, const float* norm_weight,
                                            float eps, const uint8_t* W_gate, const half* scales_gate,
                                            const uint8_t* W_up, const half* scales_up, int64_t M,
                                            int64_t N, int64_t K, int group_size = 128,
                                            void* workspace = nullptr, size_t workspace_bytes = 0) {
    detail::check("rmsnorm_mlp_gate_up_swiglu_int4",
                  xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16(detail::q(s), Y, X, norm_weight, eps, W_gate,
                                                             scales_gate, W_up, scales_up, M, N, K,
                                                             group_size, workspace, workspace_bytes));
}

// linear_int4 + add_inplace in one call: residual += X W^T (+ bias)
// (forward.cpp:229/270 with :284-290)
inline void linear_int4_residual(hipStream_t s, half* residual, const half* X, const uint8_t* W_int4,
                                 const half* scales, const float* bias, int64_t M, int64_t N, int64_t K,
                                 int group_size = 128) {
    detail::check("linear_int4_residual",
                  xinfer_linear_int4_residual_f16(detail::q(s), residual, X, W_int4, scales, bias, M, N,
                                                  K, group_size));
}

// src/ops/sampling.h:13-17 (bytes instead of an element count)
inline size_t argmax_scratch_size(int64_t vocab_size, int64_t rows = 1) {
    return xinfer_argmax_scratch_bytes(vocab_size, rows);
}

// Synchronous device->host copy of the id; supplied by the caller because
// this header does not include the HIP runtime.  Returns hipSuccess (0) on
// success.  A caller using HIP passes e.g.
//   [](void* dst, const void* src, size_t n, hipStream_t s) {
//       return (int)hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s) ||
//              (int)hipStreamSynchronize(s); }
using CopyToHostFn = int (*)(void* dst, const void* src, size_t bytes, hipStream_t s);

// src/ops/sampling.h:22-26: blocking greedy argmax -> token id.  `id_dev`
// is an int64 slot in device memory; `scratch` may be null (library buffer)
// or hold argmax_scratch_size(vocab_size) bytes.
inline int64_t argmax(hipStream_t s, const float* logits, int64_t vocab_size, int64_t* id_dev,
                      CopyToHostFn copy_to_host, void* scratch = nullptr,
                      size_t scratch_bytes = 0) {
    detail::check("argmax", xinfer_argmax_f32(detail::q(s), logits, vocab_size, 1, id_dev, scratch,
                                              scratch_bytes));
    int64_t id = 0;
    if (copy_to_host(&id, id_dev, sizeof(id), s) != 0) throw Error("argmax", XINFER_ERR_HIP);
    return id;
}

}  // namespace ops
}  // namespace xinfer
