// INT4-G128-SYM projection for M > 8 (chunked prefill).  Placeholder that
// runs the GEMV kernels on slabs of 8 activation rows until the MFMA GEMM
// lands.

#include "common.h"

namespace xhip_host {

int gemm_int4_f16(hipStream_t st, void* Y, bool y_f32, const void* X, const uint8_t* W,
                  const uint16_t* S, const uint8_t* W2, const uint16_t* S2, const float* bias,
                  int64_t M, int64_t N, int64_t K) {
    const size_t ysz = y_f32 ? 4 : 2;
    for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mm = (M - m0) < 8 ? (M - m0) : 8;
        const void* Xs = (const char*)X + (size_t)m0 * K * 2;
        void* Ys = (char*)Y + (size_t)m0 * N * ysz;
        int rc;
        if (W2)
            rc = xinfer_mlp_gate_up_swiglu_int4_f16(st, Ys, Xs, W, S, W2, S2, mm, N, K, 128);
        else if (y_f32)
            rc = xinfer_linear_int4_f16_f32out(st, (float*)Ys, Xs, W, S, bias, mm, N, K, 128);
        else
            rc = xinfer_linear_int4_f16(st, Ys, Xs, W, S, bias, mm, N, K, 128);
        if (rc) return rc;
    }
    return XINFER_OK;
}

}  // namespace xhip_host
