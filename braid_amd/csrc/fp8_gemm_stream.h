// The small-M FP8 GEMM kernel behind braid_fp8_gemm (host declarations).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace braid {

constexpr int64_t kStreamMaxM = 64;

// True for the shapes the streaming kernel takes: 1 <= M <= 64, N % 16 == 0
// (N < 2^24), and K = 1024 * 2^i for i < 5 (eight waves, 128 k per step, a
// power-of-two steps per wave).
bool fp8_gemm_stream_fits(int64_t M, int64_t N, int64_t K);

// Output columns per workgroup, in units of 16, for N on the current device.
int fp8_gemm_stream_columns(int64_t N);

// out[M, N] = (x * sx[0]) @ (w * sw[0])^T with fp32 accumulation, rounded once
// to out_dtype (BRAID_BF16, BRAID_F16 or BRAID_F32). x [M, K] and w [N, K]
// row-major e4m3fn codes, 16-byte aligned; sx, sw device scalars. No
// workspace. Returns a braid status.
int fp8_gemm_stream(const uint8_t* x, const float* sx, const uint8_t* w, const float* sw,
                    void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                    hipStream_t stream);

}  // namespace braid
