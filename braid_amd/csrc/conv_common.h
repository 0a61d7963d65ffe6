// Per-channel pieces of the causal depthwise conv1d decode step, shared by the
// conv kernels (conv1d_decode.hip) and the fused conv + GDN decode kernel
// (gdn_mixer_decode.hip), so every path runs the same arithmetic.
//
// Reference behaviour: braid/kernels/csrc/conv1d_decode.cu:40-75. Per channel
// c, with the window st holding the last K pre-conv inputs (oldest first):
//   w   = (st[1], ..., st[K-1], x)     window slides left, new value last
//   st <- w
//   out = SiLU(sum_i w[i] * weight[c, i] + bias[c])
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace braid {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float conv_widen(float x) { return x; }
__device__ __forceinline__ float conv_widen(uint16_t bf16) {
  return __uint_as_float((uint32_t)bf16 << 16);
}

__device__ __forceinline__ float silu(float a) { return a / (1.f + expf(-a)); }

// Loads a channel's window and weight row (vector accesses at K = 4).
template <int K>
__device__ __forceinline__ void load_window(const float* st, const float* wr, float (&w)[K],
                                            float (&wt)[K]) {
  if constexpr (K == 4) {
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(st);
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(wr);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = s4[i];
      wt[i] = w4[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      w[i] = st[i];
      wt[i] = wr[i];
    }
  }
}

template <int K>
__device__ __forceinline__ void load_weights(const float* wr, float (&wt)[K]) {
  if constexpr (K == 4) {
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(wr);
#pragma unroll
    for (int i = 0; i < 4; ++i) wt[i] = w4[i];
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) wt[i] = wr[i];
  }
}

template <int K>
__device__ __forceinline__ void store_window(float* st, const float (&w)[K]) {
  if constexpr (K == 4) {
    f32x4 s4;
#pragma unroll
    for (int i = 0; i < 4; ++i) s4[i] = w[i];
    *reinterpret_cast<f32x4*>(st) = s4;
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) st[i] = w[i];
  }
}

// The same with the bias value already read (has_bias: a bias is given).
template <int K>
__device__ __forceinline__ float conv_step_b(float (&w)[K], float x, const float (&wt)[K],
                                             float bias, bool has_bias) {
#pragma unroll
  for (int i = 0; i < K - 1; ++i) w[i] = w[i + 1];
  w[K - 1] = x;
  float acc = w[0] * wt[0];
#pragma unroll
  for (int i = 1; i < K; ++i) acc = fmaf(w[i], wt[i], acc);
  if (has_bias) acc += bias;
  return silu(acc);
}

// One token: slide the window, append x, dot with the weight row (in window
// order, as fmas), add the bias, SiLU.
template <int K>
__device__ __forceinline__ float conv_step(float (&w)[K], float x, const float (&wt)[K],
                                           const float* __restrict__ bias, int c) {
#pragma unroll
  for (int i = 0; i < K - 1; ++i) w[i] = w[i + 1];
  w[K - 1] = x;
  float acc = w[0] * wt[0];
#pragma unroll
  for (int i = 1; i < K; ++i) acc = fmaf(w[i], wt[i], acc);
  if (bias != nullptr) acc += bias[c];
  return silu(acc);
}

}  // namespace
}  // namespace braid
