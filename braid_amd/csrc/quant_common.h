// Shared device code of the FP8 e4m3fn activation quantizer: element widening,
// 128-bit loads, the NaN-propagating block max, the e4m3fn rounding and the
// quantize pass. Used by quant_act.hip (plain quantization) and gated_norm.hip
// (the gated-norm readout, whose first pass produces the amax partials).
//
// The bit-level contract (braid/kernels/csrc/quant_act.cu:90-176, matching the
// torch spelling of braid/model/quant.py:115 and :228-229):
//   scale = max(amax(|x|) * fl(1/448), 1e-12), NaN-propagating
//   q     = e4m3fn(clamp(x / scale, -448, 448)), round to nearest even.
#pragma once

#include "capi_common.h"

namespace braid {
namespace quant {
namespace {

constexpr int kThreads = 256;
constexpr int kVec = 8;
constexpr int kMaxBlocks = 1024;
constexpr float kFp8Max = 448.0f;
constexpr float kInvFp8Max = 1.0f / 448.0f;  // fl32(1/448), as torch's scalar division rounds it
constexpr float kEps = 1e-12f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct XF32 { using T = float; };
struct XF16 { using T = uint16_t; };
struct XBF16 { using T = uint16_t; };

__device__ __forceinline__ float widen(XF32, float v) { return v; }
__device__ __forceinline__ float widen(XF16, uint16_t v) {
  return (float)__builtin_bit_cast(_Float16, v);
}
__device__ __forceinline__ float widen(XBF16, uint16_t v) {
  return __uint_as_float((uint32_t)v << 16);
}

// Loads eight consecutive elements starting at x[i] (16-byte aligned).
__device__ __forceinline__ void load_vec(XF32, const float* x, long i, float (&o)[kVec]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(x + i);
  const f32x4 b = *reinterpret_cast<const f32x4*>(x + i + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o[j] = a[j];
    o[j + 4] = b[j];
  }
}
template <class Tag>
__device__ __forceinline__ void load_vec(Tag tag, const uint16_t* x, long i, float (&o)[kVec]) {
  const u32x4 r = *reinterpret_cast<const u32x4*>(x + i);
#pragma unroll
  for (int j = 0; j < kVec; ++j)
    o[j] = widen(tag, (uint16_t)((r[j >> 1] >> (16 * (j & 1))) & 0xffffu));
}

// The value v holds in lane (this lane xor S), S a power of two below 64,
// exchanged on the VALU rather than through the LDS crossbar (a ds_bpermute
// is an LDS round trip per stage): DPP inside a 16-lane row for S = 1, 2 and
// 8 (quad_perm [1,0,3,2], [2,3,0,1], row_ror:8); for S = 4, row_half_mirror
// (t[i] = v[7 - i] in each 8-lane half) then quad_perm [3,2,1,0], which reads
// t[4q + 3 - j] = v[(4q + j) xor 4]; for S = 16 and 32 the permlane swap of v
// with itself, after which the two results hold the lower and the upper
// block's value in every lane.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, true));
}
template <int S>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (S == 1) {
    return dpp_f<0xB1>(v);
  } else if constexpr (S == 2) {
    return dpp_f<0x4E>(v);
  } else if constexpr (S == 4) {
    return dpp_f<0x1B>(dpp_f<0x141>(v));
  } else if constexpr (S == 8) {
    return dpp_f<0x128>(v);
  } else {
    static_assert(S == 16 || S == 32, "a lane-index bit");
    const uint32_t u = __float_as_uint(v);
    const auto p = S == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float((__lane_id() & S) ? p[0] : p[1]);
  }
}

// NaN-propagating max: once m is NaN it stays NaN.
__device__ __forceinline__ float nan_max(float m, float v) { return (v != v || v > m) ? v : m; }

__device__ __forceinline__ float block_nan_max(float m) {
  __shared__ float waves[kThreads / 64];
  // Each lane folds in its partner's value, lane xor 1, 2, ..., 32: the
  // butterfly every lane of the wave runs alike.
  m = nan_max(m, lane_xor<1>(m));
  m = nan_max(m, lane_xor<2>(m));
  m = nan_max(m, lane_xor<4>(m));
  m = nan_max(m, lane_xor<8>(m));
  m = nan_max(m, lane_xor<16>(m));
  m = nan_max(m, lane_xor<32>(m));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) waves[wave] = m;
  __syncthreads();
  float r = waves[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) r = nan_max(r, waves[w]);
  return r;
}

// fp32 -> e4m3fn code, round to nearest even.
//   |f| >= 480 or NaN       -> 0x7f (NaN)
//   2^-6 <= |f| < 480       -> round the fp32 mantissa to 3 bits (RNE), rebias
//                              the exponent from 127 to 7; a mantissa carry
//                              rolls into the exponent, and (464, 480) lands on
//                              0x7f exactly as the RNE rule puts it past 448
//   |f| < 2^-6              -> subnormal: the code is |f| / 2^-9 rounded to an
//                              integer (RNE), 0..8 (8 is the smallest normal)
__device__ __forceinline__ uint32_t e4m3fn_code(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a >= 0x43f00000u) {            // 480.0f, and every Inf/NaN pattern above it
    code = 0x7fu;
  } else if (a < 0x3c800000u) {      // 2^-6
    code = (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  } else {
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (r >> 20) - ((127u - 7u) << 3);
  }
  return code | sign;
}

__device__ __forceinline__ float quant_value(float x, float sc) {
  float v = x / sc;
  v = (v < -kFp8Max) ? -kFp8Max : ((v > kFp8Max) ? kFp8Max : v);
  return v;
}

// Vectors each thread keeps in flight per grid-stride step: four 16-byte loads
// are issued before any of them is used.
constexpr int kUnroll = 4;

template <class Tag>
__global__ void __launch_bounds__(kThreads)
amax_partial(const typename Tag::T* __restrict__ x, float* __restrict__ partial, long n,
             int vec) {
  const long tid = (long)blockIdx.x * kThreads + threadIdx.x;
  const long stride = (long)gridDim.x * kThreads;
  float m = 0.f;
  long tail = 0;
  if (vec) {
    const long nv = n / kVec;
    long j = tid;
    for (; j + (kUnroll - 1) * stride < nv; j += kUnroll * stride) {
      float o[kUnroll][kVec];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) load_vec(Tag{}, x, (j + u * stride) * kVec, o[u]);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) m = nan_max(m, fabsf(o[u][e]));
      }
    }
    for (; j < nv; j += stride) {
      float o[kVec];
      load_vec(Tag{}, x, j * kVec, o);
#pragma unroll
      for (int e = 0; e < kVec; ++e) m = nan_max(m, fabsf(o[e]));
    }
    tail = nv * kVec;
  }
  for (long i = tail + tid; i < n; i += stride) m = nan_max(m, fabsf(widen(Tag{}, x[i])));
  m = block_nan_max(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// The per-tensor scale and what the fast path needs of it.
//
// Fast path (the scale is finite, which it is unless amax is Inf or NaN, and
// then no element is Inf or NaN either):
//   * x / sc as x * y corrected once (Markstein): y = fl(1 / sc) by one IEEE
//     division, q0 = fl(x y), r = x - sc q0 exactly by an fma, q = fl(q0 + r y).
//     With y correctly rounded and r exact this is the correctly rounded
//     quotient. r is exact unless it underflows, which needs |x| below about
//     2^-103; then |x / sc| < 2^-10 (sc >= 1e-12), below half the smallest
//     e4m3fn step, and both quotients encode to the zero of x's sign. r == 0
//     keeps q0, so a signed zero x keeps its sign. Checked on the MI355X
//     against IEEE division over every bf16 x and random fp32 x in
//     [-amax, amax] for 4096 scales (1.7e10 pairs): identical codes.
//   * the clamped value is finite, and gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn,
//     round to nearest even) gives the same code as e4m3fn_code for every
//     finite fp32 input (checked over all 2^32 patterns; the two differ only
//     on positive NaN, which the clamp cannot produce here).
// Slow path (non-finite scale): the IEEE division and e4m3fn_code.
struct QuantScale {
  float sc, y;
  bool fast;
};
__device__ __forceinline__ QuantScale quant_scale(float sc) {
  const bool fast = __builtin_isfinite(sc);
  return QuantScale{sc, fast ? 1.0f / sc : 0.f, fast};
}
__device__ __forceinline__ float quant_value_fast(float x, const QuantScale& s) {
  const float q0 = x * s.y;
  const float r = fmaf(-s.sc, q0, x);
  float v = (r == 0.f) ? q0 : fmaf(r, s.y, q0);
  v = (v < -kFp8Max) ? -kFp8Max : ((v > kFp8Max) ? kFp8Max : v);
  return v;
}
// Four finite clamped values -> four codes in one word, element e in byte e.
__device__ __forceinline__ uint32_t pack4_fast(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}
__device__ __forceinline__ uint32_t quant_code(float x, const QuantScale& s) {
  if (s.fast)
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(quant_value_fast(x, s), 0.f, 0, false) &
           0xffu;
  return e4m3fn_code(quant_value(x, s.sc));
}

__device__ __forceinline__ uint2 quant_vec(const float (&o)[kVec], const QuantScale& s) {
  if (s.fast) {
    float v[kVec];
#pragma unroll
    for (int e = 0; e < kVec; ++e) v[e] = quant_value_fast(o[e], s);
    return make_uint2(pack4_fast(v[0], v[1], v[2], v[3]), pack4_fast(v[4], v[5], v[6], v[7]));
  }
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    lo |= e4m3fn_code(quant_value(o[e], s.sc)) << (8 * e);
    hi |= e4m3fn_code(quant_value(o[e + 4], s.sc)) << (8 * e);
  }
  return make_uint2(lo, hi);
}

// Eight codes, one 8-byte nontemporal store (the codes are read once, by the
// GEMM that consumes them).
__device__ __forceinline__ void store_codes(uint8_t* p, uint2 v) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store((u32x2){v.x, v.y}, reinterpret_cast<u32x2*>(p));
}

// The first grid-stride step's loads are issued before the partials are
// reduced to the scale, so the reduction overlaps them: kUnroll vectors a
// thread when it has that many, else its first vector (a [64, 4096] input
// gives each thread one).
template <class Tag>
__global__ void __launch_bounds__(kThreads)
quantize(const typename Tag::T* __restrict__ x, const float* __restrict__ partial, int nparts,
         float* __restrict__ scale, uint8_t* __restrict__ q, long n, int vec) {
  const long tid = (long)blockIdx.x * kThreads + threadIdx.x;
  const long stride = (long)gridDim.x * kThreads;
  const long nv = vec ? n / kVec : 0;
  float o[kUnroll][kVec];
  long j = tid;
  bool full = j + (kUnroll - 1) * stride < nv;
  const bool one = !full && j < nv;
  if (full) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load_vec(Tag{}, x, (j + u * stride) * kVec, o[u]);
  } else if (one) {
    load_vec(Tag{}, x, j * kVec, o[0]);
  }

  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += kThreads) m = nan_max(m, partial[i]);
  m = block_nan_max(m);
  const float raw = m * kInvFp8Max;
  const float sc = (raw < kEps) ? kEps : raw;
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = sc;
  const QuantScale qs = quant_scale(sc);

  while (full) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      store_codes(q + (j + u * stride) * kVec, quant_vec(o[u], qs));
    j += kUnroll * stride;
    full = j + (kUnroll - 1) * stride < nv;
    if (full) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) load_vec(Tag{}, x, (j + u * stride) * kVec, o[u]);
    }
  }
  if (one) {
    store_codes(q + j * kVec, quant_vec(o[0], qs));
    j += stride;
  }
  for (; j < nv; j += stride) {
    float v1[kVec];
    load_vec(Tag{}, x, j * kVec, v1);
    store_codes(q + j * kVec, quant_vec(v1, qs));
  }
  for (long i = nv * kVec + tid; i < n; i += stride)
    q[i] = (uint8_t)quant_code(widen(Tag{}, x[i]), qs);
}

// Grid of the quantize pass (and of the plain amax pass) for n elements.
int blocks_for(int64_t n) {
  const int64_t per_block = (int64_t)kThreads * kVec;
  const int64_t want = (n + per_block - 1) / per_block;
  return (int)(want < 1 ? 1 : (want > kMaxBlocks ? kMaxBlocks : want));
}

}  // namespace
}  // namespace quant
}  // namespace braid
