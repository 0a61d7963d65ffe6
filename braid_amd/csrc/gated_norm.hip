// Gated RMSNorm readout of the GDN mixer, fused with the out_proj input's
// dynamic FP8 quantization.
//
// Reference behaviour (braid/model/gdn.py:373-387 `_readout`, braid/model/
// norm.py:48-71 `rms_norm_gated`, then braid/model/quant.py:209-229 on the
// result): for each (token, value head) unit of HD = 128 scan outputs y,
//   c    = y.to(act)                         scan output cast to the act dtype
//   xf   = c * rsqrt(mean(c^2) + eps)       F.rms_norm in fp32, no weight
//   h    = gamma * xf.to(act)                gamma fp32 [HD]; promotes to fp32
//   o    = h * silu(z.float())               silu(x) = x / (1 + exp(-x))
//   core = o.to(act)                         the out_proj input [N, H*HD]
// and, when the out_proj weight is FP8, (q, scale) = quantize_act(core) over
// the whole [N, H*HD] tensor.
//
// Launch 1 (gated_norm_amax) computes `core` and, in the same pass, one
// NaN-propagating partial max of |core| per block: it replaces the amax pass of
// the quantizer, so the readout and the quantization together are the same two
// launches as the quantization alone. Launch 2 is the quantizer's own second
// pass, reading `core` back (bf16: 2 B per element, L2/MALL-resident at
// decode sizes).
//
// Layout: a wave takes two units per iteration, 32 lanes each, four
// consecutive elements per lane (16-byte fp32 loads of y, 8-byte loads of z).
// The sum of squares is an in-lane pair sum followed by a 32-lane butterfly,
// so both halves of the wave reduce independently. The reduction order differs
// from torch's rms_norm kernel: the result agrees to fp32 rounding before the
// act-dtype casts (gated by tolerance, not bits).
#include "quant_common.h"

namespace braid {
namespace {

using namespace quant;

constexpr int kUnit = 128;                          // HD
constexpr int kLanesPerUnit = 32;                   // 4 elements per lane
constexpr int kUnitsPerBlock = (kThreads / 64) * 2;  // two units per wave

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Act-dtype narrowing of two fp32 values, round to nearest even, returned both
// packed (for the store) and widened back (for the arithmetic that follows).
// The packed vector conversion consumes the already-rounded fp32 operands; a
// scalar `(_Float16)(a * b)` may be contracted into one mixed-precision op
// that rounds the exact product once, straight to 16 bits.
template <class Tag>
struct Narrow;
template <>
struct Narrow<XF32> {
  __device__ __forceinline__ static void pair(float& a, float& b, uint32_t&) {}
};
template <>
struct Narrow<XF16> {
  __device__ __forceinline__ static void pair(float& a, float& b, uint32_t& bits) {
    const f16x2 h = __builtin_convertvector((f32x2){a, b}, f16x2);
    bits = __builtin_bit_cast(uint32_t, h);
    a = (float)h[0];
    b = (float)h[1];
  }
};
template <>
struct Narrow<XBF16> {
  __device__ __forceinline__ static void pair(float& a, float& b, uint32_t& bits) {
    bits = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
    a = __uint_as_float(bits << 16);
    b = __uint_as_float(bits & 0xffff0000u);
  }
};

// Four consecutive elements at p + i (i a multiple of 4, 16/8-byte aligned).
__device__ __forceinline__ void load4(XF32, const float* p, long i, float (&o)[4]) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(p + i);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = v[e];
}
template <class Tag>
__device__ __forceinline__ void load4(Tag tag, const uint16_t* p, long i, float (&o)[4]) {
  const u32x2 r = *reinterpret_cast<const u32x2*>(p + i);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = widen(tag, (uint16_t)((r[e >> 1] >> (16 * (e & 1))) & 0xffffu));
}

// Rounds o[0..3] to the act dtype in place and stores them at p + i. Plain
// (cacheable) stores: the quantize pass reads core back right away, and at
// prefill sizes it then comes from the Infinity Cache (4073 tokens: 42.6 ->
// 41.2 us for the readout against nontemporal stores).
__device__ __forceinline__ void round_store4(XF32, float* p, long i, float (&o)[4]) {
  *reinterpret_cast<f32x4*>(p + i) = (f32x4){o[0], o[1], o[2], o[3]};
}
template <class Tag>
__device__ __forceinline__ void round_store4(Tag, uint16_t* p, long i, float (&o)[4]) {
  uint32_t r0, r1;
  Narrow<Tag>::pair(o[0], o[1], r0);
  Narrow<Tag>::pair(o[2], o[3], r1);
  *reinterpret_cast<u32x2*>(p + i) = (u32x2){r0, r1};
}
template <class Tag>
__device__ __forceinline__ void round4(Tag, float (&o)[4]) {
  uint32_t unused;
  Narrow<Tag>::pair(o[0], o[1], unused);
  Narrow<Tag>::pair(o[2], o[3], unused);
}

// One unit's computation from its loaded y (c, widened) and z values: writes
// core and folds |core| into the running max m.
template <class ATag>
__device__ __forceinline__ void gated_unit(float (&c)[4], const float (&zf)[4], const f32x4& gm,
                                           float eps, bool live, typename ATag::T* core, long i,
                                           float& m) {
  round4(ATag{}, c);
  float ss = (c[0] * c[0] + c[1] * c[1]) + (c[2] * c[2] + c[3] * c[3]);
  static_assert(kLanesPerUnit == 32, "a unit's sum runs over lane bits 0-4");
  ss += lane_xor<1>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<16>(ss);
  const float r = rsqrtf(ss * (1.0f / kUnit) + eps);  // mean: exact power-of-two scale
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = c[e] * r;
  round4(ATag{}, o);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float h = gm[e] * o[e];
    const float s = zf[e] / (1.0f + expf(-zf[e]));
    o[e] = h * s;
  }
  if (live) {
    round_store4(ATag{}, core, i, o);
#pragma unroll
    for (int e = 0; e < 4; ++e) m = nan_max(m, fabsf(o[e]));
  }
}

// YTag: dtype of the scan output y (fp32, or already the act dtype). ATag: the
// act dtype of z and core. Each wave iteration takes one pair of units, one
// per half-wave. (Two pairs per iteration, loaded before either is computed,
// measured 3% slower at 4073 tokens, four 8%: more bytes in flight per wave
// did not pay for the registers and the longer iteration.)
template <class YTag, class ATag>
__global__ void __launch_bounds__(kThreads)
gated_norm_amax(const typename YTag::T* __restrict__ y, const typename ATag::T* __restrict__ z,
                const float* __restrict__ gamma, float eps, long units,
                typename ATag::T* __restrict__ core, float* __restrict__ partial) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane / kLanesPerUnit, sub = lane % kLanesPerUnit;
  const f32x4 gm = *reinterpret_cast<const f32x4*>(gamma + 4 * sub);
  float m = 0.f;
  const long step = (long)gridDim.x * kUnitsPerBlock;
  // Both halves of a wave run every iteration (the butterfly needs all 64
  // lanes); a half past the end works on zeros and stores nothing.
  for (long u0 = ((long)blockIdx.x * (kThreads / 64) + wave) * 2; u0 < units; u0 += step) {
    const long u = u0 + half;
    const bool live = u < units;
    const long i = u * kUnit + 4 * sub;
    float c[4] = {0.f, 0.f, 0.f, 0.f}, zz[4] = {0.f, 0.f, 0.f, 0.f};
    if (live) {
      load4(YTag{}, y, i, c);
      load4(ATag{}, z, i, zz);
    }
    gated_unit<ATag>(c, zz, gm, eps, live, core, i, m);
  }
  m = block_nan_max(m);
  if (partial != nullptr && threadIdx.x == 0) partial[blockIdx.x] = m;
}

int norm_blocks(int64_t units) {
  const int64_t want = (units + kUnitsPerBlock - 1) / kUnitsPerBlock;
  return (int)(want < 1 ? 1 : (want > kMaxBlocks ? kMaxBlocks : want));
}

template <class YTag, class ATag>
int launch(const void* yv, const void* zv, const float* gamma, float eps, int64_t units,
           void* corev, uint8_t* q, float* scale, float* partial, hipStream_t stream) {
  using AT = typename ATag::T;
  const auto* y = static_cast<const typename YTag::T*>(yv);
  const auto* z = static_cast<const AT*>(zv);
  AT* core = static_cast<AT*>(corev);
  const int blocks = norm_blocks(units);
  gated_norm_amax<YTag, ATag><<<blocks, kThreads, 0, stream>>>(y, z, gamma, eps, units, core,
                                                              q != nullptr ? partial : nullptr);
  if (q != nullptr) {
    const int64_t n = units * kUnit;
    const int vec = ((reinterpret_cast<uintptr_t>(q) & 7u) == 0) ? 1 : 0;
    quantize<ATag><<<blocks_for(n), kThreads, 0, stream>>>(core, partial, blocks, scale, q, n, vec);
  }
  const int st = hip_status(hipGetLastError(), "launching gated_rmsnorm kernels");
  return st != BRAID_OK ? st : ok();
}

template <class ATag>
int dispatch_y(int y_dtype, const void* y, const void* z, const float* gamma, float eps,
               int64_t units, void* core, uint8_t* q, float* scale, float* partial,
               hipStream_t stream, int act_dtype) {
  if (y_dtype == BRAID_F32)
    return launch<XF32, ATag>(y, z, gamma, eps, units, core, q, scale, partial, stream);
  if (y_dtype == act_dtype)
    return launch<ATag, ATag>(y, z, gamma, eps, units, core, q, scale, partial, stream);
  return fail(BRAID_EINVAL, "y must be fp32 or the activation dtype");
}

}  // namespace
}  // namespace braid

using namespace braid;

extern "C" int braid_gated_rmsnorm_workspace(int64_t units) { return norm_blocks(units); }

extern "C" int braid_gated_rmsnorm_quant(const void* y, int y_dtype, const void* z,
                                         int act_dtype, const float* gamma, float eps,
                                         int64_t units, int HD, void* core, uint8_t* q,
                                         float* scale, float* partial, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (HD != kUnit) return fail(BRAID_EINVAL, "head_dim must be 128, got " + std::to_string(HD));
  if (units < 0) return fail(BRAID_EINVAL, "negative unit count");
  const bool quant = q != nullptr;
  if (quant && (scale == nullptr || partial == nullptr))
    return fail(BRAID_EINVAL, "q, scale and partial must be given together");
  if (!quant && (scale != nullptr))
    return fail(BRAID_EINVAL, "q, scale and partial must be given together");
  if (quant && units == 0) return fail(BRAID_EINVAL, "x must not be empty");
  if (units == 0) return ok();
  if (y == nullptr || z == nullptr || gamma == nullptr || core == nullptr)
    return fail(BRAID_EINVAL, "y/z/gamma/core must be non-null");
  if (!aligned16(y) || !aligned16(z) || !aligned16(core) || !aligned16(gamma))
    return fail(BRAID_EINVAL, "y, z, gamma and core must be 16-byte aligned");
  switch (act_dtype) {
    case BRAID_F32:
      return dispatch_y<XF32>(y_dtype, y, z, gamma, eps, units, core, q, scale, partial, stream,
                              act_dtype);
    case BRAID_F16:
      return dispatch_y<XF16>(y_dtype, y, z, gamma, eps, units, core, q, scale, partial, stream,
                              act_dtype);
    case BRAID_BF16:
      return dispatch_y<XBF16>(y_dtype, y, z, gamma, eps, units, core, q, scale, partial, stream,
                               act_dtype);
    default: return fail(BRAID_EINVAL, "activation must be fp32, bf16 or fp16");
  }
}
