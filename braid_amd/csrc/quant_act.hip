// Dynamic per-tensor FP8 (e4m3fn) activation quantization in two launches.
//
// Reference behaviour: braid/kernels/csrc/quant_act.cu:90-176, which matches the
// torch spelling of braid/model/quant.py:115 and :228-229 bit for bit:
//   scale = (x.float().abs().amax() / 448).clamp(min=1e-12)
//   q     = (x.float() / scale).clamp(-448, 448).to(float8_e4m3fn)
// Operation for operation:
//   * amax is a NaN-propagating max of |x| (torch.amax returns NaN if any
//     element is NaN); max is exact, so the grid shape cannot change the bits.
//   * `amax / 448` divides by a host scalar, which torch evaluates as
//     amax * fl(1/448): one rounded reciprocal, then a multiply.
//   * clamp(min=1e-12) leaves NaN alone, so it is a comparison, not fmaxf.
//   * `x / scale` divides by a device tensor: true IEEE division.
//   * clamp(-448, 448) propagates NaN, again a comparison.
//   * the fp8 conversion rounds to nearest even; |v| >= 480 and NaN map to the
//     NaN code 0x7f, with the sign bit carried over.
//
// Pass 1 (amax_partial): each block reduces a grid-strided share to one
// partial max. Pass 2 (quantize): every block re-reduces the partials (at most
// kMaxBlocks floats, L2-resident) — a third launch would cost more than the
// redundant re-reduction — and converts its share. 128-bit loads throughout:
// eight bf16/fp16 elements (or two vectors of four fp32) per thread-iteration,
// eight fp8 codes per 64-bit store.
#include <mutex>

#include "quant_common.h"

namespace braid {
namespace {

using namespace quant;

// Device scratch of braid_quantize_act_noalloc: the pass-1 partial maxima
// (at most kMaxBlocks floats, 4 KiB). One copy per GPU, held for the life of
// the process. Host code never passes `scratch` itself to a kernel (in host
// code the name is a stand-in, not a device address): it passes the address
// hipGetSymbolAddress returned for the current device.
static __device__ __align__(256) float scratch[kMaxBlocks];
constexpr int64_t kScratchFloats = kMaxBlocks;

// Per-device address of `scratch`, looked up once per device with that
// device current (the first no-alloc call made on it).
constexpr int kMaxDevices = 64;
float* g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_for_current_device(float** out) {
  int dev = 0;
  int st = hip_status(hipGetDevice(&dev), "hipGetDevice");
  if (st != BRAID_OK) return st;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(BRAID_EINVAL, "device ordinal " + std::to_string(dev) + " beyond the " +
                                  std::to_string(kMaxDevices) + " the no-alloc quantizer serves");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                    "hipGetSymbolAddress(quantize scratch)");
    if (st != BRAID_OK) return st;
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return BRAID_OK;
}

template <class Tag>
int launch(const void* xv, int64_t n, uint8_t* q, float* scale, float* partial,
           hipStream_t stream) {
  using T = typename Tag::T;
  const T* x = static_cast<const T*>(xv);
  const int blocks = blocks_for(n);
  const int vec = (aligned16(x) && ((reinterpret_cast<uintptr_t>(q) & 7u) == 0)) ? 1 : 0;
  amax_partial<Tag><<<blocks, kThreads, 0, stream>>>(x, partial, n, vec);
  quantize<Tag><<<blocks, kThreads, 0, stream>>>(x, partial, blocks, scale, q, n, vec);
  const int st = hip_status(hipGetLastError(), "launching quantize_act kernels");
  return st != BRAID_OK ? st : ok();
}

}  // namespace
}  // namespace braid

using namespace braid;

extern "C" int braid_quantize_act_workspace(int64_t n) { return n <= 0 ? 1 : blocks_for(n); }

extern "C" int braid_quantize_act_noalloc(const void* x, int x_dtype, int64_t n, uint8_t* q,
                                          float* scale, void* stream_) {
  if (n <= 0) return fail(BRAID_EINVAL, "x must not be empty");
  if (x == nullptr || q == nullptr || scale == nullptr)
    return fail(BRAID_EINVAL, "x/q/scale must be non-null");
  if (x_dtype != BRAID_F32 && x_dtype != BRAID_F16 && x_dtype != BRAID_BF16)
    return fail(BRAID_EINVAL, "activation must be fp32, bf16 or fp16");
  if (blocks_for(n) > kScratchFloats)
    return fail(BRAID_EINVAL, "quantize_act_noalloc: " + std::to_string(blocks_for(n)) +
                                  " partials exceed the " + std::to_string(kScratchFloats) +
                                  "-float device scratch");
  float* partial = nullptr;
  const int st = scratch_for_current_device(&partial);
  if (st != BRAID_OK) return st;
  return braid_quantize_act(x, x_dtype, n, q, scale, partial, stream_);
}

extern "C" int braid_quantize_act(const void* x, int x_dtype, int64_t n, uint8_t* q,
                                  float* scale, float* partial, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (n <= 0) return fail(BRAID_EINVAL, "x must not be empty");
  if (x == nullptr || q == nullptr || scale == nullptr || partial == nullptr)
    return fail(BRAID_EINVAL, "x/q/scale/partial must be non-null");
  switch (x_dtype) {
    case BRAID_F32: return launch<XF32>(x, n, q, scale, partial, stream);
    case BRAID_F16: return launch<XF16>(x, n, q, scale, partial, stream);
    case BRAID_BF16: return launch<XBF16>(x, n, q, scale, partial, stream);
    default: return fail(BRAID_EINVAL, "activation must be fp32, bf16 or fp16");
  }
}
