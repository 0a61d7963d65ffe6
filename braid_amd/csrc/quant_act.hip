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
#include "quant_common.h"

namespace braid {
namespace {

using namespace quant;

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
