// Batched slotted causal depthwise conv1d with SiLU: one decode step
// (conv1d_decode) and a whole chunk of T tokens (conv1d_prefill).
//
// Decode reference behaviour: braid/kernels/csrc/conv1d_decode.cu:40-75. Per
// channel c of batch row b, with the window st = conv_pool[slot_idx[b], c,
// 0..K) holding the last K pre-conv inputs (oldest first, K contiguous per
// channel):
//   w   = (st[1], ..., st[K-1], x[b, c])     window slides left, new value last
//   st <- w
//   out[b, c] = SiLU(sum_i w[i] * weight[c, i] + bias[c])
// SiLU applies to every channel (Q, K and V alike); bias is added after the dot
// and before the activation.
//
// The prefill is the same step applied to tokens 0..len_b-1 of row b, with the
// token axis split into chunks across threads (see conv1d_prefill_kernel). It
// replaces the reference's prefill conv, torch F.conv1d over [window | x] plus
// a gather to save the last K real inputs of a ragged row
// (braid/model/gdn.py:171-226). Its contract is exact: the outputs and the
// saved window equal conv1d_decode applied token by token, bit for bit,
// because both run conv_step below. Pad positions (t >= len_b) write 0 and do
// not move the window.
//
// One thread per channel. At K = 4 a channel's window is one 16-byte fp32
// vector, so the pool read, the pool write and the weight read are single
// 128-bit accesses and a wave moves 1 KiB per instruction.
#include "capi_common.h"
#include "conv_common.h"

namespace braid {
namespace {

template <int K, class XT>
__global__ void __launch_bounds__(256)
conv1d_decode_kernel(float* __restrict__ conv_pool, const int* __restrict__ slot_idx,
                     const XT* __restrict__ x, const float* __restrict__ weight,
                     const float* __restrict__ bias, float* __restrict__ out, int C) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int b = blockIdx.y;
  const int slot = slot_idx[b];
  float* st = conv_pool + ((size_t)slot * C + c) * K;
  float w[K], wt[K];
  load_window<K>(st, weight + (size_t)c * K, w, wt);
  const float o = conv_step<K>(w, conv_widen(x[(size_t)b * C + c]), wt, bias, c);
  store_window<K>(st, w);
  out[(size_t)b * C + c] = o;
}

// Loads NC consecutive channels' values of one token (NC = 1 or 4; 4 is a
// single 8-byte bf16 or 16-byte fp32 vector).
template <int NC>
__device__ __forceinline__ void load_x(const float* p, float (&o)[NC]) {
  if constexpr (NC == 4) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[j];
  } else {
    o[0] = *p;
  }
}
template <int NC>
__device__ __forceinline__ void load_x(const uint16_t* p, float (&o)[NC]) {
  if constexpr (NC == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    o[0] = conv_widen((uint16_t)(v.x & 0xffffu));
    o[1] = conv_widen((uint16_t)(v.x >> 16));
    o[2] = conv_widen((uint16_t)(v.y & 0xffffu));
    o[3] = conv_widen((uint16_t)(v.y >> 16));
  } else {
    o[0] = conv_widen(*p);
  }
}
// Prefill outputs are written once and read by a later launch: nontemporal.
template <int NC>
__device__ __forceinline__ void store_out(float* p, const float (&o)[NC]) {
  if constexpr (NC == 4) {
    __builtin_nontemporal_store((f32x4){o[0], o[1], o[2], o[3]}, reinterpret_cast<f32x4*>(p));
  } else {
    __builtin_nontemporal_store(o[0], p);
  }
}

// T tokens per launch. A conv output depends only on the K most recent
// inputs, not on earlier outputs, so the token axis is cut into chunks of
// kChunk tokens and each thread runs NC adjacent channels over one chunk
// (NC = 4 gives 8- or 16-byte loads and 16-byte stores): a thread starts from
// the K - 1 inputs before its chunk (from the cached window for the first
// chunk, from x otherwise) and runs conv_step over its tokens — the same
// window values in the same order as the token-by-token decode, so the same
// bits. Only the first chunk's thread touches the pool: it reads the old window
// and afterwards writes the new one (the last K inputs of the row's live
// tokens, spliced after the old window when fewer than K), so no thread of
// another chunk can see it half-updated.
template <int K, int NC, class XT>
__global__ void __launch_bounds__(256)
conv1d_prefill_kernel(float* __restrict__ conv_pool, const int* __restrict__ slot_idx,
                      const XT* __restrict__ x, const float* __restrict__ weight,
                      const float* __restrict__ bias, float* __restrict__ out, int C, int T,
                      const int* __restrict__ seq_lens) {
  constexpr int kChunk = 16;
  const int c0 = (blockIdx.x * blockDim.x + threadIdx.x) * NC;
  if (c0 >= C) return;
  const int b = blockIdx.z;
  const int t0 = blockIdx.y * kChunk;
  int len = T;
  if (seq_lens != nullptr) len = min(max(seq_lens[b], 0), T);
  const XT* xb = x + (size_t)b * T * C + c0;
  float* ob = out + (size_t)b * T * C + c0;
  float* st = conv_pool + ((size_t)slot_idx[b] * C + c0) * K;

  float w[NC][K], wt[NC][K], old[NC][K];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (t0 == 0) {
      load_window<K>(st + j * K, weight + (size_t)(c0 + j) * K, old[j], wt[j]);
#pragma unroll
      for (int i = 0; i < K; ++i) w[j][i] = old[j][i];
    } else {
      load_weights<K>(weight + (size_t)(c0 + j) * K, wt[j]);
    }
  }
  if (t0 != 0) {
    // inputs t0-K .. t0-1 (t0 >= kChunk >= K, so all come from x); w[.][0] is
    // shifted out by the first step and never used
#pragma unroll
    for (int i = 0; i < K; ++i) {
      float xi[NC];
      load_x<NC>(xb + (size_t)(t0 - K + i) * C, xi);
#pragma unroll
      for (int j = 0; j < NC; ++j) w[j][i] = xi[j];
    }
  }
  const int t1 = min(t0 + kChunk, T);
  const int live_end = min(t1, len);
  float xs[kChunk][NC];
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    if (t0 + u < live_end) {
      load_x<NC>(xb + (size_t)(t0 + u) * C, xs[u]);
    } else {
#pragma unroll
      for (int j = 0; j < NC; ++j) xs[u][j] = 0.f;
    }
  }
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    const int t = t0 + u;
    float o[NC];
    if (t < live_end) {
#pragma unroll
      for (int j = 0; j < NC; ++j) o[j] = conv_step<K>(w[j], xs[u][j], wt[j], bias, c0 + j);
      store_out<NC>(ob + (size_t)t * C, o);
    } else if (t < t1) {
#pragma unroll
      for (int j = 0; j < NC; ++j) o[j] = 0.f;
      store_out<NC>(ob + (size_t)t * C, o);
    }
  }
  if (t0 == 0) {
    // new window = the last K entries of [old window | x_0 .. x_{len-1}]
    float nw[NC][K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int src = len - K + i;  // position in x; negative = from the old window
      float xi[NC];
      if (src >= 0) load_x<NC>(xb + (size_t)src * C, xi);
#pragma unroll
      for (int j = 0; j < NC; ++j) nw[j][i] = src >= 0 ? xi[j] : old[j][K + src];
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) store_window<K>(st + j * K, nw[j]);
  }
}

template <class XT>
int launch(int K, float* conv_pool, const int32_t* slot_idx, int B, const XT* x,
           const float* weight, const float* bias, float* out, int C, hipStream_t stream) {
  const int threads = 256;
  const dim3 grid((unsigned)((C + threads - 1) / threads), (unsigned)B);
  switch (K) {
    case 2:
      conv1d_decode_kernel<2, XT><<<grid, threads, 0, stream>>>(conv_pool, slot_idx, x, weight,
                                                                bias, out, C);
      break;
    case 3:
      conv1d_decode_kernel<3, XT><<<grid, threads, 0, stream>>>(conv_pool, slot_idx, x, weight,
                                                                bias, out, C);
      break;
    case 4:
      conv1d_decode_kernel<4, XT><<<grid, threads, 0, stream>>>(conv_pool, slot_idx, x, weight,
                                                                bias, out, C);
      break;
    default:
      conv1d_decode_kernel<8, XT><<<grid, threads, 0, stream>>>(conv_pool, slot_idx, x, weight,
                                                                bias, out, C);
      break;
  }
  const int st = hip_status(hipGetLastError(), "launching conv1d_decode_kernel");
  return st != BRAID_OK ? st : ok();
}

template <class XT>
int launch_prefill(int K, float* conv_pool, const int32_t* slot_idx, int B, int T, const XT* x,
                   const float* weight, const float* bias, float* out, int C,
                   const int32_t* seq_lens, hipStream_t stream) {
  if (T == 0) return ok();  // no tokens: nothing to compute, the windows stay as they are
  const int threads = 256;
  constexpr int kChunk = 16;
  // Four channels per thread when every vector access stays aligned: C a
  // multiple of 4 (then each row and window block is too) and 16-byte bases.
  const bool vec4 = (C % 4 == 0) && aligned16(x) && aligned16(out) && aligned16(conv_pool) &&
                    aligned16(weight);
  const int nc = vec4 ? 4 : 1;
  const int per_row = (C + nc - 1) / nc;
  const dim3 grid((unsigned)((per_row + threads - 1) / threads),
                  (unsigned)((T + kChunk - 1) / kChunk), (unsigned)B);
#define BRAID_CONV_PREFILL(KK, NC)                                                         \
  conv1d_prefill_kernel<KK, NC, XT><<<grid, threads, 0, stream>>>(conv_pool, slot_idx, x,  \
                                                                  weight, bias, out, C, T, \
                                                                  seq_lens)
#define BRAID_CONV_PREFILL_K(NC)              \
  switch (K) {                                \
    case 2: BRAID_CONV_PREFILL(2, NC); break; \
    case 3: BRAID_CONV_PREFILL(3, NC); break; \
    case 4: BRAID_CONV_PREFILL(4, NC); break; \
    default: BRAID_CONV_PREFILL(8, NC); break; \
  }
  if (vec4) {
    BRAID_CONV_PREFILL_K(4)
  } else {
    BRAID_CONV_PREFILL_K(1)
  }
#undef BRAID_CONV_PREFILL_K
#undef BRAID_CONV_PREFILL
  const int st = hip_status(hipGetLastError(), "launching conv1d_prefill_kernel");
  return st != BRAID_OK ? st : ok();
}

int check_conv(float* conv_pool, int64_t n_slots, int C, int K, const int32_t* slot_idx, int B,
               const void* x, int x_dtype, const float* weight, float* out) {
  if (K != 2 && K != 3 && K != 4 && K != 8)
    return fail(BRAID_EINVAL,
                "conv_kernel " + std::to_string(K) + " is not instantiated (have 2, 3, 4, 8)");
  if (x_dtype != BRAID_F32 && x_dtype != BRAID_BF16)
    return fail(BRAID_EINVAL, "x must be fp32 or bf16 (the activation dtypes braid runs)");
  if (C <= 0 || B < 0 || n_slots <= 0)
    return fail(BRAID_EINVAL, "conv_pool must be [S_max, C, K] with S_max, C > 0");
  if (B == 0) return BRAID_OK;
  if (conv_pool == nullptr || slot_idx == nullptr || x == nullptr || weight == nullptr ||
      out == nullptr)
    return fail(BRAID_EINVAL, "conv_pool/slot_idx/x/weight/out must be non-null");
  if (K == 4 && (!aligned16(conv_pool) || !aligned16(weight)))
    return fail(BRAID_EINVAL, "conv_pool and weight must be 16-byte aligned at K = 4");
  return BRAID_OK;
}

}  // namespace
}  // namespace braid

using namespace braid;

extern "C" int braid_conv1d_prefill(float* conv_pool, int64_t n_slots, int C, int K,
                                    const int32_t* slot_idx, int B, int T, const void* x,
                                    int x_dtype, const float* weight, const float* bias,
                                    float* out, const int32_t* seq_lens, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (T < 0) return fail(BRAID_EINVAL, "T must be non-negative");
  const int st0 = check_conv(conv_pool, n_slots, C, K, slot_idx, B, x, x_dtype, weight, out);
  if (st0 != BRAID_OK) return st0;
  if (B == 0) return ok();
  // Rows update their slot's window over the whole chunk: two rows on one slot
  // would race, so (unlike the one-step decode) slots must be distinct.
  const int st = validate_slots(slot_idx, B, n_slots, true, stream);
  if (st != BRAID_OK) return st;
  if (x_dtype == BRAID_F32)
    return launch_prefill(K, conv_pool, slot_idx, B, T, static_cast<const float*>(x), weight,
                          bias, out, C, seq_lens, stream);
  return launch_prefill(K, conv_pool, slot_idx, B, T, static_cast<const uint16_t*>(x), weight,
                        bias, out, C, seq_lens, stream);
}

extern "C" int braid_conv1d_decode(float* conv_pool, int64_t n_slots, int C, int K,
                                   const int32_t* slot_idx, int B, const void* x, int x_dtype,
                                   const float* weight, const float* bias, float* out,
                                   void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const int st0 = check_conv(conv_pool, n_slots, C, K, slot_idx, B, x, x_dtype, weight, out);
  if (st0 != BRAID_OK) return st0;
  if (B == 0) return ok();
  const int st = validate_slots(slot_idx, B, n_slots, false, stream);
  if (st != BRAID_OK) return st;
  if (x_dtype == BRAID_F32)
    return launch(K, conv_pool, slot_idx, B, static_cast<const float*>(x), weight, bias, out, C,
                  stream);
  return launch(K, conv_pool, slot_idx, B, static_cast<const uint16_t*>(x), weight, bias, out, C,
                stream);
}
