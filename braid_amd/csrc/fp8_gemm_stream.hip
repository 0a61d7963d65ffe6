// Small-M FP8 (e4m3fn) W8A8 GEMM that streams the weight once: the decode
// shapes of braid's projections (M = the batch, at most 64 rows; N x K = a
// projection's weight), where the cost is reading w from HBM.
//
// Reference behaviour: braid/model/quant.py:232-241 (`fp8_matmul`),
//   out[M, N] = (xq[M, K] * sx) @ (w[N, K] * sw)^T, fp32 accumulation.
// The FP8 products are exact in fp32; the accumulation order is this
// kernel's, fixed (below), so results are deterministic run to run.
//
// Work split: workgroup g owns 16*NT output columns (all M rows) over the whole
// of K, so the weight is read exactly once and no cross-workgroup reduction is
// needed; NT is chosen so that the grid still covers every CU. Its 8 waves
// take the 128-wide k-steps round robin (wave w: steps w, w + 8, ...). The
// activation (256 KB at M = 64, K = 4096) is read by every workgroup and
// stays L2-resident. The 8 per-wave partial tiles meet in LDS and are summed in
// a fixed tree ((w0+w1)+(w2+w3))+((w4+w5)+(w6+w7)), then scaled by sx * sw
// and rounded once to the output type.
//
// Loads: x [M, K] and w [N, K] are row-major, K-contiguous. The MFMA
// (v_mfma_f32_16x16x128_f8f6f4) wants lane l to hold row l % 16 of a 16-row
// operand, so loading its operands straight from memory puts 16 rows 4 KiB
// apart in every 16 consecutive lanes: each lane is then a separate L1 access
// of 16 bytes, and the L1's access rate (about one a clock) caps a CU at about
// 16 B a clock, a third of the weight stream it needs. Here each 16-row
// block of a step is read as two fully coalesced loads instead (eight lanes
// per 128-byte row chunk, 8 rows per instruction), written to the wave's own
// LDS stage, and read back in the MFMA's layout. The stage stores row r's
// 16-byte chunk c at slot c ^ (r & 7), so both the writes (8 lanes fill one
// row) and the MFMA-layout reads (8 lanes read 8 rows) are bank-conflict free.
// The stage is private to the wave, so no workgroup barrier is needed until
// the final reduction.
//
// MFMA operand layout: lane l = (r = l & 15, kg = l >> 4) holds row (A) or
// column (B) r and the 32 bytes of k-group kg; any placement of a step's 128 k
// values in those bytes gives the same sum as long as A and B use the same
// one. This kernel puts chunks kg and 4 + kg of the row's 128-byte step there.
// Lane l of the 16x16 result holds column l % 16 of rows 4 (l / 16) .. + 3.
//
// Rows m >= M of the A operand read row M - 1 again: row m of the product
// depends only on row m of A, and those rows are never stored.
#include <hip/hip_runtime.h>

#include "capi_common.h"
#include "fp8_gemm_stream.h"
#include "stream_shape.h"

namespace braid {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kStepK = 128;       // bytes (= k values) of one MFMA step per row
constexpr int kBlockBytes = 16 * kStepK;  // one 16-row operand block of a step

// One step's raw, coalesced loads of a wave: 2 per 16-row block.
template <int MT, int NT>
struct RawStep {
  v4i a[2 * MT];
  v4i b[2 * NT];
};

// Lane i of a coalesced load reads chunk i & 7 of row 8 q + (i >> 3).
template <int MT, int NT>
__device__ __forceinline__ void load_raw(RawStep<MT, NT>& raw, const uint8_t* const* xrow,
                                         const uint8_t* const* wrow, int off) {
#pragma unroll
  for (int q = 0; q < 2 * NT; ++q) raw.b[q] = *reinterpret_cast<const v4i*>(wrow[q] + off);
#pragma unroll
  for (int q = 0; q < 2 * MT; ++q) raw.a[q] = *reinterpret_cast<const v4i*>(xrow[q] + off);
}

// Stage byte offset of row `row`'s chunk `c` (rows of 128 bytes, swizzled).
__device__ __forceinline__ int stage_pos(int row, int c) {
  return row * kStepK + 16 * (c ^ (row & 7));
}

template <int MT, int NT>
__device__ __forceinline__ void write_stage(uint8_t* stage, const RawStep<MT, NT>& raw,
                                            int lane) {
  const int rr = lane >> 3, c = lane & 7;
#pragma unroll
  for (int q = 0; q < 2 * MT; ++q)
    *reinterpret_cast<v4i*>(stage + stage_pos(8 * q + rr, c)) = raw.a[q];
#pragma unroll
  for (int q = 0; q < 2 * NT; ++q)
    *reinterpret_cast<v4i*>(stage + MT * kBlockBytes + stage_pos(8 * q + rr, c)) = raw.b[q];
}

// The MFMA operand of 16-row block `blk` at `base`: row r, chunks kg, 4 + kg.
__device__ __forceinline__ v8i read_operand(const uint8_t* base, int blk, int r, int kg) {
  const int row = 16 * blk + r;
  const v4i lo = *reinterpret_cast<const v4i*>(base + stage_pos(row, kg));
  const v4i hi = *reinterpret_cast<const v4i*>(base + stage_pos(row, 4 + kg));
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int MT, int NT>
__device__ __forceinline__ void mma_stage(v4f (&acc)[MT][NT], const uint8_t* stage, int r,
                                          int kg) {
  v8i a[MT], b[NT];
#pragma unroll
  for (int i = 0; i < MT; ++i) a[i] = read_operand(stage, i, r, kg);
#pragma unroll
  for (int j = 0; j < NT; ++j) b[j] = read_operand(stage + MT * kBlockBytes, j, r, kg);
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
      // scale operands 0: the unscaled v_mfma_f32_16x16x128_f8f6f4, e4m3 x e4m3
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i], b[j], acc[i][j], 0, 0,
                                                                   0, 0, 0, 0);
}

template <class Out>
__device__ __forceinline__ Out narrow(float v);
template <>
__device__ __forceinline__ float narrow<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ _Float16 narrow<_Float16>(float v) {
  return (_Float16)v;
}
template <>
__device__ __forceinline__ __bf16 narrow<__bf16>(float v) {
  return (__bf16)v;
}

// Raw steps a wave keeps in flight: DEPTH steps of 8 (MT + NT) VGPRs each,
// beside the operands being consumed (the same again) and the 4 MT NT
// accumulators, within 256 VGPRs (two waves per SIMD); one step fewer for
// the longest unrolled loops (16 steps), which otherwise spill. At M = 64 and
// NT = 3 that is one step: measured, two steps in flight were 2-4% slower
// for in_proj and out_proj alike.
template <int MT, int NT, int SPW>
constexpr int ring_depth() {
  constexpr int d = (200 - 4 * MT * NT) / (8 * (MT + NT)) - 1 - (SPW >= 16 ? 1 : 0);
  return d < 1 ? 1 : (d > SPW ? SPW : d);
}

// LDS of one wave: its stage, later its slice of the reduction.
template <int MT, int NT>
constexpr int wave_lds_bytes() {
  constexpr int stage = (MT + NT) * kBlockBytes;
  constexpr int red = MT * NT * 4 * 64 * 4;
  return stage > red ? stage : red;
}

// SPW = k-steps per wave (K / 128 / 8), a template argument so the step loop
// unrolls into straight-line code: each wait then covers exactly the step it
// needs and the later steps stay in flight.
template <int MT, int NT, int SPW, class Out>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void fp8_gemm_stream_kernel(const uint8_t* __restrict__ x, const float* __restrict__ sx,
                            const uint8_t* __restrict__ w, const float* __restrict__ sw,
                            Out* __restrict__ out, int M, int N, int K) {
  constexpr int DEPTH = ring_depth<MT, NT, SPW>();
  constexpr int kWaveLds = wave_lds_bytes<MT, NT>();
  __shared__ __align__(16) uint8_t lds[kWaves * kWaveLds];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * (16 * NT);
  uint8_t* stage = lds + wave * kWaveLds;

  // coalesced row pointers (lane: row 8 q + lane / 8, chunk lane % 8), at the
  // wave's first k-step
  const int rr = lane >> 3, c = lane & 7;
  const uint8_t* wrow[2 * NT];
#pragma unroll
  for (int q = 0; q < 2 * NT; ++q)
    wrow[q] = w + (size_t)(n0 + 8 * q + rr) * K + wave * kStepK + 16 * c;
  const uint8_t* xrow[2 * MT];
#pragma unroll
  for (int q = 0; q < 2 * MT; ++q)
    xrow[q] = x + (size_t)min(8 * q + rr, M - 1) * K + wave * kStepK + 16 * c;

  v4f acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  RawStep<MT, NT> ring[DEPTH];
#pragma unroll
  for (int s = 0; s < DEPTH; ++s) load_raw<MT, NT>(ring[s], xrow, wrow, s * kWaves * kStepK);
  // the fences keep each step's loads where they are written: the scheduler
  // would otherwise sink them to their first use to save registers
  __builtin_amdgcn_sched_barrier(0);
  const int r = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    // LDS instructions of one wave execute in order: these writes land
    // before the reads below, and the reads of step s - 1 before them
    write_stage<MT, NT>(stage, ring[s % DEPTH], lane);
    __builtin_amdgcn_sched_barrier(0);
    if (s + DEPTH < SPW)
      load_raw<MT, NT>(ring[s % DEPTH], xrow, wrow, (s + DEPTH) * kWaves * kStepK);
    __builtin_amdgcn_sched_barrier(0);
    mma_stage<MT, NT>(acc, stage, r, kg);
    __builtin_amdgcn_sched_barrier(0);
  }

  // the wave's stage becomes its reduction slice [MT NT 4][64] floats
  float* red = reinterpret_cast<float*>(lds);
  constexpr int kWaveFloats = kWaveLds / 4;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[wave * kWaveFloats + ((i * NT + j) * 4 + e) * 64 + lane] = acc[i][j][e];
  __syncthreads();

  const float scale = sx[0] * sw[0];
  constexpr int kCols = 16 * NT;
  for (int idx = threadIdx.x; idx < MT * 16 * kCols; idx += kThreads) {
    const int m = idx / kCols, n = idx % kCols;
    if (m >= M) break;  // m only grows with idx
    const int slot = ((m >> 4) * NT + (n >> 4)) * 4 + (m & 3);
    const int l = (n & 15) + 16 * ((m & 15) >> 2);
    float p[kWaves];
#pragma unroll
    for (int v = 0; v < kWaves; ++v) p[v] = red[v * kWaveFloats + slot * 64 + l];
    const float sum = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    out[(size_t)m * N + n0 + n] = narrow<Out>(sum * scale);
  }
}

template <int MT, int NT, int SPW>
int launch_spw(const uint8_t* x, const float* sx, const uint8_t* w, const float* sw, void* out,
               int out_dtype, int M, int N, int K, hipStream_t stream) {
  const dim3 grid(N / (16 * NT)), block(kThreads);
  switch (out_dtype) {
    case BRAID_BF16:
      fp8_gemm_stream_kernel<MT, NT, SPW, __bf16>
          <<<grid, block, 0, stream>>>(x, sx, w, sw, static_cast<__bf16*>(out), M, N, K);
      break;
    case BRAID_F16:
      fp8_gemm_stream_kernel<MT, NT, SPW, _Float16>
          <<<grid, block, 0, stream>>>(x, sx, w, sw, static_cast<_Float16*>(out), M, N, K);
      break;
    default:
      fp8_gemm_stream_kernel<MT, NT, SPW, float>
          <<<grid, block, 0, stream>>>(x, sx, w, sw, static_cast<float*>(out), M, N, K);
      break;
  }
  return hip_status(hipGetLastError(), "fp8_gemm_stream_kernel launch");
}

template <int MT, int NT>
int launch_nt(const uint8_t* x, const float* sx, const uint8_t* w, const float* sw, void* out,
              int out_dtype, int M, int N, int K, hipStream_t stream) {
  switch (K / (kWaves * kStepK)) {
    case 1: return launch_spw<MT, NT, 1>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
    case 2: return launch_spw<MT, NT, 2>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
    case 4: return launch_spw<MT, NT, 4>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
    case 8: return launch_spw<MT, NT, 8>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
    default: return launch_spw<MT, NT, 16>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
  }
}

template <int MT>
int launch_mt(int nt, const uint8_t* x, const float* sx, const uint8_t* w, const float* sw,
              void* out, int out_dtype, int M, int N, int K, hipStream_t stream) {
  switch (nt) {
    case 3: return launch_nt<MT, 3>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
    case 2: return launch_nt<MT, 2>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
    default: return launch_nt<MT, 1>(x, sx, w, sw, out, out_dtype, M, N, K, stream);
  }
}

}  // namespace

bool fp8_gemm_stream_fits(int64_t M, int64_t N, int64_t K) {
  // K = 128 * 8 * SPW for SPW in {1, 2, 4, 8, 16}: 1,024 .. 16,384
  const int64_t spw = K / (kWaves * kStepK);
  return M >= 1 && M <= kStreamMaxM && N >= 16 && N % 16 == 0 && N <= (1 << 24) &&
         K % (kWaves * kStepK) == 0 &&
         (spw == 1 || spw == 2 || spw == 4 || spw == 8 || spw == 16);
}

int fp8_gemm_stream_columns(int64_t N) {
  // the widest column block (at most 48 columns: 64 spill registers at
  // M = 64) that still leaves a workgroup for every CU
  const int cus = device_topo().cus > 0 ? device_topo().cus : 256;
  for (int nt = 3; nt > 1; --nt)
    if (N % (16 * nt) == 0 && N / (16 * nt) >= cus) return nt;
  return 1;
}

int fp8_gemm_stream(const uint8_t* x, const float* sx, const uint8_t* w, const float* sw,
                    void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                    hipStream_t stream) {
  if (!fp8_gemm_stream_fits(M, N, K))
    return fail(BRAID_EINVAL,
                "fp8_gemm_stream: shape outside M <= 64, N % 16 == 0, K = 1024 * 2^i (i < 5)");
  const int nt = fp8_gemm_stream_columns(N);
  const int m = (int)M, n = (int)N, k = (int)K;
  switch ((m + 15) / 16) {
    case 1: return launch_mt<1>(nt, x, sx, w, sw, out, out_dtype, m, n, k, stream);
    case 2: return launch_mt<2>(nt, x, sx, w, sw, out, out_dtype, m, n, k, stream);
    case 3: return launch_mt<3>(nt, x, sx, w, sw, out, out_dtype, m, n, k, stream);
    default: return launch_mt<4>(nt, x, sx, w, sw, out, out_dtype, m, n, k, stream);
  }
}

}  // namespace braid
