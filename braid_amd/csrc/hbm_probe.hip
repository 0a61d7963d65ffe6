// HBM stream probe at the decode step's access shape, for the roofline.
//
// Not part of the drop-in ABI (include/braid_gdn.h) and not on any product
// path: bench.py loads libbraid_probe.so to measure, on the box it runs on,
// what an in-place stream of 32 KiB state tiles can reach. Each kernel moves
// exactly the decode's state bytes with the decode's lane layout (one
// 256-thread workgroup per tile; lane l of wave w owns the 16-byte chunk l % 16
// of rows 32 w + l / 16 + 4 i, i = 0..7; nontemporal 128-bit accesses), in
// the decode's launch shape (stream_shape.h: tile order and resident
// workgroups per CU), and nothing else, so decode time / probe time is the share of that ceiling
// the decode reaches with its arithmetic, q/k/v/y traffic and gates included.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "stream_shape.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kTileBytes = 128 * 128 * 2;

__device__ __forceinline__ int chunk_offset(int i) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  return (32 * w + (l >> 4) + 4 * i) * 256 + (l & 15) * 16;
}

// Read every chunk of the tile and write it back changed (the decode's
// in-place update of a state tile, without the arithmetic).
__global__ void __launch_bounds__(256)
probe_rmw(char* base, const int* __restrict__ tile_idx, int xc) {
  char* t = base + (size_t)tile_idx[braid::stream_tile(xc)] * kTileBytes;
  u32x4 s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    s[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(t + chunk_offset(i)));
#pragma unroll
  for (int i = 0; i < 8; ++i)
    __builtin_nontemporal_store(s[i] ^ 0x00010001u, reinterpret_cast<u32x4*>(t + chunk_offset(i)));
}

// Read every chunk; `sink` is written only if the data hits an impossible
// pattern, which keeps the loads live without adding traffic.
__global__ void __launch_bounds__(256) probe_read(const char* base, const int* __restrict__ tile_idx,
                                                  u32x4* sink, int xc) {
  const char* t = base + (size_t)tile_idx[braid::stream_tile(xc)] * kTileBytes;
  u32x4 s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    s[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(t + chunk_offset(i)));
  u32x4 a = s[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) a ^= s[i];
  if ((a.x ^ a.y ^ a.z ^ a.w) == 0x9e3779b9u && a.x == 0x7f4a7c15u) sink[threadIdx.x] = a;
}

// Write every chunk.
__global__ void __launch_bounds__(256)
probe_write(char* base, const int* __restrict__ tile_idx, int xc) {
  char* t = base + (size_t)tile_idx[braid::stream_tile(xc)] * kTileBytes;
  const u32x4 v = {threadIdx.x, blockIdx.x, 0x3c003c00u, 0x3c003c00u};
#pragma unroll
  for (int i = 0; i < 8; ++i)
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(t + chunk_offset(i)));
}

// One thread writes the GPU's constant-rate wall clock (s_memrealtime) to
// *out. Launched on a stream between other work, it timestamps the point
// where the work before it has finished (same-stream launches run in order).
__global__ void __launch_bounds__(64) probe_clock(unsigned long long* out) {
  if (threadIdx.x == 0) out[0] = __builtin_amdgcn_s_memrealtime();
}

}  // namespace

extern "C" {

// Enqueues probe_clock on `stream`: *out receives the wall-clock counter when
// the stream reaches it. Ticks per second: braid_probe_clock_hz(). Returns 0
// or a nonzero hipError_t.
int braid_probe_clock(void* out, void* stream) {
  if (out == nullptr) return (int)hipErrorInvalidValue;
  probe_clock<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<unsigned long long*>(out));
  return (int)hipGetLastError();
}

// Rate of the counter braid_probe_clock reads, in ticks per second (0 if the
// runtime cannot say).
double braid_probe_clock_hz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return 0.0;
  return 1000.0 * khz;
}

// One pass over n_tiles 32 KiB tiles at base + tile_idx[t] * 32 KiB, on
// `stream`. kind 0: read-modify-write in place; 1: read only (sink: 4 KiB of
// device memory); 2: write only. Returns 0, or a nonzero hipError_t.
int braid_probe_stream(int kind, void* base, int64_t n_tiles, const int32_t* tile_idx,
                       void* sink, void* stream) {
  if (base == nullptr || tile_idx == nullptr || n_tiles <= 0 || n_tiles > (1 << 30) ||
      kind < 0 || kind > 2 || (kind == 1 && sink == nullptr))
    return (int)hipErrorInvalidValue;
  const dim3 grid((unsigned)n_tiles), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The decode's launch shape for the same tile count (the decode's 16-bit
  // tiles hold its exchange buffer, 4,104 bytes of static LDS).
  // The decode's overrides, read once from the environment as the kernel
  // library reads them.
  static const int remap_env = braid::env_int("BRAID_DECODE_XCD_REMAP");
  static const int cap_env = braid::env_int("BRAID_DECODE_WGS_PER_CU");
  const braid::StreamShape sh = braid::stream_shape(n_tiles, braid::device_topo(), true, 4104, remap_env, cap_env);
  if (kind == 0)
    probe_rmw<<<grid, block, sh.lds_pad, s>>>(static_cast<char*>(base), tile_idx,
                                              sh.xcd_per);
  else if (kind == 1)
    probe_read<<<grid, block, sh.lds_pad, s>>>(static_cast<const char*>(base), tile_idx,
                                               static_cast<u32x4*>(sink), sh.xcd_per);
  else
    probe_write<<<grid, block, sh.lds_pad, s>>>(static_cast<char*>(base), tile_idx,
                                                sh.xcd_per);
  return (int)hipGetLastError();
}

}  // extern "C"
