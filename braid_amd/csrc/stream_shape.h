// Launch shape of a state stream over 32 KiB tiles (one 256-thread workgroup
// per tile): the decode kernels and the HBM probe that measures their ceiling
// share it, so the probe keeps streaming exactly what the decode streams.
//
// Two measured choices (MI355X: 256 CUs in 8 XCDs, cold slot-permuted pools),
// both taken only for a "large" launch: at least 6 tiles per CU for 16-bit
// tiles, 12 for fp32 tiles.
//
// * XCD-contiguous tiles. The dispatcher deals consecutive workgroups to the
//   8 XCDs in turn, so tile order t = blockIdx.x hands each XCD every eighth
//   tile. Remapping workgroup i to tile (i % 8) * (n / 8) + i / 8 gives XCD x
//   the contiguous range [x n / 8, (x + 1) n / 8) instead, walked in order.
//   fp16 decode at B = 96/128/192/256 (with the cap below): 39.4 -> 38.3,
//   51.6 -> 49.4, 75.6 -> 72.6, 100.0 -> 93.8 us; fp32 pool at B = 128:
//   96.9 -> 95.1 us. Up to B = 64 it changes nothing measurable (B = 8 is 2%
//   slower), hence the threshold. Needs n % 8 == 0.
// * Two resident workgroups per CU, not four, by asking for
//   dynamic LDS the kernel does not use. Measured at B = 128 (fp16 pool, cold,
//   XCD-contiguous), residency cap 2 / 3 / 4 / none: 48.5 / 48.8-49.2 / 49.6 /
//   49.6 us; the in-place stream probe alone 46.3 / 47.4 / 47.6 / 47.6 us. B =
//   96: 37.6 / 37.4-37.6 / 38.1 / 38.1 us. With the decode built for two
//   waves per SIMD at this cap (gdn_scan.hip), remap + cap 2 against neither:
//   B = 80 32.4 -> 31.2 us, B = 64 26.2 -> 25.9, B = 48 20.25 -> 20.3, B = 32
//   13.8 -> 14.8. Once the decode issued its loads at the highest wave
//   priority (gdn_scan.hip), B = 48 (6 tiles per CU) joined: default 21.6,
//   remap + cap 2 20.3 us; B = 40 (5 per CU) is the same either way and B =
//   32 is slower capped (15.0 against 12.0); hence 6 tiles per CU. fp32
//   tiles (64 KiB, large from 12
//   tiles per CU) take the cap too: cap 2 / 3 / none at B = 96, 128, 192, 256:
//   70.0 / 70.5 / 70.9, 91.8 / 92.5 / 93.4, 134.7 / 136.9 / 138.2, 178.1 /
//   181.6 / 183.3 us.
//
// The device's CU count, XCD count and LDS per CU come from its HIP
// attributes (device_topo), so a partitioned device gets its own figures:
// dispatch order where it has another XCD count, the cap sized to its LDS.
//
// The caller passes overrides for measurement (-1: no override): remap 0 / 1,
// cap 0 (uncapped) or N > 0. The kernel library takes them from its launch
// knobs, which are read from the environment once, when the library loads,
// and can be set with braid_set_launch_override; a captured graph keeps the
// launch shape it was captured with.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdlib.h>

namespace braid {

// The XCD count the remap below is written for (MI355X: 256 CUs in 8 XCDs).
constexpr int kXcds = 8;

// The tile a workgroup streams (see above): `per` = tiles per XCD (n / 8)
// for the XCD-contiguous order, 0 for dispatch order. Branch-free, from a
// kernel argument, so the tile index needs no read beyond the kernel's
// arguments.
__device__ __forceinline__ int stream_tile(int per) {
  const int remapped = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  return per > 0 ? remapped : (int)blockIdx.x;
}

// What the launch shape needs to know of the current device, from its HIP
// attributes (not assumed): CUs, XCDs (XCCs) and LDS bytes per CU. A
// partitioned MI355X (e.g. one XCD per logical device) reports its own
// partition's figures. Zeros when a query fails: no large-launch choices.
struct DeviceTopo {
  int cus = 0;
  int xcds = 0;
  long lds_per_cu = 0;
};

// Queried once per device ordinal (the attributes do not change while the
// process runs) with that device current.
inline DeviceTopo device_topo() {
  constexpr int kMaxDevices = 64;
  static DeviceTopo cached[kMaxDevices];
  static bool known[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return DeviceTopo{};
  if (dev >= 0 && dev < kMaxDevices && __atomic_load_n(&known[dev], __ATOMIC_ACQUIRE))
    return cached[dev];
  DeviceTopo t;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
    t.cus = v;
  v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess) t.xcds = v;
  v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) ==
      hipSuccess)
    t.lds_per_cu = v;
  if (dev >= 0 && dev < kMaxDevices) {
    cached[dev] = t;  // racing writers store the same values
    __atomic_store_n(&known[dev], true, __ATOMIC_RELEASE);
  }
  return t;
}

struct StreamShape {
  int xcd_per;  // argument of stream_tile
  size_t lds_pad;      // dynamic LDS bytes to request
};

// A non-negative integer from the environment, or -1 when the variable is
// unset, empty or not a whole decimal number.
inline int env_int(const char* name) {
  const char* e = getenv(name);
  if (e == nullptr || e[0] == '\0') return -1;
  char* end = nullptr;
  const long v = strtol(e, &end, 10);
  return (end == e || *end != '\0' || v < 0 || v > (1L << 30)) ? -1 : (int)v;
}

// topo: the device (cus 0: no large-launch choices); narrow: 16-bit tiles;
// static_lds: the kernel's own LDS bytes; remap_env / cap_env: overrides, -1
// for none. The XCD remap is taken only on a device with kXcds XCDs (the
// order stream_tile computes); the residency cap divides the device's own
// LDS per CU.
inline StreamShape stream_shape(long n_tiles, const DeviceTopo& topo, bool narrow,
                                size_t static_lds, int remap_env = -1, int cap_env = -1) {
  const bool large = topo.cus > 0 && n_tiles >= (narrow ? 6L : 12L) * topo.cus;
  StreamShape s{0, 0};
  const bool remap = remap_env >= 0 ? remap_env > 0 : (large && topo.xcds == kXcds);
  s.xcd_per = (remap && n_tiles % kXcds == 0) ? (int)(n_tiles / kXcds) : 0;
  const int cap = cap_env >= 0 ? cap_env : (large && topo.lds_per_cu > 0 ? 2 : 0);
  if (cap > 0 && topo.lds_per_cu > 0) {
    long pad = topo.lds_per_cu / cap - (long)static_lds - 1024;
    if (pad > 65536) pad = 65536;
    s.lds_pad = pad > 0 ? (size_t)pad : 0;
  }
  return s;
}

}  // namespace braid
