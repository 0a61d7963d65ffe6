// Launch shape of a state stream over 32 KiB tiles (one 256-thread workgroup
// per tile): the decode kernels and the HBM probe that measures their ceiling
// share it, so the probe keeps streaming exactly what the decode streams.
//
// Two measured choices (MI355X: 256 CUs in 8 XCDs, cold slot-permuted pools),
// both taken only for a "large" launch: at least 8 tiles per CU for 16-bit
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
//   13.8 -> 14.8; hence 8 tiles per CU. fp32 tiles (64 KiB, large from 12
//   tiles per CU) take the cap too: cap 2 / 3 / none at B = 96, 128, 192, 256:
//   70.0 / 70.5 / 70.9, 91.8 / 92.5 / 93.4, 134.7 / 136.9 / 138.2, 178.1 /
//   181.6 / 183.3 us.
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

constexpr int kXcds = 8;

// The tile a workgroup streams (see above): `per` = tiles per XCD (n / 8)
// for the XCD-contiguous order, 0 for dispatch order. Branch-free, from a
// kernel argument, so the tile index needs no read beyond the kernel's
// arguments.
__device__ __forceinline__ int stream_tile(int per) {
  const int remapped = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  return per > 0 ? remapped : (int)blockIdx.x;
}

struct StreamShape {
  int xcd_per;  // argument of stream_tile
  size_t lds_pad;      // dynamic LDS bytes to request
};

// An integer from the environment, or -1 when the variable is unset.
inline int env_int(const char* name) {
  const char* e = getenv(name);
  return e ? atoi(e) : -1;
}

// cus: CUs of the device (0 if unknown: no large-launch choices);
// narrow: 16-bit tiles; static_lds: the kernel's own LDS bytes;
// remap_env / cap_env: overrides, -1 for none.
inline StreamShape stream_shape(long n_tiles, int cus, bool narrow, size_t static_lds,
                                int remap_env = -1, int cap_env = -1) {
  const bool large = cus > 0 && n_tiles >= (narrow ? 8L : 12L) * cus;
  StreamShape s{0, 0};
  const bool remap = remap_env >= 0 ? remap_env > 0 : large;
  s.xcd_per = (remap && n_tiles % kXcds == 0) ? (int)(n_tiles / kXcds) : 0;
  const int cap = cap_env >= 0 ? cap_env : (large ? 2 : 0);
  if (cap > 0) {
    constexpr long kLdsPerCu = 160 * 1024;
    long pad = kLdsPerCu / cap - (long)static_lds - 1024;
    if (pad > 65536) pad = 65536;
    s.lds_pad = pad > 0 ? (size_t)pad : 0;
  }
  return s;
}

}  // namespace braid
