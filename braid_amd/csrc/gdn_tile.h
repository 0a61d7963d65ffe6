// Gated DeltaNet tile step for gfx950 (CDNA4, wave64).
//
// One (sequence slot, value head) state tile is S[s, d], s = key index (rows,
// SS = 128), d = value index (columns, HD = 128), row-major with d contiguous:
// the pool layout [n_slots, H, SS, HD] of braid/model/cache.py:127-128. A row
// is 256 bytes of an fp16 pool.
//
// A tile belongs to one 256-thread workgroup: wave w owns the 32 full rows
// [32w, 32w + 32). Lane l of a wave owns the 8-column chunk c8 = l % 16 of rows
// 32w + r + 4i (r = l / 16, i = 0..7), so each of a lane's eight state accesses
// is one 16-byte vector and every wave-wide load or store instruction covers
// four consecutive rows — 1 KiB contiguous for fp16. Measured on MI355X, this
// whole-row pattern streams ~10% faster than per-wave column panels, and the
// state goes through nontemporal loads and stores (it is touched once per
// step and never re-read by the step).
//
// Every reduction of the recurrence runs over rows s for a fixed column d, in
// one fixed order that defines the result's bits:
//   1. sequentially over a lane's eight rows (an fma chain, i = 0..7);
//   2. a butterfly over the four row groups r of a wave (lane xor 16, then xor
//      32): partners add the same two operands, so all lanes agree bitwise;
//   3. across the four waves through LDS, summed as (w0 + w1) + (w2 + w3) by
//      every lane that needs the total.
//
// The state lives in registers in its STORAGE type. Each token widens it to
// fp32, runs the recurrence in fp32 and narrows it back, exactly as a decode
// launch does between its load and its store. The prefill scan therefore
// executes, token for token, the same instructions on the same values as T
// decode launches: chunked prefill equals decode applied T times, bit for bit,
// for fp32, fp16 and bf16 pools alike.
//
// Arithmetic follows braid/kernels/csrc/gdn_decode.cu:198-271 (and the oracle
// braid/reference/gdn_ref.py:69-99):
//   q_hat = q * rsqrt(sum q^2 + 1e-6), k_hat likewise (HF additive epsilon)
//   kv[d]    = sum_s S[s,d] k_hat[s]              (undecayed state)
//   delta[d] = (v[d] - alpha * kv[d]) * beta
//   S'[s,d]  = alpha * S[s,d] + k_hat[s] * delta[d]
//   y[d]     = (sum_s S'[s,d] q_hat[s]) * 128^-0.5  (fp32 S', before narrowing)
// Head h reads key group g = h / (H / G) (grouped layout, gdn_decode.cu:173).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace braid {

constexpr int kSS = 128;                          // key dim (state rows)
constexpr int kHD = 128;                          // value dim (state columns)
constexpr int kWaves = 4;                         // waves per tile
constexpr int kRowsPerWave = kSS / kWaves;        // 32
constexpr int kChunks = kHD / 8;                  // 16 eight-column chunks per row
constexpr int kRowGroups = 64 / kChunks;          // 4 row groups per wave
constexpr int kRowsPerLane = kRowsPerWave / kRowGroups;  // 8
constexpr int kTileThreads = 64 * kWaves;
constexpr float kL2Eps = 1e-6f;
// 128^-0.5 correctly rounded to fp32 (0x3DB504F3).
constexpr float kYScale = 0.088388347648318440550f;

// ---------------------------------------------------------------------------
// Storage types. A Row8 is the eight consecutive elements of one state row a
// lane owns, held in the pool's own encoding. load_nt / store_nt are the
// streaming (nontemporal) accesses used for the state.

struct F32 {};
struct F16 {};
struct BF16 {};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (a quiet NaN).
__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_widen(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
// fp32 -> fp16 bits, round to nearest even, of the ALREADY ROUNDED fp32 value.
// The empty asm pins `f` in a register: without it the compiler may fuse
// fptrunc(fma(a, b, c)) into one mixed-precision fma that rounds straight to
// fp16 (a single rounding instead of fp32-then-fp16). That is a different
// result in rare ties, and the compiler makes the choice per call site, so
// decode and prefill could disagree. The reference narrows the fp32 value
// (gdn_decode.cu:29-30); so does this.
__device__ __forceinline__ uint32_t f16_bits_rne(float f) {
  asm volatile("" : "+v"(f));
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float f16_widen(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

template <class Tag>
struct Row8;

template <>
struct Row8<F32> {
  using elem = float;
  f32x4 lo, hi;
  __device__ __forceinline__ void load_nt(const float* p) {
    lo = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    hi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
  }
  __device__ __forceinline__ void store_nt(float* p) const {
    __builtin_nontemporal_store(lo, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(hi, reinterpret_cast<f32x4*>(p + 4));
  }
  __device__ __forceinline__ float get(int c) const { return c < 4 ? lo[c] : hi[c - 4]; }
  __device__ __forceinline__ void set(int c, float x) {
    if (c < 4) lo[c] = x; else hi[c - 4] = x;
  }
};

template <class Tag>
struct Row8Half {
  using elem = uint16_t;
  u32x4 raw;  // element c sits in bits 16*(c&1) of raw[c>>1]
  __device__ __forceinline__ void load_nt(const uint16_t* p) {
    raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ __forceinline__ void store_nt(uint16_t* p) const {
    __builtin_nontemporal_store(raw, reinterpret_cast<u32x4*>(p));
  }
  __device__ __forceinline__ uint32_t bits(int c) const {
    return (raw[c >> 1] >> (16 * (c & 1))) & 0xffffu;
  }
  __device__ __forceinline__ void put(int c, uint32_t b) {
    const int w = c >> 1, sh = 16 * (c & 1);
    raw[w] = (raw[w] & ~(0xffffu << sh)) | (b << sh);
  }
};

template <>
struct Row8<F16> : Row8Half<F16> {
  __device__ __forceinline__ float get(int c) const { return f16_widen(bits(c)); }
  __device__ __forceinline__ void set(int c, float x) { put(c, f16_bits_rne(x)); }
};

template <>
struct Row8<BF16> : Row8Half<BF16> {
  __device__ __forceinline__ float get(int c) const { return bf16_widen(bits(c)); }
  __device__ __forceinline__ void set(int c, float x) { put(c, bf16_bits_rne(x)); }
};

// ---------------------------------------------------------------------------
// Cross-lane sums. Butterflies over lane-index bits: partners add the same two
// operands (a + b == b + a), so after every stage all lanes of a group hold
// bit-identical partial sums.

__device__ __forceinline__ float xor_shuffle(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Sum over all 64 lanes.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += xor_shuffle(v, m);
  return v;
}

// Sum over a wave's four row groups sharing a column chunk (lane bits 4, 5).
__device__ __forceinline__ float rowgroup_sum(float v) {
  v += xor_shuffle(v, 16);
  v += xor_shuffle(v, 32);
  return v;
}

// ---------------------------------------------------------------------------
// Gate policies: where (alpha, beta) for (row b, head h, token t) come from.

// Gates the caller computed (gdn_decode.cu:102-110): [B, T, H] fp32.
struct PrecomputedGates {
  const float* alpha;
  const float* beta;
  __device__ __forceinline__ void get(int b, int h, int t, int H, int T, float& a,
                                      float& bt) const {
    const size_t i = ((size_t)b * T + t) * H + h;
    a = alpha[i];
    bt = beta[i];
  }
};

template <class ActTag>
struct ActRead;
template <>
struct ActRead<F32> {
  using elem = float;
  __device__ __forceinline__ static float widen(float x) { return x; }
  __device__ __forceinline__ static float round_trip(float x) { return x; }
};
template <>
struct ActRead<BF16> {
  using elem = uint16_t;
  __device__ __forceinline__ static float widen(uint16_t x) { return bf16_widen(x); }
  __device__ __forceinline__ static float round_trip(float x) {
    return bf16_widen(bf16_bits_rne(x));
  }
};

// Gates computed in-kernel from the raw projections, in torch's spelling
// (braid/model/gdn.py:299-300, gdn_decode.cu:112-136):
//   beta  = widen(round_act(1 / (1 + exp(-b))))     sigmoid in the act dtype
//   alpha = exp(A[h] * sp),  sp = x > 20 ? x : log1p(exp(x)),  x = a + dt_bias[h]
// A pad column (seq_lens given, t >= seq_lens[b]) is alpha = 1, beta = 0, which
// leaves the state bit-identical.
template <class ActTag>
struct RawGates {
  using AT = typename ActRead<ActTag>::elem;
  const AT* a_raw;
  const AT* b_raw;
  const float* A;
  const float* dt_bias;
  const int* seq_lens;  // nullptr: every column live
  __device__ __forceinline__ void get(int b, int h, int t, int H, int T, float& a,
                                      float& bt) const {
    if (seq_lens != nullptr && t >= seq_lens[b]) {
      a = 1.f;
      bt = 0.f;
      return;
    }
    const size_t i = ((size_t)b * T + t) * H + h;
    const float e = expf(-ActRead<ActTag>::widen(b_raw[i]));
    bt = ActRead<ActTag>::round_trip(1.f / (1.f + e));
    const float x = ActRead<ActTag>::widen(a_raw[i]) + dt_bias[h];
    const float sp = x > 20.f ? x : log1pf(expf(x));
    a = expf(A[h] * sp);
  }
};

// ---------------------------------------------------------------------------
// Lane geometry within a tile.
struct LaneMap {
  int wave;  // 0..3: rows [32 wave, 32 wave + 32)
  int lane;  // 0..63
  int rg;    // row group 0..3
  int c8;    // column chunk 0..15
  int col0;  // first of this lane's eight columns
  __device__ __forceinline__ LaneMap(int tid) {
    lane = tid & 63;
    wave = tid >> 6;
    rg = lane / kChunks;
    c8 = lane % kChunks;
    col0 = c8 * 8;
  }
  __device__ __forceinline__ int row(int i) const {
    return wave * kRowsPerWave + rg + kRowGroups * i;
  }
};

// Cross-wave exchange buffers for one tile: per-wave column partials of kv and
// of y, kept apart so one token's y exchange never overwrites kv partials a
// slower wave is still reading (and vice versa across tokens).
struct TileLds {
  float kv[kWaves][kHD];
  float y[kWaves][kHD];
};

// q_hat / k_hat for this lane's rows, from the dense [SS] fp32 key-group
// vectors. Every lane of every wave computes the norms with the same reduction
// tree, so every wave sees identical bits.
struct QK {
  float qh[kRowsPerLane];
  float kh[kRowsPerLane];
};

__device__ __forceinline__ void normalize_qk(const LaneMap& L, const float* __restrict__ q,
                                             const float* __restrict__ k, QK& out) {
  const float2 q2 = *reinterpret_cast<const float2*>(q + 2 * L.lane);
  const float2 k2 = *reinterpret_cast<const float2*>(k + 2 * L.lane);
  float qr[kRowsPerLane], kr[kRowsPerLane];
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
    qr[i] = q[L.row(i)];
    kr[i] = k[L.row(i)];
  }
  const float qs = wave_sum(q2.x * q2.x + q2.y * q2.y);
  const float ks = wave_sum(k2.x * k2.x + k2.y * k2.y);
  const float q_inv = rsqrtf(qs + kL2Eps);
  const float k_inv = rsqrtf(ks + kL2Eps);
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
    out.qh[i] = qr[i] * q_inv;
    out.kh[i] = kr[i] * k_inv;
  }
}

// Completes a column sum: the lane's chain value `part` for columns
// col0..col0+7 is reduced over the wave's row groups, exchanged through `buf`
// and summed over the four waves in the fixed order (w0 + w1) + (w2 + w3).
// Every lane returns the eight column totals of its chunk.
__device__ __forceinline__ void tile_column_sums(const LaneMap& L, float (&part)[8],
                                                 float (*buf)[kHD]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) part[c] = rowgroup_sum(part[c]);
  if (L.rg == 0) {
    f32x4 lo, hi;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      lo[c] = part[c];
      hi[c] = part[c + 4];
    }
    *reinterpret_cast<f32x4*>(&buf[L.wave][L.col0]) = lo;
    *reinterpret_cast<f32x4*>(&buf[L.wave][L.col0 + 4]) = hi;
  }
  __syncthreads();
  float w[kWaves][8];
#pragma unroll
  for (int j = 0; j < kWaves; ++j) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(&buf[j][L.col0]);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(&buf[j][L.col0 + 4]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      w[j][c] = lo[c];
      w[j][c + 4] = hi[c];
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) part[c] = (w[0][c] + w[1][c]) + (w[2][c] + w[3][c]);
}

// One token of the recurrence on this lane's 8 x 8 block. `v` holds the eight
// value entries of the lane's columns; `y` receives their outputs (identical
// in every lane of a column chunk). Contains two workgroup barriers, so all
// four waves of the tile must call it together.
template <class Tag>
__device__ __forceinline__ void gdn_token(const LaneMap& L, Row8<Tag> (&S)[kRowsPerLane],
                                          const QK& qk, const float (&v)[8], float alpha,
                                          float beta, TileLds& lds, float (&y)[8]) {
  float kv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) kv[c] = S[0].get(c) * qk.kh[0];
#pragma unroll
  for (int i = 1; i < kRowsPerLane; ++i) {
#pragma unroll
    for (int c = 0; c < 8; ++c) kv[c] = fmaf(S[i].get(c), qk.kh[i], kv[c]);
  }
  tile_column_sums(L, kv, lds.kv);
  float delta[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) delta[c] = (v[c] - alpha * kv[c]) * beta;

  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float nv = fmaf(qk.kh[i], delta[c], alpha * S[i].get(c));
      S[i].set(c, nv);
      acc[c] = fmaf(nv, qk.qh[i], acc[c]);
    }
  }
  tile_column_sums(L, acc, lds.y);
#pragma unroll
  for (int c = 0; c < 8; ++c) y[c] = acc[c] * kYScale;
}

__device__ __forceinline__ void load8(const float* __restrict__ p, float (&out)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    out[c] = a[c];
    out[c + 4] = b[c];
  }
}

__device__ __forceinline__ void store8(float* __restrict__ p, const float (&in)[8]) {
  f32x4 a, b;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    a[c] = in[c];
    b[c] = in[c + 4];
  }
  *reinterpret_cast<f32x4*>(p) = a;
  *reinterpret_cast<f32x4*>(p + 4) = b;
}

}  // namespace braid
