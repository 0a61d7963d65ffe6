// Gated DeltaNet tile step for gfx950 (CDNA4, wave64).
//
// One (sequence slot, value head) state tile is S[s, d], s = key index (rows,
// SS = 128), d = value index (columns, HD = 128), row-major with d contiguous:
// the pool layout [n_slots, H, SS, HD] of braid/model/cache.py:127-128. A row
// is 256 bytes of an fp16 pool.
//
// Decode layout (8 columns per lane): a tile belongs to one workgroup of four
// waves (256 threads); wave w owns the 32 full rows [32w, 32w + 32). Lane l of
// a wave owns the 8-column chunk cc = l % 16 of rows 32w + r + 4i (r = l / 16,
// i = 0..7), so each of a lane's eight state accesses is one 16-byte vector and
// every wave-wide load or store instruction covers four consecutive rows —
// 1 KiB contiguous for fp16. Measured on MI355X, this whole-row pattern streams
// ~18% faster than per-wave column panels, and the state goes through
// nontemporal loads and stores (it is touched once per step and never re-read
// by the step).
//
// Every reduction of the recurrence runs over rows s for a fixed column d, in
// one fixed order that defines the result's bits:
//   1. sequentially over a lane's eight rows (an fma chain, i = 0..7);
//   2. a butterfly over the four row groups r of a wave (lane xor 16, then xor
//      32): partners add the same two operands, so all lanes agree bitwise;
//   3. across the four row blocks through LDS, as the pairwise tree
//      (w0 + w1) + (w2 + w3), evaluated the same way by every lane that needs
//      the total.
//
// Prefill layouts (ScanMap: 2 columns per lane, or 1 for small launches, whose
// tiles are then split over two workgroups; ScanMapQuarter: 1 column and 16
// rows per lane, a tile over four workgroups): the same rows, chains and tree.
// A column's arithmetic does not depend on which lane holds it, so the results
// are the decode layout's bits.
//
// The state lives in registers in its STORAGE type. Each token widens it to
// fp32, runs the recurrence in fp32 and narrows it back, exactly as a decode
// launch does between its load and its store. The prefill scan therefore
// executes, token for token, the same operations on the same values as T
// decode launches: chunked prefill equals decode applied T times, bit for bit,
// for fp32, fp16 and bf16 pools alike.
//
// Arithmetic follows braid/kernels/csrc/gdn_decode.cu:198-271 (and the oracle
// braid/reference/gdn_ref.py:69-99):
//   q_hat = q * rsqrt(sum q^2 + 1e-6), k_hat likewise (HF additive epsilon)
//   kv[d]    = sum_s S[s,d] k_hat[s]              (undecayed state)
//   delta[d] = (v[d] - alpha * kv[d]) * beta
//   S'[s,d]  = alpha * S[s,d] + k_hat[s] * delta[d]   (as fma(alpha, S, k_hat*delta))
//   y[d]     = (sum_s S'[s,d] q_hat[s]) * 128^-0.5  (fp32 S', before narrowing)
// Head h reads key group g = h / (H / G) (grouped layout, gdn_decode.cu:173).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace braid {

constexpr int kSS = 128;                                 // key dim (state rows)
constexpr int kHD = 128;                                 // value dim (state columns)
constexpr int kWaves = 4;                                // row blocks per column group
constexpr int kRowsPerWave = kSS / kWaves;               // 32
constexpr int kRowGroups = 4;                            // row groups per wave (lane / 16)
constexpr int kLanesPerRowGroup = 64 / kRowGroups;       // 16
constexpr int kRowsPerLane = kRowsPerWave / kRowGroups;  // 8
constexpr float kL2Eps = 1e-6f;
// 128^-0.5 correctly rounded to fp32 (0x3DB504F3).
constexpr float kYScale = 0.088388347648318440550f;

// Threads of a tile's workgroup when each lane owns `cpl` columns.
constexpr int tile_threads(int cpl) { return 64 * kWaves * (8 / cpl); }
constexpr int kDecodeCols = 8;   // columns per lane, decode
constexpr int kPrefillCols = 2;  // columns per lane, prefill

// ---------------------------------------------------------------------------
// Storage types. A Row<Tag, N> is the N consecutive elements of one state row
// a lane owns, held in the pool's own encoding. load_nt / store_nt are the
// streaming (nontemporal) accesses used for the state.

struct F32 {};
struct F16 {};
struct BF16 {};

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (a quiet NaN).
// Used for the activation-dtype round trip of the gates.
__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_widen(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float f16_widen(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two already-rounded fp32 values -> packed 16-bit pair, round to nearest
// even: one v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 on gfx950. Written as a
// vector conversion on purpose: the scalar spelling (_Float16)fmaf(...) lets
// the compiler fuse the fma and the narrowing into one mixed-precision fma
// that rounds ONCE, straight to fp16, which differs in rare ties from the
// reference's fp32-then-narrow (gdn_decode.cu:29-30) and is chosen per call
// site (it broke decode == prefill bit-identity). The packed conversion
// consumes the rounded fp32 results.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, f16x2));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// Element type of a pool of each storage tag.
template <class Tag>
struct Storage;
template <>
struct Storage<F32> { using T = float; };
template <>
struct Storage<F16> { using T = uint16_t; };
template <>
struct Storage<BF16> { using T = uint16_t; };

template <class Tag, int N>
struct Row;

template <int N>
struct Row<F32, N> {
  typedef float vec __attribute__((ext_vector_type(N)));
  vec d;
  __device__ __forceinline__ void load_nt(const float* p) {
    d = __builtin_nontemporal_load(reinterpret_cast<const vec*>(p));
  }
  __device__ __forceinline__ void store_nt(float* p) const {
    __builtin_nontemporal_store(d, reinterpret_cast<vec*>(p));
  }
  __device__ __forceinline__ float get(int c) const { return d[c]; }
  // Columns c and c + 1 (c even).
  __device__ __forceinline__ void set2(int c, float x0, float x1) {
    d[c] = x0;
    d[c + 1] = x1;
  }
  // The row's elements as two halves at p0 and p1 (the split column layout).
  typedef float half_vec __attribute__((ext_vector_type(N / 2)));
  __device__ __forceinline__ void load_nt_halves(const float* p0, const float* p1) {
    const half_vec a = __builtin_nontemporal_load(reinterpret_cast<const half_vec*>(p0));
    const half_vec b = __builtin_nontemporal_load(reinterpret_cast<const half_vec*>(p1));
#pragma unroll
    for (int c = 0; c < N / 2; ++c) {
      d[c] = a[c];
      d[c + N / 2] = b[c];
    }
  }
  __device__ __forceinline__ void store_nt_halves(float* p0, float* p1) const {
    half_vec a, b;
#pragma unroll
    for (int c = 0; c < N / 2; ++c) {
      a[c] = d[c];
      b[c] = d[c + N / 2];
    }
    __builtin_nontemporal_store(a, reinterpret_cast<half_vec*>(p0));
    __builtin_nontemporal_store(b, reinterpret_cast<half_vec*>(p1));
  }
};

template <int N>
struct RowHalf {
  typedef uint32_t vec __attribute__((ext_vector_type(N / 2)));
  vec raw;  // element c sits in bits 16*(c&1) of raw[c>>1]
  __device__ __forceinline__ void load_nt(const uint16_t* p) {
    raw = __builtin_nontemporal_load(reinterpret_cast<const vec*>(p));
  }
  __device__ __forceinline__ void store_nt(uint16_t* p) const {
    __builtin_nontemporal_store(raw, reinterpret_cast<vec*>(p));
  }
  __device__ __forceinline__ uint32_t bits(int c) const {
    return (raw[c >> 1] >> (16 * (c & 1))) & 0xffffu;
  }
};

template <int N>
struct Row<F16, N> : RowHalf<N> {
  __device__ __forceinline__ float get(int c) const { return f16_widen(this->bits(c)); }
  __device__ __forceinline__ void set2(int c, float x0, float x1) {
    this->raw[c >> 1] = pack_f16x2(x0, x1);
  }
};

template <int N>
struct Row<BF16, N> : RowHalf<N> {
  __device__ __forceinline__ float get(int c) const { return bf16_widen(this->bits(c)); }
  __device__ __forceinline__ void set2(int c, float x0, float x1) {
    this->raw[c >> 1] = pack_bf16x2(x0, x1);
  }
};

// One column per lane (the split prefill layout). The 16-bit rows keep their
// element in the low half of a 32-bit register and narrow through the same
// packed conversion as the pairs (the high half is discarded), so the
// rounding is the pairs' bit for bit and the compiler cannot fuse it into the
// producing fma.
template <>
struct Row<F32, 1> {
  float d;
  __device__ __forceinline__ void load_nt(const float* p) { d = __builtin_nontemporal_load(p); }
  __device__ __forceinline__ void store_nt(float* p) const { __builtin_nontemporal_store(d, p); }
  __device__ __forceinline__ float get(int) const { return d; }
  __device__ __forceinline__ void set1(float x) { d = x; }
};

// x as an opaque fp32 register value: a narrowing of the result then starts
// from the rounded fp32 value. Without it the backend can fuse the producing
// fma with a single-element fp16 narrowing into one mixed-precision fma that
// rounds once, straight to 16 bits (seen when two scan tokens share a basic
// block). Costs a register copy when x has another use.
__device__ __forceinline__ float opaque(float x) {
  asm("" : "+v"(x));
  return x;
}

// The first term of a kv chain, S * kh, as fma(S, kh, -0): equal to the
// rounded product for every input (adding -0 changes no value and keeps a -0
// product), and one mixed-precision fma on a 16-bit S instead of a widening
// and a multiply. The -0 goes through opaque() so the fma is not folded back
// into the multiply.
__device__ __forceinline__ float first_term(float s, float kh, float neg_zero) {
  return fmaf(s, kh, neg_zero);
}

struct RowHalf1 {
  uint32_t raw;  // the element in bits 0..15
  __device__ __forceinline__ void load_nt(const uint16_t* p) {
    raw = __builtin_nontemporal_load(p);
  }
  __device__ __forceinline__ void store_nt(uint16_t* p) const {
    __builtin_nontemporal_store((uint16_t)raw, p);
  }
  __device__ __forceinline__ uint32_t bits(int) const { return raw & 0xffffu; }
};

template <>
struct Row<F16, 1> : RowHalf1 {
  __device__ __forceinline__ float get(int c) const { return f16_widen(bits(c)); }
  __device__ __forceinline__ void set1(float x) { raw = pack_f16x2(x, 0.f) & 0xffffu; }
};

template <>
struct Row<BF16, 1> : RowHalf1 {
  __device__ __forceinline__ float get(int c) const { return bf16_widen(bits(c)); }
  __device__ __forceinline__ void set1(float x) { raw = pack_bf16x2(x, 0.f) & 0xffffu; }
};

// Two rows' elements of one column (the one-column prefill layouts): row a in
// bits 0..15 of one register, row b in bits 16..31, so one packed conversion
// narrows both (the mixed-precision fma reads either half directly). Each
// element is rounded on its own, as the single-element rows round it.
template <class Tag>
struct RowPair1;
template <>
struct RowPair1<F32> {
  float d0, d1;
  __device__ __forceinline__ void load_nt(const float* a, const float* b) {
    d0 = __builtin_nontemporal_load(a);
    d1 = __builtin_nontemporal_load(b);
  }
  __device__ __forceinline__ void store_nt(float* a, float* b) const {
    __builtin_nontemporal_store(d0, a);
    __builtin_nontemporal_store(d1, b);
  }
  __device__ __forceinline__ float get(int h) const { return h ? d1 : d0; }
  __device__ __forceinline__ void set(float lo, float hi) {
    d0 = lo;
    d1 = hi;
  }
};
struct RowHalfPair {
  uint32_t raw;
  __device__ __forceinline__ void load_nt(const uint16_t* a, const uint16_t* b) {
    raw = (uint32_t)__builtin_nontemporal_load(a) | ((uint32_t)__builtin_nontemporal_load(b) << 16);
  }
  __device__ __forceinline__ void store_nt(uint16_t* a, uint16_t* b) const {
    __builtin_nontemporal_store((uint16_t)raw, a);
    __builtin_nontemporal_store((uint16_t)(raw >> 16), b);
  }
  __device__ __forceinline__ uint32_t bits(int h) const { return h ? raw >> 16 : raw & 0xffffu; }
};
template <>
struct RowPair1<F16> : RowHalfPair {
  __device__ __forceinline__ float get(int h) const { return f16_widen(bits(h)); }
  __device__ __forceinline__ void set(float lo, float hi) { raw = pack_f16x2(lo, hi); }
};
template <>
struct RowPair1<BF16> : RowHalfPair {
  __device__ __forceinline__ float get(int h) const { return bf16_widen(bits(h)); }
  __device__ __forceinline__ void set(float lo, float hi) { raw = pack_bf16x2(lo, hi); }
};

// N consecutive floats from / to 16-byte-aligned memory (global or LDS).
template <int N>
__device__ __forceinline__ void loadN(const float* __restrict__ p, float (&out)[N]) {
  typedef float vec __attribute__((ext_vector_type(N)));
  const vec a = *reinterpret_cast<const vec*>(p);
#pragma unroll
  for (int c = 0; c < N; ++c) out[c] = a[c];
}

template <int N>
__device__ __forceinline__ void storeN(float* __restrict__ p, const float (&in)[N]) {
  typedef float vec __attribute__((ext_vector_type(N)));
  vec a;
#pragma unroll
  for (int c = 0; c < N; ++c) a[c] = in[c];
  *reinterpret_cast<vec*>(p) = a;
}

// ---------------------------------------------------------------------------
// Cross-lane sums. Butterflies over lane-index bits: partners add the same two
// operands (a + b == b + a), so after every stage all lanes of a group hold
// bit-identical partial sums. Every partner exchange runs on the VALU (DPP
// and gfx950's permlane swaps), not through the LDS crossbar: a ds_bpermute
// costs an LDS round trip per stage, and the decode's reductions are a chain
// of such stages on its critical path.

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, true));
}

// v + (v of lane xor 1), xor 2: DPP quad_perm [1,0,3,2] and [2,3,0,1].
__device__ __forceinline__ float add_xor1(float v) { return v + dpp<0xB1>(v); }
__device__ __forceinline__ float add_xor2(float v) { return v + dpp<0x4E>(v); }

// v + (v of lane xor 4): DPP row_half_mirror gives t[i] = v[7 - i] within each
// 8-lane half row, then quad_perm [3,2,1,0] reads t[4q + 3 - j] at lane
// i = 4q + j, which is v[4 (1 - q) + j] = v[i xor 4]. Two DPP instructions,
// the second fused into the add.
__device__ __forceinline__ float add_xor4(float v) {
  return v + dpp<0x1B>(dpp<0x141>(v));
}

// v + (v of lane xor 8): DPP row_ror:8 (within each 16-lane row, rotating by
// 8 is xor 8).
__device__ __forceinline__ float add_xor8(float v) { return v + dpp<0x128>(v); }

// v + (v of lane xor 16 / xor 32) through v_permlane16_swap /
// v_permlane32_swap: after the swap of v with itself the two results hold the
// even and the odd row's (lane block's) value in every lane, so their sum is
// the pair's sum.
__device__ __forceinline__ float add_xor16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Sum over all 64 lanes: stages xor 1, 2, 4, 8, 16, 32.
__device__ __forceinline__ float wave_sum(float v) {
  return add_xor32(add_xor16(add_xor8(add_xor4(add_xor2(add_xor1(v))))));
}

// Sum over a wave's four row groups sharing a column chunk (lane bits 4, 5):
// v + (lane xor 16), then + (lane xor 32). kPermlane: through the permlane
// swaps (VALU); otherwise through ds_bpermute, which holds no extra registers
// (the fused conv + decode kernels have none to spare at 128 VGPRs). Same
// sums either way (a + b == b + a), so the same bits. (Swaps of v against a
// don't-care register, valid only in row group 0's lanes, which alone store
// the totals, saved a copy per stage but gained nothing on the B = 128
// decode, 47.96 -> 48.00 us, so the full-wave swaps stay.)
template <bool kPermlane = false>
__device__ __forceinline__ float rowgroup_sum(float v) {
  if constexpr (kPermlane) return add_xor32(add_xor16(v));
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// ---------------------------------------------------------------------------
// Gate policies: where (alpha, beta) for (row b, head h, token t) come from.
//
// Each policy splits into load() — the global reads for (row b, head h,
// token t) — and eval_alpha() / eval_beta() — the arithmetic — so a scan can
// issue the next token's reads early. A decode issues the token's gate reads
// (load_decode: raw values and head constants) first of all its reads and
// evaluates each gate once per tile (publish_gates).
struct GateRaw {
  float x0, x1;  // policy-defined raw values
  bool pad;      // a pad column: alpha = 1, beta = 0
};

// A head's gate constants (A[h], dt_bias[h] for raw gates), read once per
// tile alongside the token's raw values, so that a decode issues every gate
// read at its start instead of behind the arithmetic that needs it.
struct GateConst {
  float A, dt_bias;
};

// Marks kernel arguments as used here, in scalar registers: the compiler
// then reads them all in one round instead of each at its first use (a
// kernel's argument reads are scalar loads, and it waited for each group
// before issuing the next).
template <class T>
__device__ __forceinline__ void pin_arg(const T& x) {
  asm volatile("" ::"s"(x));
}
template <class... Ts>
__device__ __forceinline__ void pin_args(const Ts&... xs) {
  (pin_arg(xs), ...);
}

// A value at a wave-uniform address, read through the scalar unit (s_load,
// via the constant address space, which the kernels never write): scalar
// loads are counted apart from the vector memory queue, so a later wait for
// this value does not wait for the vector loads issued after it.
__device__ __forceinline__ int load_uniform(const int* p) {
  typedef const __attribute__((address_space(4))) int* const_i32_ptr;
  return *reinterpret_cast<const_i32_ptr>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ float load_uniform(const float* p) {
  return __int_as_float(load_uniform(reinterpret_cast<const int*>(p)));
}
// A 16-bit value, taken out of its aligned dword (an aligned 4-byte read
// cannot cross a page, so it cannot fault past the end of the tensor).
__device__ __forceinline__ uint16_t load_uniform(const uint16_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t w = (uint32_t)load_uniform(reinterpret_cast<const int*>(a & ~(uintptr_t)3));
  return (uint16_t)(w >> ((a & 2) * 8));
}

// A zero the compiler cannot prove wave-uniform. An address offset by it
// is read with a vector load even when the index is uniform: a decode issues
// its few per-tile reads (gates, head constants) as vector loads ahead of
// everything else, so they go out back to back and, completing in issue
// order, arrive before the tile; as scalar loads the compiler issued them
// one after another, each waiting for the previous, ahead of the tile's
// loads.
__device__ __forceinline__ int lane_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// Gates the caller computed (gdn_decode.cu:102-110): [B, T, H] fp32.
struct PrecomputedGates {
  const float* alpha;
  const float* beta;
  __device__ __forceinline__ GateRaw load(int b, int h, int t, int H, int T) const {
    const size_t i = ((size_t)b * T + t) * H + h;
    return GateRaw{alpha[i], beta[i], false};
  }
  // A live token's gates (t below the row's length), and the head's
  // constants, read once per tile by a scan.
  __device__ __forceinline__ GateRaw load_live(int b, int h, int t, int H, int T) const {
    return load(b, h, t, H, T);
  }
  __device__ __forceinline__ GateConst tile_consts(int) const { return GateConst{0.f, 0.f}; }
  // One decode token's gate reads (T = 1), as vector loads (lane_zero), kept
  // in their storage form until the tile's reads have been issued.
  struct DecodeIn {
    float a, b;
  };
  __device__ __forceinline__ void pin_args() const { braid::pin_args(alpha, beta); }
  __device__ __forceinline__ DecodeIn load_decode(int b, int h, int H) const {
    const size_t i = (size_t)b * H + h + lane_zero();
    return DecodeIn{alpha[i], beta[i]};
  }
  __device__ __forceinline__ static void keep(const DecodeIn& d) {
    asm volatile("" ::"v"(d.a), "v"(d.b));
  }
  // The same reads through the scalar unit, for a wave-uniform h (no vector
  // registers held); keep_uniform marks them used in scalar registers.
  __device__ __forceinline__ DecodeIn load_decode_uniform(int b, int h, int H) const {
    const size_t i = (size_t)b * H + h;
    return DecodeIn{braid::load_uniform(alpha + i), braid::load_uniform(beta + i)};
  }
  __device__ __forceinline__ static void keep_uniform(const DecodeIn& d) {
    asm volatile("" ::"s"(d.a), "s"(d.b));
  }
  __device__ __forceinline__ GateRaw raw_of(const DecodeIn& d) const {
    return GateRaw{d.a, d.b, false};
  }
  __device__ __forceinline__ GateConst consts_of(const DecodeIn&) const {
    return GateConst{0.f, 0.f};
  }
  __device__ __forceinline__ float alpha_of(const GateRaw& r, const GateConst&) const {
    return r.x0;
  }
  __device__ __forceinline__ float eval_alpha(const GateRaw& r, int) const { return r.x0; }
  __device__ __forceinline__ float eval_beta(const GateRaw& r) const { return r.x1; }
  // Live columns of row b: all T (the caller pads with alpha = 1, beta = 0,
  // gdn_decode.cu:553-579, which runs them).
  __device__ __forceinline__ int row_len(int, int T) const { return T; }
  __host__ __device__ bool ragged() const { return false; }
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
  __device__ __forceinline__ GateRaw load(int b, int h, int t, int H, int T) const {
    if (seq_lens != nullptr && t >= seq_lens[b]) return GateRaw{0.f, 0.f, true};
    const size_t i = ((size_t)b * T + t) * H + h;
    return GateRaw{ActRead<ActTag>::widen(a_raw[i]), ActRead<ActTag>::widen(b_raw[i]), false};
  }
  // A live token's gates (t below the row's length: no pad test, so no read
  // of seq_lens), and the head's constants, read once per tile by a scan.
  __device__ __forceinline__ GateRaw load_live(int b, int h, int t, int H, int T) const {
    const size_t i = ((size_t)b * T + t) * H + h;
    return GateRaw{ActRead<ActTag>::widen(a_raw[i]), ActRead<ActTag>::widen(b_raw[i]), false};
  }
  __device__ __forceinline__ GateConst tile_consts(int h) const {
    return GateConst{A[h], dt_bias[h]};
  }
  // One decode token's gate reads: the raw values and the head's constants,
  // as vector loads (lane_zero), kept in their storage form until the tile's
  // reads have been issued (a conversion here would wait for them first).
  // Decode launches carry no seq_lens (every row is live), so there is no pad
  // test: a conditional read would put a branch, and a wait, ahead of the
  // tile's loads.
  struct DecodeIn {
    AT a, b;
    float A, dt_bias;
  };
  __device__ __forceinline__ void pin_args() const { braid::pin_args(a_raw, b_raw, A, dt_bias); }
  __device__ __forceinline__ DecodeIn load_decode(int b, int h, int H) const {
    const int z = lane_zero();
    const size_t i = (size_t)b * H + h + z;
    return DecodeIn{a_raw[i], b_raw[i], A[h + z], dt_bias[h + z]};
  }
  __device__ __forceinline__ static void keep(const DecodeIn& d) {
    asm volatile("" ::"v"(d.a), "v"(d.b), "v"(d.A), "v"(d.dt_bias));
  }
  // The same reads through the scalar unit, for a wave-uniform h (no vector
  // registers held); keep_uniform marks them used in scalar registers.
  __device__ __forceinline__ DecodeIn load_decode_uniform(int b, int h, int H) const {
    const size_t i = (size_t)b * H + h;
    return DecodeIn{braid::load_uniform(a_raw + i), braid::load_uniform(b_raw + i),
                    braid::load_uniform(A + h), braid::load_uniform(dt_bias + h)};
  }
  __device__ __forceinline__ static void keep_uniform(const DecodeIn& d) {
    asm volatile("" ::"s"(d.a), "s"(d.b), "s"(d.A), "s"(d.dt_bias));
  }
  __device__ __forceinline__ GateRaw raw_of(const DecodeIn& d) const {
    return GateRaw{ActRead<ActTag>::widen(d.a), ActRead<ActTag>::widen(d.b), false};
  }
  __device__ __forceinline__ GateConst consts_of(const DecodeIn& d) const {
    return GateConst{d.A, d.dt_bias};
  }
  __device__ __forceinline__ float alpha_of(const GateRaw& r, const GateConst& c) const {
    if (r.pad) return 1.f;
    const float x = r.x0 + c.dt_bias;
    const float sp = x > 20.f ? x : log1pf(expf(x));
    return expf(c.A * sp);
  }
  __device__ __forceinline__ float eval_alpha(const GateRaw& r, int h) const {
    return alpha_of(r, GateConst{A[h], dt_bias[h]});
  }
  // Live columns of row b: seq_lens[b] clamped to [0, T] (a length beyond T
  // or below 0 is legal, test_gdn_raw_gates.py:234-256), or all T.
  __device__ __forceinline__ int row_len(int b, int T) const {
    if (seq_lens == nullptr) return T;
    const int n = seq_lens[b];
    return n < 0 ? 0 : (n > T ? T : n);
  }
  __host__ __device__ bool ragged() const { return seq_lens != nullptr; }
  __device__ __forceinline__ float eval_beta(const GateRaw& r) const {
    if (r.pad) return 0.f;
    const float e = expf(-r.x1);
    return ActRead<ActTag>::round_trip(1.f / (1.f + e));
  }
};

// ---------------------------------------------------------------------------
// Lane geometry within a tile when each lane owns CPL columns.
//
// kSplit (fp32 pools): the lane's CPL columns are two runs of CPL / 2, at
// cc * CPL / 2 and 64 columns further, instead of one run at cc * CPL. A
// lane's fp32 row chunk is then two 16-byte pieces 256 bytes apart, and every
// wave-wide load or store of a piece covers four 256-byte half rows, where
// one run of 32 bytes per lane would leave every other 16 bytes to a second
// instruction. Sums run over rows within a column, so which lane holds a
// column changes no bit.
template <int CPL, bool kSplit = false>
struct LaneMap {
  static constexpr int kGroupCols = kLanesPerRowGroup * CPL;  // columns per wave group
  static constexpr bool kSplitCols = kSplit;
  static constexpr int kRun = kSplit ? CPL / 2 : CPL;         // contiguous columns per run
  int wave;  // 0..(waves per tile - 1)
  int w;     // row block 0..3: rows [32 w, 32 w + 32)
  int lane;  // 0..63
  int rg;    // row group 0..3
  int cc;    // column chunk within the wave's column group, 0..15
  int col0;  // first of this lane's columns
  // part: which kGroupCols-column slice of the tile this workgroup owns, for
  // a tile split over several workgroups (column parts).
  __device__ __forceinline__ LaneMap(int tid, int part = 0) {
    lane = tid & 63;
    wave = tid >> 6;
    w = wave % kWaves;
    rg = lane / kLanesPerRowGroup;
    cc = lane % kLanesPerRowGroup;
    col0 = (part + wave / kWaves) * kGroupCols + cc * kRun;
  }
  __device__ __forceinline__ int row(int i) const {
    return w * kRowsPerWave + rg + kRowGroups * i;
  }
  // The lanes that write a column chunk's outputs: row group 0 of row block
  // cc / 4 (the four row blocks share the stores).
  __device__ __forceinline__ bool stores_y() const { return rg == 0 && cc / 4 == w; }
};

// The lane's CPL values of a [kHD] vector (v, y, an LDS exchange row) in its
// column order: one run, or two runs 64 columns apart.
template <int CPL, bool S>
__device__ __forceinline__ void load_cols(const LaneMap<CPL, S>& L, const float* base,
                                          float (&out)[CPL]) {
  typedef float vec __attribute__((ext_vector_type(LaneMap<CPL, S>::kRun)));
  constexpr int R = LaneMap<CPL, S>::kRun;
#pragma unroll
  for (int run = 0; run < CPL / R; ++run) {
    const vec a = *reinterpret_cast<const vec*>(base + L.col0 + run * (kHD / 2));
#pragma unroll
    for (int c = 0; c < R; ++c) out[run * R + c] = a[c];
  }
}
template <int CPL, bool S>
__device__ __forceinline__ void store_cols(const LaneMap<CPL, S>& L, float* base,
                                           const float (&in)[CPL]) {
  typedef float vec __attribute__((ext_vector_type(LaneMap<CPL, S>::kRun)));
  constexpr int R = LaneMap<CPL, S>::kRun;
#pragma unroll
  for (int run = 0; run < CPL / R; ++run) {
    vec a;
#pragma unroll
    for (int c = 0; c < R; ++c) a[c] = in[run * R + c];
    *reinterpret_cast<vec*>(base + L.col0 + run * (kHD / 2)) = a;
  }
}

// A state row's CPL elements of this lane, from / to the row starting at `row`.
template <class Tag, int CPL, bool S>
__device__ __forceinline__ void load_row(Row<Tag, CPL>& r, const LaneMap<CPL, S>& L,
                                         const typename Storage<Tag>::T* row) {
  if constexpr (S)
    r.load_nt_halves(row + L.col0, row + L.col0 + kHD / 2);
  else
    r.load_nt(row + L.col0);
}
template <class Tag, int CPL, bool S>
__device__ __forceinline__ void store_row(const Row<Tag, CPL>& r, const LaneMap<CPL, S>& L,
                                          typename Storage<Tag>::T* row) {
  if constexpr (S)
    r.store_nt_halves(row + L.col0, row + L.col0 + kHD / 2);
  else
    r.store_nt(row + L.col0);
}

// Lane geometry of the scan (prefill) layout: a lane holds all 32 rows of its
// row block w for CPL columns, so the row-group level of every column sum is
// done in-lane and a column sum crosses lanes only over the four row blocks.
// Lane bits: 0-1 row block w, 2-5 column chunk cc; a wave owns 16 * CPL whole
// columns, so a token needs no workgroup barrier. The lane's rows are indexed
// (rg, i) -> w * 32 + rg + 4 i as in the decode layout, so its four in-lane
// chains are the decode chains of row groups 0..3, combined as
// (rg0 + rg1) + (rg2 + rg3) like the decode's lane-xor-16 / xor-32 stages, and
// the row blocks as (w0 + w1) + (w2 + w3) like the decode's LDS tree: every
// sum has the decode's bits. The row blocks sit in the low lane bits so that
// their two stages are DPP quad permutes (lane xor 1, xor 2) rather than
// permlane swaps across 16 and 32 lanes: a token's kv total is on the scan's
// critical path, and a quad permute is both shorter and one instruction
// (config 4's 4 x 256 tokens 0.1233 -> 0.1203 ms, one 512-token row
// 0.241 -> 0.228 ms; the same bits).
//
// A workgroup is four waves. With two columns per lane they own the tile's
// 128 columns; with one column per lane (kParts = 2) a tile is two
// workgroups, `part` owning columns [64 part, 64 part + 64). Columns never
// meet in the recurrence, so the split changes no bit, and each wave carries
// half the per-token work.
template <int CPL>
struct ScanMap {
  static constexpr int kCPL = CPL;
  static constexpr int kLaneRowGroups = kRowGroups;  // a lane holds all 32 rows of its block
  static constexpr int kColsPerWave = 16 * CPL;
  static constexpr int kWavesPerTile = kHD / kColsPerWave;
  static constexpr int kWaves = 4;  // per workgroup
  static constexpr int kParts = kWavesPerTile / kWaves;
  int wave, lane, cc, w, col0;
  __device__ __forceinline__ ScanMap(int tid, int part) {
    lane = tid & 63;
    wave = tid >> 6;
    cc = lane >> 2;
    w = lane & 3;
    col0 = (part * kWaves + wave) * kColsPerWave + cc * CPL;
  }
  __device__ __forceinline__ int row(int rg, int i) const {
    return w * kRowsPerWave + rg + kRowGroups * i;
  }
  // Row block 0's lanes write the column totals (every lane holds them).
  __device__ __forceinline__ bool stores_y() const { return w == 0; }
};

// Quarter scan layout: one column and two of the four row groups per lane, so
// a lane holds 16 rows and a tile spreads over four workgroups of four waves
// (8 columns per wave). Lane l: row-group half rgh = l % 2 (row groups 2 rgh
// and 2 rgh + 1), row block w = (l / 2) % 4, column cc = l / 8. Column totals:
// in-lane (rg 2rgh + rg 2rgh+1), then lane xor 1 gives (rg0 + rg1) + (rg2 + rg3),
// then xor 2 and xor 4 give (w0 + w1) + (w2 + w3): the decode's order, every
// exchange a DPP stage inside a 16-lane row (no permlane swap; config 4's
// 4 x 256 tokens in this layout 0.1197 -> 0.1163 ms, the same bits).
struct ScanMapQuarter {
  static constexpr int kCPL = 1;
  static constexpr int kLaneRowGroups = 2;
  static constexpr int kColsPerWave = 8;
  static constexpr int kWavesPerTile = kHD / kColsPerWave;
  static constexpr int kWaves = 4;  // per workgroup
  static constexpr int kParts = kWavesPerTile / kWaves;
  int wave, lane, cc, rgh, w, col0;
  __device__ __forceinline__ ScanMapQuarter(int tid, int part) {
    lane = tid & 63;
    wave = tid >> 6;
    rgh = lane & 1;
    w = (lane >> 1) & 3;
    cc = lane >> 3;
    col0 = (part * kWaves + wave) * kColsPerWave + cc;
  }
  // rgl: the lane's row group 0 or 1 (row group 2 rgh + rgl).
  __device__ __forceinline__ int row(int rgl, int i) const {
    return w * kRowsPerWave + 2 * rgh + rgl + kRowGroups * i;
  }
  __device__ __forceinline__ bool stores_y() const { return w == 0 && rgh == 0; }
};

// Eighth scan layout: one column and one row group per lane, so a lane holds
// exactly one of the decode's eight-row chains (rows w * 32 + rg + 4 i) and a
// tile spreads over eight workgroups of four waves (4 columns per wave).
// Lane l: row group rg = l % 4, row block w = (l / 4) % 4, column cc = l / 16.
// Column totals: the in-lane chain, then lane xor 1 and xor 2 give
// (rg0 + rg1) + (rg2 + rg3), then xor 4 and xor 8 give (w0 + w1) + (w2 + w3):
// the decode's order, every exchange inside a 16-lane row (DPP).
struct ScanMapEighth {
  static constexpr int kCPL = 1;
  static constexpr int kLaneRowGroups = 1;
  static constexpr int kColsPerWave = 4;
  static constexpr int kWavesPerTile = kHD / kColsPerWave;
  static constexpr int kWaves = 4;  // per workgroup
  static constexpr int kParts = kWavesPerTile / kWaves;
  int wave, lane, cc, rg, w, col0;
  __device__ __forceinline__ ScanMapEighth(int tid, int part) {
    lane = tid & 63;
    wave = tid >> 6;
    rg = lane & 3;
    w = (lane >> 2) & 3;
    cc = lane >> 4;
    col0 = (part * kWaves + wave) * kColsPerWave + cc;
  }
  __device__ __forceinline__ int row(int i) const {
    return w * kRowsPerWave + rg + kRowGroups * i;
  }
  __device__ __forceinline__ bool stores_y() const { return (lane & 15) == 0; }
};

// Scan layout of a prefill launch by code: 1 and 2 columns per lane
// (ScanMap), 4 for the quarter layout (four workgroups per tile), 8 for the
// eighth layout (eight).
template <int L>
struct ScanLayoutOf {
  using type = ScanMap<L>;
};
template <>
struct ScanLayoutOf<4> {
  using type = ScanMapQuarter;
};
template <>
struct ScanLayoutOf<8> {
  using type = ScanMapEighth;
};

// Column total of the scan layout from a lane's four row-group chains:
// (rg0 + rg1) + (rg2 + rg3) in-lane, then (w0 + w1) + (w2 + w3) across the
// lanes of a quad (lane xor 1, then xor 2).
__device__ __forceinline__ float scan_column_sum(float c0, float c1, float c2, float c3) {
  return add_xor2(add_xor1((c0 + c1) + (c2 + c3)));
}

// Cross-wave exchange buffers for one tile: per-row-block column partials of
// kv and of y, kept apart so one token's y exchange never overwrites kv
// partials a slower wave is still reading (and vice versa across tokens).
struct TileLds {
  float kv[kWaves][kHD];
  float y[kWaves][kHD];
  float gate[2];  // this token's alpha, beta (see publish_gates)
};

// q_hat / k_hat for this lane's rows, from the dense [SS] fp32 key-group
// vectors. Every lane of every wave computes the norms with the same reduction
// tree, so every wave sees identical bits. Split into the loads (QKRaw) and
// the arithmetic (normalize_qk) so a scan can issue the next token's loads
// before it runs the current token.
struct QK {
  float qh[kRowsPerLane];
  float kh[kRowsPerLane];
};

struct QKRaw {
  float2 q2, k2;           // elements 2 lane, 2 lane + 1 (for the norms)
  float qr[kRowsPerLane];  // this lane's rows
  float kr[kRowsPerLane];
};

template <class LM>
__device__ __forceinline__ void load_qk(const LM& L, const float* __restrict__ q,
                                        const float* __restrict__ k, QKRaw& r) {
  r.q2 = *reinterpret_cast<const float2*>(q + 2 * L.lane);
  r.k2 = *reinterpret_cast<const float2*>(k + 2 * L.lane);
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
    r.qr[i] = q[L.row(i)];
    r.kr[i] = k[L.row(i)];
  }
}

// q / k elements 2 lane and 2 lane + 1 (what the norms reduce).
template <class LM>
__device__ __forceinline__ void load_qk2(const LM& L, const float* __restrict__ q,
                                         const float* __restrict__ k, float2& q2, float2& k2) {
  q2 = *reinterpret_cast<const float2*>(q + 2 * L.lane);
  k2 = *reinterpret_cast<const float2*>(k + 2 * L.lane);
}

// One wave's normalised q and k, in LDS in the order a lane reads its rows:
// element r = 32 w + rg + 4 i at [(4 w + rg) * 8 + i], so a lane's eight rows
// are eight consecutive floats.
struct QKLds {
  float q[kSS];
  float k[kSS];
};

__device__ __forceinline__ int qk_lds_pos(int r) {
  return ((r >> 5) * kRowGroups + (r & 3)) * kRowsPerLane + ((r >> 2) & 7);
}

// 1 / sqrt(sum x^2 + 1e-6) of a [128] vector held as x[2 lane], x[2 lane + 1]
// by the 64 lanes of a wave; every lane returns the same bits.
__device__ __forceinline__ float inv_norm(float2 x2) {
  return rsqrtf(wave_sum(x2.x * x2.x + x2.y * x2.y) + kL2Eps);
}

__device__ __forceinline__ void scale_qk(const QKRaw& r, float q_inv, float k_inv, QK& out) {
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
    out.qh[i] = r.qr[i] * q_inv;
    out.kh[i] = r.kr[i] * k_inv;
  }
}

__device__ __forceinline__ void normalize_qk(const QKRaw& r, QK& out) {
  scale_qk(r, inv_norm(r.q2), inv_norm(r.k2), out);
}

// q_hat / k_hat for this lane's rows from the pairs every lane of the wave
// loaded (load_qk2): the norms by the wave butterfly, each lane scales its
// two elements (x * factor, the bits scale_qk gives) and writes them to the
// wave's own LDS copy, and reads back its eight rows. Only this wave touches
// `buf`, so no workgroup barrier is needed.
template <class LM>
__device__ __forceinline__ void normalize_qk_lds(const LM& L, float2 q2, float2 k2, QKLds& buf,
                                                 QK& out) {
  const float qi = inv_norm(q2), ki = inv_norm(k2);
  const int p0 = qk_lds_pos(2 * L.lane), p1 = qk_lds_pos(2 * L.lane + 1);
  buf.q[p0] = q2.x * qi;
  buf.q[p1] = q2.y * qi;
  buf.k[p0] = k2.x * ki;
  buf.k[p1] = k2.y * ki;
  // The reads below take values other lanes of this wave wrote: a wave-scope
  // release/acquire keeps the compiler from moving them ahead of the writes
  // (the hardware already completes a wave's LDS operations in order, so this
  // emits no wait of its own).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int base = (L.w * kRowGroups + L.rg) * kRowsPerLane;
  loadN<kRowsPerLane>(&buf.q[base], out.qh);
  loadN<kRowsPerLane>(&buf.k[base], out.kh);
}

template <class LM>
__device__ __forceinline__ void normalize_qk(const LM& L, const float* __restrict__ q,
                                             const float* __restrict__ k, QK& out) {
  QKRaw r;
  load_qk(L, q, k, r);
  normalize_qk(r, out);
}

// Column sums of the tile are completed in two halves around a workgroup
// barrier, so a scan can put two sums behind ONE barrier:
//   column_sums_post:  reduce the lane's chain values over the wave's row
//                      groups and (row group 0) write them to buf[row block];
//   column_sums_take:  after the barrier, read the four row blocks' partials
//                      and add them by the fixed tree (w0 + w1) + (w2 + w3).
// Every lane ends with the totals of its columns.
template <bool kPermlane = false, int CPL, bool S>
__device__ __forceinline__ void column_sums_post(const LaneMap<CPL, S>& L, float (&part)[CPL],
                                                 float (*buf)[kHD]) {
#pragma unroll
  for (int c = 0; c < CPL; ++c) part[c] = rowgroup_sum<kPermlane>(part[c]);
  if (L.rg == 0) store_cols(L, buf[L.w], part);
}

template <int CPL, bool S>
__device__ __forceinline__ void column_sums_take(const LaneMap<CPL, S>& L, float (&part)[CPL],
                                                 float (*buf)[kHD]) {
  float wv[kWaves][CPL];
#pragma unroll
  for (int j = 0; j < kWaves; ++j) load_cols(L, buf[j], wv[j]);
#pragma unroll
  for (int c = 0; c < CPL; ++c) part[c] = (wv[0][c] + wv[1][c]) + (wv[2][c] + wv[3][c]);
}

// kv chain of one token: kv[c] = sum over the lane's eight rows of
// S[i][c] * k_hat[i], in row order.
template <class Tag, int CPL>
__device__ __forceinline__ void kv_partials(const Row<Tag, CPL> (&S)[kRowsPerLane], const QK& qk,
                                            float (&kv)[CPL]) {
#pragma unroll
  for (int c = 0; c < CPL; ++c) kv[c] = S[0].get(c) * qk.kh[0];
#pragma unroll
  for (int i = 1; i < kRowsPerLane; ++i) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) kv[c] = fmaf(S[i].get(c), qk.kh[i], kv[c]);
  }
}

// The update phase of one token, given the column totals kv: delta, the state
// update narrowed to the storage type, and the readout's chain values.
template <class Tag, int CPL>
__device__ __forceinline__ void update_state(Row<Tag, CPL> (&S)[kRowsPerLane], const QK& qk,
                                             const float (&v)[CPL], const float (&kv)[CPL],
                                             float alpha, float beta, float (&acc)[CPL]) {
  float delta[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) delta[c] = (v[c] - alpha * kv[c]) * beta;
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] = 0.f;
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
#pragma unroll
    for (int c = 0; c < CPL; c += 2) {
      // S' = alpha * S + k_hat * delta, contracted as fma(alpha, S, k_hat * delta):
      // the 16-bit S feeds the fma directly (v_fma_mix, exact widening), one
      // instruction fewer per element than widening, scaling, then fusing.
      const float n0 = fmaf(alpha, S[i].get(c), qk.kh[i] * delta[c]);
      const float n1 = fmaf(alpha, S[i].get(c + 1), qk.kh[i] * delta[c + 1]);
      S[i].set2(c, n0, n1);
      acc[c] = fmaf(n0, qk.qh[i], acc[c]);
      acc[c + 1] = fmaf(n1, qk.qh[i], acc[c + 1]);
    }
  }
}

// One token of the recurrence on this lane's 8 x CPL block. `v` holds the
// value entries of the lane's columns; `y` receives their outputs (identical
// in every lane of a column chunk). alpha and beta are read from lds.gate
// after the first barrier, so whoever writes them must do so before it
// (publish_gates). Contains two workgroup barriers, so all waves of the tile
// must call it together.
template <class Tag, int CPL, bool kPermlane = false, bool kSplit>
__device__ __forceinline__ void gdn_token(const LaneMap<CPL, kSplit>& L,
                                          Row<Tag, CPL> (&S)[kRowsPerLane], const QK& qk,
                                          const float (&v)[CPL], TileLds& lds,
                                          float (&y)[CPL]) {
  float kv[CPL];
  kv_partials<Tag, CPL>(S, qk, kv);
  column_sums_post<kPermlane>(L, kv, lds.kv);
  __syncthreads();
  column_sums_take(L, kv, lds.kv);
  float acc[CPL];
  update_state<Tag, CPL>(S, qk, v, kv, lds.gate[0], lds.gate[1], acc);
  column_sums_post<kPermlane>(L, acc, lds.y);
  __syncthreads();
  column_sums_take(L, acc, lds.y);
#pragma unroll
  for (int c = 0; c < CPL; ++c) y[c] = acc[c] * kYScale;
}

// One token of the scan on this lane's 32 x CPL block (S[rg][i] = row
// w * 32 + rg + 4 i), in the scan layout: the decode token's arithmetic, each
// element's operations in the decode's order. kh / qh hold the row block's 32
// normalised key / query entries in row order.
// kOpaqueNarrow: narrow each new state element through opaque() (for callers
// whose code shape lets the backend contract the narrowing).
template <class Tag, int CPL, bool kOpaqueNarrow = false>
__device__ __forceinline__ void scan_token(Row<Tag, CPL> (&S)[kRowGroups][kRowsPerLane],
                                           const float (&kh)[kRowsPerWave],
                                           const float (&qh)[kRowsPerWave],
                                           const float (&v)[CPL], float alpha, float beta,
                                           float (&y)[CPL]) {
  float ch[kRowGroups][CPL];
  const float nz = opaque(-0.0f);
#pragma unroll
  for (int rg = 0; rg < kRowGroups; ++rg) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) ch[rg][c] = first_term(S[rg][0].get(c), kh[rg], nz);
#pragma unroll
    for (int i = 1; i < kRowsPerLane; ++i) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) ch[rg][c] = fmaf(S[rg][i].get(c), kh[rg + kRowGroups * i], ch[rg][c]);
    }
  }
  float delta[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const float kv = scan_column_sum(ch[0][c], ch[1][c], ch[2][c], ch[3][c]);
    delta[c] = (v[c] - alpha * kv) * beta;
  }
#pragma unroll
  for (int rg = 0; rg < kRowGroups; ++rg) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) ch[rg][c] = 0.f;
#pragma unroll
    for (int i = 0; i < kRowsPerLane; ++i) {
      const int r = rg + kRowGroups * i;
      if constexpr (CPL == 1) {
        // Both uses of the new value take the barrier's output, so it costs
        // no register copy.
        float n0 = fmaf(alpha, S[rg][i].get(0), kh[r] * delta[0]);
        if constexpr (kOpaqueNarrow) n0 = opaque(n0);
        S[rg][i].set1(n0);
        ch[rg][0] = fmaf(n0, qh[r], ch[rg][0]);
      } else {
#pragma unroll
        for (int c = 0; c < CPL; c += 2) {
          const float n0 = fmaf(alpha, S[rg][i].get(c), kh[r] * delta[c]);
          const float n1 = fmaf(alpha, S[rg][i].get(c + 1), kh[r] * delta[c + 1]);
          S[rg][i].set2(c, n0, n1);
          ch[rg][c] = fmaf(n0, qh[r], ch[rg][c]);
          ch[rg][c + 1] = fmaf(n1, qh[r], ch[rg][c + 1]);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c)
    y[c] = scan_column_sum(ch[0][c], ch[1][c], ch[2][c], ch[3][c]) * kYScale;
}

// The one-column layout's token over row pairs: P[p][i] holds rows of row
// groups 2p (low half) and 2p + 1 (high half), i.e. rows w * 32 + rg + 4 i.
// Each element's operations and each chain's order are scan_token's.
template <class Tag, bool kOpaqueNarrow = false>
__device__ __forceinline__ void scan_token_pairs(RowPair1<Tag> (&P)[2][kRowsPerLane],
                                                 const float (&kh)[kRowsPerWave],
                                                 const float (&qh)[kRowsPerWave], float v,
                                                 float alpha, float beta, float& y) {
  float ch[kRowGroups];
  const float nz = opaque(-0.0f);
#pragma unroll
  for (int rg = 0; rg < kRowGroups; ++rg) {
    ch[rg] = first_term(P[rg >> 1][0].get(rg & 1), kh[rg], nz);
#pragma unroll
    for (int i = 1; i < kRowsPerLane; ++i)
      ch[rg] = fmaf(P[rg >> 1][i].get(rg & 1), kh[rg + kRowGroups * i], ch[rg]);
  }
  const float kv = scan_column_sum(ch[0], ch[1], ch[2], ch[3]);
  const float delta = (v - alpha * kv) * beta;
#pragma unroll
  for (int rg = 0; rg < kRowGroups; ++rg) ch[rg] = 0.f;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
#pragma unroll
    for (int i = 0; i < kRowsPerLane; ++i) {
      float n[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        n[h] = fmaf(alpha, P[p][i].get(h), kh[2 * p + h + kRowGroups * i] * delta);
        if constexpr (kOpaqueNarrow) n[h] = opaque(n[h]);
      }
      P[p][i].set(n[0], n[1]);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        ch[2 * p + h] = fmaf(n[h], qh[2 * p + h + kRowGroups * i], ch[2 * p + h]);
    }
  }
  y = scan_column_sum(ch[0], ch[1], ch[2], ch[3]) * kYScale;
}

// One token of the quarter layout on this lane's 16 rows x 1 column: S[rgl][i]
// is row w * 32 + 2 rgh + rgl + 4 i, kh / qh hold the same rows. Each
// element's operations are scan_token's (and so the decode's), in the same
// order; the column totals follow the layout's tree.
template <class Tag, bool kOpaqueNarrow = false>
__device__ __forceinline__ void scan_token_quarter(RowPair1<Tag> (&P)[kRowsPerLane],
                                                   const float (&kh)[2][kRowsPerLane],
                                                   const float (&qh)[2][kRowsPerLane], float v,
                                                   float alpha, float beta, float& y) {
  float ch[2];
  const float nz = opaque(-0.0f);
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    ch[g] = first_term(P[0].get(g), kh[g][0], nz);
#pragma unroll
    for (int i = 1; i < kRowsPerLane; ++i) ch[g] = fmaf(P[i].get(g), kh[g][i], ch[g]);
  }
  const float kv = add_xor4(add_xor2(add_xor1(ch[0] + ch[1])));
  const float delta = (v - alpha * kv) * beta;
  ch[0] = ch[1] = 0.f;
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) {
    float n[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      n[g] = fmaf(alpha, P[i].get(g), kh[g][i] * delta);
      if constexpr (kOpaqueNarrow) n[g] = opaque(n[g]);
    }
    P[i].set(n[0], n[1]);
#pragma unroll
    for (int g = 0; g < 2; ++g) ch[g] = fmaf(n[g], qh[g][i], ch[g]);
  }
  y = add_xor4(add_xor2(add_xor1(ch[0] + ch[1]))) * kYScale;
}

// One token of the eighth layout on this lane's chain of 8 rows x 1 column:
// P[m] holds rows i = 2m (low half) and 2m + 1 (high half) of the chain
// (row w * 32 + rg + 4 i); kh / qh hold the same rows. Each element's
// operations are scan_token's (and so the decode's), in the same order; the
// column totals follow the layout's tree.
template <class Tag, bool kOpaqueNarrow = false>
__device__ __forceinline__ void scan_token_eighth(RowPair1<Tag> (&P)[kRowsPerLane / 2],
                                                  const float (&kh)[kRowsPerLane],
                                                  const float (&qh)[kRowsPerLane], float v,
                                                  float alpha, float beta, float& y) {
  const float nz = opaque(-0.0f);
  float ch = first_term(P[0].get(0), kh[0], nz);
#pragma unroll
  for (int i = 1; i < kRowsPerLane; ++i) ch = fmaf(P[i >> 1].get(i & 1), kh[i], ch);
  const float kv = add_xor8(add_xor4(add_xor2(add_xor1(ch))));
  const float delta = (v - alpha * kv) * beta;
  ch = 0.f;
#pragma unroll
  for (int m = 0; m < kRowsPerLane / 2; ++m) {
    float n[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      n[h] = fmaf(alpha, P[m].get(h), kh[2 * m + h] * delta);
      if constexpr (kOpaqueNarrow) n[h] = opaque(n[h]);
    }
    P[m].set(n[0], n[1]);
#pragma unroll
    for (int h = 0; h < 2; ++h) ch = fmaf(n[h], qh[2 * m + h], ch);
  }
  y = add_xor8(add_xor4(add_xor2(add_xor1(ch)))) * kYScale;
}

// Computes one token's gates once per tile and leaves them in lds.gate for
// gdn_token: wave 0 evaluates alpha (exp, log1p, exp), wave 1 beta (exp and a
// divide), from the inputs every wave loaded. The next workgroup barrier
// publishes them. The
// arithmetic is the policy's own, so which wave runs it changes no bit.
template <class Gates, class LM>
__device__ __forceinline__ void publish_gates(const LM& L, const Gates& gates, const GateRaw& r,
                                              const GateConst& c, TileLds& lds) {
  if (L.wave == 0) {
    const float a = gates.alpha_of(r, c);
    if (L.lane == 0) lds.gate[0] = a;
  } else if (L.wave == 1) {
    const float bt = gates.eval_beta(r);
    if (L.lane == 0) lds.gate[1] = bt;
  }
}

}  // namespace braid
