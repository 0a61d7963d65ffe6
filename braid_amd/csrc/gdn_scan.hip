// Batched Gated DeltaNet decode step and chunk prefill scan for gfx950.
//
// Both kernels launch one workgroup per (batch row, value head) tile and run
// the same per-token arithmetic with the same summation trees: decode with
// four waves of 32 state rows x 128 columns (gdn_token, column sums finished
// across waves in LDS), prefill with four waves of 128 rows x 32 columns
// (scan_token, column sums finished inside each wave, no barrier per token).
// Decode loads the tile from the slot-indexed pool, runs one token and stores
// it back; prefill loads it once, runs T tokens with the tile resident in
// registers (in the pool's storage type) and stores it once. Reference behaviour: braid/kernels/csrc/gdn_decode.cu:156-272 (decode)
// and :467-551 (prefill); entry-point contracts :313-441 and :553-699.
#include <algorithm>
#include <cmath>
#include <deque>
#include <functional>
#include <map>
#include <mutex>
#include <queue>
#include <vector>
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "capi_common.h"
#include "conv_common.h"
#include "gdn_tile.h"
#include "stream_shape.h"

namespace braid {
namespace {

// One decode token for the tile (workgroup index = (b * H + h) * P + part).
//
// P column parts: the tile's 128 columns are split over P workgroups of four
// waves, part p owning columns [128 p / P, 128 (p + 1) / P) with 8 / P columns
// per lane. Every column sum runs over rows within the column, so a part
// needs nothing from the others: each lane keeps the same eight rows and its
// chains, the row-group butterfly and the cross-wave tree are unchanged, and
// the results are the one-part layout's bits. Small launches use 2 or 4 parts
// to spread each tile's arithmetic over more CUs (its latency is the
// per-lane work, which shrinks with the columns). fp32 pools split a lane's
// columns into two runs 64 apart only with one part.
//
// kWavesPerSimd bounds the register budget: 4 (128 VGPRs) where up to four
// workgroups share a CU; 2 for the large launches that stream_shape caps at
// two workgroups per CU, where 256 VGPRs cost no residency and the compiler
// schedules the prologue's loads more freely (169 VGPRs; B = 128: 47.92 ->
// 47.63 us a step in one A/B run).
template <class Tag, class Gates, int P, int kWavesPerSimd = 4>
__global__ void __launch_bounds__(tile_threads(kDecodeCols))
__attribute__((amdgpu_waves_per_eu(1, kWavesPerSimd)))
gdn_decode_kernel(typename Storage<Tag>::T* __restrict__ pool, const int* __restrict__ slot_idx,
                  const float* __restrict__ q, const float* __restrict__ k,
                  const float* __restrict__ v, Gates gates, float* __restrict__ y, int H,
                  int heads_per_group, long q_row, long k_row, long v_row, int xcd_per) {
  constexpr int CPL = kDecodeCols / P;
  static_assert(P == 1 || P == 2 || P == 4, "1, 2 or 4 column parts");
  using ST = typename Storage<Tag>::T;
  // Every argument in registers at once: one round of argument reads, not
  // one per first use.
  // The loads are issued at the highest wave priority and the arithmetic at
  // the lowest: a workgroup that starts while the CU's other workgroup is in
  // its arithmetic then puts its tile's reads in flight first, before more of
  // the other's VALU work (B = 128: 47.57 -> 47.32 us a step, bf16 and fp32
  // pools about 1% faster, over three alternated runs each).
  __builtin_amdgcn_s_setprio(3);
  pin_args(pool, slot_idx, q, k, v, y, H, heads_per_group, q_row, k_row, v_row, xcd_per);
  gates.pin_args();
  const int wg = stream_tile(xcd_per);
  const int tix = P == 1 ? wg : wg / P;
  const int part = wg - tix * P;
  const int b = tix / H;
  const int h = tix - b * H;
  const int g = h / heads_per_group;
  const LaneMap<CPL, std::is_same<Tag, F32>::value && P == 1> L(threadIdx.x, part);
  __shared__ TileLds lds;
  __shared__ QKLds qk_lds[kWaves];

  // Reads in issue order: the slot (the slot map lives in device memory, so
  // one captured graph serves any slot assignment, gdn_decode.cu:230-236);
  // the gates' inputs (vector loads, see lane_zero), so their arithmetic runs
  // while the tile is still in flight (vector loads complete in issue order);
  // for 16-bit pools q/k/v, so the norms wait only for them; then, once the
  // slot is known, the tile. An fp32 pool's body has no registers to spare
  // for early q/k/v and issues them after the tile. The scheduling barriers
  // keep this order: the slot's round trip overlaps the issue of the others.
  constexpr bool kEarly = !std::is_same<Tag, F32>::value;
  const int slot = load_uniform(slot_idx + b);
  const typename Gates::DecodeIn gin = gates.load_decode(b, h, H);
  const float* qg = q + (size_t)b * q_row + (size_t)g * kSS;
  const float* kg = k + (size_t)b * k_row + (size_t)g * kSS;
  const float* vh = v + (size_t)b * v_row + (size_t)h * kHD;
  float2 q2, k2;
  float vv[CPL];
  if (kEarly) {
    load_qk2(L, qg, kg, q2, k2);
    load_cols(L, vh, vv);
  }
  __builtin_amdgcn_sched_barrier(0);
  ST* tile = pool + ((size_t)slot * H + h) * (kSS * kHD);
  Row<Tag, CPL> S[kRowsPerLane];
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) load_row(S[i], L, tile + (size_t)L.row(i) * kHD);
  if (!kEarly) {
    load_cols(L, vh, vv);
    load_qk2(L, qg, kg, q2, k2);
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(0);
  // Every wave holds the gate inputs here, so their reads stay where they
  // were issued rather than moving into the wave that evaluates each gate.
  Gates::keep(gin);
  publish_gates(L, gates, gates.raw_of(gin), gates.consts_of(gin), lds);
  QK qk;
  normalize_qk_lds(L, q2, k2, qk_lds[L.wave], qk);

  float yy[CPL];
  // Row-group sums through the permlane swaps, not the LDS crossbar: this
  // kernel has the registers, and a B = 128 step gains 0.66 us (48.48 ->
  // 47.82) from the shorter per-tile chain.
  gdn_token<Tag, CPL, true>(L, S, qk, vv, lds, yy);

#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) store_row(S[i], L, tile + (size_t)L.row(i) * kHD);
  // Each column's totals sit in all lanes of its chunk; one lane per chunk writes them.
  if (L.stores_y()) store_cols(L, y + ((size_t)b * H + h) * kHD, yy);
}

// The conv1d decode step fused into the GDN decode step (one launch for the
// mixer's conv and recurrence): one workgroup per (batch row b, key group g)
// owns the HPG value heads of the group, HPG tiles of four waves each. Its
// threads first run the conv step (conv_step, the conv kernels' arithmetic)
// for the group's q and k channels and the heads' v channels, updating those
// channels' windows in the conv pool and leaving the outputs in LDS; then each
// tile runs the decode token on them exactly as gdn_decode_kernel does on q/k/v
// read from memory. So the outputs, the state and the windows equal
// conv1d_decode followed by gdn_decode, bit for bit. A group's q/k windows are
// advanced once because one workgroup owns all heads that read them. The conv
// outputs never go to memory: nothing but the recurrence reads them.
template <int HPG>
struct ConvDecodeLds {
  TileLds tile[HPG];
  float qkv[2 + HPG][kHD];  // conv outputs: q, k, then each head's v
};

// The decode token of tile t of a conv + decode workgroup, on the conv
// outputs in LDS (after the barrier that publishes them), then the stores.
template <class Tag, int HPG, class LM>
__device__ __forceinline__ void decode_token_from_lds(const LM& L,
                                                      Row<Tag, kDecodeCols> (&S)[kRowsPerLane],
                                                      ConvDecodeLds<HPG>& lds, int t,
                                                      typename Storage<Tag>::T* tile,
                                                      float* y_row) {
  constexpr int CPL = kDecodeCols;
  float vv[CPL];
  load_cols(L, lds.qkv[2 + t], vv);
  QK qk;
  normalize_qk(L, lds.qkv[0], lds.qkv[1], qk);
  float yy[CPL];
  gdn_token<Tag, CPL>(L, S, qk, vv, lds.tile[t], yy);
#pragma unroll
  for (int i = 0; i < kRowsPerLane; ++i) store_row(S[i], L, tile + (size_t)L.row(i) * kHD);
  if (L.stores_y()) store_cols(L, y_row, yy);
}

template <class Tag, class XT, class Gates, int HPG>
__device__ __forceinline__ void conv_decode_body(typename Storage<Tag>::T* __restrict__ pool,
                                                 float* __restrict__ conv_pool,
                                                 const int* __restrict__ slot_idx,
                                                 const XT* __restrict__ x,
                                                 const float* __restrict__ conv_w,
                                                 const float* __restrict__ conv_b, Gates gates,
                                                 float* __restrict__ y, int H, int G, int C) {
  constexpr int CPL = kDecodeCols, kK = 4;
  constexpr int kTileThreads = tile_threads(CPL);
  using ST = typename Storage<Tag>::T;
  pin_args(pool, conv_pool, slot_idx, x, conv_w, conv_b, y, H, G, C);
  gates.pin_args();
  const int b = blockIdx.x / G;
  const int g = blockIdx.x - b * G;
  // The conv-first order below serves 16-bit pools with two heads per group
  // (every Qwen3.5 GDN layer); other shapes load the state first, which their
  // registers allow without spilling.
  constexpr bool kConvFirst = sizeof(typename Storage<Tag>::T) == 2 && HPG == 2;
  // The tile of this wave's threads, uniform in the wave (in the conv-first
  // order, where the head and the tile's address then live in scalar
  // registers).
  const int t = kConvFirst ? __builtin_amdgcn_readfirstlane(threadIdx.x / kTileThreads)
                           : (int)(threadIdx.x / kTileThreads);
  const int h = g * HPG + t;
  const LaneMap<CPL, std::is_same<Tag, F32>::value> L(threadIdx.x % kTileThreads);

  __shared__ ConvDecodeLds<HPG> lds;

  // The group's conv channels: segment 0 = q (channels g*SS..), 1 = k
  // (G*SS + g*SS..), 2 + j = v of head g*HPG + j (2*G*SS + head*HD..).
  // Loads complete in issue order, so in the conv-first order the conv's small
  // loads are issued before the state's and the conv arithmetic then overlaps
  // the state's arrival; an fp32 tile, or one head per group (two channels
  // per thread), leaves no registers for that at four waves per SIMD, so
  // there the state is loaded first.
  constexpr int kConv = (2 + HPG) * kHD;
  constexpr int kThreads = kTileThreads * HPG;
  constexpr int kPer = (kConv + kThreads - 1) / kThreads;
  auto channel = [&](int e) {
    const int seg = e / kHD, off = e - seg * kHD;
    return seg < 2 ? seg * G * kSS + g * kSS + off
                   : 2 * G * kSS + (g * HPG + seg - 2) * kHD + off;
  };
  Row<Tag, CPL> S[kRowsPerLane];
  if constexpr (kConvFirst) {
    // Reads in issue order: the slot (scalar); what does not need it (gate
    // inputs, conv weights, biases and inputs); then, once the slot is known,
    // the conv windows and then the state. Loads complete in issue order, so
    // the gate and conv arithmetic overlaps the state's arrival (windows
    // ahead of the state: 24 config-3 layers 730.6 -> 720.6 us). The
    // scheduling barriers keep this order.
    const int slot = load_uniform(slot_idx + b);
    const typename Gates::DecodeIn gin = gates.load_decode_uniform(b, h, H);
    float w[kPer][kK], wt[kPer][kK], bv[kPer];
    XT xr[kPer];  // widened where used: a conversion here would wait for the read
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
      const int e = threadIdx.x + m * kThreads;
      if (kConv % kThreads == 0 || e < kConv) {
        const int c = channel(e);
        load_weights<kK>(conv_w + (size_t)c * kK, wt[m]);
        xr[m] = x[(size_t)b * C + c];
        bv[m] = conv_b != nullptr ? conv_b[c] : 0.f;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    ST* tile = pool + ((size_t)slot * H + h) * (kSS * kHD);
    // The slot's windows: a wave-uniform base and a 32-bit per-lane offset,
    // so the window store needs one vector register for its address.
    float* const win = conv_pool + (size_t)slot * C * kK;
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
      const int e = threadIdx.x + m * kThreads;
      if (kConv % kThreads == 0 || e < kConv)
        load_weights<kK>(win + (unsigned)channel(e) * kK, w[m]);
    }
#pragma unroll
    for (int i = 0; i < kRowsPerLane; ++i) load_row(S[i], L, tile + (size_t)L.row(i) * kHD);
    __builtin_amdgcn_sched_barrier(0);
    Gates::keep_uniform(gin);
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
      const int e = threadIdx.x + m * kThreads;
      if (kConv % kThreads == 0 || e < kConv) {
        const int c = channel(e), seg = e / kHD;
        lds.qkv[seg][e - seg * kHD] = conv_step_b<kK>(w[m], conv_widen(xr[m]), wt[m], bv[m],
                                                      conv_b != nullptr);
        store_window<kK>(win + (unsigned)c * kK, w[m]);
      }
    }
    publish_gates(L, gates, gates.raw_of(gin), gates.consts_of(gin), lds.tile[t]);
    __syncthreads();
    decode_token_from_lds<Tag, HPG>(L, S, lds, t, tile, y + ((size_t)b * H + h) * kHD);
  } else {
    const int slot = slot_idx[b];
    ST* tile = pool + ((size_t)slot * H + h) * (kSS * kHD);
#pragma unroll
    for (int i = 0; i < kRowsPerLane; ++i) load_row(S[i], L, tile + (size_t)L.row(i) * kHD);
    for (int e = threadIdx.x; e < kConv; e += kThreads) {
      const int c = channel(e), seg = e / kHD;
      float* st = conv_pool + ((size_t)slot * C + c) * kK;
      float w[kK], wt[kK];
      load_window<kK>(st, conv_w + (size_t)c * kK, w, wt);
      lds.qkv[seg][e - seg * kHD] = conv_step<kK>(w, conv_widen(x[(size_t)b * C + c]), wt,
                                                  conv_b, c);
      store_window<kK>(st, w);
    }
    __syncthreads();
    publish_gates(L, gates, gates.load(b, h, 0, H, 1), GateConst{gates.A[h], gates.dt_bias[h]},
                  lds.tile[t]);
    decode_token_from_lds<Tag, HPG>(L, S, lds, t, tile, y + ((size_t)b * H + h) * kHD);
  }
}

// Two entry kernels over the same body. A 16-bit pool's body fits in 128
// VGPRs (four waves per SIMD) only when the compiler is told to aim for that
// occupancy; an fp32 pool's body spills under that constraint and is left to
// the default, where it also lands at 128.
template <class Tag, class XT, class Gates, int HPG>
__global__ void __launch_bounds__(tile_threads(kDecodeCols) * HPG)
__attribute__((amdgpu_waves_per_eu(4)))
gdn_conv_decode_kernel(typename Storage<Tag>::T* __restrict__ pool,
                       float* __restrict__ conv_pool, const int* __restrict__ slot_idx,
                       const XT* __restrict__ x, const float* __restrict__ conv_w,
                       const float* __restrict__ conv_b, Gates gates, float* __restrict__ y,
                       int H, int G, int C) {
  conv_decode_body<Tag, XT, Gates, HPG>(pool, conv_pool, slot_idx, x, conv_w, conv_b, gates, y,
                                        H, G, C);
}

template <class XT, class Gates, int HPG>
__global__ void __launch_bounds__(tile_threads(kDecodeCols) * HPG)
gdn_conv_decode_kernel_f32(float* __restrict__ pool, float* __restrict__ conv_pool,
                           const int* __restrict__ slot_idx, const XT* __restrict__ x,
                           const float* __restrict__ conv_w, const float* __restrict__ conv_b,
                           Gates gates, float* __restrict__ y, int H, int G, int C) {
  conv_decode_body<F32, XT, Gates, HPG>(pool, conv_pool, slot_idx, x, conv_w, conv_b, gates, y,
                                        H, G, C);
}

// A prefill stage: the next kStage tokens' per-token inputs, staged in LDS by
// a parallel prologue so that the serial loop reads nothing from global memory:
//   qk   normalised q and k (q_hat, k_hat), each kStageVec floats holding the
//        kSS rows in the order the launch's layout reads them (StageOrder);
//   v    the value row [kHD];
//   gate alpha, beta.
constexpr int kStage = 32;

// Where row r of q_hat / k_hat sits in a stage vector, per layout:
//   kRowOrder      r (the whole and split layouts read 32-row blocks);
//   kEighthOrder   an eighth-layout lane's chain of eight rows (row block w,
//                  row group rg, i = 0..7) as two runs of four: i < 4 at
//                  (w * 4 + rg) * 4 + i, i >= 4 at 64 + (w * 4 + rg) * 4 + i - 4,
//                  so that a wave's 16-byte reads cover consecutive banks
//                  (eight-float runs put a read's 16 chains on half the banks:
//                  18-24 M bank-conflict cycles a launch; config 4 in this
//                  layout 0.1616 -> 0.159 ms, the same bits);
//   kQuarterOrder  a quarter-layout lane's 16 rows (row block w, row groups
//                  2 rgh and 2 rgh + 1) are 16 consecutive floats, (i, rgl)
//                  at 2 i + rgl, in groups of kQuarterGroup floats: the group
//                  stride of 20 (not 16) puts the eight groups a read touches
//                  on distinct LDS banks. Four 16-byte reads per vector instead
//                  of eight 8-byte pairs (quarter-layout tokens: config 4's
//                  4 x 256 0.1255 -> 0.120 ms, one 512-token row 0.161 ->
//                  0.155 ms; the same bits).
enum StageOrder { kRowOrder, kEighthOrder, kQuarterOrder };
constexpr int kQuarterGroup = 20;
constexpr int kStageVec = 8 * kQuarterGroup;  // >= kSS
__device__ __forceinline__ int eighth_stage_pos(int w, int rg, int i) {
  return (i >> 2) * 64 + (w * kRowGroups + rg) * 4 + (i & 3);
}
__device__ __forceinline__ int quarter_stage_pos(int w, int rgh, int i, int rgl) {
  return (w * 2 + rgh) * kQuarterGroup + 2 * i + rgl;
}

struct alignas(16) StageLds {
  float qk[kStage][2][kStageVec];
  float v[kStage][kHD];
  float gate[kStage][2];
};

// One thread's share of a stage's global inputs, loaded a whole stage ahead so
// that the loads are in flight while the previous stage's serial loop runs:
// every thread kV4 of the stage's 16-byte v pieces, lane j of the last two
// waves token j's raw gate values, and the q and k vectors of the wave's
// tokens w, w + waves, ... in rounds of four vectors: in round u, the 16-lane
// row (lane / 16) = 2 x + c holds vector c (0: q, 1: k) of the wave's token
// 2u + x, each lane eight consecutive elements (8 (lane % 16) ...), as two
// 16-byte pieces (see write_stage for why).
template <int kTileWaves>
struct StageRegs {
  static constexpr int kTok = kStage / kTileWaves;
  static constexpr int kRounds = kTok / 2;
  static constexpr int kV4 = kStage * (kHD / 4) / (64 * kTileWaves);
  float4 qk[kRounds][2];
  float4 v[kV4];
  GateRaw gate;
};

template <int kTileWaves, class Gates>
__device__ __forceinline__ void load_stage(StageRegs<kTileWaves>& r, int wave, int lane,
                                           const Gates& gates, const float* __restrict__ q,
                                           const float* __restrict__ k,
                                           const float* __restrict__ v, int b, int h, int g,
                                           int H, int G, int T, int t0, int n) {
  constexpr int kThreads = 64 * kTileWaves;
  // Lane j of each of the last two waves: token j's raw gates (alpha is
  // evaluated by the first of them, beta by the second).
  if (wave >= kTileWaves - 2 && lane < n) r.gate = gates.load_live(b, h, t0 + lane, H, T);
#pragma unroll
  for (int m = 0; m < StageRegs<kTileWaves>::kV4; ++m) {
    const int e = threadIdx.x + m * kThreads, j = e / (kHD / 4), c4 = e % (kHD / 4);
    if (j < n)
      r.v[m] = *reinterpret_cast<const float4*>(v + (((size_t)b * T + t0 + j) * H + h) * kHD +
                                                4 * c4);
  }
  const float* const src = ((lane >> 4) & 1) ? k : q;
  const int x = lane >> 5, e0 = 8 * (lane & 15);
#pragma unroll
  for (int u = 0; u < StageRegs<kTileWaves>::kRounds; ++u) {
    const int j = wave + (2 * u + x) * kTileWaves;
    if (j < n) {
      const float* p = src + (((size_t)b * T + t0 + j) * G + g) * kSS + e0;
      r.qk[u][0] = *reinterpret_cast<const float4*>(p);
      r.qk[u][1] = *reinterpret_cast<const float4*>(p + 4);
    }
  }
}

// Turns the prefetched inputs of tokens [t0, t0 + n) into the stage in LDS.
// Gates: the policy's own arithmetic, alpha on one wave and beta on another.
//
// q and k: q_hat = q * factor with the decode's factor, inv_norm: 1 /
// sqrt(S + 1e-6), S the sum of the 64 leaves p_l = x[2l]^2 + x[2l+1]^2 over
// the butterfly lane xor 1, 2, 4, 8, 16, 32, which is the balanced tree that
// first adds neighbouring leaves, then neighbouring pairs, and so on. Here a
// lane holds eight consecutive elements, so it forms four neighbouring leaves
// and their first two tree levels in-lane, ((p0 + p1) + (p2 + p3)); the other
// four levels pair neighbouring lanes of its 16-lane row, lane xor 1, 2, 4
// and 8. The same additions in the same order, so the decode's bits, at about
// a third of the instructions (one 16-lane row per vector: four vectors per
// wave instruction, and no exchange across rows).
//
// kOrder: where each row of q_hat and k_hat goes in LDS (StageOrder).
template <int kTileWaves, StageOrder kOrder, class Gates>
__device__ __forceinline__ void write_stage(const StageRegs<kTileWaves>& r, int wave, int lane,
                                            const Gates& gates, const GateConst& gc, int n,
                                            StageLds& st) {
  constexpr int kThreads = 64 * kTileWaves;
  // The gates' transcendental chains on two waves, alpha and beta in
  // parallel, while the other two start on their norms.
  if (lane < n) {
    if (wave == kTileWaves - 2) st.gate[lane][0] = gates.alpha_of(r.gate, gc);
    if (wave == kTileWaves - 1) st.gate[lane][1] = gates.eval_beta(r.gate);
  }
#pragma unroll
  for (int m = 0; m < StageRegs<kTileWaves>::kV4; ++m) {
    const int e = threadIdx.x + m * kThreads, j = e / (kHD / 4), c4 = e % (kHD / 4);
    if (j < n) *reinterpret_cast<float4*>(&st.v[j][4 * c4]) = r.v[m];
  }
  constexpr int kRounds = StageRegs<kTileWaves>::kRounds;
  const int c = (lane >> 4) & 1, x = lane >> 5, e0 = 8 * (lane & 15);
  float f[kRounds];
#pragma unroll
  for (int u = 0; u < kRounds; ++u) {
    const float4 a = r.qk[u][0], b = r.qk[u][1];
    const float p0 = a.x * a.x + a.y * a.y, p1 = a.z * a.z + a.w * a.w;
    const float p2 = b.x * b.x + b.y * b.y, p3 = b.z * b.z + b.w * b.w;
    f[u] = (p0 + p1) + (p2 + p3);
  }
#pragma unroll
  for (int u = 0; u < kRounds; ++u) f[u] = add_xor1(f[u]);
#pragma unroll
  for (int u = 0; u < kRounds; ++u) f[u] = add_xor2(f[u]);
#pragma unroll
  for (int u = 0; u < kRounds; ++u) f[u] = add_xor4(f[u]);
#pragma unroll
  for (int u = 0; u < kRounds; ++u) f[u] = add_xor8(f[u]);
#pragma unroll
  for (int u = 0; u < kRounds; ++u) {
    const int j = wave + (2 * u + x) * kTileWaves;
    if (j < n) {
      const float fu = rsqrtf(f[u] + kL2Eps);
      const float4 a = r.qk[u][0], b = r.qk[u][1];
      float* dst = &st.qk[j][c][0];
      if constexpr (kOrder == kQuarterOrder) {
        // Rows e0 + k (e0 a multiple of 8): row block e0 / 32, row group k % 4,
        // chain index (e0 % 32) / 4 + k / 4.
        const int wb = e0 >> 5, i0 = (e0 & 31) >> 2;
        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int rg = kk & 3;
          dst[quarter_stage_pos(wb, rg >> 1, i0 + (kk >> 2), rg & 1)] = xs[kk] * fu;
        }
      } else if constexpr (kOrder == kEighthOrder) {
        // Rows e0 + k (e0 a multiple of 8): row block e0 / 32, row group k % 4,
        // chain index (e0 / 4) % 8 + k / 4.
        const int wb = e0 >> 5, i0 = (e0 >> 2) & 7;
        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) dst[eighth_stage_pos(wb, kk & 3, i0 + (kk >> 2))] = xs[kk] * fu;
      } else {
        *reinterpret_cast<float4*>(dst + e0) = make_float4(a.x * fu, a.y * fu, a.z * fu, a.w * fu);
        *reinterpret_cast<float4*>(dst + e0 + 4) =
            make_float4(b.x * fu, b.y * fu, b.z * fu, b.w * fu);
      }
    }
  }
}

// One token's inputs for a lane of the scan layout, read from the stage.
template <int CPL>
struct TokenIn {
  float kh[kRowsPerWave], qh[kRowsPerWave];  // the lane's row block, row order
  float v[CPL];
  float alpha, beta;
};

// v and the gates are read first: issued behind the 16 row reads, the
// compiler placed them after the kv chain and waited for them there.
template <int CPL>
__device__ __forceinline__ void read_token(const StageLds& st, int j, int r0, int col0,
                                           TokenIn<CPL>& t) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const float2 ab = *reinterpret_cast<const float2*>(&st.gate[j][0]);
  t.alpha = ab.x;
  t.beta = ab.y;
  if constexpr (CPL == 2) {
    const float2 v2 = *reinterpret_cast<const float2*>(&st.v[j][col0]);
    t.v[0] = v2.x;
    t.v[1] = v2.y;
  } else {
    static_assert(CPL == 1, "one or two columns per lane");
    t.v[0] = st.v[j][col0];
  }
#pragma unroll
  for (int r = 0; r < kRowsPerWave; r += 4) {
    const f32x4 k4 = *reinterpret_cast<const f32x4*>(&st.qk[j][1][r0 + r]);
    const f32x4 q4 = *reinterpret_cast<const f32x4*>(&st.qk[j][0][r0 + r]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t.kh[r + e] = k4[e];
      t.qh[r + e] = q4[e];
    }
  }
}

// The quarter layout's token: its 16 rows' k_hat / q_hat (rows w * 32 + 2 rgh +
// rgl + 4 i, consecutive in the stage's quarter order from `pos`), its
// column's v, and the gates.
struct TokenInQ {
  float kh[2][kRowsPerLane], qh[2][kRowsPerLane];
  float v, alpha, beta;
};

__device__ __forceinline__ void read_token_quarter(const StageLds& st, int j, int pos, int col0,
                                                   TokenInQ& t) {
  const float2 ab = *reinterpret_cast<const float2*>(&st.gate[j][0]);
  t.alpha = ab.x;
  t.beta = ab.y;
  t.v = st.v[j][col0];
  // Four 16-byte reads per vector (a group is 16-byte aligned, not 64).
#pragma unroll
  for (int p = 0; p < kRowsPerLane / 2; ++p) {
    float k4[4], q4[4];
    loadN<4>(&st.qk[j][1][pos + 4 * p], k4);
    loadN<4>(&st.qk[j][0][pos + 4 * p], q4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t.kh[e & 1][2 * p + (e >> 1)] = k4[e];
      t.qh[e & 1][2 * p + (e >> 1)] = q4[e];
    }
  }
}

// The eighth layout's token: its chain's 8 rows of k_hat / q_hat (two 16-byte
// reads each, the stage being in lane order), its column's v, and the gates.
struct TokenInE {
  float kh[kRowsPerLane], qh[kRowsPerLane];
  float v, alpha, beta;
};

__device__ __forceinline__ void read_token_eighth(const StageLds& st, int j, int pos, int col0,
                                                  TokenInE& t) {
  const float2 ab = *reinterpret_cast<const float2*>(&st.gate[j][0]);
  t.alpha = ab.x;
  t.beta = ab.y;
  t.v = st.v[j][col0];
  float lo[4], hi[4];
  loadN<4>(&st.qk[j][1][pos], lo);
  loadN<4>(&st.qk[j][1][pos + 64], hi);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    t.kh[i] = lo[i];
    t.kh[4 + i] = hi[i];
  }
  loadN<4>(&st.qk[j][0][pos], lo);
  loadN<4>(&st.qk[j][0][pos + 64], hi);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    t.qh[i] = lo[i];
    t.qh[4 + i] = hi[i];
  }
}

// The eighth layout's state: the lane's chain, rows i = 2m and 2m + 1 in
// p[m].
template <class Tag>
struct ScanStateE {
  RowPair1<Tag> p[kRowsPerLane / 2];
  template <class ST>
  __device__ __forceinline__ void load(const ScanMapEighth& L, const ST* tile) {
#pragma unroll
    for (int m = 0; m < kRowsPerLane / 2; ++m)
      p[m].load_nt(tile + (size_t)L.row(2 * m) * kHD, tile + (size_t)L.row(2 * m + 1) * kHD);
  }
  template <class ST>
  __device__ __forceinline__ void store(const ScanMapEighth& L, ST* tile) const {
#pragma unroll
    for (int m = 0; m < kRowsPerLane / 2; ++m)
      p[m].store_nt(tile + (size_t)L.row(2 * m) * kHD, tile + (size_t)L.row(2 * m + 1) * kHD);
  }
};

template <class Tag, int CPL, int kLRG>
struct ScanState;

// One token of a ScanMap layout (one or two columns per lane) on its state.
template <class Tag, int CPL, bool kOpaqueNarrow = false>
__device__ __forceinline__ void scan_token_any(ScanState<Tag, CPL, kRowGroups>& S,
                                               const TokenIn<CPL>& in, float (&y)[CPL]) {
  if constexpr (CPL == 1)
    scan_token_pairs<Tag, kOpaqueNarrow>(S.p, in.kh, in.qh, in.v[0], in.alpha, in.beta, y[0]);
  else
    scan_token<Tag, CPL, kOpaqueNarrow>(S.s, in.kh, in.qh, in.v, in.alpha, in.beta, y);
}

// A lane's state in a scan layout: a Row<Tag, CPL> per (row group, i), or,
// with one column per lane, row pairs (RowPair1) over row groups 2p and 2p + 1
// so that one packed conversion narrows two elements.
template <class Tag, int CPL, int kLRG>
struct ScanState {
  Row<Tag, CPL> s[kLRG][kRowsPerLane];
  template <class LM, class ST>
  __device__ __forceinline__ void load(const LM& L, const ST* tile) {
#pragma unroll
    for (int rg = 0; rg < kLRG; ++rg) {
#pragma unroll
      for (int i = 0; i < kRowsPerLane; ++i) s[rg][i].load_nt(tile + (size_t)L.row(rg, i) * kHD);
    }
  }
  template <class LM, class ST>
  __device__ __forceinline__ void store(const LM& L, ST* tile) const {
#pragma unroll
    for (int rg = 0; rg < kLRG; ++rg) {
#pragma unroll
      for (int i = 0; i < kRowsPerLane; ++i) s[rg][i].store_nt(tile + (size_t)L.row(rg, i) * kHD);
    }
  }
};
template <class Tag, int kLRG>
struct ScanState<Tag, 1, kLRG> {
  RowPair1<Tag> p[kLRG / 2][kRowsPerLane];
  template <class LM, class ST>
  __device__ __forceinline__ void load(const LM& L, const ST* tile) {
#pragma unroll
    for (int q = 0; q < kLRG / 2; ++q) {
#pragma unroll
      for (int i = 0; i < kRowsPerLane; ++i)
        p[q][i].load_nt(tile + (size_t)L.row(2 * q, i) * kHD,
                        tile + (size_t)L.row(2 * q + 1, i) * kHD);
    }
  }
  template <class LM, class ST>
  __device__ __forceinline__ void store(const LM& L, ST* tile) const {
#pragma unroll
    for (int q = 0; q < kLRG / 2; ++q) {
#pragma unroll
      for (int i = 0; i < kRowsPerLane; ++i)
        p[q][i].store_nt(tile + (size_t)L.row(2 * q, i) * kHD,
                         tile + (size_t)L.row(2 * q + 1, i) * kHD);
    }
  }
};

// The live tokens of one tile (or of its workgroup's share of the columns),
// with the state resident in registers. Scan layouts (ScanLayoutOf<Layout>):
// four waves; a lane holds the 32 rows of its row block for CPL columns
// (ScanMap), or 16 of them for one column (ScanMapQuarter); the column sums
// finish in-lane and over the row groups and blocks with DPP / permlane swaps,
// by the decode's summation tree, so the bits are the decode's and no token
// needs a workgroup barrier. kTokenPairs runs two tokens per loop iteration. Tokens run in stages of
// kStage: their inputs are loaded a stage ahead (StageRegs) and staged in LDS
// (StageLds) between stages, so the serial loop carries only the recurrence
// and the output stores.
//
// Only the row's live tokens [0, len) run: a pad token (alpha = 1, beta = 0)
// is an identity on the state, so skipping it leaves the state exactly as the
// reference's pad steps do (gdn.py:301-316), up to their turning a -0 entry
// into +0. y at the pad positions [len, T) is written as 0 (the reference
// leaves arbitrary values there that nothing reads; zeros also keep a later
// per-tensor FP8 scale of the readout independent of the pads).
template <class Tag, class Gates, int Layout, bool kTokenPairs = false>
__device__ __forceinline__ void prefill_tile(typename Storage<Tag>::T* __restrict__ pool,
                                             const int* __restrict__ slot_idx,
                                             const float* __restrict__ q,
                                             const float* __restrict__ k,
                                             const float* __restrict__ v, const Gates& gates,
                                             float* __restrict__ y, int H, int G,
                                             int heads_per_group, int T, int b, int h, int part,
                                             int len, StageLds& st) {
  using LM = typename ScanLayoutOf<Layout>::type;
  constexpr int CPL = LM::kCPL;
  constexpr int kLRG = LM::kLaneRowGroups;
  using ST = typename Storage<Tag>::T;
  const int g = h / heads_per_group;
  const LM L(threadIdx.x, part);
  const int slot = slot_idx[b];
  ST* tile = pool + ((size_t)slot * H + h) * (kSS * kHD) + L.col0;

  typename std::conditional<Layout == 8, ScanStateE<Tag>, ScanState<Tag, CPL, kLRG>>::type S;
  S.load(L, tile);

  constexpr int kW = LM::kWaves;
  // Where the lane's rows start in a stage vector: its row block's first row
  // (row order), its group (quarter order) or its chain (eighth order).
  int r0 = L.w * kRowsPerWave;
  if constexpr (Layout == 4) r0 = quarter_stage_pos(L.w, L.rgh, 0, 0);
  // The eighth layout's chain in the lane-ordered stage.
  if constexpr (Layout == 8) r0 = eighth_stage_pos(L.w, L.rg, 0);
  // The head's gate constants, read once (a read per stage would wait on
  // memory in the middle of the prologue).
  const GateConst gc = gates.tile_consts(h);
  StageRegs<kW> pre;
  // (Loads nothing when len == 0; a branch around it costs ~30 VGPRs.)
  load_stage<kW>(pre, L.wave, L.lane, gates, q, k, v, b, h, g, H, G, T, 0, min(kStage, len));
  for (int t0 = 0; t0 < len; t0 += kStage) {
    const int n = min(kStage, len - t0);
    // Every wave has finished reading the previous stage (the barrier at the
    // end of the stage loop), so it may be overwritten.
    write_stage<kW, Layout == 8 ? kEighthOrder : (Layout == 4 ? kQuarterOrder : kRowOrder)>(
        pre, L.wave, L.lane, gates, gc, n, st);
    __syncthreads();
    // The next stage's loads fly while this stage's tokens run.
    if (t0 + kStage < len)
      load_stage<kW>(pre, L.wave, L.lane, gates, q, k, v, b, h, g, H, G, T, t0 + kStage,
                     min(kStage, len - t0 - kStage));
    float* yt = y + (((size_t)b * T + t0) * H + h) * kHD + L.col0;
    const size_t y_tok = (size_t)H * kHD;
    int j = 0;
    if constexpr (Layout == 8) {
      // The next pair's inputs are read from the stage while this pair runs
      // (the layout runs one wave per SIMD, so the 36 registers are free).
      // Two pairs per iteration, so the buffers trade roles without copies;
      // reads past the stage's live tokens stay inside it and go unused.
      auto clamp = [](int t) { return min(t, kStage - 1); };
      auto pair = [&](int jj, const TokenInE& a, const TokenInE& c) {
        float y0[1], y1[1];
        scan_token_eighth<Tag, true>(S.p, a.kh, a.qh, a.v, a.alpha, a.beta, y0[0]);
        scan_token_eighth<Tag, true>(S.p, c.kh, c.qh, c.v, c.alpha, c.beta, y1[0]);
        if (L.stores_y()) {
          storeN<1>(yt + jj * y_tok, y0);
          storeN<1>(yt + (jj + 1) * y_tok, y1);
        }
      };
      TokenInE c0, c1, n0, n1;
      read_token_eighth(st, 0, r0, L.col0, c0);
      read_token_eighth(st, 1, r0, L.col0, c1);
      for (; j + 3 < n; j += 4) {
        read_token_eighth(st, j + 2, r0, L.col0, n0);
        read_token_eighth(st, j + 3, r0, L.col0, n1);
        pair(j, c0, c1);
        read_token_eighth(st, clamp(j + 4), r0, L.col0, c0);
        read_token_eighth(st, clamp(j + 5), r0, L.col0, c1);
        pair(j + 2, n0, n1);
      }
      if (j + 1 < n) {
        read_token_eighth(st, clamp(j + 2), r0, L.col0, n0);
        pair(j, c0, c1);
        c0 = n0;
        j += 2;
      }
      if (j < n) {
        float yy[1];
        scan_token_eighth<Tag>(S.p, c0.kh, c0.qh, c0.v, c0.alpha, c0.beta, yy[0]);
        if (L.stores_y()) storeN<1>(yt + j * y_tok, yy);
      }
    } else if constexpr (Layout == 4) {
      if constexpr (kTokenPairs) {
        for (; j + 1 < n; j += 2) {
          TokenInQ in0, in1;
          read_token_quarter(st, j, r0, L.col0, in0);
          read_token_quarter(st, j + 1, r0, L.col0, in1);
          float y0[1], y1[1];
          scan_token_quarter<Tag, true>(S.p[0], in0.kh, in0.qh, in0.v, in0.alpha, in0.beta,
                                        y0[0]);
          scan_token_quarter<Tag, true>(S.p[0], in1.kh, in1.qh, in1.v, in1.alpha, in1.beta,
                                        y1[0]);
          if (L.stores_y()) {
            storeN<1>(yt + j * y_tok, y0);
            storeN<1>(yt + (j + 1) * y_tok, y1);
          }
        }
      }
      for (; j < n; ++j) {
        TokenInQ in;
        read_token_quarter(st, j, r0, L.col0, in);
        float yy[1];
        scan_token_quarter<Tag>(S.p[0], in.kh, in.qh, in.v, in.alpha, in.beta, yy[0]);
        if (L.stores_y()) storeN<1>(yt + j * y_tok, yy);
      }
    } else if constexpr (kTokenPairs) {
      // Two tokens per iteration, both y stores after both tokens, so the two
      // token bodies form one basic block the scheduler can interleave (the
      // second token's loads and kv chain with the first's readout). Used by
      // the one-column layout of gdn_prefill_kernel: it is latency-bound (a
      // wave issues VALU about half its cycles) and runs at most one
      // workgroup per CU, so the extra registers cost nothing. Measured:
      // config 4's 4 x 256 tokens 0.189 -> 0.181 ms, one 512-token row
      // 0.340 -> 0.316 ms. In the planned kernel, whose register count both
      // layouts set and which may hold two workgroups per CU, it was 8-20%
      // slower.
      for (; j + 1 < n; j += 2) {
        TokenIn<CPL> in0, in1;
        read_token<CPL>(st, j, r0, L.col0, in0);
        read_token<CPL>(st, j + 1, r0, L.col0, in1);
        float y0[CPL], y1[CPL];
        scan_token_any<Tag, CPL, true>(S, in0, y0);
        scan_token_any<Tag, CPL, true>(S, in1, y1);
        if (L.stores_y()) {
          storeN<CPL>(yt + j * y_tok, y0);
          storeN<CPL>(yt + (j + 1) * y_tok, y1);
        }
      }
    }
    if constexpr (Layout != 4 && Layout != 8) {
      for (; j < n; ++j) {
        TokenIn<CPL> in;
        read_token<CPL>(st, j, r0, L.col0, in);
        float yy[CPL];
        scan_token_any<Tag, CPL>(S, in, yy);
        if (L.stores_y()) storeN<CPL>(yt + j * y_tok, yy);
      }
    }
    __syncthreads();
  }

  S.store(L, tile);

  // Zeros at the pad positions, the workgroup's columns, 16 bytes per thread.
  constexpr int kCols = LM::kWaves * LM::kColsPerWave;  // this workgroup's columns
  constexpr int kV4 = kCols / 4;
  const int c0 = part * kCols;
  for (int e = threadIdx.x; e < (T - len) * kV4; e += 64 * kW) {
    const int t = len + e / kV4, c = c0 + 4 * (e % kV4);
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store((f32x4){0.f, 0.f, 0.f, 0.f},
                                reinterpret_cast<f32x4*>(y + (((size_t)b * T + t) * H + h) * kHD + c));
  }
}

// A scan wave issues at most one VALU instruction per about five clocks and
// waits on its own dependency chains between them, so its SIMD has issue
// cycles to spare. A decode launched beside it (MixedTick: a memory-bound
// launch on a side stream) shares those SIMDs; at the highest wave priority
// the scan's instruction is the one chosen whenever it is ready, and the
// decode issues in the cycles the scan leaves idle (config 4's tick, bucket
// 96: 133.2 -> 129.3 us; a prefill alone is unchanged).
__device__ __forceinline__ void raise_scan_priority() { __builtin_amdgcn_s_setprio(3); }

// One tile (layout 2), a half tile (layout 1, kParts = 2), a quarter tile
// (layout 4, kParts = 4) or an eighth (layout 8, kParts = 8) per workgroup:
// blockIdx.x = (b * H + h) * kParts + part. Layouts 1, 4 and 8 run token
// pairs.
template <class Tag, class Gates, int Layout>
__global__ void __launch_bounds__(64 * ScanLayoutOf<Layout>::type::kWaves)
gdn_prefill_kernel(typename Storage<Tag>::T* __restrict__ pool,
                   const int* __restrict__ slot_idx,
                   const float* __restrict__ q, const float* __restrict__ k,
                   const float* __restrict__ v, Gates gates, float* __restrict__ y,
                   int H, int G, int heads_per_group, int T) {
  using LM = typename ScanLayoutOf<Layout>::type;
  raise_scan_priority();
  const int tile_id = blockIdx.x / LM::kParts;
  const int part = blockIdx.x - tile_id * LM::kParts;
  const int b = tile_id / H;
  const int h = tile_id - b * H;
  __shared__ StageLds st;
  prefill_tile<Tag, Gates, Layout, Layout != 2>(pool, slot_idx, q, k, v, gates, y, H, G,
                                                heads_per_group, T, b, h, part,
                                                gates.row_len(b, T), st);
}

// Ragged batches of up to four tiles per CU: the rows' live lengths decide
// the layout. Every workgroup derives the same plan from seq_lens:
//   * rows ranked by live length, longest first (ties by row index);
//   * three tiers by rank: the first n4 rows run in the quarter layout (four
//     workgroups per tile), the next n2 split over two workgroups (one column
//     per lane), the rest whole (two columns per lane). A tier's per-token
//     time, relative to a whole tile's, is about kSplitCost and kQuarterCost
//     (measured on single rows), so splitting shortens a row's chain but costs
//     more workgroup time in all. (n4, n2) minimise the estimated makespan:
//     the larger of the critical path and the total workgroup time over the
//     CUs, with at most one extra workgroup per CU (the first plan found wins
//     ties);
//   * workgroup order: quarter tiles, then split tiles, then whole tiles,
//     longest rows first within each, so the longest chains start on CUs of
//     their own and the short rows fill in. Workgroups beyond the plan return.
// A row's tiles compute the same bits in any layout.
constexpr float kSplitCost = 0.745f;
constexpr float kQuarterCost = 0.47f;
constexpr int kMaxPlanRows = 1024;

template <class Tag, class Gates>
__global__ void __launch_bounds__(256)
gdn_prefill_planned_kernel(typename Storage<Tag>::T* __restrict__ pool,
                           const int* __restrict__ slot_idx,
                           const float* __restrict__ q, const float* __restrict__ k,
                           const float* __restrict__ v, Gates gates, float* __restrict__ y,
                           int B, int H, int G, int heads_per_group, int T, int cus,
                           int max_extra, int forced_plan) {
  raise_scan_priority();
  __shared__ StageLds st;
  __shared__ int lens[kMaxPlanRows];
  __shared__ int order[kMaxPlanRows];  // row of each rank
  __shared__ int plan[3];  // n4, n2, n8
  for (int r = threadIdx.x; r < B; r += blockDim.x) lens[r] = gates.row_len(r, T);
  __syncthreads();
  for (int r = threadIdx.x; r < B; r += blockDim.x) {
    int rank = 0;
    for (int o = 0; o < B; ++o)
      rank += (lens[o] > lens[r] || (lens[o] == lens[r] && o < r)) ? 1 : 0;
    order[rank] = r;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    // Estimated makespan of a plan, in whole-tile token times: the larger of
    // its critical path (each tier's longest row x the tier's per-token cost)
    // and its total workgroup time spread over the CUs (a quarter tile costs
    // 4 kQuarterCost of a whole tile's time, a split one 2 kSplitCost). At
    // most max_extra workgroups beyond one per tile: 3 H per quarter row, H
    // per split row.
    const int extra = max_extra / H;
    const float per_cu = (float)H / (float)cus;
    float total = 0.f;
    for (int r = 0; r < B; ++r) total += (float)lens[r];
    float best = fmaxf((float)lens[order[0]], total * per_cu);
    int b4 = 0, b2 = 0;
    float sum4 = 0.f;  // lengths of the quarter rows
    for (int n4 = 0; n4 <= B && 3 * n4 <= extra; ++n4) {
      if (n4 > 0) sum4 += (float)lens[order[n4 - 1]];
      const float m4 = n4 > 0 ? kQuarterCost * (float)lens[order[0]] : 0.f;
      float sum2 = 0.f;  // lengths of the split rows
      for (int n2 = 0; n4 + n2 <= B && 3 * n4 + n2 <= extra; ++n2) {
        if (n2 > 0) sum2 += (float)lens[order[n4 + n2 - 1]];
        const float fixed = fmaxf(m4, n2 > 0 ? kSplitCost * (float)lens[order[n4]] : 0.f);
        const float whole = n4 + n2 < B ? (float)lens[order[n4 + n2]] : 0.f;
        const float work = (total + (4.f * kQuarterCost - 1.f) * sum4 +
                            (2.f * kSplitCost - 1.f) * sum2) * per_cu;
        const float m = fmaxf(fmaxf(fixed, whole), work);
        if (m < best) {
          best = m;
          b4 = n4;
          b2 = n2;
        }
        // Once the whole tier no longer sets the critical path, splitting
        // more rows cannot lower the estimate.
        if (whole <= fixed) break;
      }
    }
    plan[0] = b4;
    plan[1] = b2;
    plan[2] = 0;
    // A plan chosen on the host or forced for measurement (n8 * 2^20 + n4 *
    // 2^10 + n2; the launch sized the grid for it).
    if (forced_plan >= 0) {
      plan[2] = min(forced_plan >> 20, B);
      plan[0] = min((forced_plan >> 10) & 1023, B - plan[2]);
      plan[1] = min(forced_plan & 1023, B - plan[2] - plan[0]);
    }
  }
  __syncthreads();
  const int n4 = plan[0], n2 = plan[1], n8 = plan[2];
  int i = blockIdx.x;
  // Ranks: the n8 longest rows in the eighth layout, the next n4 quarter,
  // then n2 split, the rest whole; workgroups in that order.
  if (i < 8 * n8 * H) {
    const int rank = i / (8 * H), rem = i - rank * 8 * H;
    const int b = order[rank];
    prefill_tile<Tag, Gates, 8, true>(pool, slot_idx, q, k, v, gates, y, H, G, heads_per_group, T,
                                      b, rem >> 3, rem & 7, lens[b], st);
    return;
  }
  i -= 8 * n8 * H;
  if (i < 4 * n4 * H) {
    const int rank = n8 + i / (4 * H), rem = i - (rank - n8) * 4 * H;
    const int b = order[rank];
    prefill_tile<Tag, Gates, 4, true>(pool, slot_idx, q, k, v, gates, y, H, G, heads_per_group, T,
                                      b, rem >> 2, rem & 3, lens[b], st);
    return;
  }
  i -= 4 * n4 * H;
  if (i < 2 * n2 * H) {
    const int rank = n8 + n4 + i / (2 * H), rem = i - (rank - n8 - n4) * 2 * H;
    const int b = order[rank];
    prefill_tile<Tag, Gates, 1>(pool, slot_idx, q, k, v, gates, y, H, G, heads_per_group, T, b,
                                rem >> 1, rem & 1, lens[b], st);
    return;
  }
  i -= 2 * n2 * H;
  if (i < (B - n8 - n4 - n2) * H) {
    const int rank = n8 + n4 + n2 + i / H;
    const int b = order[rank];
    prefill_tile<Tag, Gates, 2>(pool, slot_idx, q, k, v, gates, y, H, G, heads_per_group, T, b,
                                i - (i / H) * H, 0, lens[b], st);
  }
}

// ---------------------------------------------------------------------------
// Host-side checks shared by the four entry points.

int check_common(void* pool, int pool_dtype, int64_t n_slots, int H, int G, int SS, int HD,
                 const int32_t* slot_idx, int B) {
  if (pool_dtype != BRAID_F32 && pool_dtype != BRAID_F16 && pool_dtype != BRAID_BF16)
    return fail(BRAID_EINVAL, "state pool must be fp32, fp16 or bf16");
  if (SS != kSS || HD != kHD) return fail(BRAID_EINVAL, "only SS=HD=128 is instantiated");
  if (H <= 0 || G <= 0 || H % G != 0)
    return fail(BRAID_EINVAL, "n_heads must be divisible by n_groups");
  if (B < 0) return fail(BRAID_EINVAL, "batch must be non-negative");
  if (n_slots <= 0) return fail(BRAID_EINVAL, "pool must hold at least one slot");
  if (B > 0 && (pool == nullptr || slot_idx == nullptr))
    return fail(BRAID_EINVAL, "pool and slot_idx must be non-null");
  if (!aligned16(pool)) return fail(BRAID_EINVAL, "pool must be 16-byte aligned");
  return BRAID_OK;
}

int check_rows(const float* p, int64_t row, int64_t inner, const char* name) {
  if (p == nullptr) return fail(BRAID_EINVAL, std::string(name) + " must be non-null");
  if (row < inner) return fail(BRAID_EINVAL, std::string(name) + " rows overlap");
  if (!aligned16(p) || (row % 4) != 0)
    return fail(BRAID_EINVAL, std::string(name) +
                                  " must be 16-byte aligned with a row stride that is a "
                                  "multiple of 4 elements");
  return BRAID_OK;
}

int check_act(const void* a_raw, const void* b_raw, int act_dtype, const float* A,
              const float* dt_bias) {
  if (act_dtype != BRAID_F32 && act_dtype != BRAID_BF16)
    return fail(BRAID_EINVAL,
                "a_raw/b_raw must be fp32 or bf16 (the activation dtypes braid runs)");
  if (a_raw == nullptr || b_raw == nullptr || A == nullptr || dt_bias == nullptr)
    return fail(BRAID_EINVAL, "a_raw/b_raw/A/dt_bias must be non-null");
  return BRAID_OK;
}

// CUs of the current device (0 if the runtime cannot say), cached per device:
// the decode launch consults it every step.
int device_cus() { return device_topo().cus; }

// Column parts of a decode launch (gdn_decode_kernel): 2 when a launch has
// at most as many tiles as the GPU has CUs, else 1. Measured per step on
// MI355X (fp16 pool, H = 32, cold slots, graph-replayed), parts 1 / 2 / 4:
// B=1 3.95 / 3.31 / 3.55 us, B=4 4.56 / 3.88 / 4.99, B=8 5.33 / 4.84 / 7.74,
// B=16 7.20 / 8.65 / 12.29. Four parts never win: two columns per lane make
// every state access 4 bytes. The DECODE_PARTS launch knob (1, 2 or 4)
// overrides the choice.
int decode_parts(long n_tiles, int cus) {
  const int forced = launch_knob(BRAID_KNOB_DECODE_PARTS);
  if (forced == 1 || forced == 2 || forced == 4) return forced;
  return cus > 0 && n_tiles <= cus ? 2 : 1;
}

template <class Tag, class Gates, int P>
void launch_decode_as(void* pool, const int32_t* slot_idx, int B, int H, int G, const float* q,
                      int64_t q_row, const float* k, int64_t k_row, const float* v,
                      int64_t v_row, Gates gates, float* y, int cus, hipStream_t stream) {
  const long n_wg = (long)B * H * P;
  const dim3 grid((unsigned)n_wg), block(tile_threads(kDecodeCols));
  const DeviceTopo topo = device_topo();
  const StreamShape shape =
      stream_shape(n_wg, topo, !std::is_same<Tag, F32>::value,
                   sizeof(TileLds) + kWaves * sizeof(QKLds),
                   launch_knob(BRAID_KNOB_DECODE_XCD_REMAP),
                   launch_knob(BRAID_KNOB_DECODE_WGS_PER_CU));
  // A launch capped at two resident workgroups per CU (its LDS request) takes
  // the two-waves-per-SIMD register budget.
  const size_t lds_per_wg = shape.lds_pad + sizeof(TileLds) + kWaves * sizeof(QKLds);
  if constexpr (P == 1 && !std::is_same<Tag, F32>::value) {
    if (shape.lds_pad > 0 && (size_t)topo.lds_per_cu / lds_per_wg <= 2) {
      gdn_decode_kernel<Tag, Gates, P, 2><<<grid, block, shape.lds_pad, stream>>>(
          static_cast<typename Storage<Tag>::T*>(pool), slot_idx, q, k, v, gates, y, H, H / G,
          q_row, k_row, v_row, shape.xcd_per);
      return;
    }
  }
  gdn_decode_kernel<Tag, Gates, P><<<grid, block, shape.lds_pad, stream>>>(
      static_cast<typename Storage<Tag>::T*>(pool), slot_idx, q, k, v, gates, y, H, H / G,
      q_row, k_row, v_row, shape.xcd_per);
}

template <class Tag, class Gates>
void launch_decode_parts(int parts, void* pool, const int32_t* slot_idx, int B, int H, int G,
                         const float* q, int64_t q_row, const float* k, int64_t k_row,
                         const float* v, int64_t v_row, Gates gates, float* y, int cus,
                         hipStream_t stream) {
  if (parts == 4)
    launch_decode_as<Tag, Gates, 4>(pool, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                                    gates, y, cus, stream);
  else if (parts == 2)
    launch_decode_as<Tag, Gates, 2>(pool, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                                    gates, y, cus, stream);
  else
    launch_decode_as<Tag, Gates, 1>(pool, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                                    gates, y, cus, stream);
}

template <class Gates>
int launch_decode(void* pool, int pool_dtype, const int32_t* slot_idx, int B, int H, int G,
                  const float* q, int64_t q_row, const float* k, int64_t k_row, const float* v,
                  int64_t v_row, Gates gates, float* y, hipStream_t stream) {
  const int cus = device_cus();
  const int parts = decode_parts((long)B * H, cus);
  switch (pool_dtype) {
    case BRAID_F32:
      launch_decode_parts<F32>(parts, pool, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                               gates, y, cus, stream);
      break;
    case BRAID_F16:
      launch_decode_parts<F16>(parts, pool, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                               gates, y, cus, stream);
      break;
    default:
      launch_decode_parts<BF16>(parts, pool, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                                gates, y, cus, stream);
      break;
  }
  const int st = hip_status(hipGetLastError(), "launching gdn_decode_kernel");
  return st != BRAID_OK ? st : ok();
}

// Prefill layout of a launch:
//   8: the eighth layout (one column and 8 rows per lane, eight workgroups
//      per tile), when that leaves no CU with a second workgroup;
//   4: the quarter layout (one column and 16 rows per lane, four workgroups
//      per tile), likewise;
//   1: one column per lane for every tile (two workgroups per tile), likewise;
//   2: two columns per lane for every tile;
//   0: planned per row from seq_lens (gdn_prefill_planned_kernel), for larger
//      ragged batches.
// Measured (MI355X, 256 CUs): one 512-token row 0.315 ms in layout 1, 0.225 ms
// in layout 4; rows (300, 700) 0.425 -> 0.301 ms; config 4's 128 tiles, where
// layout 4 would put two workgroups on every CU, 0.183 in layout 1 against
// 0.190 ms; one 512-token row in layout 8 0.126 ms against 0.164 in layout
// 4, 1024 tokens 0.245 against 0.320 (half the VALU per token again, and the
// column sums inside 16-lane rows). With up to two eighth-layout workgroups
// per CU the eighth layout still wins once the chunk is long enough for its
// per-token cost to outweigh the shared CU (two rows of H = 32, quarter
// against eighth: T = 64 0.0265 against 0.030 ms, T = 256 0.0879 against
// 0.0844, T = 1024 0.325 against 0.305; at three rows, three per CU, the
// eighth loses, 0.130 against 0.119 in layout 1). The PREFILL_LAYOUT launch
// knob (1, 2, 4, 8, or 0 for planned when seq_lens is given) overrides the
// choice.
constexpr int kEighthSharedMinT = 256;

int prefill_layout(int n_tiles, int B, int T, bool ragged, int cus) {
  const int forced = launch_knob(BRAID_KNOB_PREFILL_LAYOUT);
  if (forced == 1 || forced == 2 || forced == 4 || forced == 8) return forced;
  if (forced == 0 && ragged && B <= kMaxPlanRows) return 0;
  if (cus > 0 && 8 * n_tiles <= cus) return 8;
  if (cus > 0 && 8 * n_tiles <= 2 * cus && T >= kEighthSharedMinT) return 8;
  if (cus > 0 && 4 * n_tiles <= cus) return 4;
  if (cus > 0 && 2 * n_tiles <= cus) return 1;
  return ragged && B <= kMaxPlanRows && cus > 0 && n_tiles <= 4 * cus ? 0 : 2;
}

template <class Gates, int Layout>
void launch_prefill_cols(void* pool, int pool_dtype, const int32_t* slot_idx, int B, int T,
                         int H, int G, const float* q, const float* k, const float* v,
                         Gates gates, float* y, hipStream_t stream) {
  using LM = typename ScanLayoutOf<Layout>::type;
  const dim3 grid((unsigned)B * (unsigned)H * LM::kParts), block(64 * LM::kWaves);
  const int hpg = H / G;
  switch (pool_dtype) {
    case BRAID_F32:
      gdn_prefill_kernel<F32, Gates, Layout><<<grid, block, 0, stream>>>(
          static_cast<float*>(pool), slot_idx, q, k, v, gates, y, H, G, hpg, T);
      break;
    case BRAID_F16:
      gdn_prefill_kernel<F16, Gates, Layout><<<grid, block, 0, stream>>>(
          static_cast<uint16_t*>(pool), slot_idx, q, k, v, gates, y, H, G, hpg, T);
      break;
    default:
      gdn_prefill_kernel<BF16, Gates, Layout><<<grid, block, 0, stream>>>(
          static_cast<uint16_t*>(pool), slot_idx, q, k, v, gates, y, H, G, hpg, T);
      break;
  }
}

template <class Gates>
void launch_prefill_planned(void* pool, int pool_dtype, const int32_t* slot_idx, int B, int T,
                            int H, int G, const float* q, const float* k, const float* v,
                            Gates gates, float* y, int cus, int forced, hipStream_t stream) {
  // At most one extra workgroup per CU for split tiles; the grid has room for
  // whatever the plan uses (the rest return at once).
  const int max_extra = std::min(cus, 3 * B * H);
  // forced: a plan chosen on the host (n8 * 2^20 + n4 * 2^10 + n2), or -1 for the
  // kernel's own; the grid holds whichever plan runs.
  int n_wg = B * H + max_extra;
  if (forced >= 0) {
    const int n8 = std::min(forced >> 20, B), n4 = std::min((forced >> 10) & 1023, B - n8);
    const int n2 = std::min(forced & 1023, B - n8 - n4);
    n_wg = std::max(n_wg, (8 * n8 + 4 * n4 + 2 * n2 + (B - n8 - n4 - n2)) * H);
  }
  const dim3 grid((unsigned)n_wg), block(256);
  const int hpg = H / G;
  switch (pool_dtype) {
    case BRAID_F32:
      gdn_prefill_planned_kernel<F32, Gates><<<grid, block, 0, stream>>>(
          static_cast<float*>(pool), slot_idx, q, k, v, gates, y, B, H, G, hpg, T, cus,
          max_extra, forced);
      break;
    case BRAID_F16:
      gdn_prefill_planned_kernel<F16, Gates><<<grid, block, 0, stream>>>(
          static_cast<uint16_t*>(pool), slot_idx, q, k, v, gates, y, B, H, G, hpg, T, cus,
          max_extra, forced);
      break;
    default:
      gdn_prefill_planned_kernel<BF16, Gates><<<grid, block, 0, stream>>>(
          static_cast<uint16_t*>(pool), slot_idx, q, k, v, gates, y, B, H, G, hpg, T, cus,
          max_extra, forced);
      break;
  }
}

// Host plan of a ragged prefill (the planned kernel's tiers), from the live
// lengths when the call can read them on the host (an eager call, which
// copies the slot map there anyway). Each candidate (n4 quarter rows, n2
// split rows, the rest whole; longest rows first, in the kernel's grid order)
// is scored by simulating the launch on `cus` CUs of two workgroup slots:
// workgroup i takes the first slot of CU i, workgroup cus + i the second,
// later ones the slots as they free (in grid order). A workgroup runs its
// row's tokens at a per-token cost of its tier, solo or sharing its CU, and
// the cost changes whenever its partner starts or ends. CUs with the same
// contents form one class, so a simulation is a few dozen events. The costs,
// relative, were fitted on MI355X to every plan (n8 <= 2, n4 <= 6, n2 <= 8)
// timed over 11 ragged batches (fp16 pool, H = 32), per token: eighth 0.268
// solo / 0.308 shared, quarter 0.344 / 0.469, split 0.416 / 0.499, whole
// 0.619 / 0.871. Against the best measured plan of each batch the chosen ones
// are 6.4% slower in sum over the 11 (at most 4.3%; config 2's is its best,
// 0.426 ms); the kernel's own
// estimate had chosen plans up to 35% slower (config 2: 0.538 against 0.474
// ms; 4 rows of ~1000 and ~300 tokens: 0.484 against 0.359 ms).
struct TierCost {
  float solo, shared;
};
// Tiers: 0 eighth, 1 quarter, 2 split, 3 whole.
constexpr TierCost kPlanCost[4] = {
    {0.268f, 0.308f}, {0.344f, 0.469f}, {0.416f, 0.499f}, {0.619f, 0.871f}};
constexpr int kTierParts[4] = {8, 4, 2, 1};

struct PlanJob {
  float rem, solo, shared;  // fraction of the job left; its duration solo / shared
};
struct PlanClass {
  long m;  // CUs in the class
  int n;   // jobs on each (0..2)
  PlanJob job[2];
};

// The simulation's state, kept between candidates so its buffers are
// allocated once per plan.
struct PlanSim {
  struct Row {
    long count;
    float solo, shared;
  };
  std::vector<Row> rows;
  size_t qi = 0;  // queue front: the next row with workgroups left
  std::vector<PlanClass> cls, next, groups, g2;

  // Fills one free slot on each CU of `c` from the queue (grid order),
  // splitting the class where the queue's rows change; appends to `out`.
  void fill_slot(PlanClass c, std::vector<PlanClass>& out) {
    long m = c.m;
    while (m > 0 && qi < rows.size()) {
      Row& r = rows[qi];
      const long t = std::min(m, r.count);
      PlanClass d = c;
      d.m = t;
      d.job[d.n++] = PlanJob{1.f, r.solo, r.shared};
      out.push_back(d);
      r.count -= t;
      m -= t;
      if (r.count == 0) ++qi;
    }
    if (m > 0) {
      c.m = m;
      out.push_back(c);
    }
  }

  float makespan(const std::vector<int>& sorted_lens, int n8, int n4, int n2, int H, int cus) {
    const int B = (int)sorted_lens.size();
    rows.clear();
    qi = 0;
    for (int r = 0; r < B; ++r) {
      const int tier = r < n8 ? 0 : (r < n8 + n4 ? 1 : (r < n8 + n4 + n2 ? 2 : 3));
      const float L = (float)sorted_lens[r];
      if (sorted_lens[r] > 0)
        rows.push_back({(long)kTierParts[tier] * H, kPlanCost[tier].solo * L,
                        kPlanCost[tier].shared * L});
    }
    next.clear();
    cls.clear();
    fill_slot(PlanClass{cus, 0, {}}, next);  // first slots
    for (const PlanClass& c : next)
      if (c.n > 0) fill_slot(c, cls);         // second slots
    float t = 0.f;
    for (int guard = 0; !cls.empty() && guard < 100000; ++guard) {
      float dt = INFINITY;
      for (const PlanClass& c : cls)
        for (int j = 0; j < c.n; ++j)
          dt = std::min(dt, c.job[j].rem * (c.n == 1 ? c.job[j].solo : c.job[j].shared));
      t += dt;
      next.clear();
      for (PlanClass c : cls) {
        int kept = 0;
        for (int j = 0; j < c.n; ++j) {
          PlanJob jb = c.job[j];
          jb.rem -= dt / (c.n == 1 ? jb.solo : jb.shared);
          if (jb.rem > 1e-6f) c.job[kept++] = jb;
        }
        const int freed = c.n - kept;
        c.n = kept;
        if (freed == 0) {
          next.push_back(c);
          continue;
        }
        groups.clear();
        groups.push_back(c);
        for (int f = 0; f < freed; ++f) {
          g2.clear();
          for (const PlanClass& g : groups) fill_slot(g, g2);
          groups.swap(g2);
        }
        for (const PlanClass& g : groups)
          if (g.n > 0) next.push_back(g);
      }
      cls.swap(next);
    }
    return t;
  }
};

// The plan (n8 * 2^20 + n4 * 2^10 + n2) with the least simulated makespan,
// over n8 <= 2 eighth rows, n4 <= 6 quarter rows and n2 <= 8 split rows
// (ties: the first found, fewer upgraded rows). A candidate is not simulated
// when a lower bound already reaches the best plan so far: its longest row
// in each tier alone and solo, or all its work spread over every slot at the
// shared costs.
int simulate_prefill_plans(const std::vector<int>& lens, int H, int cus);

// Plans already chosen, by (sorted live lengths, H, CUs): a scheduler's ticks
// repeat their chunk lengths, and a simulation costs 2-95 us of host time
// (16 ragged rows: 95 us) against about 1 us for the lookup. Bounded: at
// kPlanCacheMax entries the oldest entry is evicted for each new one (first
// in, first out), so a serving loop past the bound re-plans only the lengths
// it has not seen lately instead of all of them at once.
constexpr size_t kPlanCacheMax = 4096;

int host_prefill_plan(const std::vector<int32_t>& seq_lens, int T, int H, int cus) {
  std::vector<int> lens(seq_lens.size());
  for (size_t r = 0; r < lens.size(); ++r) lens[r] = std::min(std::max((int)seq_lens[r], 0), T);
  std::sort(lens.begin(), lens.end(), std::greater<int>());
  static std::mutex mu;
  static std::map<std::vector<int>, int> cache;
  static std::deque<std::map<std::vector<int>, int>::iterator> order;
  std::vector<int> key(lens);
  key.push_back(H);
  key.push_back(cus);
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  const int plan = simulate_prefill_plans(lens, H, cus);
  std::lock_guard<std::mutex> lock(mu);
  const auto ins = cache.emplace(std::move(key), plan);
  if (ins.second) {  // another thread may have planned the same lengths meanwhile
    order.push_back(ins.first);
    if (order.size() > kPlanCacheMax) {
      cache.erase(order.front());
      order.pop_front();
    }
  }
  return plan;
}

// The simulation behind host_prefill_plan, over lengths sorted longest first.
int simulate_prefill_plans(const std::vector<int>& lens, int H, int cus) {
  const int B = (int)lens.size();
  std::vector<double> prefix(B + 1, 0.0);
  for (int r = 0; r < B; ++r) prefix[r + 1] = prefix[r] + lens[r];
  PlanSim sim;
  float best = INFINITY;
  int plan = 0;
  for (int n8 = 0; n8 <= std::min(B, 2); ++n8)
    for (int n4 = 0; n4 <= std::min(B - n8, 6); ++n4)
      for (int n2 = 0; n2 <= std::min(B - n8 - n4, 8); ++n2) {
        const int first[4] = {0, n8, n8 + n4, n8 + n4 + n2};
        const int count[4] = {n8, n4, n2, B - n8 - n4 - n2};
        float bound = 0.f;
        double work = 0.0;
        for (int t = 0; t < 4; ++t) {
          if (count[t] == 0) continue;
          bound = std::max(bound, kPlanCost[t].solo * lens[first[t]]);
          work += kTierParts[t] * kPlanCost[t].shared *
                  (prefix[first[t] + count[t]] - prefix[first[t]]);
        }
        bound = std::max(bound, (float)(H * work / (2.0 * cus)));
        if (bound >= best) continue;
        const float m = sim.makespan(lens, n8, n4, n2, H, cus);
        if (m < best) {
          best = m;
          plan = (n8 << 20) | (n4 << 10) | n2;
        }
      }
  return plan;
}

template <class Gates>
int launch_prefill(void* pool, int pool_dtype, const int32_t* slot_idx, int B, int T, int H,
                   int G, const float* q, const float* k, const float* v, Gates gates,
                   float* y, const std::vector<int32_t>* host_lens, hipStream_t stream,
                   int plan_hint = -1) {
  const int cus = device_cus();
  int layout = prefill_layout(B * H, B, T, gates.ragged(), cus);
  // With the live lengths on the host, every ragged batch the planned kernel
  // takes is planned there. A plan that puts every row in one tier runs that
  // layout's own kernel instead (its split layout runs token pairs, which
  // the planned kernel's does not: config 4's 4 x 256 tokens 0.155 ms
  // planned, 0.132 ms in the split kernel).
  int host_plan = -1;
  if (host_lens != nullptr && layout != 8 && launch_knob(BRAID_KNOB_PREFILL_LAYOUT) < 0 &&
      launch_knob(BRAID_KNOB_PREFILL_PLAN) < 0 && B <= kMaxPlanRows && cus > 0 &&
      B * H <= 4 * cus) {
    host_plan = host_prefill_plan(*host_lens, T, H, cus);
    const int n8 = host_plan >> 20, n4 = (host_plan >> 10) & 1023, n2 = host_plan & 1023;
    layout = n8 == B ? 8 : (n4 == B ? 4 : (n2 == B ? 1 : 0));
  } else if (plan_hint >= 0 && gates.ragged() && layout != 8 &&
             launch_knob(BRAID_KNOB_PREFILL_LAYOUT) < 0 &&
             launch_knob(BRAID_KNOB_PREFILL_PLAN) < 0 && B <= kMaxPlanRows && cus > 0 &&
             B * H <= 4 * cus) {
    // The caller's plan (braid_gdn_prefill_raw_plan), taken as the host's.
    const int n8 = std::min(plan_hint >> 20, B);
    const int n4 = std::min((plan_hint >> 10) & 1023, B - n8);
    const int n2 = std::min(plan_hint & 1023, B - n8 - n4);
    host_plan = (n8 << 20) | (n4 << 10) | n2;
    layout = n8 == B ? 8 : (n4 == B ? 4 : (n2 == B ? 1 : 0));
  }
  if (layout == 8)
    launch_prefill_cols<Gates, 8>(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y,
                                  stream);
  else if (layout == 4)
    launch_prefill_cols<Gates, 4>(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y,
                                  stream);
  else if (layout == 1)
    launch_prefill_cols<Gates, 1>(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y,
                                  stream);
  else if (layout == 2)
    launch_prefill_cols<Gates, 2>(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y,
                                  stream);
  else {
    // The PREFILL_PLAN knob (measurement) forces a plan; otherwise an eager
    // call runs the host's plan and a captured one leaves it to the kernel.
    int forced = launch_knob(BRAID_KNOB_PREFILL_PLAN);
    if (forced < 0) forced = host_plan;
    launch_prefill_planned<Gates>(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y,
                                  cus > 0 ? cus : 256, forced, stream);
  }
  const int st = hip_status(hipGetLastError(), "launching gdn_prefill_kernel");
  return st != BRAID_OK ? st : ok();
}

int check_dense(const void* p, const char* name) {
  if (p == nullptr) return fail(BRAID_EINVAL, std::string(name) + " must be non-null");
  if (!aligned16(p)) return fail(BRAID_EINVAL, std::string(name) + " must be 16-byte aligned");
  return BRAID_OK;
}

}  // namespace
}  // namespace braid

using namespace braid;

#define BRAID_TRY(expr)            \
  do {                             \
    const int _st = (expr);        \
    if (_st != BRAID_OK) return _st; \
  } while (0)

extern "C" int braid_gdn_decode(void* pool, int pool_dtype, int64_t n_slots, int H, int G,
                                int SS, int HD, const int32_t* slot_idx, int B, const float* q,
                                int64_t q_row, const float* k, int64_t k_row, const float* v,
                                int64_t v_row, const float* alpha, const float* beta, float* y,
                                void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  BRAID_TRY(check_common(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B));
  if (B == 0) return ok();
  BRAID_TRY(check_rows(q, q_row, (int64_t)G * SS, "q"));
  BRAID_TRY(check_rows(k, k_row, (int64_t)G * SS, "k"));
  BRAID_TRY(check_rows(v, v_row, (int64_t)H * HD, "v"));
  if (alpha == nullptr || beta == nullptr)
    return fail(BRAID_EINVAL, "alpha/beta must be non-null");
  BRAID_TRY(check_dense(y, "y"));
  BRAID_TRY(validate_slots(slot_idx, B, n_slots, true, stream));
  return launch_decode(pool, pool_dtype, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                       PrecomputedGates{alpha, beta}, y, stream);
}

extern "C" int braid_gdn_decode_raw(void* pool, int pool_dtype, int64_t n_slots, int H, int G,
                                    int SS, int HD, const int32_t* slot_idx, int B,
                                    const float* q, int64_t q_row, const float* k,
                                    int64_t k_row, const float* v, int64_t v_row,
                                    const void* a_raw, const void* b_raw, int act_dtype,
                                    const float* A, const float* dt_bias, float* y,
                                    void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  BRAID_TRY(check_common(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B));
  BRAID_TRY(check_act(a_raw, b_raw, act_dtype, A, dt_bias));
  if (B == 0) return ok();
  BRAID_TRY(check_rows(q, q_row, (int64_t)G * SS, "q"));
  BRAID_TRY(check_rows(k, k_row, (int64_t)G * SS, "k"));
  BRAID_TRY(check_rows(v, v_row, (int64_t)H * HD, "v"));
  BRAID_TRY(check_dense(y, "y"));
  BRAID_TRY(validate_slots(slot_idx, B, n_slots, true, stream));
  if (act_dtype == BRAID_F32) {
    RawGates<F32> gates{static_cast<const float*>(a_raw), static_cast<const float*>(b_raw), A,
                        dt_bias, nullptr};
    return launch_decode(pool, pool_dtype, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row,
                         gates, y, stream);
  }
  RawGates<BF16> gates{static_cast<const uint16_t*>(a_raw), static_cast<const uint16_t*>(b_raw),
                       A, dt_bias, nullptr};
  return launch_decode(pool, pool_dtype, slot_idx, B, H, G, q, q_row, k, k_row, v, v_row, gates,
                       y, stream);
}

extern "C" int braid_gdn_prefill(void* pool, int pool_dtype, int64_t n_slots, int H, int G,
                                 int SS, int HD, const int32_t* slot_idx, int B, int T,
                                 const float* q, const float* k, const float* v,
                                 const float* alpha, const float* beta, float* y,
                                 void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  BRAID_TRY(check_common(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B));
  if (T < 0) return fail(BRAID_EINVAL, "T must be non-negative");
  if (B == 0) return ok();
  if (T > 0) {
    BRAID_TRY(check_dense(q, "q"));
    BRAID_TRY(check_dense(k, "k"));
    BRAID_TRY(check_dense(v, "v"));
    BRAID_TRY(check_dense(y, "y"));
    if (alpha == nullptr || beta == nullptr)
      return fail(BRAID_EINVAL, "alpha/beta must be non-null");
  }
  BRAID_TRY(validate_slots(slot_idx, B, n_slots, true, stream));
  return launch_prefill(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v,
                        PrecomputedGates{alpha, beta}, y, nullptr, stream);
}

namespace braid {
namespace {

int prefill_raw(void* pool, int pool_dtype, int64_t n_slots, int H, int G, int SS, int HD,
                const int32_t* slot_idx, int B, int T, const float* q, const float* k,
                const float* v, const void* a_raw, const void* b_raw, int act_dtype,
                const float* A, const float* dt_bias, float* y, const int32_t* seq_lens,
                int plan_hint, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  BRAID_TRY(check_common(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B));
  if (T < 0) return fail(BRAID_EINVAL, "T must be non-negative");
  BRAID_TRY(check_act(a_raw, b_raw, act_dtype, A, dt_bias));
  if (B == 0) return ok();
  if (T > 0) {
    BRAID_TRY(check_dense(q, "q"));
    BRAID_TRY(check_dense(k, "k"));
    BRAID_TRY(check_dense(v, "v"));
    BRAID_TRY(check_dense(y, "y"));
  }
  // An eager call reads the live lengths on the host for the ragged plan, in
  // the slot check's round trip (one synchronisation for both copies).
  std::vector<int32_t> host_lens;
  int cap_st = BRAID_OK;
  const bool capturing = stream_capturing(stream, &cap_st);
  if (cap_st != BRAID_OK) return cap_st;
  if (seq_lens != nullptr && !capturing && T > 0) host_lens.resize(B);
  BRAID_TRY(validate_slots(slot_idx, B, n_slots, true, stream,
                           host_lens.empty() ? nullptr : seq_lens,
                           host_lens.empty() ? nullptr : host_lens.data()));
  const std::vector<int32_t>* lens_p = host_lens.empty() ? nullptr : &host_lens;
  if (act_dtype == BRAID_F32) {
    RawGates<F32> gates{static_cast<const float*>(a_raw), static_cast<const float*>(b_raw), A,
                        dt_bias, seq_lens};
    return launch_prefill(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y, lens_p,
                          stream, plan_hint);
  }
  RawGates<BF16> gates{static_cast<const uint16_t*>(a_raw), static_cast<const uint16_t*>(b_raw),
                       A, dt_bias, seq_lens};
  return launch_prefill(pool, pool_dtype, slot_idx, B, T, H, G, q, k, v, gates, y, lens_p,
                        stream, plan_hint);
}

}  // namespace
}  // namespace braid

extern "C" int braid_gdn_prefill_raw(void* pool, int pool_dtype, int64_t n_slots, int H, int G,
                                     int SS, int HD, const int32_t* slot_idx, int B, int T,
                                     const float* q, const float* k, const float* v,
                                     const void* a_raw, const void* b_raw, int act_dtype,
                                     const float* A, const float* dt_bias, float* y,
                                     const int32_t* seq_lens, void* stream_) {
  return prefill_raw(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B, T, q, k, v, a_raw,
                     b_raw, act_dtype, A, dt_bias, y, seq_lens, -1, stream_);
}

extern "C" int braid_gdn_prefill_raw_plan(void* pool, int pool_dtype, int64_t n_slots, int H,
                                          int G, int SS, int HD, const int32_t* slot_idx, int B,
                                          int T, const float* q, const float* k, const float* v,
                                          const void* a_raw, const void* b_raw, int act_dtype,
                                          const float* A, const float* dt_bias, float* y,
                                          const int32_t* seq_lens, int plan, void* stream_) {
  if (plan >= 0 && seq_lens == nullptr)
    return fail(BRAID_EINVAL, "a prefill plan needs seq_lens (it plans ragged batches)");
  return prefill_raw(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B, T, q, k, v, a_raw,
                     b_raw, act_dtype, A, dt_bias, y, seq_lens, plan, stream_);
}

namespace braid {
namespace {

template <class Tag, class XT, class Gates, int HPG>
void launch_conv_decode_as(void* pool, float* conv_pool, const int32_t* slot_idx, int B, int H,
                           int G, int C, const void* x, const float* w, const float* bias,
                           Gates gates, float* y, hipStream_t stream) {
  const dim3 grid((unsigned)B * (unsigned)G), block(tile_threads(kDecodeCols) * HPG);
  if constexpr (std::is_same<Tag, F32>::value)
    gdn_conv_decode_kernel_f32<XT, Gates, HPG><<<grid, block, 0, stream>>>(
        static_cast<float*>(pool), conv_pool, slot_idx, static_cast<const XT*>(x), w, bias,
        gates, y, H, G, C);
  else
    gdn_conv_decode_kernel<Tag, XT, Gates, HPG><<<grid, block, 0, stream>>>(
        static_cast<typename Storage<Tag>::T*>(pool), conv_pool, slot_idx,
        static_cast<const XT*>(x), w, bias, gates, y, H, G, C);
}

template <class Tag, class XT, class Gates>
void launch_conv_decode_hpg(int hpg, void* pool, float* conv_pool, const int32_t* slot_idx,
                            int B, int H, int G, int C, const void* x, const float* w,
                            const float* bias, Gates gates, float* y, hipStream_t stream) {
  if (hpg == 1)
    launch_conv_decode_as<Tag, XT, Gates, 1>(pool, conv_pool, slot_idx, B, H, G, C, x, w, bias,
                                             gates, y, stream);
  else
    launch_conv_decode_as<Tag, XT, Gates, 2>(pool, conv_pool, slot_idx, B, H, G, C, x, w, bias,
                                             gates, y, stream);
}

template <class XT, class Gates>
void launch_conv_decode(int pool_dtype, int hpg, void* pool, float* conv_pool,
                        const int32_t* slot_idx, int B, int H, int G, int C, const void* x,
                        const float* w, const float* bias, Gates gates, float* y,
                        hipStream_t stream) {
  switch (pool_dtype) {
    case BRAID_F32:
      launch_conv_decode_hpg<F32, XT, Gates>(hpg, pool, conv_pool, slot_idx, B, H, G, C, x, w,
                                             bias, gates, y, stream);
      break;
    case BRAID_F16:
      launch_conv_decode_hpg<F16, XT, Gates>(hpg, pool, conv_pool, slot_idx, B, H, G, C, x, w,
                                             bias, gates, y, stream);
      break;
    default:
      launch_conv_decode_hpg<BF16, XT, Gates>(hpg, pool, conv_pool, slot_idx, B, H, G, C, x, w,
                                              bias, gates, y, stream);
      break;
  }
}

}  // namespace
}  // namespace braid

extern "C" int braid_gdn_conv_decode_raw(void* pool, int pool_dtype, int64_t n_slots, int H,
                                         int G, int SS, int HD, float* conv_pool, int K,
                                         const int32_t* slot_idx, int B, const void* x,
                                         int x_dtype, const float* conv_weight,
                                         const float* conv_bias, const void* a_raw,
                                         const void* b_raw, int act_dtype, const float* A,
                                         const float* dt_bias, float* y, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  BRAID_TRY(check_common(pool, pool_dtype, n_slots, H, G, SS, HD, slot_idx, B));
  BRAID_TRY(check_act(a_raw, b_raw, act_dtype, A, dt_bias));
  const int hpg = H / G;
  if (hpg != 1 && hpg != 2)
    return fail(BRAID_EINVAL, "the fused conv decode takes 1 or 2 value heads per key group");
  if (K != 4) return fail(BRAID_EINVAL, "the fused conv decode takes conv_kernel == 4");
  if (x_dtype != BRAID_F32 && x_dtype != BRAID_BF16)
    return fail(BRAID_EINVAL, "x must be fp32 or bf16 (the activation dtypes braid runs)");
  if (B == 0) return ok();
  if (conv_pool == nullptr || x == nullptr || conv_weight == nullptr)
    return fail(BRAID_EINVAL, "conv_pool, x and conv_weight must be non-null");
  if (!aligned16(conv_pool) || !aligned16(conv_weight))
    return fail(BRAID_EINVAL, "conv_pool and conv_weight must be 16-byte aligned");
  BRAID_TRY(check_dense(y, "y"));
  BRAID_TRY(validate_slots(slot_idx, B, n_slots, true, stream));
  const int C = 2 * G * SS + H * HD;
  auto go = [&](auto gates) {
    if (x_dtype == BRAID_F32)
      launch_conv_decode<float>(pool_dtype, hpg, pool, conv_pool, slot_idx, B, H, G, C, x,
                                conv_weight, conv_bias, gates, y, stream);
    else
      launch_conv_decode<uint16_t>(pool_dtype, hpg, pool, conv_pool, slot_idx, B, H, G, C, x,
                                   conv_weight, conv_bias, gates, y, stream);
    const int st = hip_status(hipGetLastError(), "launching gdn_conv_decode_kernel");
    return st != BRAID_OK ? st : ok();
  };
  if (act_dtype == BRAID_F32)
    return go(RawGates<F32>{static_cast<const float*>(a_raw), static_cast<const float*>(b_raw),
                            A, dt_bias, nullptr});
  return go(RawGates<BF16>{static_cast<const uint16_t*>(a_raw),
                           static_cast<const uint16_t*>(b_raw), A, dt_bias, nullptr});
}

extern "C" int braid_prefill_plan(const int32_t* seq_lens_host, int B, int T, int H, int cus) {
  if (seq_lens_host == nullptr || B <= 0 || T < 0 || H <= 0 || cus <= 0)
    return -fail(BRAID_EINVAL,
                 "braid_prefill_plan needs host lengths, B > 0, T >= 0, H > 0, cus > 0");
  return host_prefill_plan(std::vector<int32_t>(seq_lens_host, seq_lens_host + B), T, H, cus);
}
