/*
 * braid_gdn.h — C ABI of the MI355X (gfx950) Gated DeltaNet mixer hot path.
 *
 * One shared library, libbraid_gdn.so, exports these entry points. They take
 * plain device pointers, element counts/strides and a hipStream_t (passed as
 * void* so this header needs no HIP include), enqueue work on that stream and
 * return 0 on success. On failure they return a nonzero braid_status and
 * braid_last_error() returns a thread-local, human-readable message. Nothing
 * here allocates device memory; every output buffer and workspace belongs to
 * the caller.
 *
 * Each entry replaces one function of the reference's pybind11 module
 * (braid/kernels/csrc/bindings.cpp:25-34); the citation on each declaration
 * names the reference function whose behaviour it reproduces.
 *
 * Slot validation: every state-pool entry point checks the device slot map
 * (range and, for the GDN scans, distinctness) by copying it to the host —
 * unless the stream is capturing a graph, where a device->host copy would be
 * illegal. This mirrors braid/kernels/csrc/gdn_decode.cu:280-297 and
 * conv1d_decode.cu:77-89.
 */
#ifndef BRAID_GDN_H
#define BRAID_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of the state pool, the activations and the conv input. */
enum braid_dtype {
  BRAID_F32 = 0,
  BRAID_F16 = 1,
  BRAID_BF16 = 2,
};

enum braid_status {
  BRAID_OK = 0,
  BRAID_EINVAL = 1,    /* bad argument: shape, dtype, null pointer, overlap */
  BRAID_ESLOT = 2,     /* slot map out of range or (GDN scans) not distinct */
  BRAID_EHIP = 3,      /* a HIP runtime call failed */
};

/* ABI version; bumped on any signature change. */
int braid_abi_version(void);

/* Message for the last failing call on this thread ("" when none). */
const char* braid_last_error(void);

/*
 * Launch knobs: overrides of the launch-shape choices the library makes per
 * launch, for measurement and for tests that force each shape. No entry
 * point's results depend on them (every shape gives the same bits); only the
 * time does. No counterpart in the reference, which has one launch shape per
 * kernel. Each knob starts from its environment variable, read once when the
 * library loads; -1 (or unset) means "the library's own choice".
 *
 *   BRAID_KNOB_DECODE_XCD_REMAP  (BRAID_DECODE_XCD_REMAP)  0 / 1
 *   BRAID_KNOB_DECODE_WGS_PER_CU (BRAID_DECODE_WGS_PER_CU) 0 uncapped, N
 *   BRAID_KNOB_PREFILL_LAYOUT    (BRAID_PREFILL_COLS)      1, 2, 4, 8, or 0 planned
 *   BRAID_KNOB_DECODE_PARTS      (BRAID_DECODE_PARTS)      1, 2 or 4 column parts
 *   BRAID_KNOB_PREFILL_PLAN      (BRAID_PREFILL_PLAN)      n8 * 2^20 + n4 * 2^10 + n2:
 *                                a planned prefill runs its n8 longest rows in the
 *                                eighth layout, the next n4 quarter, the next n2
 *                                split
 *   BRAID_KNOB_FP8_GEMM          (BRAID_FP8_GEMM)          0 hipBLASLt, 1 the streaming
 *                                small-M kernel (where its shape rules allow)
 *
 * A captured graph keeps the launch shape it was captured with. An environment
 * value that is not a whole decimal number in [0, 2^30] leaves the knob unset.
 * The knobs are process-wide: an override set on one thread shapes the
 * launches of every thread.
 */
enum braid_launch_knob {
  BRAID_KNOB_DECODE_XCD_REMAP = 0,
  BRAID_KNOB_DECODE_WGS_PER_CU = 1,
  BRAID_KNOB_PREFILL_LAYOUT = 2,
  BRAID_KNOB_DECODE_PARTS = 3,
  BRAID_KNOB_PREFILL_PLAN = 4,
  BRAID_KNOB_FP8_GEMM = 5,
};
/*
 * The plan an eager braid_gdn_prefill_raw with seq_lens chooses for a ragged
 * batch: n8 * 2^20 + n4 * 2^10 + n2 (its n8 longest rows in the eighth layout,
 * eight workgroups per tile; the next n4 quarter, four; the next n2 split
 * over two; the rest whole), from host lengths, for `cus` CUs; -BRAID_EINVAL
 * on bad arguments. Host-only (no GPU call), for measurement and tests. No
 * counterpart in the reference.
 */
int braid_prefill_plan(const int32_t* seq_lens_host, int B, int T, int H, int cus);

/* Sets a knob (value < 0 clears it). BRAID_EINVAL for an unknown knob. */
int braid_set_launch_override(int knob, int value);
/* The knob's current value, -1 when unset or unknown. */
int braid_get_launch_override(int knob);

/*
 * Batched GDN decode step, precomputed gates.
 * Replaces gdn_decode (braid/kernels/csrc/gdn_decode.cu:313-360).
 *
 *   pool     [n_slots, H, SS, HD] of pool_dtype, updated in place at the rows
 *            named by slot_idx only
 *   slot_idx [B] int32, device
 *   q, k     [B, G, SS] fp32; the last two dims dense, batch row stride
 *            q_row / k_row elements (>= G*SS)
 *   v        [B, H, HD] fp32, batch row stride v_row (>= H*HD)
 *   alpha, beta [B, H] fp32 dense
 *   y        [B, H, HD] fp32 dense, written
 * SS and HD must be 128; H % G == 0.
 */
int braid_gdn_decode(void* pool, int pool_dtype, int64_t n_slots, int H, int G,
                     int SS, int HD, const int32_t* slot_idx, int B,
                     const float* q, int64_t q_row, const float* k,
                     int64_t k_row, const float* v, int64_t v_row,
                     const float* alpha, const float* beta, float* y,
                     void* stream);

/*
 * Batched GDN decode step with the gates computed in-kernel from the raw
 * projections. Replaces gdn_decode_raw (gdn_decode.cu:367-441).
 *
 *   a_raw, b_raw [B, H] of act_dtype (BRAID_F32 or BRAID_BF16), dense
 *   A, dt_bias   [H] fp32 (A already -exp(A_log))
 *   beta  = widen(round_act(1 / (1 + exp(-b))))
 *   alpha = exp(A * softplus(a + dt_bias)), softplus(x) = x > 20 ? x : log1p(exp(x))
 */
int braid_gdn_decode_raw(void* pool, int pool_dtype, int64_t n_slots, int H,
                         int G, int SS, int HD, const int32_t* slot_idx, int B,
                         const float* q, int64_t q_row, const float* k,
                         int64_t k_row, const float* v, int64_t v_row,
                         const void* a_raw, const void* b_raw, int act_dtype,
                         const float* A, const float* dt_bias, float* y,
                         void* stream);

/*
 * The conv1d decode step fused into the GDN decode step with in-kernel gates:
 * braid_conv1d_decode followed by braid_gdn_decode_raw on the conv output's
 * q/k/v column views, in one launch and bit for bit the same outputs, state
 * and windows. Replaces the pair the reference's decode runs back to back
 * (braid/model/gdn.py:131-160: conv1d_decode, then gdn_decode_raw on
 * split/unflatten views of its output); the conv output is not written.
 *
 *   conv_pool [n_slots, C, K] fp32 with C = 2*G*SS + H*HD ([Q | K | V]);
 *             K must be 4; updated in place at the slot rows
 *   x         [B, C] of x_dtype (BRAID_F32 or BRAID_BF16), dense
 *   conv_weight [C, K] fp32; conv_bias [C] fp32 or NULL
 *   H / G must be 1 or 2. Other arguments as braid_gdn_decode_raw; slots must
 *   be distinct.
 */
int braid_gdn_conv_decode_raw(void* pool, int pool_dtype, int64_t n_slots, int H,
                              int G, int SS, int HD, float* conv_pool, int K,
                              const int32_t* slot_idx, int B, const void* x,
                              int x_dtype, const float* conv_weight,
                              const float* conv_bias, const void* a_raw,
                              const void* b_raw, int act_dtype, const float* A,
                              const float* dt_bias, float* y, void* stream);

/*
 * Chunk prefill scan: T tokens per launch, state held on chip between them.
 * Replaces gdn_prefill (gdn_decode.cu:553-603).
 *
 *   q, k [B, T, G, SS], v and y [B, T, H, HD], alpha/beta [B, T, H]; all fp32
 *   dense. The caller pads with alpha = 1, beta = 0 (an exact identity step).
 * The result equals braid_gdn_decode applied T times, bit for bit, for every
 * pool dtype (the on-chip state is kept in the pool's storage type).
 */
int braid_gdn_prefill(void* pool, int pool_dtype, int64_t n_slots, int H,
                      int G, int SS, int HD, const int32_t* slot_idx, int B,
                      int T, const float* q, const float* k, const float* v,
                      const float* alpha, const float* beta, float* y,
                      void* stream);

/*
 * Chunk prefill scan with in-kernel gates and ragged lengths.
 * Replaces gdn_prefill_raw (gdn_decode.cu:611-699).
 *
 *   a_raw, b_raw [B, T, H] of act_dtype, dense
 *   seq_lens     [B] int32 device, or NULL (every column live). A column
 *                t >= seq_lens[b] runs alpha = 1, beta = 0. 0 and values > T
 *                are legal.
 */
int braid_gdn_prefill_raw(void* pool, int pool_dtype, int64_t n_slots, int H,
                          int G, int SS, int HD, const int32_t* slot_idx,
                          int B, int T, const float* q, const float* k,
                          const float* v, const void* a_raw, const void* b_raw,
                          int act_dtype, const float* A, const float* dt_bias,
                          float* y, const int32_t* seq_lens, void* stream);

/*
 * braid_gdn_prefill_raw with the caller's launch plan for a ragged batch
 * (plan: what braid_prefill_plan returns for the lengths the caller expects,
 * or < 0 for none). An eager call reads seq_lens on the host and plans from
 * them, so it ignores the plan; a call under graph capture cannot, and
 * without a plan it runs the kernel's own cruder estimate. Any plan computes
 * the same bits for any lengths (the kernel ranks the rows by their actual
 * lengths); the plan only shapes the launch. A plan needs seq_lens
 * (BRAID_EINVAL without). No counterpart in the reference, whose prefill is
 * not captured.
 */
int braid_gdn_prefill_raw_plan(void* pool, int pool_dtype, int64_t n_slots, int H,
                               int G, int SS, int HD, const int32_t* slot_idx,
                               int B, int T, const float* q, const float* k,
                               const float* v, const void* a_raw, const void* b_raw,
                               int act_dtype, const float* A, const float* dt_bias,
                               float* y, const int32_t* seq_lens, int plan, void* stream);

/*
 * Batched slotted causal depthwise conv1d, one decode step, SiLU fused.
 * Replaces conv1d_decode (braid/kernels/csrc/conv1d_decode.cu:91-149).
 *
 *   conv_pool [n_slots, C, K] fp32, window of the last K pre-conv inputs,
 *             oldest first, K contiguous per channel; updated in place
 *   x         [B, C] of x_dtype (BRAID_F32 or BRAID_BF16), dense
 *   weight    [C, K] fp32; bias [C] fp32 or NULL
 *   out       [B, C] fp32: SiLU(sum_i window[i] * weight[c, i] + bias[c])
 * K must be 2, 3, 4 or 8. Slots are range-checked only (no distinctness).
 */
int braid_conv1d_decode(float* conv_pool, int64_t n_slots, int C, int K,
                        const int32_t* slot_idx, int B, const void* x,
                        int x_dtype, const float* weight, const float* bias,
                        float* out, void* stream);

/*
 * Chunked causal conv1d (prefill), SiLU fused: T tokens per launch.
 * Replaces the reference's prefill conv, which is torch code rather than a
 * kernel: F.conv1d over [cached window | x] plus a gather that saves the last
 * K real inputs of each ragged row (braid/model/gdn.py:171-226).
 *
 *   conv_pool [n_slots, C, K] fp32, as for braid_conv1d_decode
 *   x         [B, T, C] of x_dtype (BRAID_F32 or BRAID_BF16), dense
 *   out       [B, T, C] fp32
 *   seq_lens  [B] int32 device, or NULL (all T tokens live). Row b runs tokens
 *             0..min(seq_lens[b], T)-1; 0 and values > T are legal.
 * For live tokens the outputs and the window left in the pool equal
 * braid_conv1d_decode applied token by token, bit for bit. Pad positions
 * (t >= len) are written as 0 and do not move the window. Slots must be
 * distinct (each row rewrites its window).
 */
int braid_conv1d_prefill(float* conv_pool, int64_t n_slots, int C, int K,
                         const int32_t* slot_idx, int B, int T, const void* x,
                         int x_dtype, const float* weight, const float* bias,
                         float* out, const int32_t* seq_lens, void* stream);

/*
 * Number of fp32 partials braid_quantize_act needs as workspace for an
 * n-element activation.
 */
int braid_quantize_act_workspace(int64_t n);

/*
 * Dynamic per-tensor FP8 e4m3fn activation quantization, two launches.
 * Replaces quantize_act (braid/kernels/csrc/quant_act.cu:140-176), which
 * allocated its outputs; here the caller passes them.
 *
 *   x       n contiguous elements of x_dtype (F32, F16 or BF16), n > 0
 *   q       n bytes, e4m3fn codes
 *   scale   1 fp32: max(amax(|x|) * fl(1/448), 1e-12), NaN if x holds NaN
 *   partial braid_quantize_act_workspace(n) fp32 scratch
 * q = e4m3fn(clamp(x / scale, -448, 448)), round to nearest even.
 */
int braid_quantize_act(const void* x, int x_dtype, int64_t n, uint8_t* q,
                       float* scale, float* partial, void* stream);

/*
 * braid_quantize_act without a workspace argument: the pass-1 partial maxima
 * go to a device scratch array inside the library (1024 floats, 4 KiB, one
 * copy per GPU, held until the process ends), so the call allocates nothing
 * and needs no caller buffer beyond x, q and scale. No counterpart in the
 * reference: it is for callers that cannot allocate, such as code under
 * graph capture or a serving loop that forbids allocation. Codes and scale
 * equal braid_quantize_act's bit for bit. Single-stream contract: every call
 * on one GPU shares that GPU's scratch, so the caller issues all of a GPU's
 * calls on one stream (or otherwise orders them, e.g. with events); calls
 * that overlap on one GPU (different streams, or different threads) race and
 * may return wrong codes and scales. The library does not detect this. A call fully
 * rewrites the partials it reads, so nothing needs clearing between calls.
 * The partial count never exceeds the scratch for any n (it is capped at
 * 1024); a larger count would be rejected with BRAID_EINVAL. Arguments and
 * errors otherwise as braid_quantize_act.
 */
int braid_quantize_act_noalloc(const void* x, int x_dtype, int64_t n, uint8_t* q,
                               float* scale, void* stream);

/*
 * Number of fp32 partials braid_gated_rmsnorm_quant needs as workspace for
 * `units` (token, head) units.
 */
int braid_gated_rmsnorm_workspace(int64_t units);

/*
 * Gated RMSNorm readout of the mixer, optionally fused with the out_proj
 * input's dynamic FP8 quantization. Replaces the torch readout
 * GatedDeltaNet._readout + rms_norm_gated (braid/model/gdn.py:373-387,
 * braid/model/norm.py:48-71) followed by quantize_act (quant.py:209-229) on
 * its result.
 *
 *   y      [units, HD] of y_dtype (BRAID_F32, or act_dtype), dense: the scan
 *          output, units = tokens * H
 *   z      [units, HD] of act_dtype (F32, F16 or BF16), dense: the gate
 *   gamma  [HD] fp32 (stored directly, no unit offset)
 *   core   [units, HD] of act_dtype, written:
 *            c = round_act(y); xf = c * rsqrt(mean(c^2) + eps)
 *            core = round_act(gamma * round_act(xf) * silu(z))
 *   q, scale, partial: NULL for the norm alone (one launch); else q
 *          [units*HD] e4m3fn codes and scale [1] fp32 = quantize_act(core)
 *          bit for bit, with braid_gated_rmsnorm_workspace(units) partials.
 * HD must be 128; y, z, gamma and core 16-byte aligned. units == 0 is a no-op
 * for the norm alone and an error with q (quantize_act rejects empty input).
 */
int braid_gated_rmsnorm_quant(const void* y, int y_dtype, const void* z,
                              int act_dtype, const float* gamma, float eps,
                              int64_t units, int HD, void* core, uint8_t* q,
                              float* scale, float* partial, void* stream);

/*
 * Workspace bytes braid_fp8_gemm plans for (the algorithm it selects needs at
 * most this much).
 */
size_t braid_fp8_gemm_workspace(void);

/*
 * FP8 e4m3fn W8A8 GEMM with per-tensor dequant scales. Decode shapes
 * (1 <= M <= 64, K = 1024 * 2^i for i < 5) run a hand-written kernel that
 * streams the weight once (no workspace used, fixed summation order, so
 * repeated calls give the same bits); other shapes, and every shape under
 * BRAID_FP8_GEMM=0, run one hipBLASLt matmul.
 * Replaces fp8_matmul's torch._scaled_mm(xq, w.t(), scale_a=sx, scale_b=sw)
 * (braid/model/quant.py:232-241).
 *
 *   x        [M, K] e4m3fn codes, row-major (the quantized activation)
 *   x_scale  [1] fp32 device: x's dequant scale
 *   w        [N, K] e4m3fn codes, row-major (the weight, as FP8Weight.data)
 *   w_scale  [1] fp32 device
 *   out      [M, N] of out_dtype (BRAID_BF16, F16 or F32), row-major:
 *            out = (x * x_scale) @ (w * w_scale)^T, fp32 accumulation
 *   workspace  device scratch of workspace_bytes (>= braid_fp8_gemm_workspace())
 * N and K must be multiples of 16. On the hipBLASLt path the first call for a
 * shape selects the algorithm on the host; later calls only enqueue, and may
 * be captured (the streaming kernel needs no such first call). Calls sharing
 * one workspace must not overlap.
 */
int braid_fp8_gemm(const uint8_t* x, const float* x_scale, const uint8_t* w,
                   const float* w_scale, void* out, int out_dtype, int64_t M,
                   int64_t N, int64_t K, void* workspace,
                   size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BRAID_GDN_H */
