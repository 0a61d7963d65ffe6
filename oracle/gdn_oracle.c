/*
 * CPU oracle for the GDN mixer hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, scalar, fp32 restatement of the reference's arithmetic, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. Nothing in the product links, loads or calls this file.
 *
 * Built with -O2 -ffp-contract=off and no fast-math: every multiply and add
 * below rounds separately, in source order, and libm's expf / log1pf / sqrtf
 * are used as is.
 *
 * Functions and the reference lines they restate:
 *   oracle_gdn_decode     braid/reference/gdn_ref.py:42-99 (operator order) and
 *                         braid/kernels/csrc/gdn_decode.cu:198-271 (in-kernel
 *                         l2norm with the additive 1e-6 epsilon, y scaled after
 *                         the dot, grouped head->group map g = h / (H/G))
 *   oracle_gdn_gates      braid/model/gdn.py:299-300 (beta's sigmoid rounded
 *                         through the activation dtype; alpha in fp32 with
 *                         softplus' threshold-20 branch), pad rule
 *                         gdn_decode.cu:120-124
 *   oracle_conv1d_decode  tests/test_conv1d_decode.py:10-21 and the window
 *                         layout of braid/kernels/csrc/conv1d_decode.cu:21-27
 *   oracle_quantize_act   braid/model/quant.py:115 and :228-229 as spelled out
 *                         in braid/kernels/csrc/quant_act.cu:43-56, 117-130
 *   oracle_e4m3fn         float -> float8_e4m3fn, round to nearest even, by
 *                         exhaustive nearest-code search (not bit tricks)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- bf16 helpers (round to nearest even; NaN -> 0x7FC0) ---------------- */

static uint16_t bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static float bf16_value(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float oracle_bf16_round(float f) { return bf16_value(bf16_bits(f)); }

/* ---- the recurrence --------------------------------------------------- */

/*
 * One decode token for B rows whose fp32 states have been gathered into
 * S[B, H, SS, HD] (updated in place). q, k: [B, G, SS] with batch stride
 * q_row / k_row; v: [B, H, HD] with batch stride v_row; alpha, beta: [B, H];
 * y: [B, H, HD] dense. qk_scratch holds 2 * SS floats.
 */
void oracle_gdn_decode(float* S, int B, int H, int G, int SS, int HD, const float* q,
                       int64_t q_row, const float* k, int64_t k_row, const float* v,
                       int64_t v_row, const float* alpha, const float* beta, float* y,
                       float* scratch /* 2*SS + 2*HD floats */) {
  const int hpg = H / G;
  const float yscale = (float)(1.0 / sqrt((double)HD)); /* fl32(HD^-0.5) */
  float* qh = scratch;
  float* kh = scratch + SS;
  float* kv = scratch + 2 * SS;
  float* acc = kv + HD;
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < H; ++h) {
      const int g = h / hpg;
      const float* qi = q + (int64_t)b * q_row + (int64_t)g * SS;
      const float* ki = k + (int64_t)b * k_row + (int64_t)g * SS;
      float qs = 0.f, ks = 0.f;
      for (int s = 0; s < SS; ++s) {
        qs += qi[s] * qi[s];
        ks += ki[s] * ki[s];
      }
      const float qinv = 1.0f / sqrtf(qs + 1e-6f);
      const float kinv = 1.0f / sqrtf(ks + 1e-6f);
      for (int s = 0; s < SS; ++s) {
        qh[s] = qi[s] * qinv;
        kh[s] = ki[s] * kinv;
      }
      const float a = alpha[b * H + h], bt = beta[b * H + h];
      float* St = S + ((int64_t)b * H + h) * SS * HD;
      const float* vi = v + (int64_t)b * v_row + (int64_t)h * HD;
      /* kv[d] = sum_s S[s,d] k_hat[s], summed over s in order (per column d) */
      for (int d = 0; d < HD; ++d) kv[d] = 0.f;
      for (int s = 0; s < SS; ++s) {
        const float* row = St + (int64_t)s * HD;
        for (int d = 0; d < HD; ++d) kv[d] += row[d] * kh[s];
      }
      /* delta[d] = (v - alpha * kv) * beta, kept in kv */
      for (int d = 0; d < HD; ++d) {
        kv[d] = (vi[d] - a * kv[d]) * bt;
        acc[d] = 0.f;
      }
      /* S' = alpha S + k_hat delta; y accumulates the fp32 S' in the same pass */
      for (int s = 0; s < SS; ++s) {
        float* row = St + (int64_t)s * HD;
        for (int d = 0; d < HD; ++d) {
          const float nv = a * row[d] + kh[s] * kv[d];
          row[d] = nv;
          acc[d] += nv * qh[s];
        }
      }
      float* yo = y + ((int64_t)b * H + h) * HD;
      for (int d = 0; d < HD; ++d) yo[d] = acc[d] * yscale;
    }
  }
}

/* ---- gates ------------------------------------------------------------ */

/*
 * a_raw, b_raw: [B, T, H] widened to fp32 by the caller (bf16 -> fp32 is
 * exact). act_bf16 != 0 rounds beta's sigmoid through bf16. seq_lens: [B] or
 * NULL; a column t >= seq_lens[b] yields alpha = 1, beta = 0.
 */
void oracle_gdn_gates(const float* a_raw, const float* b_raw, int B, int T, int H,
                      const float* A, const float* dt_bias, int act_bf16,
                      const int32_t* seq_lens, float* alpha, float* beta) {
  for (int b = 0; b < B; ++b) {
    for (int t = 0; t < T; ++t) {
      for (int h = 0; h < H; ++h) {
        const int64_t i = ((int64_t)b * T + t) * H + h;
        if (seq_lens && t >= seq_lens[b]) {
          alpha[i] = 1.f;
          beta[i] = 0.f;
          continue;
        }
        float sig = 1.0f / (1.0f + expf(-b_raw[i]));
        if (act_bf16) sig = oracle_bf16_round(sig);
        beta[i] = sig;
        const float x = a_raw[i] + dt_bias[h];
        const float sp = x > 20.0f ? x : log1pf(expf(x));
        alpha[i] = expf(A[h] * sp);
      }
    }
  }
}

/* ---- conv1d decode ---------------------------------------------------- */

/*
 * state: gathered windows [B, C, K] (updated in place), x: [B, C] fp32,
 * weight [C, K], bias [C] or NULL, out [B, C].
 */
void oracle_conv1d_decode(float* state, int B, int C, int K, const float* x,
                          const float* weight, const float* bias, float* out) {
  for (int b = 0; b < B; ++b) {
    for (int c = 0; c < C; ++c) {
      float* st = state + ((int64_t)b * C + c) * K;
      for (int i = 0; i < K - 1; ++i) st[i] = st[i + 1];
      st[K - 1] = x[(int64_t)b * C + c];
      float acc = 0.f;
      for (int i = 0; i < K; ++i) acc += st[i] * weight[(int64_t)c * K + i];
      if (bias) acc += bias[c];
      out[(int64_t)b * C + c] = acc * (1.0f / (1.0f + expf(-acc)));
    }
  }
}

/* ---- FP8 e4m3fn ------------------------------------------------------- */

/* Value of a non-negative e4m3fn code 0..0x7e; 0x7f is given the value 480,
 * the next step of the binade, so that nearest-even search sends exactly the
 * inputs the format cannot hold (|f| > 464) to the NaN code. */
static double e4m3_value(int code) {
  if (code == 0x7f) return 480.0;
  const int e = (code >> 3) & 0xf, m = code & 7;
  if (e == 0) return ldexp((double)m, -9);
  return ldexp(1.0 + m / 8.0, e - 7);
}

uint8_t oracle_e4m3fn(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  if (isnan(f)) return (uint8_t)(0x7f | sign);
  const double a = fabs((double)f);
  if (a >= 480.0) return (uint8_t)(0x7f | sign);
  int best = 0;
  double best_err = a;
  for (int c = 1; c <= 0x7f; ++c) {
    const double err = fabs(a - e4m3_value(c));
    if (err < best_err || (err == best_err && (c & 1) == 0 && (best & 1) == 1)) {
      best = c;
      best_err = err;
    }
  }
  return (uint8_t)(best | sign);
}

/* NaN-propagating max, as torch.amax. */
static float nan_max(float m, float v) { return (isnan(v) || v > m) ? v : m; }

/*
 * x: n fp32 values (the activation widened), q: n codes, *scale out.
 *   scale = max(amax(|x|) * fl(1/448), 1e-12)   (NaN passes through)
 *   q     = e4m3fn(clamp(x / scale, -448, 448))
 */
void oracle_quantize_act(const float* x, int64_t n, uint8_t* q, float* scale) {
  float m = 0.f;
  for (int64_t i = 0; i < n; ++i) m = nan_max(m, fabsf(x[i]));
  const float inv448 = 1.0f / 448.0f;
  const float raw = m * inv448;
  const float sc = (raw < 1e-12f) ? 1e-12f : raw;
  *scale = sc;
  for (int64_t i = 0; i < n; ++i) {
    float v = x[i] / sc;
    v = (v < -448.0f) ? -448.0f : ((v > 448.0f) ? 448.0f : v);
    q[i] = oracle_e4m3fn(v);
  }
}
