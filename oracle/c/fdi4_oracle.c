/*
 * C restatement of the reference's CPU algorithm -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (and bench.py's cpu_baseline leg) as a checker; never linked
 * into the product library. Build: oracle/Makefile -> oracle/liboracle_c.so.
 *
 *   oracle_quantize_group   reference src/quantize_int4_ref.py:46-84 for one
 *                           group [rows, C] (row stride in elements): plain
 *                           sequential float32 arithmetic, rintf (the default
 *                           round-to-nearest-even mode) -- an implementation
 *                           independent of NumPy's vectorized one.
 *   oracle_pack             reference src/int4_pack.py:14-29
 *   oracle_fake_quantize    reference scripts/validate_llama.py:126-154 (and,
 *                           with rounding 1, src/quantize_int4_ref.py:139-158
 *                           per block) for one key stream [rows, C].
 *   oracle_f32_to_bf16      round-to-nearest-even float32 -> bfloat16 bits.
 *   oracle_paged_attention_f64
 *                           the float64 arbiter (reference
 *                           tests/test_pallas_flash_decode.py:53-78) over the
 *                           paged layout: exact dequantization in double, one
 *                           full softmax per (sequence, q-head).
 *
 * Compiled with -O2 -ffp-contract=off and no fast-math so every float
 * operation is one IEEE single-precision operation.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oracle_quantize_group(const float* x, int rows, int C, int64_t stride, uint8_t* q,
                           int64_t q_stride, float* scale, float* zp) {
  for (int c = 0; c < C; ++c) {
    float mn = x[c], mx = x[c];
    for (int r = 1; r < rows; ++r) {
      const float v = x[(int64_t)r * stride + c];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    float span = mx - mn;
    const float floor_ = 1e-8f;
    if (span < floor_) span = floor_;
    const float s = span / 15.0f;
    const float z = (-mn) / s;
    scale[c] = s;
    zp[c] = z;
    for (int r = 0; r < rows; ++r) {
      float b = rintf((x[(int64_t)r * stride + c] - mn) / s);
      if (b < 0.0f) b = 0.0f;
      if (b > 15.0f) b = 15.0f;
      q[(int64_t)r * q_stride + c] = (uint8_t)b;
    }
  }
}

void oracle_pack(const uint8_t* q, int64_t rows, int C, uint8_t* out) {
  const int pc = (C + 1) / 2;
  for (int64_t r = 0; r < rows; ++r)
    for (int j = 0; j < pc; ++j) {
      const unsigned lo = q[r * C + 2 * j];
      const unsigned hi = (2 * j + 1 < C) ? q[r * C + 2 * j + 1] : 0u;
      out[r * pc + j] = (uint8_t)(lo | (hi << 4));
    }
}

/* Quantize-dequantize of x [rows, C] (contiguous) in blocks of `block` rows:
 * rounding 0 = floor(t + 0.5f) with dq = q*s + mn, rounding 1 = rintf(t) with
 * dq = q*s - zp*s, t = (x - mn) / s, s = max(mx - mn, 1e-8f) / 15 (recip = 0)
 * or max(mx - mn, 1e-8f) * float(1/15) (recip = 1). */
void oracle_fake_quantize(const float* x, int rows, int C, int block, int rounding, int recip,
                          float* out) {
  const volatile float fifteen = 15.0f;
  const float r15 = 1.0f / fifteen; /* float32(1/15), rounded at run time */
  for (int r0 = 0; r0 < rows; r0 += block) {
    const int n = rows - r0 < block ? rows - r0 : block;
    for (int c = 0; c < C; ++c) {
      float mn = x[(int64_t)r0 * C + c], mx = mn;
      for (int r = 1; r < n; ++r) {
        const float v = x[(int64_t)(r0 + r) * C + c];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
      }
      float span = mx - mn;
      if (span < 1e-8f) span = 1e-8f;
      const float s = recip ? span * r15 : span / 15.0f;
      const float z = (-mn) / s;
      for (int r = 0; r < n; ++r) {
        const int64_t i = (int64_t)(r0 + r) * C + c;
        const float t = (x[i] - mn) / s;
        float q = rounding == 0 ? floorf(t + 0.5f) : rintf(t);
        if (q < 0.0f) q = 0.0f;
        if (q > 15.0f) q = 15.0f;
        if (rounding == 0) {
          const float qs = q * s;
          out[i] = qs + mn;
        } else {
          const float qs = q * s, zs = z * s;
          out[i] = qs - zs;
        }
      }
    }
  }
}

void oracle_f32_to_bf16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &x[i], 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
      out[i] = 0x7FC0u;
      continue;
    }
    /* Ties go to the even upper half: add 0x7FFF plus the upper half's low bit. */
    out[i] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
}

/* query [B, Hq, D]; k_pages [P, Hkv, R, D/2]; v_pages [P, Hkv, R, D] float;
 * k_scale/k_zp [B, Hkv, G, D]; page_table [B, max_pages]; seq_lens [B];
 * out [B, Hq, D] double. q-head h reads kv-head h / (Hq/Hkv). */
void oracle_paged_attention_f64(const float* query, int B, int Hq, int D,
                                const uint8_t* k_pages, const float* v_pages, int Hkv, int R,
                                const float* k_scale, const float* k_zp, int G,
                                const int32_t* page_table, int max_pages,
                                const int32_t* seq_lens, int ppg, double* out) {
  const int rep = Hq / Hkv;
  int tmax = 0;
  for (int b = 0; b < B; ++b)
    if (seq_lens[b] > tmax) tmax = seq_lens[b];
  double* logit = (double*)malloc(sizeof(double) * (tmax > 0 ? tmax : 1));
  double* acc = (double*)malloc(sizeof(double) * D);
  for (int b = 0; b < B; ++b) {
    const int T = seq_lens[b];
    for (int h = 0; h < Hq; ++h) {
      const int hk = h / rep;
      const float* qv = query + ((int64_t)b * Hq + h) * D;
      double m = -INFINITY;
      for (int t = 0; t < T; ++t) {
        const int lp = t / R, r = t % R;
        const int64_t phys = page_table[(int64_t)b * max_pages + lp];
        const uint8_t* krow = k_pages + ((phys * Hkv + hk) * R + r) * (D / 2);
        const float* sc = k_scale + (((int64_t)b * Hkv + hk) * G + lp / ppg) * D;
        const float* zc = k_zp + (((int64_t)b * Hkv + hk) * G + lp / ppg) * D;
        double s = 0.0;
        for (int d = 0; d < D; ++d) {
          const unsigned nib = (d & 1) ? (krow[d / 2] >> 4) : (krow[d / 2] & 15u);
          const double k = (double)nib * (double)sc[d] - (double)zc[d] * (double)sc[d];
          s += (double)qv[d] * k;
        }
        logit[t] = s;
        if (s > m) m = s;
      }
      double l = 0.0;
      for (int d = 0; d < D; ++d) acc[d] = 0.0;
      for (int t = 0; t < T; ++t) {
        const int lp = t / R, r = t % R;
        const int64_t phys = page_table[(int64_t)b * max_pages + lp];
        const float* vrow = v_pages + ((phys * Hkv + hk) * R + r) * D;
        const double p = exp(logit[t] - m);
        l += p;
        for (int d = 0; d < D; ++d) acc[d] += p * (double)vrow[d];
      }
      double* o = out + ((int64_t)b * Hq + h) * D;
      for (int d = 0; d < D; ++d) o[d] = (T > 0) ? acc[d] / l : 0.0;
    }
  }
  free(logit);
  free(acc);
}
