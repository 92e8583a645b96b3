/* CPU restatement of the reference's oracle GEMV for the CPU baseline and the oracle cross-check (TEST
 * INFRASTRUCTURE ONLY: never linked into the product).
 *
 * The reference's CPU path dequantizes a whole matrix in float32 (monolith/formats/nvfp4.py:139-144,
 * int4_affine.py:85-91) and multiplies in float32 (monolith/nn/oracle.py:20-22). This file computes the same numbers
 * row by row, streaming the packed weights once: w = (e2m1 · e4m3) · s2 (one rounding) or code · scale + bias, and
 * y = Σ x·w accumulated in float64 (reported as float32), rows split over OpenMP threads. */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float e4m3_value(uint8_t c) {
  const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7) return NAN;
  const float v = e == 0 ? (float)m * 0.001953125f /* 2^-9 */ : ldexpf(1.0f + m / 8.0f, e - 7);
  return s ? -v : v;
}

static const float kE2M1[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};

/* codes [n][k/2] (low nibble first), scales [n][k/16] E4M3, tensor scale s2; x [m][k]; y [m][n] */
void oracle_nvfp4_gemv(const uint8_t* codes, const uint8_t* scales, float s2, const float* x, int m, int n, int k,
                       float* y, int threads) {
  float lut[256];
  for (int c = 0; c < 256; ++c) lut[c] = e4m3_value((uint8_t)c);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int row = 0; row < n; ++row) {
    const uint8_t* cr = codes + (size_t)row * (k / 2);
    const uint8_t* sr = scales + (size_t)row * (k / 16);
    double acc[16];
    for (int t = 0; t < m; ++t) acc[t] = 0.0;
    for (int b = 0; b < k / 16; ++b) {
      const float bs = lut[sr[b]];
      float w[16];
      for (int i = 0; i < 8; ++i) {
        const uint8_t byte = cr[b * 8 + i];
        w[2 * i] = (kE2M1[byte & 15] * bs) * s2;
        w[2 * i + 1] = (kE2M1[byte >> 4] * bs) * s2;
      }
      for (int t = 0; t < m; ++t) {
        const float* xr = x + (size_t)t * k + b * 16;
        double s = 0.0;
        for (int i = 0; i < 16; ++i) s += (double)w[i] * xr[i];
        acc[t] += s;
      }
    }
    for (int t = 0; t < m; ++t) y[(size_t)t * n + row] = (float)acc[t];
  }
}

/* codes [n][k/2], scales / biases [n][k/64] float (BF16-valued) */
void oracle_int4_gemv(const uint8_t* codes, const float* scales, const float* biases, const float* x, int m, int n,
                      int k, float* y, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int row = 0; row < n; ++row) {
    const uint8_t* cr = codes + (size_t)row * (k / 2);
    double acc[16];
    for (int t = 0; t < m; ++t) acc[t] = 0.0;
    for (int g = 0; g < k / 64; ++g) {
      const float sc = scales[(size_t)row * (k / 64) + g], bi = biases[(size_t)row * (k / 64) + g];
      float w[64];
      for (int i = 0; i < 32; ++i) {
        const uint8_t byte = cr[g * 32 + i];
        w[2 * i] = (float)(byte & 15) * sc + bi;
        w[2 * i + 1] = (float)(byte >> 4) * sc + bi;
      }
      for (int t = 0; t < m; ++t) {
        const float* xr = x + (size_t)t * k + g * 64;
        double s = 0.0;
        for (int i = 0; i < 64; ++i) s += (double)w[i] * xr[i];
        acc[t] += s;
      }
    }
    for (int t = 0; t < m; ++t) y[(size_t)t * n + row] = (float)acc[t];
  }
}
