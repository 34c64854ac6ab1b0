/*
 * C restatement of the MXFP4 dequant + float64 GEMM oracle.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through oracle/c_oracle.py) as
 * an independent second restatement of the reference semantics.  The product
 * library never links or calls it.
 *
 * Semantics follow konradha/cdna3-bench python/mxfp4_cdna3/ref.py:50-78, but
 * each value is decoded from the E2M1 bit fields rather than from the
 * magnitude table at ref.py:3, so the two restatements cannot share a
 * transcription error:
 *   value = (-1)^s * mag(e, m) * 2^(scale - 127)
 *   mag   = m * 0.5                      (e == 0, subnormal)
 *         = (1 + m/2) * 2^(e - 1)        (e > 0)
 * Code 8 yields -0.0 (ref.py:67).  Scale byte 0 yields 2^-127 and 255 yields
 * 2^128 -> inf once rounded to float, as ref.py:69 does through float32.
 * Layouts: 0 = [K/2, N] codes with [K/32, N] scales (csrc/mxfp4_ext.cpp:20-24),
 *          1 = [N, K/2] codes with [N, K/32] scales.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static double e2m1_bits(unsigned code) {
  unsigned s = (code >> 3) & 1u, e = (code >> 1) & 3u, m = code & 1u;
  double mag = (e == 0) ? 0.5 * (double)m : (1.0 + 0.5 * (double)m) * ldexp(1.0, (int)e - 1);
  return s ? -mag : mag;
}

/* Float32 value of one weight element, as ref.py computes it in float32. */
static float weight_f32(const uint8_t* B, const uint8_t* S, int64_t K, int64_t N, int layout,
                        int64_t k, int64_t n) {
  uint8_t byte, sbyte;
  if (layout == 0) {
    byte = B[(k / 2) * N + n];
    sbyte = S[(k / 32) * N + n];
  } else {
    byte = B[n * (K / 2) + k / 2];
    sbyte = S[n * (K / 32) + k / 32];
  }
  unsigned code = (k & 1) ? (byte >> 4) : (byte & 0x0Fu);
  float scale = (float)ldexp(1.0, (int)sbyte - 127); /* float64 power cast to f32 */
  float v = (float)e2m1_bits(code);
  return v * scale;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7FC0u);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* out[k*N + n] = bf16 bits of the dequantized weight (the [K, N] tile). */
void mxo_dequant_bf16(const uint8_t* B, const uint8_t* S, int64_t K, int64_t N, int layout,
                      uint16_t* out) {
  for (int64_t k = 0; k < K; ++k)
    for (int64_t n = 0; n < N; ++n) out[k * N + n] = f32_to_bf16_rne(weight_f32(B, S, K, N, layout, k, n));
}

/* C[m*N+n] = sum_k A[m,k] W[k,n] in float64; Cabs = sum_k |A||W|.  A is bf16 bits [M,K]. */
int mxo_gemm_f64(const uint16_t* A, const uint8_t* B, const uint8_t* S, int64_t M, int64_t N,
                 int64_t K, int layout, double* C, double* Cabs) {
  double* W = (double*)malloc(sizeof(double) * (size_t)K * (size_t)N);
  if (!W) return -1;
  for (int64_t k = 0; k < K; ++k)
    for (int64_t n = 0; n < N; ++n) W[k * N + n] = (double)weight_f32(B, S, K, N, layout, k, n);
  for (int64_t m = 0; m < M; ++m) {
    double* c = C + m * N;
    double* ca = Cabs ? Cabs + m * N : NULL;
    for (int64_t n = 0; n < N; ++n) {
      c[n] = 0.0;
      if (ca) ca[n] = 0.0;
    }
    for (int64_t k = 0; k < K; ++k) {
      double a = (double)bf16_to_f32(A[m * K + k]);
      const double* w = W + k * N;
      for (int64_t n = 0; n < N; ++n) c[n] += a * w[n];
      if (ca)
        for (int64_t n = 0; n < N; ++n) ca[n] += fabs(a) * fabs(w[n]);
    }
  }
  free(W);
  return 0;
}
