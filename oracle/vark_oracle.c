/* C restatement of the variable-K grouped wgrad oracle (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker. It restates the same algorithm as oracle/vark_oracle.py with
 * independent code: fp8 bytes decoded by bit arithmetic (not a table), per-group accumulation in
 * fp32 in token order, then round-to-nearest-even to bf16. Semantics: reference bench.py:182-193
 * ("dW = x^T @ dy"), launch contract reference launcher.cpp:16-33 / README.md:88-97.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float vo_e4m3_to_f32(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 0xF, m = b & 7;
  float v;
  if (e == 0xF && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);            /* m/8 * 2^-6 */
  else v = ldexpf((float)(8 + m), e - 10);         /* (1+m/8) * 2^(e-7) */
  return s ? -v : v;
}

float vo_e5m2_to_f32(uint8_t b) {
  const int s = b >> 7, e = (b >> 2) & 0x1F, m = b & 3;
  float v;
  if (e == 0x1F) v = m ? NAN : INFINITY;
  else if (e == 0) v = ldexpf((float)m, -16);      /* m/4 * 2^-14 */
  else v = ldexpf((float)(4 + m), e - 17);         /* (1+m/4) * 2^(e-15) */
  return s ? -v : v;
}

uint16_t vo_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* Tensorwise grouped wgrad; out_bits: bf16 [G, OUT_M, OUT_N]. Returns 0, or -1 on bad offsets,
 * -2 on allocation failure. */
int vo_vark_tensorwise(const uint8_t* lhs, const uint8_t* rhs, float sl, float sr, const int64_t* offs, int G,
                       int64_t M, int OUT_M, int OUT_N, int64_t slm, int64_t srm, uint16_t* out_bits) {
  if (offs[0] != 0) return -1;
  for (int g = 0; g < G; ++g)
    if (offs[g + 1] < offs[g] || offs[g + 1] > M) return -1;
  float* acc = (float*)malloc(sizeof(float) * (size_t)OUT_M * OUT_N);
  float* a = (float*)malloc(sizeof(float) * (size_t)OUT_M);
  float* b = (float*)malloc(sizeof(float) * (size_t)OUT_N);
  if (!acc || !a || !b) { free(acc); free(a); free(b); return -2; }
  for (int g = 0; g < G; ++g) {
    memset(acc, 0, sizeof(float) * (size_t)OUT_M * OUT_N);
    for (int64_t k = offs[g]; k < offs[g + 1]; ++k) {
      for (int m = 0; m < OUT_M; ++m) a[m] = vo_e4m3_to_f32(lhs[k * slm + m]) * sl;
      for (int n = 0; n < OUT_N; ++n) b[n] = vo_e5m2_to_f32(rhs[k * srm + n]) * sr;
      for (int m = 0; m < OUT_M; ++m) {
        const float am = a[m];
        float* row = acc + (size_t)m * OUT_N;
        for (int n = 0; n < OUT_N; ++n) row[n] += am * b[n];
      }
    }
    uint16_t* o = out_bits + (size_t)g * OUT_M * OUT_N;
    for (size_t i = 0; i < (size_t)OUT_M * OUT_N; ++i) o[i] = vo_f32_to_bf16(acc[i]);
  }
  free(acc); free(a); free(b);
  return 0;
}

/* Persistent fwd / dgrad grouped GEMM (reference bench.py:153-181,238-247): out_bits[r, n] =
 * bf16(sum_k (sa * A[r, k]) (sb * B[g, n, k])) for the rows r of group g, accumulated in fp32 in
 * k order; A is e4m3 (a_e5m2 = 0) or e5m2 (a_e5m2 = 1), B e4m3 [G, N, K] (trans_b); rows outside
 * every group are left as they are. Returns 0, or -1 on bad offsets, -2 on allocation failure. */
int vo_persistent_fp8(const uint8_t* a, const uint8_t* b, float sa, float sb, const int64_t* offs, int G,
                      int64_t M, int N, int K, int64_t sam, int64_t sbg, int64_t sbn, int a_e5m2,
                      uint16_t* out_bits, int64_t som) {
  if (offs[0] < 0) return -1;
  for (int g = 0; g < G; ++g)
    if (offs[g + 1] < offs[g] || offs[g + 1] > M) return -1;
  float* x = (float*)malloc(sizeof(float) * (size_t)K);
  float* w = (float*)malloc(sizeof(float) * (size_t)N * K);
  if (!x || !w) { free(x); free(w); return -2; }
  for (int g = 0; g < G; ++g) {
    for (int n = 0; n < N; ++n)
      for (int k = 0; k < K; ++k) w[(size_t)n * K + k] = vo_e4m3_to_f32(b[g * sbg + n * sbn + k]) * sb;
    for (int64_t r = offs[g]; r < offs[g + 1]; ++r) {
      for (int k = 0; k < K; ++k)
        x[k] = (a_e5m2 ? vo_e5m2_to_f32(a[r * sam + k]) : vo_e4m3_to_f32(a[r * sam + k])) * sa;
      for (int n = 0; n < N; ++n) {
        float acc = 0.0f;
        const float* wn = w + (size_t)n * K;
        for (int k = 0; k < K; ++k) acc += x[k] * wn[k];
        out_bits[r * som + n] = vo_f32_to_bf16(acc);
      }
    }
  }
  free(x); free(w);
  return 0;
}
