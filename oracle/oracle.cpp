// CPU ORACLE — TEST INFRASTRUCTURE ONLY.
//
// A plain C++17 restatement of the reference's verify-step semantics (ingot, Swift + Metal), written from the source
// text. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the checker or
// the timed CPU baseline; the product (ingot_amd/libingot_hip.so) never links, loads or calls it.
//
// Every function cites the reference file:line it follows. Each function's pin (golden vector, known-answer test,
// closed form or brute force) lives in tests/test_oracle.py; a function without one says "parity unpinned" here.
//
// Arithmetic: fp32 dequantisation and fp32 accumulation (the reference's CPU mirrors, Tests/IngotTests/
// KernelHarness.swift:95-115,189-195), row loops parallelised with OpenMP; summation orders are fixed, so results are
// deterministic for a given thread count and independent of it.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

extern "C" {

// ---------------------------------------------------------------------------------------------------------------
// Number formats.

// bf16 → fp32 and fp32 → bf16 round-to-nearest-even: Sources/Ingot/Loader/Quant.swift:119-125.
float or_bf16_to_f32(uint16_t v) {
  uint32_t u = uint32_t(v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// e2m1 code → float (sign bit 3; magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6): Sources/Ingot/Loader/Quant.swift:188-194.
float or_fp4_e2m1(uint32_t q) {
  const int e = int((q >> 1) & 3);
  const float m = float(q & 1);
  const float mag = e == 0 ? 0.5f * m : std::ldexp(1.0f + 0.5f * m, e - 1);
  return (q & 8) ? -mag : mag;
}

// e8m0 scale → 2^(s − 127), 255 → NaN: Sources/Ingot/Loader/Quant.swift:196-202.
float or_e8m0(uint8_t s) {
  if (s == 255) return std::numeric_limits<float>::quiet_NaN();
  return std::ldexp(1.0f, int(s) - 127);
}

// Dequantise rows of an MLX affine int4 g64 matrix to fp32: w = scale·q + bias, value j of a row in bits 4j…4j+3 of
// word j/8 (low nibble first). Sources/Ingot/Loader/Quant.swift:4-12 (format), 127-147 (unpackQ), 161-187
// (dequantizeRows).
void or_dequant_int4(const uint32_t* w, const uint16_t* s, const uint16_t* b, int N, int K, float* out) {
  const int wpr = K / 8, gpr = K / 64;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) {
      const uint32_t q = (w[size_t(n) * wpr + k / 8] >> (4 * (k % 8))) & 15u;
      const float sc = or_bf16_to_f32(s[size_t(n) * gpr + k / 64]), bi = or_bf16_to_f32(b[size_t(n) * gpr + k / 64]);
      out[size_t(n) * K + k] = sc * float(q) + bi;
    }
  }
}

// Dequantise an MLX mxfp4 matrix (e2m1 codes packed like int4, one e8m0 scale per 32): w = 2^(s−127)·fp4(q).
// Sources/Ingot/Loader/Quant.swift:9-12,176-178; Tests/IngotTests/KernelCaseMXFP4.swift:35-44 (SynMXFP4.dense).
void or_dequant_mxfp4(const uint32_t* w, const uint8_t* s, int N, int K, float* out) {
  const int wpr = K / 8, gpr = K / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) {
      const uint32_t q = (w[size_t(n) * wpr + k / 8] >> (4 * (k % 8))) & 15u;
      out[size_t(n) * K + k] = or_e8m0(s[size_t(n) * gpr + k / 32]) * or_fp4_e2m1(q);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Quantised matmul (fp32 dequant + fp32 matmul): Y[M, N] = X[M, K] · Wᵀ, X given as fp32 values. The reference's CPU
// mirror is Syn.q4 + CPU.matmulT (Tests/IngotTests/KernelHarness.swift:95-115,189-195); the kernel it checks is
// qmv_acc (Sources/Ingot/Shaders/verify.metal:89-105). Dot products in fp32 with 16 interleaved partial sums combined
// in a fixed order.
static inline float dot_f32(const float* a, const float* b, int K) {
  float acc[16] = {0};
  int k = 0;
  for (; k + 16 <= K; k += 16)
    for (int j = 0; j < 16; ++j) acc[j] += a[k + j] * b[k + j];
  float tail = 0.f;
  for (; k < K; ++k) tail += a[k] * b[k];
  for (int w = 8; w >= 1; w /= 2)
    for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
  return acc[0] + tail;
}

void or_qmm_int4(const float* x, int M, const uint32_t* w, const uint16_t* s, const uint16_t* b, int N, int K,
                 float* y) {
  const int wpr = K / 8, gpr = K / 64;
#pragma omp parallel
  {
    std::vector<float> row(K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int g = 0; g < gpr; ++g) {
        const float sc = or_bf16_to_f32(s[size_t(n) * gpr + g]), bi = or_bf16_to_f32(b[size_t(n) * gpr + g]);
        for (int j = 0; j < 64; ++j) {
          const int k = 64 * g + j;
          const uint32_t q = (w[size_t(n) * wpr + k / 8] >> (4 * (k % 8))) & 15u;
          row[k] = sc * float(q) + bi;
        }
      }
      for (int m = 0; m < M; ++m) y[size_t(m) * N + n] = dot_f32(x + size_t(m) * K, row.data(), K);
    }
  }
}

void or_qmm_mxfp4(const float* x, int M, const uint32_t* w, const uint8_t* s, int N, int K, float* y) {
  const int wpr = K / 8, gpr = K / 32;
#pragma omp parallel
  {
    std::vector<float> row(K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int k = 0; k < K; ++k) {
        const uint32_t q = (w[size_t(n) * wpr + k / 8] >> (4 * (k % 8))) & 15u;
        row[k] = or_e8m0(s[size_t(n) * gpr + k / 32]) * or_fp4_e2m1(q);
      }
      for (int m = 0; m < M; ++m) y[size_t(m) * N + n] = dot_f32(x + size_t(m) * K, row.data(), K);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// argmax per row, ties to the lowest index; NaN never wins (the comparison `x > m` is false for NaN):
// argmax_rows, Sources/Ingot/Shaders/verify.metal:525-547.
void or_argmax_rows(const float* x, int rows, int N, uint32_t* out) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + size_t(r) * N;
    float m = -std::numeric_limits<float>::infinity();
    uint32_t mi = 0;
    for (int i = 0; i < N; ++i)
      if (xr[i] > m) {
        m = xr[i];
        mi = uint32_t(i);
      }
    out[r] = mi;
  }
}

// Greedy acceptance of one verify round: m = number of drafts vtok[1..m] that equal the argmax of the previous row
// (top1[0..m-1]), m ≤ B − 1; emitted = vtok[1..m] followed by top1[m] (the new anchor). Returns m.
// spec_accept, Sources/Ingot/Shaders/yy_model.metal:616-642; host form Sources/Ingot/Generate.swift:155-158.
int or_accept(const uint32_t* vtok, const uint32_t* top1, int B, uint32_t* emitted) {
  int m = 0;
  while (m + 1 < B && vtok[m + 1] == top1[m]) ++m;
  for (int i = 1; i <= m; ++i) emitted[i - 1] = vtok[i];
  emitted[m] = top1[m];
  return m;
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

}  // extern "C"
