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


// ---------------------------------------------------------------------------------------------------------------
// Synthetic data (the benchmark's generator, restated): counter-based SplitMix64 streams. h(key, i) is output i of
// SplitMix64 seeded with key (the reference's SplitMix64, Sources/Ingot/Sampling.swift:50-62); key = mix(seed·φ +
// mix(tensor + c)). sm_normal sums the four 16-bit fields of one output, centred, times √3/65536 (≈ N(0,1)).
static inline uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static inline uint64_t sm_key(uint64_t seed, uint64_t tensor) {
  return sm_mix(seed * 0x9E3779B97F4A7C15ull + sm_mix(tensor + 0x632BE59BD9B4E019ull));
}
static inline uint64_t sm_at(uint64_t key, uint64_t i) { return sm_mix(key + (i + 1) * 0x9E3779B97F4A7C15ull); }
static inline float sm_normal(uint64_t key, uint64_t i) {
  const uint64_t h = sm_at(key, i);
  const int s = int(h & 0xFFFF) + int((h >> 16) & 0xFFFF) + int((h >> 32) & 0xFFFF) + int(h >> 48) - 131070;
  return float(s) * 2.642936E-05f;
}

uint64_t or_sm_at(uint64_t key, uint64_t i) { return sm_at(key, i); }
uint64_t or_sm_key(uint64_t seed, uint64_t tensor) { return sm_key(seed, tensor); }
float or_sm_normal(uint64_t key, uint64_t i) { return sm_normal(key, i); }

// MLX int4 tensor [N, K] of the synthetic model: codes from stream 2·tensor, scales from 2·tensor + 1.
void or_synth_int4(uint64_t seed, uint64_t tensor, int N, int K, float sd, uint32_t* w, uint16_t* s, uint16_t* b) {
  const uint64_t kw = sm_key(seed, 2 * tensor), ks = sm_key(seed, 2 * tensor + 1);
  const size_t nw = size_t(N) * K / 8, ng = size_t(N) * K / 64;
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < nw; ++i) {
    const uint64_t h = sm_at(kw, i >> 1);
    w[i] = uint32_t((i & 1) ? (h >> 32) : h);
  }
#pragma omp parallel for schedule(static)
  for (size_t g = 0; g < ng; ++g) {
    const uint16_t sb = or_f32_to_bf16(std::fabs(sm_normal(ks, g)) * sd);
    s[g] = sb;
    b[g] = or_f32_to_bf16(-8.0f * or_bf16_to_f32(sb));
  }
}

// MLX mxfp4 tensor [N, K] of the synthetic model: codes as or_synth_int4; e8m0 of group g = 119 + h(key_s, g) mod 7.
void or_synth_mxfp4(uint64_t seed, uint64_t tensor, int N, int K, uint32_t* w, uint8_t* s) {
  const uint64_t kw = sm_key(seed, 2 * tensor), ks = sm_key(seed, 2 * tensor + 1);
  const size_t nw = size_t(N) * K / 8, ng = size_t(N) * K / 32;
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < nw; ++i) {
    const uint64_t h = sm_at(kw, i >> 1);
    w[i] = uint32_t((i & 1) ? (h >> 32) : h);
  }
  for (size_t g = 0; g < ng; ++g) s[g] = uint8_t(119 + sm_at(ks, g) % 7);
}

void or_synth_bf16(uint64_t seed, uint64_t tensor, size_t n, float base, float amp, uint16_t* out) {
  const uint64_t k = sm_key(seed, 2 * tensor);
  for (size_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(base + amp * sm_normal(k, i));
}

void or_synth_f32(uint64_t seed, uint64_t tensor, size_t n, float base, float amp, float* out) {
  const uint64_t k = sm_key(seed, 2 * tensor);
  for (size_t i = 0; i < n; ++i) out[i] = base + amp * sm_normal(k, i);
}

// fp32 → fp16 bits, round to nearest even (normal, subnormal, overflow to inf).
uint16_t or_f32_to_f16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int e = int((u >> 23) & 0xFF) - 127;
  uint32_t m = u & 0x7FFFFFu;
  if (((u >> 23) & 0xFF) == 0xFF) return uint16_t(sign | 0x7C00u | (m ? 0x200u : 0u));
  if (e > 15) return uint16_t(sign | 0x7C00u);
  if (e >= -14) {
    uint32_t r = (uint32_t(e + 15) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return uint16_t(sign | r);
  }
  if (e < -25) return uint16_t(sign);
  m |= 0x800000u;
  const int shift = -e - 1;  // e ≤ −15: value = m · 2^(e−23) → units of 2^−24
  uint32_t r = m >> (shift);
  const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (r & 1u))) ++r;
  return uint16_t(sign | r);
}
float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  float f;
  if (e == 0) f = std::ldexp(float(m), -24);
  else if (e == 31) f = m ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
  else f = std::ldexp(float(m | 0x400u), int(e) - 25);
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u |= sign;
  std::memcpy(&f, &u, 4);
  return f;
}

// Symmetric int8 of one head vector with an fp16 scale: sc = fp16(amax/127) (1 when amax = 0), q = clamp(rint(x/sc),
// ±127). CPU.quantI8 (Tests/IngotTests/KernelHarness.swift:249-254) and vattn_prework_i8 (verify_attn_nax.metal:112-139),
// with the scale stored in fp16 (benchmark configuration 1) instead of fp32.
static void quant_i8(const float* x, int n, int8_t* q, uint16_t* sc16) {
  float amax = 0.f;
  for (int i = 0; i < n; ++i) amax = std::max(amax, std::fabs(x[i]));
  const uint16_t h = or_f32_to_f16(amax > 0.f ? amax / 127.0f : 1.0f);
  const float sc = or_f16_to_f32(h);
  for (int i = 0; i < n; ++i) q[i] = int8_t(std::min(127.f, std::max(-127.f, std::nearbyint(x[i] / sc))));
  *sc16 = h;
}

// Synthetic KV of one layer for positions pos0 … pos0+npos−1: k/v int8 [KVH][npos][HD], scales fp16 bits [KVH][npos].
void or_synth_kv(uint64_t seed, uint64_t tensor, int KVH, int HD, int pos0, int npos, int8_t* k, int8_t* v,
                 uint16_t* ks, uint16_t* vs) {
  const uint64_t kk = sm_key(seed, 2 * tensor), kv = sm_key(seed, 2 * tensor + 1);
#pragma omp parallel for collapse(2) schedule(static)
  for (int h = 0; h < KVH; ++h)
    for (int p = 0; p < npos; ++p) {
      float x[256];
      const int pos = pos0 + p;
      const size_t o = (size_t(h) * npos + p);
      for (int which = 0; which < 2; ++which) {
        const uint64_t key = which ? kv : kk;
        for (int d = 0; d < HD; ++d) x[d] = sm_normal(key, ((uint64_t(h) << 24) + uint64_t(pos)) * HD + d);
        quant_i8(x, HD, (which ? v : k) + o * HD, (which ? vs : ks) + o);
      }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Row operations of the round.

// RMSNorm: bf16(x · 1/sqrt(mean x² + eps) · w). rmsnorm_rows, Sources/Ingot/Shaders/verify.metal:501-523.
void or_rmsnorm(const float* x, int rows, int D, const uint16_t* w, float eps, float* out) {
  for (int r = 0; r < rows; ++r) {
    double ss = 0;
    for (int i = 0; i < D; ++i) ss += double(x[size_t(r) * D + i]) * x[size_t(r) * D + i];
    const float rr = 1.0f / std::sqrt(float(ss) / float(D) + eps);
    for (int i = 0; i < D; ++i)
      out[size_t(r) * D + i] = or_bf16_to_f32(or_f32_to_bf16(x[size_t(r) * D + i] * rr * or_bf16_to_f32(w[i])));
  }
}

// RMSNorm split as the verify step computes it: the matmul input is x = bf16(h ⊙ w) and the per-row factor
// r = 1/sqrt(mean h² + eps) multiplies the matmul output (RMSNorm is a per-row scale, so
// (h·r ⊙ w)·Wᵀ = r · ((h ⊙ w)·Wᵀ); only the bf16 rounding point moves). rmsnorm_rows (verify.metal:501-523).
void or_rms_split(const float* h, int rows, int D, const uint16_t* w, float eps, float* x, float* r) {
  for (int i = 0; i < rows; ++i) {
    double ss = 0;
    for (int j = 0; j < D; ++j) ss += double(h[size_t(i) * D + j]) * h[size_t(i) * D + j];
    r[i] = 1.0f / std::sqrt(float(ss) / float(D) + eps);
    for (int j = 0; j < D; ++j)
      x[size_t(i) * D + j] = or_bf16_to_f32(or_f32_to_bf16(h[size_t(i) * D + j] * or_bf16_to_f32(w[j])));
  }
}

// The same with the matmul input rounded to fp16 (the input of MXFP4 experts, whose products run in fp16 as the
// reference's half activations, verify_nax.metal:78-79).
void or_rms_split_f16(const float* h, int rows, int D, const uint16_t* w, float eps, float* x, float* r) {
  for (int i = 0; i < rows; ++i) {
    double ss = 0;
    for (int j = 0; j < D; ++j) ss += double(h[size_t(i) * D + j]) * h[size_t(i) * D + j];
    r[i] = 1.0f / std::sqrt(float(ss) / float(D) + eps);
    for (int j = 0; j < D; ++j)
      x[size_t(i) * D + j] = or_f16_to_f32(or_f32_to_f16(h[size_t(i) * D + j] * or_bf16_to_f32(w[j])));
  }
}

static void scale_rows(float* y, int rows, int N, const float* r) {
  for (int i = 0; i < rows; ++i)
    for (int j = 0; j < N; ++j) y[size_t(i) * N + j] *= r[i];
}

// Gated activation (lab_glu, Sources/Ingot/Shaders/qmm.metal:18-30): act 0 = SiLU(g)·u, act 1 = swiglu_oai
// (CPU.swigluOAI, Tests/IngotTests/KernelHarness.swift:185-188). Output rounded to bf16.
float or_glu(float g, float u, int act, float limit) {
  if (act == 0) return g / (1.0f + std::exp(-g)) * u;
  const float gc = std::min(g, limit), uc = std::min(std::max(u, -limit), limit);
  return gc / (1.0f + std::exp(-1.702f * gc)) * (uc + 1.0f);
}

// Unnormalised Sylvester Walsh–Hadamard in place, stages h = 1, 2, 4, … (CPU.fwht, KernelHarness.swift:197-210).
void or_fwht(float* v, int n) {
  for (int h = 1; h < n; h *= 2)
    for (int i = 0; i < n; i += 2 * h)
      for (int j = i; j < i + h; ++j) {
        const float a = v[j], b = v[j + h];
        v[j] = a + b;
        v[j + h] = a - b;
      }
}

// RoPE of one head (non-interleaved halves over all HD dims; angle pos·θ^(−i/(HD/2)) in double), then the orthonormal
// WHT if hadk. normRope + hadamard, Tests/IngotTests/KernelHarness.swift:379-420; vattn_prework_i8.
// RoPE of the first `rot` dims (pairs d, d + rot/2; AT_ROT of vattn_prework_i8, verify_attn_nax.metal:92-98), the
// angle of pair i at `pos` = pos·θ^(−i/(rot/2)) or, with a frequency table inv (a scaled RoPE, RopeTable), pos·inv[i]
// with cos and sin times mscale (AT_ROPE_ANG / AT_ROPE_SCALE, verify_attn.metal:66-84); then the orthonormal
// Walsh–Hadamard rotation of the head when hadk.
void or_rope_wht_ex(float* x, int HD, int rot, int pos, float theta, const float* inv, float mscale, int hadk) {
  float y[256];
  const int RH = rot / 2;
  for (int d = 0; d < HD; ++d) {
    if (d >= rot) {
      y[d] = x[d];
      continue;
    }
    const int i = d % RH;
    float c, s;
    if (inv) {
      const double ang = double(pos) * double(inv[i]);
      c = float(std::cos(ang) * double(mscale));
      s = float(std::sin(ang) * double(mscale));
    } else {
      const double ang = double(pos) * std::pow(double(theta), -double(i) / double(RH));
      c = float(std::cos(ang));
      s = float(std::sin(ang));
    }
    y[d] = d < RH ? x[d] * c - x[d + RH] * s : x[d] * c + x[d - RH] * s;
  }
  if (hadk) {
    or_fwht(y, HD);
    const float sc = HD == 128 ? 0.088388347648318441f : (HD == 64 ? 0.125f : 0.0625f);
    for (int d = 0; d < HD; ++d) y[d] *= sc;
  }
  std::memcpy(x, y, sizeof(float) * HD);
}

void or_rope_wht(float* x, int HD, int pos, float theta, int hadk) {
  or_rope_wht_ex(x, HD, HD, pos, theta, nullptr, 1.0f, hadk);
}

// The frequency table of a scaled RoPE over `dims` rotated dims (RopeTable.make, Sources/Ingot/Loader/RopeTable.swift:
// 98-137; mlx-lm initialize_rope): kind 1 linear, 2 yarn, 3 proportional. Every frequency is formed in double from
// the period θ^(2i/dims) and rounded to float once; inv [dims/2]; returns mscale.
float or_rope_table(int kind, double theta, int dims, double factor, double orig_max, double beta_fast,
                    double beta_slow, double mscale_in, double attn_factor, int truncate, double partial, float* inv) {
  const int rh = dims / 2;
  double mscale = 1.0;
  for (int i = 0; i < rh; ++i) {
    const double period = std::pow(theta, 2.0 * i / dims);
    double f = 1.0 / period;
    if (kind == 1) f = f / factor;
    if (kind == 3) f = (i < int(dims * partial) / 2) ? 1.0 / (factor * period) : 0.0;
    if (kind == 2) {
      // Correction range (yarn_find_correction_range): the dim at which `r` full rotations fit in orig_max positions.
      const double lo0 = dims * std::log(orig_max / (beta_fast * 2 * M_PI)) / (2 * std::log(theta));
      const double hi0 = dims * std::log(orig_max / (beta_slow * 2 * M_PI)) / (2 * std::log(theta));
      double lo = truncate ? std::floor(lo0) : lo0, hi = truncate ? std::ceil(hi0) : hi0;
      if (lo < 0) lo = 0;
      if (hi > dims - 1) hi = dims - 1;
      if (hi == lo) hi += 0.001;
      double ramp = (i - lo) / (hi - lo);
      ramp = ramp < 0 ? 0 : (ramp > 1 ? 1 : ramp);
      // weight (1 − ramp) on the original frequency, ramp on the interpolated one (frequency / factor)
      f = f * (1 - ramp) + (f / factor) * ramp;
    }
    inv[i] = float(f);
  }
  if (kind == 2) mscale = attn_factor > 0 ? attn_factor : (factor <= 1 ? 1.0 : 0.1 * mscale_in * std::log(factor) + 1.0);
  return float(mscale);
}

// Causal GQA attention of B rows at positions P…P+B−1 over an int8 cache of P+B keys (the block's own keys already
// written): S = (q·k8)·ks/√HD, masked to key ≤ P + t (and key > P + t − window), softmax with an optional sink logit
// in the denominator, O = Σ p·vs·v8. AttnFixture.reference (Tests/IngotTests/KernelHarness.swift:420-501).
// q fp32 [B][QH][HD] (already rounded as the kernel stores it), k/v [KVH][npos][HD], scales fp16 bits; out [B][QH·HD].
// With p16 set, each probability times its V scale is rounded to fp16 before it weights V, as the reference's
// attention does (`half(p0 * vsv[e])`, Sources/Ingot/Shaders/verify_attn_pf.metal:268-276; the GPU path rounds at the
// same point, against its running maximum). Off by default: the oracle's attention is fp32, and the difference of the
// two measures how far that rounding point alone moves the logits (the tests' tolerance for it).
static int g_p16 = 0;
void or_set_attn_p16(int on) { g_p16 = on; }

void or_attention(const float* q, int B, int P, int QH, int KVH, int HD, const int8_t* k, const int8_t* v,
                  const uint16_t* ks, const uint16_t* vs, int npos, int window, const float* sinks, float* out) {
  const int G = QH / KVH;
  const float scale = float(1.0 / std::sqrt(double(HD)));
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < B; ++t)
    for (int h = 0; h < QH; ++h) {
      const int kvh = h / G, n = P + t + 1;
      const int lo = window > 0 ? std::max(0, n - window) : 0;
      std::vector<float> s(n);
      const float* qr = q + (size_t(t) * QH + h) * HD;
      float mx = -std::numeric_limits<float>::infinity();
      for (int j = lo; j < n; ++j) {
        const int8_t* kr = k + (size_t(kvh) * npos + j) * HD;
        float dot = 0.f;
        for (int d = 0; d < HD; ++d) dot += qr[d] * float(kr[d]);
        s[j] = dot * or_f16_to_f32(ks[size_t(kvh) * npos + j]) * scale;
        mx = std::max(mx, s[j]);
      }
      if (sinks) mx = std::max(mx, sinks[h]);
      float l = sinks ? std::exp(sinks[h] - mx) : 0.f;
      std::vector<float> o(HD, 0.f);
      for (int j = lo; j < n; ++j) {
        const float p = std::exp(s[j] - mx);
        l += p;
        float pv = p * or_f16_to_f32(vs[size_t(kvh) * npos + j]);
        if (g_p16) pv = or_f16_to_f32(or_f32_to_f16(pv));
        const int8_t* vr = v + (size_t(kvh) * npos + j) * HD;
        for (int d = 0; d < HD; ++d) o[d] += pv * float(vr[d]);
      }
      for (int d = 0; d < HD; ++d) out[size_t(t) * QH * HD + h * HD + d] = o[d] / l;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// The whole verify step of the synthetic dense model (HybridModel.encodeVerify, Sources/Ingot/ModelRound.swift:48-82),
// with the weights and the KV history regenerated from the seeds. Layout of or_model_desc = ih_model_desc.
struct or_model_desc {
  int n_layers, hidden, n_q_heads, n_kv_heads, head_dim, intermediate, vocab;
  float rope_theta, rms_eps;
  int n_experts, top_k, expert_intermediate, expert_format, router_bias, expert_bias, act;
  float swiglu_limit;
  int sliding_window, sinks, hadamard_k, qk_norm, qkv_bias;
  int iid_routing, rotary_dims, attn_gate, o_bias, rope_type;
  float rope_factor, rope_orig_max, rope_beta_fast, rope_beta_slow, rope_mscale, rope_attn_factor;
  int rope_no_truncate;
  float rope_partial;
  int router_int4;
};

static uint64_t layer_tensor(int l, uint64_t kind) { return 1000 + 100 * uint64_t(l) + kind; }

// A synthetic int4 matrix held in host memory (MLX layout).
struct QMat {
  int N = 0, K = 0;
  std::vector<uint32_t> w;
  std::vector<uint16_t> s, b;
  void make(uint64_t seed, uint64_t tensor, int n, int k, float sd) {
    N = n;
    K = k;
    w.resize(size_t(N) * K / 8);
    s.resize(size_t(N) * K / 64);
    b.resize(size_t(N) * K / 64);
    or_synth_int4(seed, tensor, N, K, sd, w.data(), s.data(), b.data());
  }
  void apply(const float* x, int B, float* y) const { or_qmm_int4(x, B, w.data(), s.data(), b.data(), N, K, y); }
};

// An int4 or mxfp4 matrix (MoE experts and router).
struct AnyMat {
  int fmt = 0, N = 0, K = 0;
  QMat q4;
  std::vector<uint32_t> w;
  std::vector<uint8_t> s;
  void make(int f, uint64_t seed, uint64_t tensor, int n, int k, float sd) {
    fmt = f;
    N = n;
    K = k;
    if (fmt == 0) {
      q4.make(seed, tensor, n, k, sd);
      return;
    }
    w.resize(size_t(N) * K / 8);
    s.resize(size_t(N) * K / 32);
    or_synth_mxfp4(seed, tensor, N, K, w.data(), s.data());
  }
  void apply(const float* x, int B, float* y) const {
    if (fmt == 0) q4.apply(x, B, y);
    else or_qmm_mxfp4(x, B, w.data(), s.data(), N, K, y);
  }
};

static uint64_t expert_tensor(int l, uint64_t kind, int e) { return 3000000 + 10000 * uint64_t(l) + 1000 * kind + e; }

struct OrLayer {
  std::vector<uint16_t> attn_norm, mlp_norm, q_norm, k_norm;
  std::vector<float> sinks, qkv_bias, o_bias;
  QMat qkv, o, gate_up, down;
  // MoE: router [E][H], per expert gate|up [2I][H] (gate rows then up rows) and down [H][I], optional biases.
  AnyMat router;
  std::vector<AnyMat> egu, edn;
  std::vector<float> router_bias;
  std::vector<uint16_t> gu_bias, dn_bias;
  // KV of positions 0 … P−1 (history) followed by room for the block.
  std::vector<int8_t> k, v;
  std::vector<uint16_t> ks, vs;
};

struct OrModel {
  or_model_desc d;
  int P = 0, cap = 0;
  uint64_t seed = 0;
  std::vector<float> rinv;  // scaled RoPE: frequencies of the rotated pairs (empty: the default RoPE)
  float rmscale = 1.0f;
  // Captured residual rows after the listed layers, bf16 [B][n · H] (capture_rows, yy_model.metal:94-104).
  std::vector<int> cap_layers;
  std::vector<uint16_t> caps;
  std::vector<OrLayer> layers;
  QMat embed, head;
  std::vector<uint16_t> final_norm;
};

// Builds the synthetic model in host memory (weights of every layer, KV history of P positions from kv_seed).
void* or_model_create(const or_model_desc* d, uint64_t seed, uint64_t kv_seed, int P, int max_rows) {
  OrModel* m = new OrModel();
  m->d = *d;
  m->P = P;
  m->seed = seed;
  m->cap = P + max_rows;
  const int H = d->hidden, QH = d->n_q_heads, KVH = d->n_kv_heads, HD = d->head_dim, I = d->intermediate;
  const int QP = QH * HD * (d->attn_gate ? 2 : 1) + 2 * KVH * HD;
  const float sd = 0.02f;
  if (d->rope_type != 0) {
    const int rot = d->rotary_dims > 0 ? d->rotary_dims : HD;
    m->rinv.resize(rot / 2);
    m->rmscale = or_rope_table(d->rope_type, d->rope_theta, rot, d->rope_factor > 0 ? d->rope_factor : 1.0,
                               d->rope_orig_max, d->rope_beta_fast > 0 ? d->rope_beta_fast : 32.0,
                               d->rope_beta_slow > 0 ? d->rope_beta_slow : 1.0,
                               d->rope_mscale > 0 ? d->rope_mscale : 1.0, d->rope_attn_factor, !d->rope_no_truncate,
                               d->rope_partial > 0 ? d->rope_partial : 1.0, m->rinv.data());
  }
  m->embed.make(seed, 1, d->vocab, H, sd);
  m->head.make(seed, 3, d->vocab, H, sd);
  m->final_norm.resize(H);
  or_synth_bf16(seed, 2, H, 1.0f, 0.125f, m->final_norm.data());
  m->layers.resize(d->n_layers);
  for (int l = 0; l < d->n_layers; ++l) {
    OrLayer& L = m->layers[l];
    L.attn_norm.resize(H);
    L.mlp_norm.resize(H);
    or_synth_bf16(seed, layer_tensor(l, 0), H, 1.0f, 0.125f, L.attn_norm.data());
    or_synth_bf16(seed, layer_tensor(l, 3), H, 1.0f, 0.125f, L.mlp_norm.data());
    if (d->sinks) {
      L.sinks.resize(QH);
      or_synth_f32(seed, layer_tensor(l, 9), QH, 0.0f, 1.0f, L.sinks.data());
    }
    if (d->qk_norm) {
      L.q_norm.resize(HD);
      L.k_norm.resize(HD);
      or_synth_bf16(seed, layer_tensor(l, 10), HD, 1.0f, 0.125f, L.q_norm.data());
      or_synth_bf16(seed, layer_tensor(l, 11), HD, 1.0f, 0.125f, L.k_norm.data());
    }
    if (d->qkv_bias) {
      L.qkv_bias.resize(QP);
      or_synth_f32(seed, layer_tensor(l, 12), QP, 0.0f, 0.1f, L.qkv_bias.data());
    }
    L.qkv.make(seed, layer_tensor(l, 1), QP, H, sd);
    L.o.make(seed, layer_tensor(l, 2), H, QH * HD, sd);
    if (d->o_bias) {
      L.o_bias.resize(H);
      or_synth_f32(seed, layer_tensor(l, 14), H, 0.0f, 0.1f, L.o_bias.data());
    }
    if (d->n_experts > 0) {
      const int E = d->n_experts, IE = d->expert_intermediate, f = d->expert_format;
      L.router.make(d->router_int4 ? 0 : f, seed, layer_tensor(l, 6), E, H, sd);
      L.egu.resize(E);
      L.edn.resize(E);
      for (int e = 0; e < E; ++e) {
        L.egu[e].make(f, seed, expert_tensor(l, 0, e), 2 * IE, H, sd);
        L.edn[e].make(f, seed, expert_tensor(l, 1, e), H, IE, sd);
      }
      if (d->router_bias) {
        L.router_bias.resize(E);
        or_synth_f32(seed, layer_tensor(l, 7), E, 0.0f, 0.5f, L.router_bias.data());
      }
      if (d->expert_bias) {
        L.gu_bias.resize(size_t(E) * 2 * IE);
        L.dn_bias.resize(size_t(E) * H);
        for (int e = 0; e < E; ++e) {
          or_synth_bf16(seed, expert_tensor(l, 2, e), 2 * IE, 0.0f, 0.1f, L.gu_bias.data() + size_t(e) * 2 * IE);
          or_synth_bf16(seed, expert_tensor(l, 3, e), H, 0.0f, 0.1f, L.dn_bias.data() + size_t(e) * H);
        }
      }
    } else {
      L.gate_up.make(seed, layer_tensor(l, 4), 2 * I, H, sd);
      L.down.make(seed, layer_tensor(l, 5), H, I, sd);
    }
    L.k.resize(size_t(KVH) * m->cap * HD);
    L.v.resize(size_t(KVH) * m->cap * HD);
    L.ks.resize(size_t(KVH) * m->cap);
    L.vs.resize(size_t(KVH) * m->cap);
    std::vector<int8_t> kh(size_t(KVH) * P * HD), vh(size_t(KVH) * P * HD);
    std::vector<uint16_t> ksh(size_t(KVH) * P), vsh(size_t(KVH) * P);
    or_synth_kv(kv_seed, 500000 + uint64_t(l), KVH, HD, 0, P, kh.data(), vh.data(), ksh.data(), vsh.data());
    for (int hh = 0; hh < KVH; ++hh) {
      std::memcpy(&L.k[size_t(hh) * m->cap * HD], &kh[size_t(hh) * P * HD], size_t(P) * HD);
      std::memcpy(&L.v[size_t(hh) * m->cap * HD], &vh[size_t(hh) * P * HD], size_t(P) * HD);
      std::memcpy(&L.ks[size_t(hh) * m->cap], &ksh[size_t(hh) * P], size_t(P) * 2);
      std::memcpy(&L.vs[size_t(hh) * m->cap], &vsh[size_t(hh) * P], size_t(P) * 2);
    }
  }
  return m;
}

void or_model_free(void* h) { delete static_cast<OrModel*>(h); }

void or_route(const float* logits, int rows, int E, int K, int sigmoid, const float* sel_bias, const float* logit_bias,
              const float* pes, float scale, float eps, int32_t* inds, float* wts);
int or_expert_union(const int32_t* inds, int rows, int K, int E, int32_t* entries, int32_t* pairs);

// The MoE FFN of one layer (MoELayer.encode, Sources/Ingot/Layers/MoE.swift:346-428; MoEReference,
// Tests/IngotTests/KernelHarness.swift:720-766): x = round(h ⊙ w) and r as the RMSNorm split (fp16 for MXFP4 experts,
// bf16 for int4), router logits r·(x·Wrᵀ) (+ router bias), softmax top-k and the expert union; per pair h_p =
// round(act(r·g + bg, r·u + bu)), o_p = h_p·Wdᵀ + bd; y[row] = Σ_slot w·o in slot order; h += y.
// With iid_key ≠ 0 (the synthetic i.i.d. routing of ih_model_desc.iid_routing) the router logit of row r and expert e
// is draw (P + r)·E + e of that N(0,1) stream instead of the router's product.
static void moe_forward(const or_model_desc* d, const OrLayer& L, float* hres, int B, uint64_t iid_key, int P) {
  const int H = d->hidden, E = d->n_experts, K = d->top_k, IE = d->expert_intermediate;
  const bool f16 = d->expert_format == 1;
  auto round_act = [&](float v) { return f16 ? or_f16_to_f32(or_f32_to_f16(v)) : or_bf16_to_f32(or_f32_to_bf16(v)); };
  std::vector<float> x(size_t(B) * H), rr(B), lg(size_t(B) * E);
  if (f16) or_rms_split_f16(hres, B, H, L.mlp_norm.data(), d->rms_eps, x.data(), rr.data());
  else or_rms_split(hres, B, H, L.mlp_norm.data(), d->rms_eps, x.data(), rr.data());
  if (iid_key) {
    for (int r = 0; r < B; ++r)
      for (int e = 0; e < E; ++e) lg[size_t(r) * E + e] = sm_normal(iid_key, uint64_t(P + r) * uint64_t(E) + uint64_t(e));
  } else {
    L.router.apply(x.data(), B, lg.data());
    scale_rows(lg.data(), B, E, rr.data());
  }
  std::vector<int32_t> inds(size_t(B) * K), entries(size_t(B) * K * 3), pairs(size_t(B) * K * 2);
  std::vector<float> wts(size_t(B) * K);
  or_route(lg.data(), B, E, K, 0, nullptr, L.router_bias.empty() ? nullptr : L.router_bias.data(), nullptr, 1.0f, 0.0f,
           inds.data(), wts.data());
  const int U = or_expert_union(inds.data(), B, K, E, entries.data(), pairs.data());
  std::vector<float> o(size_t(B) * K * H);
  std::vector<int> pair_of(size_t(B) * K);
  for (int u = 0; u < U; ++u) {
    const int e = entries[3 * u], start = entries[3 * u + 1], cnt = entries[3 * u + 2];
    std::vector<float> xe(size_t(cnt) * H), gu(size_t(cnt) * 2 * IE), he(size_t(cnt) * IE), oe(size_t(cnt) * H);
    for (int j = 0; j < cnt; ++j) {
      const int r = pairs[2 * (start + j)];
      pair_of[size_t(r) * K + pairs[2 * (start + j) + 1]] = start + j;
      std::memcpy(&xe[size_t(j) * H], &x[size_t(r) * H], sizeof(float) * H);
    }
    L.egu[e].apply(xe.data(), cnt, gu.data());
    for (int j = 0; j < cnt; ++j) {
      const int r = pairs[2 * (start + j)];
      for (int i = 0; i < IE; ++i) {
        float g = gu[size_t(j) * 2 * IE + i] * rr[r], uu = gu[size_t(j) * 2 * IE + IE + i] * rr[r];
        if (!L.gu_bias.empty()) {
          g += or_bf16_to_f32(L.gu_bias[size_t(e) * 2 * IE + i]);
          uu += or_bf16_to_f32(L.gu_bias[size_t(e) * 2 * IE + IE + i]);
        }
        he[size_t(j) * IE + i] = round_act(or_glu(g, uu, d->act, d->swiglu_limit));
      }
    }
    L.edn[e].apply(he.data(), cnt, oe.data());
    for (int j = 0; j < cnt; ++j)
      for (int c = 0; c < H; ++c)
        o[size_t(start + j) * H + c] =
            oe[size_t(j) * H + c] + (L.dn_bias.empty() ? 0.f : or_bf16_to_f32(L.dn_bias[size_t(e) * H + c]));
  }
  for (int r = 0; r < B; ++r)
    for (int c = 0; c < H; ++c) {
      float y = 0.f;
      for (int k = 0; k < K; ++k) {
        const int pr = pair_of[size_t(r) * K + k];
        y += wts[size_t(r) * K + k] * o[size_t(pr) * H + c];
      }
      hres[size_t(r) * H + c] += y;
    }
}

static void capture(OrModel* m, int l, const float* hres, int B) {
  const int H = m->d.hidden, n = int(m->cap_layers.size());
  for (int j = 0; j < n; ++j) {
    if (m->cap_layers[j] != l) continue;
    m->caps.resize(size_t(B) * n * H);
    for (int r = 0; r < B; ++r)
      for (int c = 0; c < H; ++c) m->caps[(size_t(r) * n + j) * H + c] = or_f32_to_bf16(hres[size_t(r) * H + c]);
  }
}

// tie_word_embeddings: the head is the embedding table itself (Sources/Ingot/Model.swift:269-276).
void or_model_tie_head(void* h) {
  OrModel* m = static_cast<OrModel*>(h);
  m->head = m->embed;
}

void or_model_set_capture(void* h, int n, const int* layers) {
  OrModel* m = static_cast<OrModel*>(h);
  m->cap_layers.assign(layers, layers + n);
}

void or_model_captures(void* h, uint16_t* out) {
  OrModel* m = static_cast<OrModel*>(h);
  std::memcpy(out, m->caps.data(), m->caps.size() * 2);
}

// One verify step of B rows at position P (not advancing it): logits [B][vocab], top1 [B].
int or_model_verify(void* h, const uint32_t* tokens, int B, float* logits, uint32_t* top1) {
  OrModel* m = static_cast<OrModel*>(h);
  const or_model_desc* d = &m->d;
  const int H = d->hidden, QH = d->n_q_heads, KVH = d->n_kv_heads, HD = d->head_dim, I = d->intermediate;
  // q heads QS apart in the projection row ([q | gate] per head with a gate: AT_QS, verify_attn.metal:28-45).
  const int QS = HD * (d->attn_gate ? 2 : 1), QP = QH * QS + 2 * KVH * HD, P = m->P, cap = m->cap;
  const int rot = d->rotary_dims > 0 ? d->rotary_dims : HD;
  const float* rinv = m->rinv.empty() ? nullptr : m->rinv.data();
  auto col = [&](int hh) { return hh < QH ? hh * QS : QH * QS + (hh - QH) * HD; };
  if (B < 1 || P + B > cap) return 1;
  std::vector<float> hres(size_t(B) * H);
  for (int r = 0; r < B; ++r)
    or_dequant_int4(m->embed.w.data() + size_t(tokens[r]) * H / 8, m->embed.s.data() + size_t(tokens[r]) * H / 64,
                    m->embed.b.data() + size_t(tokens[r]) * H / 64, 1, H, hres.data() + size_t(r) * H);
  std::vector<float> x(size_t(B) * H), proj(size_t(B) * QP), q(size_t(B) * QH * HD), att(size_t(B) * QH * HD);
  std::vector<float> y(size_t(B) * H), gu(size_t(B) * 2 * I), a(size_t(B) * I), rr(B);
  for (int l = 0; l < d->n_layers; ++l) {
    OrLayer& L = m->layers[l];
    or_rms_split(hres.data(), B, H, L.attn_norm.data(), d->rms_eps, x.data(), rr.data());
    L.qkv.apply(x.data(), B, proj.data());
    scale_rows(proj.data(), B, QP, rr.data());
    // q|k|v bias, then the per-head RMSNorm of q and k (vattn_prework_i8's AT_QKVB and AT_QKN, verify_attn_nax.metal:
    // 76-89), before RoPE.
    for (int t = 0; t < B && !L.qkv_bias.empty(); ++t)
      for (int i = 0; i < QP; ++i) proj[size_t(t) * QP + i] += L.qkv_bias[i];
    if (!L.q_norm.empty())
      for (int t = 0; t < B; ++t)
        for (int hh = 0; hh < QH + KVH; ++hh) {
          float* xr = proj.data() + size_t(t) * QP + col(hh);
          double ss = 0;
          for (int dd = 0; dd < HD; ++dd) ss += double(xr[dd]) * xr[dd];
          const float r = 1.0f / std::sqrt(float(ss) / float(HD) + d->rms_eps);
          const uint16_t* w = hh < QH ? L.q_norm.data() : L.k_norm.data();
          for (int dd = 0; dd < HD; ++dd) xr[dd] = xr[dd] * r * or_bf16_to_f32(w[dd]);
        }
    for (int t = 0; t < B; ++t) {
      const float* pr = proj.data() + size_t(t) * QP;
      for (int hh = 0; hh < QH; ++hh) {
        float xq[256];
        std::memcpy(xq, pr + col(hh), sizeof(float) * HD);
        or_rope_wht_ex(xq, HD, rot, P + t, d->rope_theta, rinv, m->rmscale, d->hadamard_k);
        for (int dd = 0; dd < HD; ++dd) q[(size_t(t) * QH + hh) * HD + dd] = or_f16_to_f32(or_f32_to_f16(xq[dd]));
      }
      for (int hh = 0; hh < KVH; ++hh) {
        float xk[256], xv[256];
        std::memcpy(xk, pr + col(QH + hh), sizeof(float) * HD);
        std::memcpy(xv, pr + col(QH + KVH + hh), sizeof(float) * HD);
        or_rope_wht_ex(xk, HD, rot, P + t, d->rope_theta, rinv, m->rmscale, d->hadamard_k);
        const size_t o = size_t(hh) * cap + P + t;
        quant_i8(xk, HD, &L.k[o * HD], &L.ks[o]);
        quant_i8(xv, HD, &L.v[o * HD], &L.vs[o]);
      }
    }
    const int window = (d->sliding_window > 0 && l % 2 == 0) ? d->sliding_window : 0;
    or_attention(q.data(), B, P, QH, KVH, HD, L.k.data(), L.v.data(), L.ks.data(), L.vs.data(), cap, window,
                 d->sinks ? L.sinks.data() : nullptr, att.data());
    // Gated output: × sigmoid(gate) per (row, head, dim) (at_gate in vattn_reduce, verify_attn.metal:94-99,190).
    if (d->attn_gate)
      for (int t = 0; t < B; ++t)
        for (int hh = 0; hh < QH; ++hh)
          for (int dd = 0; dd < HD; ++dd) {
            const float g = proj[size_t(t) * QP + size_t(hh) * QS + HD + dd];
            att[(size_t(t) * QH + hh) * HD + dd] *= 1.0f / (1.0f + std::exp(-g));
          }
    for (auto& z : att) z = or_bf16_to_f32(or_f32_to_bf16(z));
    L.o.apply(att.data(), B, y.data());
    if (!L.o_bias.empty())
      for (int t = 0; t < B; ++t)
        for (int i = 0; i < H; ++i) y[size_t(t) * H + i] += L.o_bias[i];
    for (size_t i = 0; i < hres.size(); ++i) hres[i] += y[i];
    if (d->n_experts > 0) {
      moe_forward(d, L, hres.data(), B, d->iid_routing ? sm_key(m->seed, layer_tensor(l, 13)) : 0, P);
      capture(m, l, hres.data(), B);
      continue;
    }
    or_rms_split(hres.data(), B, H, L.mlp_norm.data(), d->rms_eps, x.data(), rr.data());
    L.gate_up.apply(x.data(), B, gu.data());
    scale_rows(gu.data(), B, 2 * I, rr.data());
    for (int t = 0; t < B; ++t)
      for (int i = 0; i < I; ++i)
        a[size_t(t) * I + i] = or_bf16_to_f32(or_f32_to_bf16(
            or_glu(gu[size_t(t) * 2 * I + i], gu[size_t(t) * 2 * I + I + i], d->act, d->swiglu_limit)));
    L.down.apply(a.data(), B, y.data());
    for (size_t i = 0; i < hres.size(); ++i) hres[i] += y[i];
    capture(m, l, hres.data(), B);
  }
  or_rms_split(hres.data(), B, H, m->final_norm.data(), d->rms_eps, x.data(), rr.data());
  m->head.apply(x.data(), B, logits);
  scale_rows(logits, B, d->vocab, rr.data());
  or_argmax_rows(logits, B, d->vocab, top1);
  return 0;
}

// Convenience: create, one step, free. logits [B][vocab], top1 [B].
int or_verify_dense(const or_model_desc* d, uint64_t seed, uint64_t kv_seed, int P, const uint32_t* tokens, int B,
                    float* logits, uint32_t* top1) {
  void* m = or_model_create(d, seed, kv_seed, P, B);
  const int rc = or_model_verify(m, tokens, B, logits, top1);
  or_model_free(m);
  return rc;
}


// ---------------------------------------------------------------------------------------------------------------
// MoE router: top-k by score (plus a selection bias), ties to the lower index, NaN logits → −inf; weights from the
// unbiased scores: softmax over the chosen logits (renormalised top-k) or sigmoid p / (Σp + eps); times `scale` and a
// per-expert scale. A router linear bias is part of the logits. RouterVector.reference
// (Tests/IngotTests/KernelCaseRouter.swift:54-80) and vmoe_route (Sources/Ingot/Shaders/verify.metal:160-240).
void or_route(const float* logits, int rows, int E, int K, int sigmoid, const float* sel_bias, const float* logit_bias,
              const float* pes, float scale, float eps, int32_t* inds, float* wts) {
  std::vector<float> l(E), p(E), sel(E);
  std::vector<int> order(E);
  for (int r = 0; r < rows; ++r) {
    for (int e = 0; e < E; ++e) {
      float v = logits[size_t(r) * E + e] + (logit_bias ? logit_bias[e] : 0.f);
      if (std::isnan(v)) v = -std::numeric_limits<float>::infinity();
      l[e] = v;
      p[e] = sigmoid ? 1.0f / (1.0f + std::exp(-v)) : v;
      sel[e] = p[e] + (sel_bias ? sel_bias[e] : 0.f);
      order[e] = e;
    }
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return sel[a] > sel[b]; });
    float w[64], sum = 0.f;
    for (int k = 0; k < K; ++k) {
      const int e = order[k];
      w[k] = sigmoid ? p[e] : std::exp(l[e] - l[order[0]]);
      sum += w[k];
    }
    if (sigmoid) sum += eps;
    for (int k = 0; k < K; ++k) {
      const int e = order[k];
      inds[size_t(r) * K + k] = e;
      wts[size_t(r) * K + k] = w[k] / sum * scale * (pes ? pes[e] : 1.0f);
    }
  }
}

// Expert union of a round by counting sort: entries (expert, start, count) in increasing expert order, pairs (row,
// slot) in row order inside each expert, slot = the rank k of the expert in the row's top-k. vmoe_route
// (Sources/Ingot/Shaders/verify.metal:262-318) and MoEPipeline.round (Tests/IngotTests/KernelHarness.swift:630-652).
// Returns U, the number of distinct experts; entries [U][3], pairs [rows·K][2].
int or_expert_union(const int32_t* inds, int rows, int K, int E, int32_t* entries, int32_t* pairs) {
  int U = 0, off = 0;
  for (int e = 0; e < E; ++e) {
    int cnt = 0;
    for (int i = 0; i < rows * K; ++i)
      if (inds[i] == e) {
        pairs[2 * (off + cnt)] = i / K;
        pairs[2 * (off + cnt) + 1] = i % K;
        ++cnt;
      }
    if (cnt == 0) continue;
    entries[3 * U] = e;
    entries[3 * U + 1] = off;
    entries[3 * U + 2] = cnt;
    ++U;
    off += cnt;
  }
  return U;
}

// ---------------------------------------------------------------------------------------------------------------
// Copy-from-context lookup. The rule (CopySpecTests.naive, Tests/IngotTests/CopySpecTests.swift:9-28): among the
// three most recent earlier occurrences p < cur of the last trigram (the index keeps four ends, the current one
// included), the one with the longest backward match (at most 64, len ≤ p), ties to the most recent; at least 3;
// propose h[p+1 … min(cur, p + maxK)]. Returns the proposal length and leaves the match length in *match.
int or_copy_naive(const uint32_t* h, int n, int maxK, int minMatch, int maxMatch, uint32_t* out, int* match) {
  *match = 0;
  if (n < 4 || maxK <= 0) return 0;
  const int cur = n - 1;
  int cand[3], nc = 0;
  for (int p = cur - 1; p >= 2 && nc < 3; --p)
    if (h[p] == h[cur] && h[p - 1] == h[cur - 1] && h[p - 2] == h[cur - 2]) cand[nc++] = p;
  int bestEnd = 0, bestLen = 0;
  for (int i = 0; i < nc; ++i) {
    const int p = cand[i];
    int len = 0;
    while (len < maxMatch && len <= p && h[p - len] == h[cur - len]) ++len;
    if (len > bestLen) { bestLen = len; bestEnd = p; }
  }
  if (bestLen < minMatch) return 0;
  *match = bestLen;
  const int end = std::min(cur, bestEnd + maxK);
  for (int i = bestEnd + 1; i <= end; ++i) out[i - bestEnd - 1] = h[i];
  return end - bestEnd;
}

// The reference's index restated (CopyIndex, Sources/Ingot/CopySpec.swift:15-139): a 4-way table of the most recent
// ends of each trigram key, key = mix(a·φ ^ mix(b + c1) ^ (c << 1)) | 1, open addressing, rebuilt at occupancy > 1/2.
struct OrCopyIndex {
  static constexpr int WAYS = 4;
  int minMatch = 3, maxMatch = 64;
  std::vector<uint32_t> hist;
  std::vector<uint64_t> keys;
  std::vector<uint32_t> pos;
  std::vector<uint8_t> cnt;
  size_t mask = 0, used = 0;
  static uint64_t mix(uint64_t x) {
    x ^= x >> 33; x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33; x *= 0xc4ceb9fe1a85ec53ull;
    return x ^ (x >> 33);
  }
  void allocate(size_t tokens) {
    size_t cap = 1;
    while (cap < tokens * 2) cap <<= 1;
    keys.assign(cap, 0);
    pos.assign(cap * WAYS, 0);
    cnt.assign(cap, 0);
    mask = cap - 1;
    used = 0;
  }
  uint64_t key_at(size_t end) const {
    const uint64_t a = hist[end - 2], b = hist[end - 1], c = hist[end];
    return mix((a * 0x9E3779B97F4A7C15ull) ^ mix(b + 0x632BE59BD9B4E019ull) ^ (c << 1)) | 1ull;
  }
  long find(uint64_t key) const {
    size_t i = key & mask;
    while (true) {
      if (keys[i] == key) return long(i);
      if (keys[i] == 0) return -1;
      i = (i + 1) & mask;
    }
  }
  void index(size_t end) {
    if (used * 2 > keys.size()) { rebuild(hist.size() * 2); return; }
    const uint64_t key = key_at(end);
    size_t i = key & mask;
    while (keys[i] != 0 && keys[i] != key) i = (i + 1) & mask;
    if (keys[i] == 0) { keys[i] = key; ++used; }
    const size_t b = i * WAYS;
    for (int w = WAYS - 1; w > 0; --w) pos[b + w] = pos[b + w - 1];
    pos[b] = uint32_t(end);
    if (cnt[i] < WAYS) ++cnt[i];
  }
  void rebuild(size_t capacity) {
    allocate(std::max(capacity, size_t(1) << 16));
    std::vector<uint32_t> h;
    h.swap(hist);
    for (uint32_t t : h) append(t);
  }
  void append(uint32_t t) {
    hist.push_back(t);
    if (hist.size() >= 3) index(hist.size() - 1);
  }
  int propose(int maxK, uint32_t* out, int* match) {
    *match = 0;
    const size_t n = hist.size();
    if (n < 4 || maxK <= 0) return 0;
    const long s = find(key_at(n - 1));
    if (s < 0) return 0;
    const long cur = long(n) - 1;
    long bestEnd = 0;
    int bestLen = 0;
    for (int w = 0; w < cnt[s]; ++w) {
      const long p = pos[size_t(s) * WAYS + w];
      if (p >= cur) continue;
      int len = 0;
      while (len < maxMatch && len <= p && hist[p - len] == hist[cur - len]) ++len;
      if (len > bestLen) { bestLen = len; bestEnd = p; }
    }
    if (bestLen < minMatch) return 0;
    *match = bestLen;
    const long end = std::min(cur, bestEnd + maxK);
    for (long i = bestEnd + 1; i <= end; ++i) out[i - bestEnd - 1] = hist[i];
    return int(end - bestEnd);
  }
};

void* or_copy_index_new(int capacity) {
  auto* c = new OrCopyIndex();
  c->allocate(size_t(capacity));
  return c;
}
void or_copy_index_free(void* h) { delete static_cast<OrCopyIndex*>(h); }
void or_copy_index_append(void* h, const uint32_t* toks, int n) {
  for (int i = 0; i < n; ++i) static_cast<OrCopyIndex*>(h)->append(toks[i]);
}
int or_copy_index_propose(void* h, int maxK, uint32_t* out, int* match) {
  return static_cast<OrCopyIndex*>(h)->propose(maxK, out, match);
}

// SplitMix64 output stream of `seed` (Sources/Ingot/Sampling.swift:50-62), for the reference's randomized tests.
void or_splitmix64(uint64_t seed, int n, uint64_t* out) {
  uint64_t s = seed;
  for (int i = 0; i < n; ++i) {
    s += 0x9E3779B97F4A7C15ull;
    out[i] = sm_mix(s);
  }
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}


// ---------------------------------------------------------------------------------------------------------------
// Sampling (temperature > 0). topk64_part/topk64_merge (Sources/Ingot/Shaders/zz_sample.metal:27-171): per row the
// 64 best logits sorted by value, ties to the lower id (tk_better, yy_model.metal:503), and (max, Σ exp((x − max)/T))
// over the row (in double here; NaN logits left out). idx/val [rows][64], z [rows][2].
void or_topk64(const float* x, int rows, int V, float temp, uint32_t* idx, float* val, float* z) {
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + size_t(r) * V;
    std::vector<int> ids;
    ids.reserve(V);
    for (int i = 0; i < V; ++i)
      if (!std::isnan(xr[i]) && xr[i] > -std::numeric_limits<float>::max()) ids.push_back(i);
    const int k = std::min<int>(64, int(ids.size()));
    std::partial_sort(ids.begin(), ids.begin() + k, ids.end(),
                      [&](int a, int b) { return xr[a] > xr[b] || (xr[a] == xr[b] && a < b); });
    for (int j = 0; j < 64; ++j) {
      idx[size_t(r) * 64 + j] = j < k ? uint32_t(ids[j]) : 0xFFFFFFFFu;
      val[size_t(r) * 64 + j] = j < k ? xr[ids[j]] : -std::numeric_limits<float>::max();
    }
    double M = -std::numeric_limits<float>::max();
    for (int i = 0; i < V; ++i)
      if (!std::isnan(xr[i])) M = std::max(M, double(xr[i]));
    double Z = 0;
    for (int i = 0; i < V; ++i)
      if (!std::isnan(xr[i])) Z += std::exp((double(xr[i]) - M) / temp);
    z[2 * r] = float(M);
    z[2 * r + 1] = float(Z);
  }
}

struct or_sample_params {
  float temp, top_p;
  int top_k;
  float min_p;
};

// sample_dist (zz_sample.metal:196-226): the candidates' probabilities after temperature → top-k → min-p → top-p,
// renormalised; returns how many remain.
int or_sample_dist(const uint32_t* ci, const float* cv, float M, float Z, const or_sample_params* p, float* pr) {
  const float it = 1.0f / p->temp;
  int n = 0;
  while (n < 64 && ci[n] != 0xFFFFFFFFu) ++n;
  float tot = Z;
  if (p->top_k > 0 && p->top_k < n) n = p->top_k;
  if (p->top_k > 0) {
    tot = 0;
    for (int j = 0; j < n; ++j) tot += std::exp((cv[j] - M) * it);
  }
  for (int j = 0; j < n; ++j) pr[j] = std::exp((cv[j] - M) * it) / tot;
  if (p->min_p > 0) {
    const float thr = p->min_p * pr[0];
    int k = 1;
    while (k < n && pr[k] >= thr) ++k;
    n = k;
    float s = 0;
    for (int j = 0; j < n; ++j) s += pr[j];
    for (int j = 0; j < n; ++j) pr[j] /= s;
  }
  if (p->top_p < 1.0f) {
    float c = 0;
    int k = n;
    for (int j = 0; j < n; ++j) {
      c += pr[j];
      if (c >= p->top_p) {
        k = j + 1;
        break;
      }
    }
    n = std::max(k, 1);
  }
  float s = 0;
  for (int j = 0; j < n; ++j) s += pr[j];
  for (int j = 0; j < n; ++j) pr[j] /= s;
  return n;
}

// sample_pick (zz_sample.metal:228-239): the token whose cumulative mass (without `skip`) first exceeds u·(1 − q).
static uint32_t or_sample_pick(const uint32_t* ci, const float* pr, int n, uint32_t skip, float q, float u) {
  const float target = u * (1.0f - q);
  float acc = 0;
  uint32_t last = 0xFFFFFFFFu;
  for (int j = 0; j < n; ++j) {
    if (ci[j] == skip) continue;
    acc += pr[j];
    last = ci[j];
    if (acc > target) return ci[j];
  }
  return last == 0xFFFFFFFFu ? ci[0] : last;
}

// spec_accept_sample (zz_sample.metal:241-281) on the host: rows' candidates, uniforms u[2i] (accept) and u[2i + 1]
// (resample) of row i; returns m and writes the emitted tokens (drafts 1..m, then the sampled token) to emitted.
int or_accept_sample(const uint32_t* vtok, int nr, const uint32_t* cidx, const float* cval, const float* z,
                     const float* u, const or_sample_params* p, uint32_t* emitted) {
  float pr[64];
  int m = 0;
  uint32_t next = 0;
  for (int i = 0; i < nr; ++i) {
    const uint32_t* ci = cidx + size_t(i) * 64;
    const int n = or_sample_dist(ci, cval + size_t(i) * 64, z[2 * i], z[2 * i + 1], p, pr);
    if (i + 1 < nr) {
      const uint32_t d = vtok[i + 1];
      float q = 0;
      for (int j = 0; j < n; ++j)
        if (ci[j] == d) q = pr[j];
      if (u[2 * i] < q) {
        ++m;
        continue;
      }
      next = or_sample_pick(ci, pr, n, d, q, u[2 * i + 1]);
    } else {
      next = or_sample_pick(ci, pr, n, 0xFFFFFFFFu, 0, u[2 * i + 1]);
    }
    break;
  }
  for (int i = 0; i < m; ++i) emitted[i] = vtok[i + 1];
  emitted[m] = next;
  return m;
}

// spec_rows_choose (yy_model.metal:654-675; SpecRowsConfig.chooseCPU, SpecRows.swift:93-105).
int or_rows_choose(const float* conf, const float* a, const float* b, const float* cost, int kmin, int kmax) {
  float acc = 1, lp = 1, bv = -1;
  int best = kmax;
  for (int t = 0; t + 1 < kmax; ++t) {
    const int g = std::min(t, 3);
    const float c = std::min(std::max(conf[t], 1e-6f), 1.0f - 1e-6f);
    const float q = 1.0f / (1.0f + std::exp(-(a[g] * std::log(c / (1.0f - c)) + b[g])));
    lp *= q;
    acc += lp;
    const int k = t + 2;
    if (k >= kmin) {
      const float v = acc / cost[k];
      if (v > bv) {
        bv = v;
        best = k;
      }
    }
  }
  return best;
}


// ---------------------------------------------------------------------------------------------------------------
// The DFlash2 drafter (DFlash2Drafter, Sources/Ingot/Drafter.swift:300-550; yy_model.metal:151-614), with the synthetic
// weights of the library's generator and the rounding points of its GPU path: bf16 activations into every projection
// (the RMSNorm outputs, the conv outputs, the attention output, the SwiGLU), fp16 q and K/V in the rings.
struct or_drafter_desc {
  int n_layers, hidden, n_q_heads, head_dim, intermediate, block, window, n_targets;
  int target_layers[8];
  int rank, dyn_conv;
  uint32_t mask_token;
  float rope_theta, rms_eps;
};

static uint64_t dl_tensor(int l, uint64_t kind) { return 7000000 + 1000 * uint64_t(l) + kind; }
static uint64_t dg_tensor(uint64_t kind) { return 7900000 + kind; }
static float rbf(float x) { return or_bf16_to_f32(or_f32_to_bf16(x)); }
static float rhf(float x) { return or_f16_to_f32(or_f32_to_f16(x)); }

struct OrDLayer {
  std::vector<uint16_t> n1, n2, qn, kn, abase, mbase;
  QMat qkv, o, gu, down, aproj, mproj;
  std::vector<float> kc, vc;  // [8][slots][HD], fp16 values
};

struct OrDrafter {
  or_drafter_desc d;
  int H = 0, HD = 0, QH = 0, QP = 0, I = 0, V = 0, slots = 0, G = 0, DYN = 0, Ht = 0;
  std::vector<OrDLayer> layers;
  QMat fc, hproj, embed, head;
  std::vector<uint16_t> hnorm, fnorm, pred, succ;
};

void* or_drafter_create(const or_drafter_desc* d, uint64_t seed, const or_model_desc* td, uint64_t tseed) {
  OrDrafter* r = new OrDrafter();
  r->d = *d;
  r->H = d->hidden;
  r->HD = d->head_dim;
  r->QH = d->n_q_heads;
  r->QP = (r->QH + 16) * r->HD;
  r->I = d->intermediate;
  r->V = td->vocab;
  r->Ht = td->hidden;
  r->G = r->QH / 8;
  r->slots = (d->window + 16 + 31) / 32 * 32;
  r->DYN = 4 * (r->H / 16);
  const int H = r->H, HD = r->HD;
  const float sd = 0.02f;
  r->embed.make(tseed, 1, td->vocab, td->hidden, sd);
  r->head.make(tseed, 3, td->vocab, td->hidden, sd);
  r->layers.resize(d->n_layers);
  for (int l = 0; l < d->n_layers; ++l) {
    OrDLayer& L = r->layers[l];
    L.n1.resize(H); L.n2.resize(H); L.qn.resize(HD); L.kn.resize(HD);
    or_synth_bf16(seed, dl_tensor(l, 0), H, 1.0f, 0.125f, L.n1.data());
    or_synth_bf16(seed, dl_tensor(l, 1), H, 1.0f, 0.125f, L.n2.data());
    or_synth_bf16(seed, dl_tensor(l, 2), HD, 1.0f, 0.125f, L.qn.data());
    or_synth_bf16(seed, dl_tensor(l, 3), HD, 1.0f, 0.125f, L.kn.data());
    L.qkv.make(seed, dl_tensor(l, 4), r->QP, H, sd);
    L.o.make(seed, dl_tensor(l, 5), H, r->QH * HD, sd);
    L.gu.make(seed, dl_tensor(l, 6), 2 * r->I, H, sd);
    L.down.make(seed, dl_tensor(l, 7), H, r->I, sd);
    if (d->dyn_conv) {
      L.aproj.make(seed, dl_tensor(l, 8), r->DYN, H, sd);
      L.mproj.make(seed, dl_tensor(l, 9), r->DYN, H, sd);
      L.abase.resize(4 * H);
      L.mbase.resize(4 * H);
      for (int k = 0; k < 4; ++k) {
        or_synth_bf16(seed, dl_tensor(l, 10) + 100 * k, H, k % 2 ? 0.0f : 1.0f, 0.1f, L.abase.data() + k * H);
        or_synth_bf16(seed, dl_tensor(l, 11) + 100 * k, H, k % 2 ? 0.0f : 1.0f, 0.1f, L.mbase.data() + k * H);
      }
    }
    L.kc.assign(size_t(8) * r->slots * HD, 0.f);
    L.vc.assign(size_t(8) * r->slots * HD, 0.f);
  }
  r->fc.make(seed, dg_tensor(1), H, d->n_targets * td->hidden, sd);
  r->hnorm.resize(H);
  r->fnorm.resize(H);
  or_synth_bf16(seed, dg_tensor(2), H, 1.0f, 0.125f, r->hnorm.data());
  or_synth_bf16(seed, dg_tensor(3), H, 1.0f, 0.125f, r->fnorm.data());
  if (d->rank > 0) {
    r->hproj.make(seed, dg_tensor(4), d->rank, H, sd);
    r->pred.resize(size_t(r->V) * d->rank);
    r->succ.resize(size_t(r->V) * d->rank);
    or_synth_bf16(seed, dg_tensor(5), r->pred.size(), 0.0f, 0.25f, r->pred.data());
    or_synth_bf16(seed, dg_tensor(6), r->succ.size(), 0.0f, 0.25f, r->succ.data());
  }
  return r;
}

void or_drafter_free(void* h) { delete static_cast<OrDrafter*>(h); }

// bf16(x · rsqrt(mean x² + eps) · w) of `rows` rows.
static void dnorm(const float* x, int rows, int H, const uint16_t* w, float eps, float* out) {
  for (int t = 0; t < rows; ++t) {
    double ss = 0;
    for (int c = 0; c < H; ++c) ss += double(x[size_t(t) * H + c]) * x[size_t(t) * H + c];
    const float rr = 1.0f / std::sqrt(float(ss) / float(H) + eps);
    for (int c = 0; c < H; ++c) out[size_t(t) * H + c] = rbf(x[size_t(t) * H + c] * rr * or_bf16_to_f32(w[c]));
  }
}

// Per-head RMSNorm + RoPE at position pos (dnorm_rope), in place on HD values.
static void dnorm_rope(float* x, int HD, const uint16_t* w, float pos, float eps, float theta) {
  double ss = 0;
  for (int i = 0; i < HD; ++i) ss += double(x[i]) * x[i];
  const float rr = 1.0f / std::sqrt(float(ss) / float(HD) + eps);
  float y[256];
  for (int i = 0; i < HD; ++i) y[i] = x[i] * rr * or_bf16_to_f32(w[i]);
  const int RH = HD / 2;
  for (int d = 0; d < HD; ++d) {
    const int i = d % RH;
    const double ang = double(pos) * std::pow(double(theta), -double(i) / double(RH));
    const float c = float(std::cos(ang)), s = float(std::sin(ang));
    x[d] = d < RH ? y[d] * c - y[d + RH] * s : y[d] * c + y[d - RH] * s;
  }
}

// Context rows: captures (bf16 values [rows][nT·Ht]) of positions pos0 + t, t < nvalid, into every layer's ring.
void or_drafter_context(void* h, const uint16_t* caps, int rows, int nvalid, int pos0) {
  OrDrafter* r = static_cast<OrDrafter*>(h);
  const int H = r->H, HD = r->HD, K = r->d.n_targets * r->Ht;
  std::vector<float> c(size_t(rows) * K), y(size_t(rows) * H), e(size_t(rows) * H), kv(size_t(rows) * 16 * HD);
  for (size_t i = 0; i < c.size(); ++i) c[i] = or_bf16_to_f32(caps[i]);
  r->fc.apply(c.data(), rows, y.data());
  dnorm(y.data(), rows, H, r->hnorm.data(), r->d.rms_eps, e.data());
  for (auto& L : r->layers) {
    // The k|v rows of q|k|v.
    QMat kvm;
    kvm.N = 16 * HD;
    kvm.K = H;
    const size_t w0 = size_t(r->QH) * HD * H / 8, s0 = size_t(r->QH) * HD * H / 64;
    kvm.w.assign(L.qkv.w.begin() + w0, L.qkv.w.end());
    kvm.s.assign(L.qkv.s.begin() + s0, L.qkv.s.end());
    kvm.b.assign(L.qkv.b.begin() + s0, L.qkv.b.end());
    kvm.apply(e.data(), rows, kv.data());
    for (int t = 0; t < nvalid; ++t) {
      const int pos = pos0 + t, ring = pos % r->d.window;
      for (int hh = 0; hh < 8; ++hh) {
        float xk[256];
        std::memcpy(xk, &kv[size_t(t) * 16 * HD + hh * HD], sizeof(float) * HD);
        dnorm_rope(xk, HD, L.kn.data(), float(pos), r->d.rms_eps, r->d.rope_theta);
        for (int i = 0; i < HD; ++i) {
          L.kc[(size_t(hh) * r->slots + ring) * HD + i] = rhf(xk[i]);
          L.vc[(size_t(hh) * r->slots + ring) * HD + i] = rhf(kv[size_t(t) * 16 * HD + (8 + hh) * HD + i]);
        }
      }
    }
  }
}

static bool dvisible(int n, int t, int P, int B, int W) {
  if (n >= W) return n < W + B;
  int back = (P - 1 - n) % W;
  if (back < 0) back += W;
  const int k = P - 1 - back;
  return k >= 0 && P + t - k < W;
}

// Draft block at position P with the anchor; drafts [block − 1], conf [block − 1].
void or_drafter_block(void* h, uint32_t anchor, int P, uint32_t* drafts, float* conf) {
  OrDrafter* r = static_cast<OrDrafter*>(h);
  const auto& d = r->d;
  const int B = d.block, M = B - 1, H = r->H, HD = r->HD, QH = r->QH, I = r->I, G = r->G, GC = H / 16;
  const bool conv = d.dyn_conv != 0;
  std::vector<float> x(size_t(B) * H), xn(size_t(B) * H), a(size_t(B) * H), dyn(size_t(B) * r->DYN);
  std::vector<float> qkv(size_t(B) * r->QP), att(size_t(B) * QH * HD), y(size_t(B) * H), gu(size_t(B) * 2 * I),
      hb(size_t(B) * I);
  for (int t = 0; t < B; ++t) {
    const uint32_t tok = t == 0 ? anchor : d.mask_token;
    or_dequant_int4(r->embed.w.data() + size_t(tok) * H / 8, r->embed.s.data() + size_t(tok) * H / 64,
                    r->embed.b.data() + size_t(tok) * H / 64, 1, H, x.data() + size_t(t) * H);
  }
  auto conv_prep = [&](const std::vector<uint16_t>& base) {
    for (int t = 0; t < B; ++t)
      for (int c = 0; c < H; ++c) {
        const int g = c / 16;
        const float x0 = xn[size_t(t) * H + c], x1 = t > 0 ? xn[size_t(t - 1) * H + c] : 0.f;
        const float k0 = or_bf16_to_f32(base[c]) + dyn[size_t(t) * r->DYN + g];
        const float k1 = or_bf16_to_f32(base[H + c]) + dyn[size_t(t) * r->DYN + GC + g];
        a[size_t(t) * H + c] = rbf(k0 * x0 + k1 * x1);
      }
  };
  auto conv_fin = [&](const std::vector<uint16_t>& base) {
    for (int t = 0; t < B; ++t)
      for (int c = 0; c < H; ++c) {
        const float y0 = y[size_t(t) * H + c];
        if (!conv) { x[size_t(t) * H + c] += y0; continue; }
        const int g = c / 16;
        const float y1 = t > 0 ? y[size_t(t - 1) * H + c] : 0.f;
        const float k0 = or_bf16_to_f32(base[2 * H + c]) + dyn[size_t(t) * r->DYN + 2 * GC + g];
        const float k1 = or_bf16_to_f32(base[3 * H + c]) + dyn[size_t(t) * r->DYN + 3 * GC + g];
        x[size_t(t) * H + c] += k0 * y0 + k1 * y1;
      }
  };
  const float scale = float(1.0 / std::sqrt(double(HD)));
  for (auto& L : r->layers) {
    dnorm(x.data(), B, H, L.n1.data(), d.rms_eps, xn.data());
    if (conv) {
      L.aproj.apply(xn.data(), B, dyn.data());
      conv_prep(L.abase);
    } else {
      a = xn;
    }
    L.qkv.apply(a.data(), B, qkv.data());
    // Block rows: q (fp16), k and v into the ring's block slots.
    std::vector<float> q(size_t(B) * QH * HD);
    for (int t = 0; t < B; ++t) {
      for (int hh = 0; hh < QH + 8; ++hh) {
        float xv[256];
        std::memcpy(xv, &qkv[size_t(t) * r->QP + hh * HD], sizeof(float) * HD);
        dnorm_rope(xv, HD, hh < QH ? L.qn.data() : L.kn.data(), float(P + t), d.rms_eps, d.rope_theta);
        for (int i = 0; i < HD; ++i) {
          if (hh < QH) q[(size_t(t) * QH + hh) * HD + i] = rhf(xv[i]);
          else L.kc[(size_t(hh - QH) * r->slots + d.window + t) * HD + i] = rhf(xv[i]);
        }
      }
      for (int hh = 0; hh < 8; ++hh)
        for (int i = 0; i < HD; ++i)
          L.vc[(size_t(hh) * r->slots + d.window + t) * HD + i] = rhf(qkv[size_t(t) * r->QP + (QH + 8 + hh) * HD + i]);
    }
    // Attention: every visible slot, softmax in fp32.
    for (int t = 0; t < B; ++t)
      for (int hh = 0; hh < QH; ++hh) {
        const int kvh = hh / G;
        std::vector<float> s(r->slots, -std::numeric_limits<float>::infinity());
        float mx = -std::numeric_limits<float>::infinity();
        for (int n = 0; n < r->slots; ++n) {
          if (!dvisible(n, t, P, B, d.window)) continue;
          float acc = 0;
          for (int i = 0; i < HD; ++i) acc += q[(size_t(t) * QH + hh) * HD + i] * L.kc[(size_t(kvh) * r->slots + n) * HD + i];
          s[n] = acc * scale;
          mx = std::max(mx, s[n]);
        }
        float l = 0;
        std::vector<float> o(HD, 0.f);
        for (int n = 0; n < r->slots; ++n) {
          if (s[n] == -std::numeric_limits<float>::infinity()) continue;
          const float p = std::exp(s[n] - mx);
          l += p;
          for (int i = 0; i < HD; ++i) o[i] += p * L.vc[(size_t(kvh) * r->slots + n) * HD + i];
        }
        for (int i = 0; i < HD; ++i) att[size_t(t) * QH * HD + hh * HD + i] = rbf(o[i] / l);
      }
    L.o.apply(att.data(), B, y.data());
    conv_fin(L.abase);
    dnorm(x.data(), B, H, L.n2.data(), d.rms_eps, xn.data());
    if (conv) {
      L.mproj.apply(xn.data(), B, dyn.data());
      conv_prep(L.mbase);
    } else {
      a = xn;
    }
    L.gu.apply(a.data(), B, gu.data());
    for (int t = 0; t < B; ++t)
      for (int i = 0; i < I; ++i) {
        const float g = gu[size_t(t) * 2 * I + i], u = gu[size_t(t) * 2 * I + I + i];
        hb[size_t(t) * I + i] = rbf(g / (1.0f + std::exp(-g)) * u);
      }
    L.down.apply(hb.data(), B, y.data());
    conv_fin(L.mbase);
  }
  std::vector<float> hid(size_t(M) * H), logits(size_t(M) * r->V), hp(size_t(M) * std::max(1, d.rank));
  dnorm(x.data() + H, M, H, r->fnorm.data(), d.rms_eps, hid.data());
  r->head.apply(hid.data(), M, logits.data());
  if (d.rank > 0) r->hproj.apply(hid.data(), M, hp.data());
  uint32_t prev = anchor;
  for (int t = 0; t < M; ++t) {
    const float* lr = logits.data() + size_t(t) * r->V;
    std::vector<int> ids(r->V);
    for (int i = 0; i < r->V; ++i) ids[i] = i;
    std::partial_sort(ids.begin(), ids.begin() + 16, ids.end(),
                      [&](int u, int v) { return lr[u] > lr[v] || (lr[u] == lr[v] && u < v); });
    float scs[16], bs = -std::numeric_limits<float>::infinity();
    int best = 0;
    for (int j = 0; j < 16; ++j) {
      double e = 0;
      for (int q = 0; q < d.rank; ++q)
        e += double(or_bf16_to_f32(r->pred[size_t(prev) * d.rank + q])) * hp[size_t(t) * d.rank + q] *
             or_bf16_to_f32(r->succ[size_t(ids[j]) * d.rank + q]);
      scs[j] = lr[ids[j]] + float(e);
      if (scs[j] > bs) { bs = scs[j]; best = j; }
    }
    drafts[t] = uint32_t(ids[best]);
    float z = 0;
    for (int j = 0; j < 16; ++j) z += std::exp((scs[j] - bs) / 1.5f);
    conf[t] = 1.0f / z;
    prev = drafts[t];
  }
}

}  // extern "C"
