// Device helpers shared by the kernels that produce qmm activations (the fragment layout of ih_internal.h) and by
// the synthetic-data generators.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace ih {

__device__ __forceinline__ float dbf16(unsigned v16) { return __uint_as_float(v16 << 16); }

__device__ __forceinline__ unsigned short dround_bf16(float f) {
  unsigned u = __float_as_uint(f);
  return (unsigned short)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Writes one 8-value chunk c (values x[8c … 8c+7] of token `tok`, already final fp32) into the fragment layout as
// bf16, and the 64-value group sums. The 8 chunks of a group must be held by 8 consecutive lanes (lane & 7 = c & 7),
// all lanes of the wave calling together; `valid` false gives zeros.
__device__ __forceinline__ void act_store_chunk(uint4* frag, float* xsum, int nkb, int tok, int c, const float (&v)[8],
                                                bool valid, int max_tok) {
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = valid ? dbf16(dround_bf16(v[e])) : 0.f;
  float sum = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  if (c < nkb * 16) {
    const int kb = c >> 4, w = c & 15, t = w >> 2, qd = w & 3;
    unsigned u[4];
    u[0] = dround_bf16(r[0]) | (unsigned(dround_bf16(r[4])) << 16);
    u[1] = dround_bf16(r[1]) | (unsigned(dround_bf16(r[5])) << 16);
    u[2] = dround_bf16(r[2]) | (unsigned(dround_bf16(r[6])) << 16);
    u[3] = dround_bf16(r[3]) | (unsigned(dround_bf16(r[7])) << 16);
    frag[((size_t(tok) * nkb + kb) * 4 + qd) * 4 + t] = make_uint4(u[0], u[1], u[2], u[3]);
    if ((c & 7) == 0) xsum[(c >> 3) * max_tok + tok] = sum;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Synthetic data: SplitMix64 streams keyed by (seed, tensor id). h(key, i) is output i of SplitMix64 seeded with key
// (Sources/Ingot/Sampling.swift:50-62 is the reference's generator).
__host__ __device__ __forceinline__ uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t sm_key(uint64_t seed, uint64_t tensor) {
  return sm_mix(seed * 0x9E3779B97F4A7C15ull + sm_mix(tensor + 0x632BE59BD9B4E019ull));
}
__host__ __device__ __forceinline__ uint64_t sm_at(uint64_t key, uint64_t i) {
  return sm_mix(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}
// Approximately N(0, 1): sum of the four 16-bit fields of one output, centred and scaled to unit variance (exact
// integer sum, one rounding), so CPU and GPU produce the same float.
__host__ __device__ __forceinline__ float sm_normal(uint64_t key, uint64_t i) {
  const uint64_t h = sm_at(key, i);
  const int s = int(h & 0xFFFF) + int((h >> 16) & 0xFFFF) + int((h >> 32) & 0xFFFF) + int(h >> 48) - 131070;
  return float(s) * 2.642936E-05f;  // sqrt(3) / 65536
}

}  // namespace ih
