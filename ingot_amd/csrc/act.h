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

// Fragment layout (ih_internal.h): 16-byte unit of (K-block kb, token tok, MFMA step t, lane group qd) in a buffer of
// ntile 16-token tiles. One (kb, tile, t) is 1024 contiguous bytes [token 16][qd 4][8 values]: the A operand of one
// MFMA step for a whole wave, read as one coalesced dwordx4 load.
__device__ __forceinline__ size_t frag_index(int ntile, int kb, int tok, int t, int qd) {
  return ((size_t(kb) * ntile + (tok >> 4)) * 4 + t) * 64 + (tok & 15) * 4 + qd;
}

// Writes one 8-value chunk c (values x[8c … 8c+7] of token `tok`, final fp32) into the fragment layout as bf16.
__device__ __forceinline__ void frag_store_chunk(uint4* frag, int nkb, int ntile, int tok, int c, const float (&v)[8]) {
  if (c >= nkb * 16) return;
  const int kb = c >> 4, w = c & 15, t = w >> 2, qd = w & 3;
  uint4 u;
  u.x = dround_bf16(v[0]) | (unsigned(dround_bf16(v[4])) << 16);
  u.y = dround_bf16(v[1]) | (unsigned(dround_bf16(v[5])) << 16);
  u.z = dround_bf16(v[2]) | (unsigned(dround_bf16(v[6])) << 16);
  u.w = dround_bf16(v[3]) | (unsigned(dround_bf16(v[7])) << 16);
  frag[frag_index(ntile, kb, tok, t, qd)] = u;
}

// The same chunk as fp16 (round to nearest even): the activation of MXFP4 experts, whose MFMA runs in fp16.
__device__ __forceinline__ void frag_store_chunk_f16(uint4* frag, int nkb, int ntile, int tok, int c,
                                                     const float (&v)[8]) {
  if (c >= nkb * 16) return;
  const int kb = c >> 4, w = c & 15, t = w >> 2, qd = w & 3;
  auto h = [](float f) { return unsigned(__half_as_ushort(__float2half_rn(f))); };
  uint4 u;
  u.x = h(v[0]) | (h(v[4]) << 16);
  u.y = h(v[1]) | (h(v[5]) << 16);
  u.z = h(v[2]) | (h(v[6]) << 16);
  u.w = h(v[3]) | (h(v[7]) << 16);
  frag[frag_index(ntile, kb, tok, t, qd)] = u;
}

__device__ __forceinline__ void frag_store(bool f16, uint4* frag, int nkb, int ntile, int tok, int c,
                                           const float (&v)[8]) {
  if (f16) frag_store_chunk_f16(frag, nkb, ntile, tok, c, v);
  else frag_store_chunk(frag, nkb, ntile, tok, c, v);
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
