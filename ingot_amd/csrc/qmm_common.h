// Device helpers shared by the quantized-matmul kernels (qmm.hip: dense int4; moe.hip: MXFP4 and gathered experts).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#include "lanes.h"

namespace ih {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16f(unsigned v16) { return __uint_as_float(v16 << 16); }

__device__ __forceinline__ unsigned short f2bf(float f) {
  unsigned u = __float_as_uint(f);
  return (unsigned short)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// (w & km) | kb. With km in a VGPR (see vgpr_of) and kb in an SGPR, LLVM selects one v_and_or_b32 (gfx9 VOP3 reads at
// most one scalar operand and no literal). The instruction is not written as inline assembly: the hazard recognizer
// does not see into asm blocks, and an asm v_and_or_b32 feeding the MFMA operands produced wrong results.
__device__ __forceinline__ unsigned and_or(unsigned w, unsigned km, unsigned kb) { return (w & km) | kb; }

// A uniform value copied into a VGPR once (an opaque move, so the compiler keeps it in a vector register).
__device__ __forceinline__ unsigned vgpr_of(unsigned s) {
  unsigned v;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "s"(s));
  return v;
}

// Eight nibbles of one word → eight bf16 values 128 + q in the element order {0,4,1,5,2,6,3,7}. km = 0x000F000F,
// kb = 0x43004300 (runtime values, see QmmParams).
__device__ __forceinline__ bf16x8 nib_bf16(unsigned w, unsigned km, unsigned kb) {
  u32x4 v;
  v.x = and_or(w, km, kb);
  v.y = and_or(w >> 4, km, kb);
  v.z = and_or(w >> 8, km, kb);
  v.w = and_or(w >> 12, km, kb);
  return __builtin_bit_cast(bf16x8, v);
}

// Two words of one group → their sixteen bf16 values (nib_bf16 of each): the three shifts of both words are three
// 64-bit shifts of the pair (the low word's top bits, which the shifted pair fills from the high word, are masked
// off), 11 instructions instead of 14. The shift amounts sh = {4, 8, 12} come in VGPRs (vgpr_of): with a constant
// amount the compiler splits a 64-bit shift into two 32-bit instructions.
__device__ __forceinline__ void nib_bf16_pair(unsigned wa, unsigned wb, unsigned km, unsigned kb, const unsigned (&sh)[3],
                                              bf16x8& a, bf16x8& b) {
  const uint64_t p = (uint64_t(wb) << 32) | wa;
  const uint64_t s4 = p >> sh[0], s8 = p >> sh[1], s12 = p >> sh[2];
  u32x4 va, vb;
  va.x = and_or(wa, km, kb);
  va.y = and_or(unsigned(s4), km, kb);
  va.z = and_or(unsigned(s8), km, kb);
  va.w = and_or(unsigned(s12), km, kb);
  vb.x = and_or(wb, km, kb);
  vb.y = and_or(unsigned(s4 >> 32), km, kb);
  vb.z = and_or(unsigned(s8 >> 32), km, kb);
  vb.w = and_or(unsigned(s12 >> 32), km, kb);
  a = __builtin_bit_cast(bf16x8, va);
  b = __builtin_bit_cast(bf16x8, vb);
}

// Buffer resources (base in SGPRs, 32-bit offsets; an offset past num_records reads as zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr unsigned OOB = 0x80000000u;  // offset that reads as zero

// Gated activation (lab_glu, Sources/Ingot/Shaders/qmm.metal:18-30): act 0 = SiLU(g)·u; act 1 = swiglu_oai,
// (clip(u, ±limit) + 1)·g'·σ(1.702·g') with g' = min(g, limit) (CPU.swigluOAI, Tests/IngotTests/KernelHarness.swift:
// 183-188).
__device__ __forceinline__ float glu_f(float g, float u, int act, float limit) {
  if (act == 0) return g / (1.0f + expf(-g)) * u;
  const float gc = fminf(g, limit), uc = fminf(fmaxf(u, -limit), limit);
  return gc / (1.0f + expf(-1.702f * gc)) * (uc + 1.0f);
}

// RMSNorm factors of M ≤ 32 activation rows from the producers' sum-of-squares partials, token-major with leading
// dimension ld (ss_in[t·ld + j], j < nss ≤ ld, ld a multiple of 256): rsc[t] = 1/sqrt(Σ_j ss_in[t][j] / D + eps).
// Wave w of nwaves takes rows w, w + nwaves, …; lane l adds partials 4l … 4l+3, then 256 + 4l …, in order, and the
// lanes are combined by a fixed butterfly, so a row's factor depends neither on M nor on the caller's launch shape.
// One 16-byte load per lane covers 256 partials of a row. Split in two so that a kernel can issue the first chunk of
// its rows (NR per wave) at entry and finish after its main loop: the partials were just written by another kernel,
// and their latency then hides under the weight stream.
typedef float f32x4v __attribute__((ext_vector_type(4)));
template <int NR>  // rows per wave
struct RmsPrefetch {
  f32x4v v[NR];
};
template <int NR>
__device__ __forceinline__ void rms_prefetch(RmsPrefetch<NR>& pf, const float* __restrict__ ss_in, int ld, int M,
                                             int wave, int nwaves, int lane) {
  const int nt = (M - wave + nwaves - 1) / nwaves;  // rows of this wave (wave-uniform, at most NR)
#pragma unroll
  for (int k = 0; k < NR; ++k)
    if (k < nt) pf.v[k] = *reinterpret_cast<const f32x4v*>(ss_in + size_t(wave + k * nwaves) * ld + 4 * lane);
}
template <int NR>
__device__ __forceinline__ void rms_finish(const RmsPrefetch<NR>& pf, const float* __restrict__ ss_in, int ld, int nss,
                                           int D, float eps, int M, float* rsc, int wave, int nwaves, int lane) {
  const int nt = (M - wave + nwaves - 1) / nwaves;
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    if (k >= nt) break;
    float ss = 0.f;
    for (int j0 = 0; j0 < nss; j0 += 256) {
      const int j = j0 + 4 * lane;
      const f32x4v v =
          j0 == 0 ? pf.v[k] : *reinterpret_cast<const f32x4v*>(ss_in + size_t(wave + k * nwaves) * ld + j);
      ss += j < nss ? v[0] : 0.f;
      ss += j + 1 < nss ? v[1] : 0.f;
      ss += j + 2 < nss ? v[2] : 0.f;
      ss += j + 3 < nss ? v[3] : 0.f;
    }
    ss += lane_xor<32>(ss);
    ss += lane_xor<16>(ss);
    ss += lane_xor<8>(ss);
    ss += lane_xor<4>(ss);
    ss += lane_xor<2>(ss);
    ss += lane_xor<1>(ss);
    if (lane == 0) rsc[wave + k * nwaves] = 1.0f / sqrtf(ss / float(D) + eps);
  }
}
// Both halves at once, rows in groups of eight (callers without a main loop to hide the latency under).
__device__ __forceinline__ void rms_factors(const float* __restrict__ ss_in, int ld, int nss, int D, float eps, int M,
                                            float* rsc, int wave, int nwaves, int lane) {
  const int nt = (M - wave + nwaves - 1) / nwaves;
  for (int k0 = 0; k0 < nt; k0 += 8) {
    // Rows wave + (k0 + k)·nwaves, k < 8: the same function on the rows from k0·nwaves on.
    const float* base = ss_in + size_t(k0) * nwaves * ld;
    const int Mk = M - k0 * nwaves;
    RmsPrefetch<8> pf;
    rms_prefetch(pf, base, ld, Mk, wave, nwaves, lane);
    rms_finish(pf, base, ld, nss, D, eps, Mk, rsc + k0 * nwaves, wave, nwaves, lane);
  }
}

}  // namespace ih
