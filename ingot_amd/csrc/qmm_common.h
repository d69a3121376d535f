// Device helpers shared by the quantized-matmul kernels (qmm.hip: dense int4; moe.hip: MXFP4 and gathered experts).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

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

}  // namespace ih
