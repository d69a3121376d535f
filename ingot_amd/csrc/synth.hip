// Synthetic weights and KV of the benchmark configurations (benchmark configurations: random int4 weights, N(0,1) int8 KV),
// generated on the GPU from counter-based SplitMix64 streams (act.h) so that any element is a pure function of
// (seed, tensor id, index) and the CPU oracle regenerates the same bits.
//
//   int4 codes   word j of a tensor = 32-bit half (j & 1) of h(key_w, j >> 1)            (uniform nibbles 0..15)
//   scales       bf16(|n(key_s, g)| · sd), n ≈ N(0,1) (act.h sm_normal), biases bf16(−8 · scale)  (benchmark configuration 0)
//   mxfp4        codes as int4; e8m0 scale of group g = 119 + h(key_s, g) mod 7      (2^-8 … 2^-2, benchmark configuration 4)
//   norm weights bf16(1 + 0.125 · n(key, i))
//   KV           per (head, position): x_d = n(key, ((head << 24) + pos) · HD + d), symmetric int8 with fp16 scale
//                sc = fp16(amax / 127) (1 when amax = 0), q = clamp(rint(x / sc), ±127)
#include "act.h"
#include "attn_args.h"
#include "ih_internal.h"

namespace ih {

__global__ void synth_int4_kernel(uint32_t* w, uint16_t* s, uint16_t* b, size_t nwords, size_t ngroups, uint64_t kw,
                                  uint64_t ks, float sd) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nwords; i += stride) {
    const uint64_t h = sm_at(kw, i >> 1);
    w[i] = uint32_t((i & 1) ? (h >> 32) : h);
  }
  for (size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x; g < ngroups; g += stride) {
    const float sc = fabsf(sm_normal(ks, g)) * sd;
    const unsigned short sb = dround_bf16(sc);
    s[g] = sb;
    b[g] = dround_bf16(-8.0f * dbf16(sb));
  }
}

__global__ void synth_mxfp4_kernel(uint32_t* w, uint8_t* s, size_t nwords, size_t ngroups, uint64_t kw, uint64_t ks) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nwords; i += stride) {
    const uint64_t h = sm_at(kw, i >> 1);
    w[i] = uint32_t((i & 1) ? (h >> 32) : h);
  }
  for (size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x; g < ngroups; g += stride)
    s[g] = uint8_t(119 + sm_at(ks, g) % 7);
}

__global__ void synth_bf16_kernel(uint16_t* out, size_t n, uint64_t key, float base, float amp) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = dround_bf16(base + amp * sm_normal(key, i));
}

__global__ void synth_f32_kernel(float* out, size_t n, uint64_t key, float base, float amp) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = base + amp * sm_normal(key, i);
}

// One block per (position, KV head): HD threads (64 or 128). K of the cache layout [head][slot][HD] int8, V transposed
// [head][HD][vld] (v_index), and the fp16 scales [head][slot].
__global__ void synth_kv_kernel(int8_t* kc, int8_t* vc, __half* ks, __half* vs, int HD, int cap, int ring, int pos0,
                                uint64_t kk, uint64_t kv) {
  __shared__ float red[4];
  const int pos = pos0 + blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int slot = ring ? pos % ring : pos;
  for (int which = 0; which < 2; ++which) {
    const uint64_t key = which ? kv : kk;
    const float x = sm_normal(key, ((uint64_t(h) << 24) + uint64_t(pos)) * HD + d);
    float a = fabsf(x);
    for (int o = 32; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
    __syncthreads();
    if ((d & 63) == 0) red[d >> 6] = a;
    __syncthreads();
    float amax = red[0];
    for (int i = 1; i < HD / 64; ++i) amax = fmaxf(amax, red[i]);
    const __half sc16 = __float2half_rn(amax > 0.f ? amax / 127.0f : 1.0f);
    const float sc = __half2float(sc16);
    const float q = fminf(127.f, fmaxf(-127.f, rintf(x / sc)));
    if (which) vc[v_index(h, slot, d, HD, v_row(cap))] = int8_t(q);
    else kc[(size_t(h) * cap + slot) * HD + d] = int8_t(q);
    if (d == 0) (which ? vs : ks)[size_t(h) * cap + slot] = sc16;
  }
}

static unsigned grid_for(size_t n) { return unsigned(std::min<size_t>((n + 255) / 256, 8192)); }

int synth_int4(ih_ctx* c, uint32_t* w, uint16_t* s, uint16_t* b, size_t N, size_t K, uint64_t seed, uint64_t tensor,
               float sd) {
  const size_t nw = N * K / 8, ng = N * K / 64;
  synth_int4_kernel<<<grid_for(nw), 256, 0, c->stream>>>(w, s, b, nw, ng, sm_key(seed, 2 * tensor),
                                                         sm_key(seed, 2 * tensor + 1), sd);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int synth_mxfp4(ih_ctx* c, uint32_t* w, uint8_t* s, size_t N, size_t K, uint64_t seed, uint64_t tensor) {
  const size_t nw = N * K / 8, ng = N * K / 32;
  synth_mxfp4_kernel<<<grid_for(nw), 256, 0, c->stream>>>(w, s, nw, ng, sm_key(seed, 2 * tensor),
                                                          sm_key(seed, 2 * tensor + 1));
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int synth_bf16(ih_ctx* c, uint16_t* out, size_t n, uint64_t seed, uint64_t tensor, float base, float amp) {
  synth_bf16_kernel<<<grid_for(n), 256, 0, c->stream>>>(out, n, sm_key(seed, 2 * tensor), base, amp);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int synth_f32(ih_ctx* c, float* out, size_t n, uint64_t seed, uint64_t tensor, float base, float amp) {
  synth_f32_kernel<<<grid_for(n), 256, 0, c->stream>>>(out, n, sm_key(seed, 2 * tensor), base, amp);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int synth_kv(ih_ctx* c, int8_t* kc, int8_t* vc, __half* ks, __half* vs, int KVH, int HD, int cap, int ring, int pos0,
             int npos, uint64_t seed, uint64_t tensor) {
  if (npos <= 0) return IH_OK;
  dim3 grid(npos, KVH);
  synth_kv_kernel<<<grid, HD, 0, c->stream>>>(kc, vc, ks, vs, HD, cap, ring, pos0, sm_key(seed, 2 * tensor),
                                              sm_key(seed, 2 * tensor + 1));
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih
