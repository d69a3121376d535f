// Verify-block attention over the int8 KV cache on gfx950: prework (RoPE, Hadamard, int8 K/V write), split-key
// flash-decoding on MFMA, and the fixed-order reduction of the splits.
//
// Reference: AttentionLayer.encode pieces prework → attn → reduce (Sources/Ingot/Layers/Attention.swift:398-525);
// kernels vattn_prework_i8 (Shaders/verify_attn_nax.metal:47-146), pattn_i8<RG, DEC=true> (Shaders/verify_attn_pf.metal:
// 49-398) and vattn_reduce (Shaders/verify_attn.metal:149-192).
//
// Cache layout (this build): K and V int8 [KV head][slot][HD] (key-major, 128-byte rows), scales fp16 [KV head][slot]
// (per token and head, symmetric). K holds H·k (orthonormal Walsh–Hadamard of the roped key) when hadk is set, and q is
// rotated the same way, so (Hq)·(Hk) = q·k.
//
// MI355X design: one workgroup per (key split, KV head, query group) with 4 waves. Each 32-key block of the split is
// read once by the workgroup, converted int8 → fp16 exactly into LDS (K key-major, V transposed), and every wave runs
// its 16-query tiles over it: Sᵀ = K·Qᵀ (v_mfma_f32_16x16x32_f16, keys as rows so each lane holds 4 keys of one query),
// online softmax in base 2 per query column, P stays in registers as the B operand of Oᵀ += Vᵀ·Pᵀ. A query's result
// does not depend on the other rows of the block: blocks start at fixed key positions, the split boundaries are fixed
// multiples of C, and the splits are combined in split order.
#include <hip/hip_fp16.h>

#include "act.h"
#include "attn_args.h"
#include "ih_internal.h"

namespace ih {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// AttnArgs: attn_args.h.

// ---------------------------------------------------------------------------------------------------------------
// Prework: grid (QH + 2·KVH, B), HD threads. vattn_prework_i8 (verify_attn_nax.metal:47-146) without QK-norm and gate
// (the configurations have neither): RoPE on all HD dims (non-interleaved halves, angle pos·θ^(−i/(HD/2)) evaluated in
// double), orthonormal WHT (Sylvester order, stages 1, 2, 4, …, then ×1/√HD) of q and k, int8 quantisation of k and v
// per (token, head): sc = fp16(amax/127) (1 when amax = 0), q = clamp(rint(x/sc), ±127), written at slot P + t.
__global__ void prework_kernel(AttnArgs a) {
  __shared__ float xs[256];
  __shared__ float red[4];
  const int slot = blockIdx.x, t = blockIdx.y, d = threadIdx.x, HD = a.HD;
  int col;
  if (slot < a.QH) col = slot * HD + d;
  else if (slot < a.QH + a.KVH) col = a.QH * HD + (slot - a.QH) * HD + d;
  else col = (a.QH + a.KVH) * HD + (slot - a.QH - a.KVH) * HD + d;
  float x = a.proj[size_t(t) * a.ldp + col];
  const int pos = a.P + t;
  const int kpos = a.ring ? pos % a.ring : pos;
  if (slot < a.QH + a.KVH) {
    xs[d] = x;
    __syncthreads();
    const int RH = HD / 2, i = d % RH;
    const double ang = double(pos) * pow(double(a.theta), -double(i) / double(RH));
    const float cs = float(cos(ang)), sn = float(sin(ang));
    x = d < RH ? x * cs - xs[d + RH] * sn : x * cs + xs[d - RH] * sn;
    if (a.hadk) {
      for (int h = 1; h < HD; h <<= 1) {
        __syncthreads();
        xs[d] = x;
        __syncthreads();
        const float o = xs[d ^ h];
        x = (d & h) ? o - x : x + o;
      }
      x *= HD == 128 ? 0.088388347648318441f : (HD == 64 ? 0.125f : 0.0625f);
    }
    if (slot < a.QH) {
      const int kvh = slot / a.G;
      a.q[(size_t(kvh) * a.Qpad + t * a.G + slot % a.G) * HD + d] = __float2half_rn(x);
      return;
    }
  }
  // K or V: symmetric int8 with one fp16 scale per (token, head).
  float am = fabsf(x);
  for (int o = 32; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
  if ((d & 63) == 0) red[d >> 6] = am;
  __syncthreads();
  float amax = red[0];
  for (int w = 1; w < HD / 64; ++w) amax = fmaxf(amax, red[w]);
  const __half sc16 = __float2half_rn(amax > 0.f ? amax / 127.0f : 1.0f);
  const float sc = __half2float(sc16);
  const int8_t qv = int8_t(fminf(127.f, fmaxf(-127.f, rintf(x / sc))));
  const bool isk = slot < a.QH + a.KVH;
  const int h = isk ? slot - a.QH : slot - a.QH - a.KVH;
  (isk ? a.kc : a.vc)[(size_t(h) * a.cap + kpos) * HD + d] = qv;
  if (d == 0) (isk ? a.ks : a.vs)[size_t(h) * a.cap + kpos] = sc16;
}

// ---------------------------------------------------------------------------------------------------------------
// Four signed bytes → four exact fp16 values: bytes ^ 0x80 are u = v + 128 ∈ [1, 255]; interleaved with the byte 0x64
// they read as the halves 1024 + u; minus 1152 gives v.
__device__ __forceinline__ void i8x4_to_h(unsigned w, __half2& lo, __half2& hi) {
  const unsigned x = w ^ 0x80808080u;
  const unsigned l = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
  const unsigned h = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
  const __half2 off = __halves2half2(__float2half(1152.f), __float2half(1152.f));
  lo = __hsub2(__builtin_bit_cast(__half2, l), off);
  hi = __hsub2(__builtin_bit_cast(__half2, h), off);
}

constexpr int KROW = 128 + 8;  // LDS row of K in halves (HD ≤ 128, padded)
constexpr int VROW = 32 + 8;   // LDS row of Vᵀ in halves

// Slot of key k (0…31) in a 32-key block of Vᵀ: the PV MFMA pairs lane group qd's element e with key 4·qd + e (e < 4,
// first 16-key tile) or 16 + 4·qd + e − 4 (second tile): the keys each lane holds after the Sᵀ MFMAs.
__device__ __forceinline__ int vslot(int k) { return k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3); }

// K/V of one 32-key block in flight: per thread one 16-byte K item (key, 16 dims) and one V item (key pair, 8 dims:
// 8 bytes of each key), so V can be written transposed as 32-bit key pairs.
template <int HD>
struct KVStage {
  uint4 k;
  uint2 v0, v1;
  float ks, vs;
};

template <int HD>
__global__ __launch_bounds__(512) void attn_kernel(AttnArgs a) {
  constexpr int NC = HD / 32;           // 32-dim chunks (MFMA K steps of Sᵀ)
  constexpr int NDT = HD / 16;          // 16-dim tiles of Oᵀ
  constexpr int KITEMS = 32 * HD / 16;  // 16-byte K items of a block
  constexpr int VITEMS = 16 * HD / 8;   // (key pair, 8 dims) V items of a block
  __shared__ _Float16 Kf[32 * KROW];
  __shared__ _Float16 Vt[HD * VROW];
  __shared__ float ksf[32], vsf[32];

  // Partials are stored by launched split (blockIdx.x); the key range is that of split blockIdx.x + s0 (a sliding
  // window does not launch the splits that end before the first row's window).
  const int sidx = blockIdx.x, split = sidx + a.s0, kvh = blockIdx.y;
  const int nthreads = blockDim.x, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, j = lane & 15, qd = lane >> 4;
  const int Q = a.G * a.B;
  const int k0 = split * a.C, k1 = min(k0 + a.C, a.P + a.B);

  // One 16-query tile per wave.
  const int qt = blockIdx.z * (nthreads >> 6) + wave;
  const bool qlive = 16 * qt < Q;
  const int m = 16 * qt + j;
  f16x8 qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (qlive && m < Q) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(a.q + (size_t(kvh) * a.Qpad + m) * HD + 32 * c + 8 * qd);
      qf[c] = __builtin_bit_cast(f16x8, v);
    } else {
      qf[c] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  f32x4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lsum = 0.f;
  const int tok = m / a.G;
  const int lim = a.P + tok;  // last visible key (causal)
  const int lo_key = a.window > 0 ? lim - a.window + 1 : -2147483647;

  const int8_t* kh = a.kc + size_t(kvh) * a.cap * HD;
  const int8_t* vh = a.vc + size_t(kvh) * a.cap * HD;
  const __half* ksh = a.ks + size_t(kvh) * a.cap;
  const __half* vsh = a.vs + size_t(kvh) * a.cap;
  auto slot_of = [&](int key) { return a.ring ? key % a.ring : key; };

  // Loader items of this thread (at most one K and one V item, since blockDim ≥ 256 for HD 128 and ≥ 128 for 64
  // is not guaranteed: threads beyond the item count load nothing).
  const bool hask = tid < KITEMS, hasv = tid < VITEMS;
  const int kkey = tid / (HD / 16), kcol = (tid % (HD / 16)) * 16;
  const int vpair = tid / (HD / 8), vcol = (tid % (HD / 8)) * 8;
  KVStage<HD> st;
  auto load = [&](int kb) {
    if (hask) {
      const int key = kb + kkey;
      st.k = key < k1 ? *reinterpret_cast<const uint4*>(kh + size_t(slot_of(key)) * HD + kcol) : make_uint4(0, 0, 0, 0);
    }
    if (hasv) {
      const int key0 = kb + 2 * vpair, key1 = key0 + 1;
      st.v0 = key0 < k1 ? *reinterpret_cast<const uint2*>(vh + size_t(slot_of(key0)) * HD + vcol) : make_uint2(0, 0);
      st.v1 = key1 < k1 ? *reinterpret_cast<const uint2*>(vh + size_t(slot_of(key1)) * HD + vcol) : make_uint2(0, 0);
    }
    if (tid < 32) {
      const int key = kb + tid;
      st.ks = key < k1 ? __half2float(ksh[slot_of(key)]) * a.scale_log2 : 0.f;
      st.vs = key < k1 ? __half2float(vsh[slot_of(key)]) : 0.f;
    }
  };
  auto store = [&]() {
    if (hask) {
      const unsigned kw[4] = {st.k.x, st.k.y, st.k.z, st.k.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __half2 lo, hi;
        i8x4_to_h(kw[i], lo, hi);
        *reinterpret_cast<__half2*>(&Kf[kkey * KROW + kcol + 4 * i]) = lo;
        *reinterpret_cast<__half2*>(&Kf[kkey * KROW + kcol + 4 * i + 2]) = hi;
      }
    }
    if (hasv) {
      // Keys 2·vpair and 2·vpair + 1 occupy adjacent slots: one 32-bit (key pair) store per dim.
      const int sl = vslot(2 * vpair);
      const unsigned a0[2] = {st.v0.x, st.v0.y}, a1[2] = {st.v1.x, st.v1.y};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        __half2 l0, h0, l1, h1;
        i8x4_to_h(a0[i], l0, h0);
        i8x4_to_h(a1[i], l1, h1);
        const int d = vcol + 4 * i;
        *reinterpret_cast<__half2*>(&Vt[(d + 0) * VROW + sl]) = __halves2half2(__low2half(l0), __low2half(l1));
        *reinterpret_cast<__half2*>(&Vt[(d + 1) * VROW + sl]) = __halves2half2(__high2half(l0), __high2half(l1));
        *reinterpret_cast<__half2*>(&Vt[(d + 2) * VROW + sl]) = __halves2half2(__low2half(h0), __low2half(h1));
        *reinterpret_cast<__half2*>(&Vt[(d + 3) * VROW + sl]) = __halves2half2(__high2half(h0), __high2half(h1));
      }
    }
    if (tid < 32) {
      ksf[tid] = st.ks;
      vsf[tid] = st.vs;
    }
  };

  if (k0 < k1) load(k0);
  for (int kb = k0; kb < k1; kb += 32) {
    __syncthreads();  // the previous block's readers are done with LDS
    store();
    __syncthreads();
    if (kb + 32 < k1) load(kb + 32);  // next block in flight during this one's products
    if (!qlive) continue;             // uniform per wave
    // Sᵀ for the two 16-key tiles: lane (j, qd) holds keys 16h + 4qd + r of query m.
    f32x4 sacc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sacc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f16x8 kf = *reinterpret_cast<const f16x8*>(&Kf[(16 * h + j) * KROW + 32 * c + 8 * qd]);
        sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[c], sacc[h], 0, 0, 0);
      }
    }
    float s[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = 16 * h + 4 * qd + r, key = kb + kk;
        const bool vis = m < Q && key < k1 && key <= lim && key >= lo_key;
        s[h][r] = vis ? sacc[h][r] * ksf[kk] : -INFINITY;
        mx = fmaxf(mx, s[h][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(mrun, mx);
    const float alpha = mnew == -INFINITY ? 1.f : exp2f(mrun - mnew);
    mrun = mnew;
    float ps = 0.f;
    f16x8 pb;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = s[h][r] == -INFINITY ? 0.f : exp2f(s[h][r] - mnew);
        ps += p;
        pb[4 * h + r] = (_Float16)(p * vsf[16 * h + 4 * qd + r]);
      }
    lsum = lsum * alpha + ps;
    // Rescale Oᵀ only when some column's maximum moved (alpha = 1 is exact and is skipped).
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const f16x8 vf = *reinterpret_cast<const f16x8*>(&Vt[(16 * dt + j) * VROW + 8 * qd]);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb, o[dt], 0, 0, 0);
    }
  }

  // Partials of this split: (max, sum) per query and the unnormalised Oᵀ (lane holds dims 16dt + 4qd + r of query m).
  if (!qlive) return;
  float l = lsum;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (m >= Q) return;
  const size_t base = (size_t(kvh) * a.nsplit + sidx) * a.Qpad;
  if (qd == 0) a.ml[base + m] = make_float2(mrun, l);
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
    *reinterpret_cast<f32x4*>(a.opart + (base + m) * HD + 16 * dt + 4 * qd) = o[dt];
}

// ---------------------------------------------------------------------------------------------------------------
// Reduction of the splits (vattn_reduce, verify_attn.metal:149-192): M = max over splits (and the sink), L = Σ e^(m−M)·l
// (+ e^(sink−M)), o = Σ e^(m−M)·O / L, in split order; written into the o_proj activation layout (column h·HD + d).
// Grid (B, QH·HD/512), 64 threads (one per 8 values).
__global__ __launch_bounds__(64) void attn_reduce_kernel(AttnArgs a, uint4* __restrict__ frag, int nkb) {
  const int t = blockIdx.x, c = blockIdx.y * 64 + threadIdx.x, HD = a.HD;
  const int h = (8 * c) / HD, d0 = (8 * c) % HD;
  const int kvh = h / a.G, m = t * a.G + h % a.G;
  const float2* mlh = a.ml + size_t(kvh) * a.nsplit * a.Qpad + m;
  float M = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, mlh[size_t(s) * a.Qpad].x);
  float L = 0.f;
  if (a.sinks) {
    const float sk = a.sinks[h] * 1.4426950408889634f;
    M = fmaxf(M, sk);
    L = exp2f(sk - M);
  }
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll 4
  for (int s = 0; s < a.nsplit; ++s) {
    const size_t idx = (size_t(kvh) * a.nsplit + s) * a.Qpad + m;
    const float2 v = a.ml[idx];
    const f32x4* src = reinterpret_cast<const f32x4*>(a.opart + idx * HD + d0);
    const f32x4 p0 = src[0], p1 = src[1];
    // An empty split carries (−inf, 0) and a zero O: its weight is 0.
    const float w = v.x == -INFINITY ? 0.f : exp2f(v.x - M);
    L += w * v.y;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] += w * p0[e];
      o[4 + e] += w * p1[e];
    }
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] *= inv;
  frag_store_chunk(frag, nkb, t, c, o);
}

int launch_prework(ih_ctx* c, const AttnArgs& a) {
  TimedLaunch tl(c, TC_PREWORK, double(a.B) * (a.QH + 2 * a.KVH) * a.HD * 4 + double(a.B) * a.KVH * (2 * a.HD + 4) +
                                    double(a.B) * a.QH * a.HD * 2);
  dim3 grid(a.QH + 2 * a.KVH, a.B);
  prework_kernel<<<grid, a.HD, 0, c->stream>>>(a);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_attention(ih_ctx* c, const AttnArgs& a) {
  const int Q = a.G * a.B;
  const int qtiles = (Q + 15) / 16;
  const int nz = (qtiles + 7) / 8;        // query groups of ≤ 8 tiles, one wave per tile
  const int waves = (qtiles + nz - 1) / nz;
  // The block loader needs 32·HD/16 threads (256 for HD 128, 128 for HD 64).
  const int threads = std::max(64 * waves, a.HD * 2);
  dim3 grid(a.nsplit, a.KVH, nz);
  // Algorithmic bytes: the int8 K and V and their fp16 scales of every key the launched splits cover, and q.
  const double keys = double(a.P + a.B) - double(a.s0) * a.C;
  TimedLaunch tl(c, TC_ATTN, double(a.KVH) * keys * (2 * a.HD + 4) + double(a.KVH) * Q * a.HD * 2);
  if (a.HD == 128) attn_kernel<128><<<grid, threads, 0, c->stream>>>(a);
  else if (a.HD == 64) attn_kernel<64><<<grid, threads, 0, c->stream>>>(a);
  else return fail(IH_EINVAL, "attention: head_dim must be 64 or 128");
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_attn_reduce(ih_ctx* c, const AttnArgs& a, ActBuf& out) {
  IH_CHECK((a.QH * a.HD) % 512 == 0, IH_EINVAL, "attention reduce: QH·HD must be a multiple of 512");
  TimedLaunch tl(c, TC_REDUCE, double(a.KVH) * a.nsplit * a.G * a.B * (a.HD + 2) * 4 + double(a.B) * a.QH * a.HD * 2);
  attn_reduce_kernel<<<dim3(a.B, a.QH * a.HD / 512), 64, 0, c->stream>>>(a, static_cast<uint4*>(out.frag), out.nkb);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih
