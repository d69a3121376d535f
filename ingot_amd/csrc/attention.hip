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

template <int HD>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  constexpr int NC = HD / 32;    // 32-dim chunks (MFMA K steps of Sᵀ)
  constexpr int NDT = HD / 16;   // 16-dim tiles of Oᵀ
  constexpr int QTW = 2;         // query tiles per wave (8 per workgroup)
  __shared__ _Float16 Kf[32 * KROW];
  __shared__ _Float16 Vt[HD * VROW];
  __shared__ float ksf[32], vsf[32];

  // Partials are stored by launched split (blockIdx.x); the key range is that of split blockIdx.x + s0 (a sliding
  // window does not launch the splits that end before the first row's window).
  const int sidx = blockIdx.x, split = sidx + a.s0, kvh = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15, qd = lane >> 4;
  const int Q = a.G * a.B;
  const int kend_all = a.P + a.B;
  const int k0 = split * a.C, k1 = min(k0 + a.C, kend_all);

  // This wave's query tiles.
  int qt[QTW];
  bool qlive[QTW];
#pragma unroll
  for (int u = 0; u < QTW; ++u) {
    qt[u] = blockIdx.z * 4 * QTW + wave + 4 * u;
    qlive[u] = 16 * qt[u] < Q;
  }
  f16x8 qf[QTW][NC];
  f32x4 o[QTW][NDT];
  float mrun[QTW], lsum[QTW];
#pragma unroll
  for (int u = 0; u < QTW; ++u) {
    mrun[u] = -INFINITY;
    lsum[u] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[u][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int m = 16 * qt[u] + j;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (qlive[u] && m < Q) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(a.q + (size_t(kvh) * a.Qpad + m) * HD + 32 * c + 8 * qd);
        qf[u][c] = __builtin_bit_cast(f16x8, v);
      } else {
        qf[u][c] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  }

  const int8_t* kh = a.kc + size_t(kvh) * a.cap * HD;
  const int8_t* vh = a.vc + size_t(kvh) * a.cap * HD;
  const __half* ksh = a.ks + size_t(kvh) * a.cap;
  const __half* vsh = a.vs + size_t(kvh) * a.cap;

  // Loader mapping: 32 keys × HD bytes of K and of V; each thread moves 16 bytes of each (HD = 128) or 8 (HD = 64).
  constexpr int BPT = HD / 8;                   // bytes per thread per tensor
  const int lk = threadIdx.x / (HD / BPT);      // key within the block
  const int ld0 = (threadIdx.x % (HD / BPT)) * BPT;

  for (int kb = k0; kb < k1; kb += 32) {
    // Stage the block: keys kb … kb+31 (slots wrap in a ring cache; keys past k1 read as zero and are masked).
    {
      const int key = kb + lk;
      const bool ok = key < k1;
      const int slot = a.ring ? key % a.ring : key;
      unsigned kw[BPT / 4], vw[BPT / 4];
#pragma unroll
      for (int i = 0; i < BPT / 4; ++i) {
        kw[i] = ok ? *reinterpret_cast<const unsigned*>(kh + size_t(slot) * HD + ld0 + 4 * i) : 0u;
        vw[i] = ok ? *reinterpret_cast<const unsigned*>(vh + size_t(slot) * HD + ld0 + 4 * i) : 0u;
      }
      __syncthreads();  // the previous block's readers are done with LDS
#pragma unroll
      for (int i = 0; i < BPT / 4; ++i) {
        __half2 lo, hi;
        i8x4_to_h(kw[i], lo, hi);
        *reinterpret_cast<__half2*>(&Kf[lk * KROW + ld0 + 4 * i]) = lo;
        *reinterpret_cast<__half2*>(&Kf[lk * KROW + ld0 + 4 * i + 2]) = hi;
        i8x4_to_h(vw[i], lo, hi);
        const int vsl = vslot(lk);
        Vt[(ld0 + 4 * i + 0) * VROW + vsl] = __builtin_bit_cast(_Float16, __low2half(lo));
        Vt[(ld0 + 4 * i + 1) * VROW + vsl] = __builtin_bit_cast(_Float16, __high2half(lo));
        Vt[(ld0 + 4 * i + 2) * VROW + vsl] = __builtin_bit_cast(_Float16, __low2half(hi));
        Vt[(ld0 + 4 * i + 3) * VROW + vsl] = __builtin_bit_cast(_Float16, __high2half(hi));
      }
      if (threadIdx.x < 32) {
        const int key2 = kb + threadIdx.x;
        const int sl2 = a.ring ? key2 % a.ring : key2;
        ksf[threadIdx.x] = key2 < k1 ? __half2float(ksh[sl2]) * a.scale_log2 : 0.f;
        vsf[threadIdx.x] = key2 < k1 ? __half2float(vsh[sl2]) : 0.f;
      }
      __syncthreads();
    }

#pragma unroll
    for (int u = 0; u < QTW; ++u) {
      if (!qlive[u]) continue;   // uniform per wave
      // Sᵀ for the two 16-key tiles.
      f32x4 sacc[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        sacc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const f16x8 kf = *reinterpret_cast<const f16x8*>(&Kf[(16 * h + j) * KROW + 32 * c + 8 * qd]);
          sacc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[u][c], sacc[h], 0, 0, 0);
        }
      }
      // Lane (j, qd) holds keys 16h + 4qd + r of query m = 16·qt + j.
      const int m = 16 * qt[u] + j;
      const int tok = m / a.G;
      const int lim = a.P + tok;  // last visible key (causal)
      const int lo_key = a.window > 0 ? lim - a.window + 1 : -2147483647;
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
      const float mnew = fmaxf(mrun[u], mx);
      const float alpha = mnew == -INFINITY ? 1.f : exp2f(mrun[u] - mnew);
      mrun[u] = mnew;
      float ps = 0.f;
      _Float16 pv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = s[h][r] == -INFINITY ? 0.f : exp2f(s[h][r] - mnew);
          ps += p;
          pv[4 * h + r] = (_Float16)(p * vsf[16 * h + 4 * qd + r]);
        }
      lsum[u] = lsum[u] * alpha + ps;
      // Rescale Oᵀ only when some column's maximum moved (alpha = 1 is exact and is skipped).
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[u][dt] *= alpha;
      }
      f16x8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = pv[e];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f16x8 vf = *reinterpret_cast<const f16x8*>(&Vt[(16 * dt + j) * VROW + 8 * qd]);
        o[u][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb, o[u][dt], 0, 0, 0);
      }
    }
  }

  // Partials of this split: (max, sum) per query and the unnormalised Oᵀ (lane holds dims 16dt + 4qd + r of query m).
  const size_t base = (size_t(kvh) * a.nsplit + sidx) * a.Qpad;
#pragma unroll
  for (int u = 0; u < QTW; ++u) {
    if (!qlive[u]) continue;
    float l = lsum[u];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int m = 16 * qt[u] + j;
    if (m >= Q) continue;
    if (qd == 0) a.ml[base + m] = make_float2(mrun[u], l);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      *reinterpret_cast<f32x4*>(a.opart + (base + m) * HD + 16 * dt + 4 * qd) = o[u][dt];
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Reduction of the splits (vattn_reduce, verify_attn.metal:149-192): M = max over splits (and the sink), L = Σ e^(m−M)·l
// (+ e^(sink−M)), o = Σ e^(m−M)·O / L, in split order; written into the o_proj activation layout (column h·HD + d).
// Grid (B), QH·HD/8 threads (one per 8 values).
__global__ __launch_bounds__(1024) void attn_reduce_kernel(AttnArgs a, uint4* __restrict__ frag, float* __restrict__ xsum,
                                                           int nkb) {
  const int t = blockIdx.x, c = threadIdx.x, HD = a.HD;
  const int h = (8 * c) / HD, d0 = (8 * c) % HD;
  const int kvh = h / a.G, m = t * a.G + h % a.G;
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.ml[(size_t(kvh) * a.nsplit + s) * a.Qpad + m].x);
  float L = 0.f;
  if (a.sinks) {
    const float sk = a.sinks[h] * 1.4426950408889634f;
    M = fmaxf(M, sk);
    L = exp2f(sk - M);
  }
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    const size_t idx = (size_t(kvh) * a.nsplit + s) * a.Qpad + m;
    const float2 v = a.ml[idx];
    if (v.x == -INFINITY) continue;
    const float w = exp2f(v.x - M);
    L += w * v.y;
    const f32x4* src = reinterpret_cast<const f32x4*>(a.opart + idx * HD + d0);
    const f32x4 p0 = src[0], p1 = src[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] += w * p0[e];
      o[4 + e] += w * p1[e];
    }
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] *= inv;
  act_store_chunk(frag, xsum, nkb, t, c, o, true, MAX_TOK);
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
  const int nz = (qtiles + 7) / 8;
  dim3 grid(a.nsplit, a.KVH, nz);
  // Algorithmic bytes: the int8 K and V and their fp16 scales of every key the launched splits cover, and q.
  const double keys = double(a.P + a.B) - double(a.s0) * a.C;
  TimedLaunch tl(c, TC_ATTN, double(a.KVH) * keys * (2 * a.HD + 4) + double(a.KVH) * Q * a.HD * 2);
  if (a.HD == 128) attn_kernel<128><<<grid, 256, 0, c->stream>>>(a);
  else if (a.HD == 64) attn_kernel<64><<<grid, 256, 0, c->stream>>>(a);
  else return fail(IH_EINVAL, "attention: head_dim must be 64 or 128");
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_attn_reduce(ih_ctx* c, const AttnArgs& a, ActBuf& out) {
  const int threads = a.QH * a.HD / 8;
  IH_CHECK(threads <= 1024 && threads % 64 == 0, IH_EINVAL, "attention reduce: QH·HD/8 must be a multiple of 64 ≤ 1024");
  TimedLaunch tl(c, TC_REDUCE, double(a.KVH) * a.nsplit * a.G * a.B * (a.HD + 2) * 4 + double(a.B) * a.QH * a.HD * 2);
  attn_reduce_kernel<<<a.B, threads, 0, c->stream>>>(a, static_cast<uint4*>(out.frag), out.xsum, out.nkb);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih
