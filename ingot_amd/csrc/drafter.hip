// The DFlash2 drafter behind the C ABI: the producer of the draft block (anchor + block − 1 drafts) of the verify step,
// and the hidden-state captures of the target model it reads.
//
// Reference: DFlash2Drafter (Sources/Ingot/Drafter.swift:1-554) with its kernels (Shaders/yy_model.metal:94-104,
// 151-614): the target's residual rows after its `target layers` are captured (capture_rows); the accepted rows'
// captures go through fc → RMSNorm → per layer k|v → k_norm + RoPE into a window ring of the drafter's layers
// (encodeContext, dctx_write); a block [anchor, mask × (block − 1)] embedded with the target's table runs through dense
// qwen3 layers whose attention sees the window of context plus the whole block (non-causal, dattn_*), with the two-tap
// dynamic conv of DFlash2 around the attention and the MLP (dconv_prep / dconv_fin_add); the target's lm_head scores
// rows 1 … block − 1, the top-16 candidates of each go to the greedy selector (dselect: logit + Σ_r pred[prev]·hp·succ
// over rank-r codebooks), which writes the drafts and their confidences (softmax(score/1.5) of the chosen one). DFlash
// v1 (no conv, rank 0): the drafts are each row's best candidate (dpick_top1).
//
// MI355X design: the projections run on the library's int4 qmm (bf16 activations, fp32 accumulate); the attention is
// one workgroup per (KV head, 128-key chunk) over fp16 K/V rings in HBM with the chunks' (max, sum, O) merged in key
// order by a second kernel; the selector is one workgroup of `rank` threads with wave sums.
#include <hip/hip_fp16.h>

#include <cmath>
#include <vector>

#include <algorithm>
#include "act.h"
#include "lanes.h"
#include "drafter_ckpt.h"
#include "model_internal.h"

namespace ih {

int synth_int4(ih_ctx* c, uint32_t* w, uint16_t* s, uint16_t* b, size_t N, size_t K, uint64_t seed, uint64_t tensor,
               float sd);
int synth_bf16(ih_ctx* c, uint16_t* out, size_t n, uint64_t seed, uint64_t tensor, float base, float amp);
int launch_embed_act(ih_ctx* c, const uint32_t* tok, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     float* h, int B, int H, int V, const uint16_t* nw, ActBuf& a, float2* rope, int P, float theta,
                     int RH, const uint32_t* pos_dev, int pos_max, const float* rinv = nullptr,
                     float rmscale = 1.0f);

constexpr int DKVH = 8;          // KV heads of the drafter attention (DF_KVH)
constexpr int DCHUNK = 128;      // keys per attention workgroup
constexpr int DCG = 16;          // channels per dynamic-conv group (DF_GS)
constexpr int DTOPK = 16;        // candidates per draft position (topk16_rows)
constexpr float CONF_TAU = 1.5f; // DFlash2Drafter.confTau

// Synthetic tensor ids of the drafter: 7·10^6 + 1000·layer + kind; globals 7.9·10^6 + kind.
enum : uint64_t { D_N1 = 0, D_N2 = 1, D_QN = 2, D_KN = 3, D_QKV = 4, D_O = 5, D_GU = 6, D_DOWN = 7, D_APROJ = 8,
                  D_MPROJ = 9, D_ABASE = 10, D_MBASE = 11 };
enum : uint64_t { D_FC = 1, D_HNORM = 2, D_FNORM = 3, D_HPROJ = 4, D_PRED = 5, D_SUCC = 6 };
constexpr uint64_t dl_tensor(int l, uint64_t kind) { return 7000000 + 1000 * uint64_t(l) + kind; }
constexpr uint64_t dg_tensor(uint64_t kind) { return 7900000 + kind; }

}  // namespace ih

using namespace ih;

struct ih_drafter_layer {
  uint16_t *n1 = nullptr, *n2 = nullptr, *qn = nullptr, *kn = nullptr;  // bf16 [H], [H], [HD], [HD]
  uint16_t *abase = nullptr, *mbase = nullptr;                          // bf16 [2 (prep|finish)][2 (tap)][H]
  ih_qmat *qkv = nullptr, *kv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr, *aproj = nullptr,
          *mproj = nullptr;
  __half *kc = nullptr, *vc = nullptr;  // rings [KVH][slots][HD]: window positions, then the block's rows
};

struct ih_drafter {
  ih_ctx* ctx = nullptr;
  ih_drafter_desc d{};
  int QP = 0, slots = 0, G = 0, DYN = 0;
  std::vector<ih_drafter_layer> layers;
  ih_qmat *fc = nullptr, *hproj = nullptr;
  uint16_t *hnorm = nullptr, *fnorm = nullptr;
  uint16_t *pred = nullptr, *succ = nullptr;  // bf16 [V][rank]
  // The target model whose embedding and head the drafter uses, and whose verify step writes the captures.
  ih_model* target = nullptr;
  uint16_t* caps = nullptr;  // bf16 [MAX_TOK][n_targets · H] (row r: the block row r of the last verify step)
  // Scratch of one pass.
  uint32_t* dtok = nullptr;  // [block]: anchor, masks
  float2* rope = nullptr;    // scratch of the embedding kernel's RoPE table
  float *x = nullptr, *proj = nullptr, *dyn = nullptr, *y = nullptr, *gu = nullptr, *logits = nullptr,
        *hp = nullptr;
  uint16_t* xn = nullptr;   // bf16 [MAX_TOK][H] normalised rows (conv input)
  __half* q = nullptr;      // [KVH][G·block][HD]
  float* opart = nullptr;   // [KVH][nchunk][G·block][HD]
  float2* ml = nullptr;     // [KVH][nchunk][G·block]
  uint32_t* cidx = nullptr; // [block][64] candidates (the first 16 are the top-16)
  float *cval = nullptr, *cz = nullptr, *conf = nullptr;
  float* esel = nullptr;      // [block][16][16] selector scores per (position, previous pick, candidate)
  ActBuf act_h, act_a, act_i, act_c, act_f;  // [H]: norm/conv outputs; [QH·HD]: attention; [I]: MLP; caps; fc out
};

namespace ih {

// ---------------------------------------------------------------------------------------------------------------
// Kernels.

// Captured residual rows (capture_rows, yy_model.metal:94-104): caps[r][j·H + c] = bf16(h[r][c]). Grid (rows).
__global__ __launch_bounds__(256) void capture_kernel(const float* __restrict__ h, int H, uint16_t* __restrict__ caps,
                                                      int ldc, int col0) {
  const int r = blockIdx.x;
  for (int c = threadIdx.x; c < H; c += 256) caps[size_t(r) * ldc + col0 + c] = dround_bf16(h[size_t(r) * H + c]);
}

// RMSNorm of fp32 rows: x·rsqrt(mean x² + eps)·w, to the fragment layout (rows out_row0 + r) and, if xn is set, to
// natural bf16 rows. Grid (rows), 256 threads; rows r ≥ first.
__global__ __launch_bounds__(256) void dnorm_kernel(const float* __restrict__ x, int H, const uint16_t* __restrict__ w,
                                                    float eps, int first, uint4* __restrict__ frag, int nkb, int ntile,
                                                    uint16_t* __restrict__ xn) {
  __shared__ float red[4];
  const int r = blockIdx.x + first;
  const float* xr = x + size_t(r) * H;
  float ss = 0.f;
  for (int c = threadIdx.x; c < H; c += 256) ss += xr[c] * xr[c];
  ss += lane_xor<32>(ss);
  ss += lane_xor<16>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<1>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float rr = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / float(H) + eps);
  for (int c8 = threadIdx.x; c8 < H / 8; c8 += 256) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = xr[8 * c8 + j] * rr * dbf16(w[8 * c8 + j]);
      if (xn) xn[size_t(r) * H + 8 * c8 + j] = dround_bf16(v[j]);
    }
    frag_store_chunk(frag, nkb, ntile, blockIdx.x, c8, v);
  }
}

// Two-tap dynamic conv before a sublayer (dconv_prep): a_t = (base[0][0] + dyn_t[0][g])·x_t + (base[0][1] +
// dyn_t[1][g])·x_{t−1}, x_{−1} = 0, g = c / 16; to the fragment layout. Grid (rows), 256 threads.
__global__ __launch_bounds__(256) void dconv_prep_kernel(const uint16_t* __restrict__ xn, const float* __restrict__ dyn,
                                                         int ldd, const uint16_t* __restrict__ base, int H, int G,
                                                         uint4* __restrict__ frag, int nkb, int ntile) {
  const int t = blockIdx.x;
  // Eight consecutive channels (one conv group) per thread and chunk, 16-byte loads of the bf16 rows.
#pragma unroll 2
  for (int c8 = threadIdx.x; c8 < H / 8; c8 += 256) {
    const int c = 8 * c8, g = c / DCG;
    const uint4 a0 = *reinterpret_cast<const uint4*>(xn + size_t(t) * H + c);
    const uint4 a1 = t > 0 ? *reinterpret_cast<const uint4*>(xn + size_t(t - 1) * H + c) : make_uint4(0, 0, 0, 0);
    const uint4 b0 = *reinterpret_cast<const uint4*>(base + c), b1 = *reinterpret_cast<const uint4*>(base + H + c);
    const float d0 = dyn[size_t(t) * ldd + g], d1 = dyn[size_t(t) * ldd + G + g];
    const uint32_t x0w[4] = {a0.x, a0.y, a0.z, a0.w}, x1w[4] = {a1.x, a1.y, a1.z, a1.w};
    const uint32_t k0w[4] = {b0.x, b0.y, b0.z, b0.w}, k1w[4] = {b1.x, b1.y, b1.z, b1.w};
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int sh = 16 * (j & 1);
      const float x0 = dbf16(uint16_t(x0w[j / 2] >> sh)), x1 = dbf16(uint16_t(x1w[j / 2] >> sh));
      const float k0 = dbf16(uint16_t(k0w[j / 2] >> sh)) + d0;
      const float k1 = dbf16(uint16_t(k1w[j / 2] >> sh)) + d1;
      v[j] = k0 * x0 + k1 * x1;
    }
    frag_store_chunk(frag, nkb, ntile, t, c8, v);
  }
}

// The conv after a sublayer added to the residual (dconv_fin_add): x_t += (base[1][0] + dyn_t[2][g])·y_t +
// (base[1][1] + dyn_t[3][g])·y_{t−1}, without dyn (DFlash v1) x += y; then, in the same launch, the next RMSNorm of
// the row (rows t ≥ first; fragment row t − first). Grid (rows), 256 threads; H a multiple of 8.
__global__ __launch_bounds__(256) void dfin_norm_kernel(const float* __restrict__ y, const float* __restrict__ dyn,
                                                        int ldd, const uint16_t* __restrict__ base, int H, int G,
                                                        float* __restrict__ x, const uint16_t* __restrict__ w,
                                                        float eps, int first, uint4* __restrict__ frag, int nkb,
                                                        int ntile, uint16_t* __restrict__ xn) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  float* xr = x + size_t(t) * H;
  float ss = 0.f;
  // Eight consecutive channels per thread (one conv group: DCG is a multiple of 8), 16-byte loads, two chunks of
  // eight per pass so that their loads are in flight together.
#pragma unroll 2
  for (int c8 = threadIdx.x; c8 < H / 8; c8 += 256) {
    const int c = 8 * c8;
    const float4* yp = reinterpret_cast<const float4*>(y + size_t(t) * H + c);
    float4* xp = reinterpret_cast<float4*>(xr + c);
    const float4 ya = yp[0], yb = yp[1], xa = xp[0], xb = xp[1];
    float y0[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
    float nx[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    if (!dyn) {
#pragma unroll
      for (int j = 0; j < 8; ++j) nx[j] += y0[j];
    } else {
      const int g = c / DCG;
      float y1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (t > 0) {
        const float4* qp = reinterpret_cast<const float4*>(y + size_t(t - 1) * H + c);
        const float4 qa = qp[0], qb = qp[1];
        y1[0] = qa.x; y1[1] = qa.y; y1[2] = qa.z; y1[3] = qa.w;
        y1[4] = qb.x; y1[5] = qb.y; y1[6] = qb.z; y1[7] = qb.w;
      }
      const uint4 b2 = *reinterpret_cast<const uint4*>(base + 2 * H + c);
      const uint4 b3 = *reinterpret_cast<const uint4*>(base + 3 * H + c);
      const float d2 = dyn[size_t(t) * ldd + 2 * G + g], d3 = dyn[size_t(t) * ldd + 3 * G + g];
      const uint32_t w2[4] = {b2.x, b2.y, b2.z, b2.w}, w3[4] = {b3.x, b3.y, b3.z, b3.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float k0 = dbf16(uint16_t(w2[j / 2] >> (16 * (j & 1)))) + d2;
        const float k1 = dbf16(uint16_t(w3[j / 2] >> (16 * (j & 1)))) + d3;
        nx[j] = nx[j] + (k0 * y0[j] + k1 * y1[j]);
      }
    }
    xp[0] = make_float4(nx[0], nx[1], nx[2], nx[3]);
    xp[1] = make_float4(nx[4], nx[5], nx[6], nx[7]);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += nx[j] * nx[j];
  }
  if (t < first) return;  // whole workgroup
  ss += lane_xor<32>(ss);
  ss += lane_xor<16>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<1>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();  // also makes the row's new values visible across the workgroup
  const float rr = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / float(H) + eps);
  for (int c8 = threadIdx.x; c8 < H / 8; c8 += 256) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = xr[8 * c8 + j] * rr * dbf16(w[8 * c8 + j]);
      if (xn) xn[size_t(t) * H + 8 * c8 + j] = dround_bf16(v[j]);
    }
    frag_store_chunk(frag, nkb, ntile, t - first, c8, v);
  }
}

// SwiGLU of gate | up rows (fp32 [rows][2I]) into the fragment layout (dswiglu). Grid (rows), 256 threads.
__global__ __launch_bounds__(256) void dswiglu_kernel(const float* __restrict__ gu, int I, uint4* __restrict__ frag,
                                                      int nkb, int ntile) {
  const int t = blockIdx.x;
  for (int c8 = threadIdx.x; c8 < I / 8; c8 += 256) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float g = gu[size_t(t) * 2 * I + 8 * c8 + j], u = gu[size_t(t) * 2 * I + I + 8 * c8 + j];
      v[j] = g / (1.0f + __expf(-g)) * u;
    }
    frag_store_chunk(frag, nkb, ntile, t, c8, v);
  }
}

// Per-head RMSNorm with weight, then RoPE over the whole head (non-interleaved halves) at position pos, of the value
// x held by lane d % 64 as x[e] = dim d + 64e (dnorm_rope, yy_model.metal:242-266).
template <int NE>
__device__ __forceinline__ void dnorm_rope(float (&x)[NE], int lane, const uint16_t* w, float pos, float eps,
                                           float theta) {
  constexpr int HD = 64 * NE, RH = HD / 2;
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) ss += x[e] * x[e];
  ss += lane_xor<32>(ss);
  ss += lane_xor<16>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<1>(ss);
  const float r = rsqrtf(ss / float(HD) + eps);
#pragma unroll
  for (int e = 0; e < NE; ++e) x[e] = x[e] * r * dbf16(w[lane + 64 * e]);
  const int i = lane % RH;
  const float ang = pos * powf(theta, -float(i) / float(RH));
  float c, s;
  sincosf(ang, &s, &c);
  if constexpr (NE == 2) {
    const float a = x[0], b = x[1];
    x[0] = a * c - b * s;
    x[1] = b * c + a * s;
  } else {
    const float o = lane_xor<32>(x[0]);
    x[0] = lane < RH ? x[0] * c - o * s : x[0] * c + o * s;
  }
}

struct DAttn {
  const float* qkv;  // [B][QP]
  int QP, QH, G, HD, B, win, slots;
  const uint16_t *qn, *kn;
  __half *q, *kc, *vc;
  float eps, theta;
  const uint32_t* st;  // round state (P = st[0]) or null
  int P;
};

// Block rows (dattn_prework): q heads → q (norm + RoPE at P + t), k → ring slot win + t (norm + RoPE), v → slot
// win + t. One wave per (head slot, row): grid ((QH + 16 + 3) / 4, B), 256 threads.
template <int HD>
__global__ __launch_bounds__(256) void dprework_kernel(DAttn a) {
  constexpr int NE = HD / 64;
  const int slot = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y, lane = threadIdx.x & 63;
  if (slot >= a.QH + 2 * DKVH) return;
  const int P = a.st ? int(a.st[0]) : a.P;
  float x[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) x[e] = a.qkv[size_t(t) * a.QP + slot * HD + lane + 64 * e];
  if (slot >= a.QH + DKVH) {
    const int h = slot - a.QH - DKVH;
#pragma unroll
    for (int e = 0; e < NE; ++e) a.vc[(size_t(h) * a.slots + a.win + t) * HD + lane + 64 * e] = __float2half_rn(x[e]);
    return;
  }
  const bool isq = slot < a.QH;
  dnorm_rope(x, lane, isq ? a.qn : a.kn, float(P + t), a.eps, a.theta);
  if (isq) {
    __half* q = a.q + (size_t(slot / a.G) * a.G * a.B + t * a.G + slot % a.G) * HD;
#pragma unroll
    for (int e = 0; e < NE; ++e) q[lane + 64 * e] = __float2half_rn(x[e]);
  } else {
    const int h = slot - a.QH;
#pragma unroll
    for (int e = 0; e < NE; ++e) a.kc[(size_t(h) * a.slots + a.win + t) * HD + lane + 64 * e] = __float2half_rn(x[e]);
  }
}

// Context rows (dctx_write): k|v rows [rows][16·HD] of positions pos0 + t (t < nvalid) into ring slot pos % win, k with
// k_norm + RoPE. nvalid and pos0 from the round state (st[2], st[3]) when st is set. Grid (4, rows), 256 threads.
template <int HD>
__global__ __launch_bounds__(256) void dctx_kernel(const float* __restrict__ kv, const uint16_t* __restrict__ kn,
                                                   __half* __restrict__ kc, __half* __restrict__ vc, int win,
                                                   int slots, float eps, float theta, const uint32_t* st, int nvalid,
                                                   int pos0) {
  constexpr int NE = HD / 64;
  const int slot = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y, lane = threadIdx.x & 63;
  if (st) {
    nvalid = int(st[2]);
    pos0 = int(st[3]);
  }
  if (t >= nvalid || slot >= 2 * DKVH) return;
  const int pos = pos0 + t, ring = pos % win;
  float x[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) x[e] = kv[size_t(t) * (2 * DKVH * HD) + slot * HD + lane + 64 * e];
  if (slot >= DKVH) {
#pragma unroll
    for (int e = 0; e < NE; ++e) vc[(size_t(slot - DKVH) * slots + ring) * HD + lane + 64 * e] = __float2half_rn(x[e]);
    return;
  }
  dnorm_rope(x, lane, kn, float(pos), eps, theta);
#pragma unroll
  for (int e = 0; e < NE; ++e) kc[(size_t(slot) * slots + ring) * HD + lane + 64 * e] = __float2half_rn(x[e]);
}

// Does block row t see slot n (dvisible, yy_model.metal:336-342)? A ring slot n < W holds the latest position k < P
// with k ≡ n (mod W), visible when written (k ≥ 0) and inside the row's window (P + t − k < W); the block's slots
// W … W + B − 1 are seen by every row.
__device__ __forceinline__ bool dvisible(int n, int t, int P, int B, int W) {
  if (n >= W) return n < W + B;
  int back = (P - 1 - n) % W;
  if (back < 0) back += W;
  const int k = P - 1 - back;
  return k >= 0 && P + t - k < W;
}

// Attention of the block's Q = G·B queries of one KV head over one chunk of 128 slots: scores in fp32 (q·k / √HD),
// the chunk's (max, Σ e^(s − max)) per query and its unnormalised O = Σ e^(s − max)·v. Grid (nchunk, KVH), 256
// threads; the queries, the chunk's K, then its V, staged in LDS (HD ≤ 128, Q ≤ 64). Wave w takes query tile w (16
// rows): S = Q·Kᵀ on v_mfma_f32_16x16x32_f16 (fp16 products exact in fp32), O += P·V on v_mfma_f32_16x16x4_f32 with
// the weights in fp32 (no rounding of P).
typedef _Float16 dh8 __attribute__((ext_vector_type(8)));
typedef float df4 __attribute__((ext_vector_type(4)));
template <int HD>
__global__ __launch_bounds__(256) void dattn_kernel(DAttn a, float* __restrict__ opart, float2* __restrict__ ml,
                                                    int nchunk) {
  constexpr int KS = HD + 8;  // halves per LDS row: 16-byte aligned fragment reads, rows 4 banks apart
  constexpr int RV = HD / 8;  // 16-byte vectors per row
  const int ch = blockIdx.x, kvh = blockIdx.y, Q = a.G * a.B;
  const int P = a.st ? int(a.st[0]) : a.P;
  const int n0 = ch * DCHUNK, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, qd = lane >> 4;
  __shared__ __attribute__((aligned(16))) __half ks[DCHUNK][KS];
  __shared__ __attribute__((aligned(16))) __half qs[64][KS];
  __shared__ float sc[64][DCHUNK + 4];
  // Rows of fp16 staged 16 bytes at a time (rows past the cache or the block read as zero).
  auto stage = [&](__half (*dst)[KS], const __half* src, int rows, int live) {
    for (int i = tid; i < rows * RV; i += 256) {
      const int r = i / RV, c = i % RV;
      const uint4 v = r < live ? *reinterpret_cast<const uint4*>(src + size_t(r) * HD + 8 * c) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&dst[r][8 * c]) = v;
    }
  };
  const int live_keys = max(0, min(DCHUNK, a.slots - n0));
  stage(ks, a.kc + (size_t(kvh) * a.slots + n0) * HD, DCHUNK, live_keys);
  stage(qs, a.q + size_t(kvh) * Q * HD, 64, Q);
  __syncthreads();
  const float scale = 1.0f / sqrtf(float(HD));
  // Scores of query tile `wave` against the chunk's 8 key tiles: lane (n, qd) holds S[16w + 4qd + e][16t + n].
  df4 sacc[DCHUNK / 16];
#pragma unroll
  for (int t = 0; t < DCHUNK / 16; ++t) {
    df4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
      const dh8 qa = *reinterpret_cast<const dh8*>(&qs[16 * wave + n][32 * s + 8 * qd]);
      const dh8 kb = *reinterpret_cast<const dh8*>(&ks[16 * t + n][32 * s + 8 * qd]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa, kb, acc, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * wave + 4 * qd + e, key = 16 * t + n;
      const bool vis = m < Q && key < live_keys && dvisible(n0 + key, m / a.G, P, a.B, a.win);
      acc[e] = vis ? acc[e] * scale : -INFINITY;
    }
    sacc[t] = acc;
  }
  // Per query row (4qd + e of the tile): the chunk's max and Σ e^(s − max) over its 128 keys — 8 in each lane, then
  // across the row's 16 lanes — and the weights e^(s − max) to LDS for the products.
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < DCHUNK / 16; ++t) mx = fmaxf(mx, sacc[t][e]);
    mx = fmaxf(mx, lane_xor<1>(mx));
    mx = fmaxf(mx, lane_xor<2>(mx));
    mx = fmaxf(mx, lane_xor<4>(mx));
    mx = fmaxf(mx, lane_xor<8>(mx));
    const int m = 16 * wave + 4 * qd + e;
    float l = 0.f;
#pragma unroll
    for (int t = 0; t < DCHUNK / 16; ++t) {
      const float p = mx == -INFINITY ? 0.f : __expf(sacc[t][e] - mx);
      sc[m][16 * t + n] = p;
      l += p;
    }
    l += lane_xor<1>(l);
    l += lane_xor<2>(l);
    l += lane_xor<4>(l);
    l += lane_xor<8>(l);
    if (n == 0 && m < Q) ml[(size_t(kvh) * nchunk + ch) * Q + m] = make_float2(mx, l);
  }
  __syncthreads();
  // The chunk's V replaces its K in LDS.
  stage(ks, a.vc + (size_t(kvh) * a.slots + n0) * HD, DCHUNK, live_keys);
  __syncthreads();
  // O of query tile `wave`: dims tile d, four keys per step; lane (n, qd) ends with O[16w + 4qd + e][16d + n].
  for (int d = 0; d < HD / 16; ++d) {
    df4 o = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < DCHUNK; k += 4) {
      const float pa = sc[16 * wave + n][k + qd];
      const float vb = __half2float(ks[k + qd][16 * d + n]);
      o = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vb, o, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * wave + 4 * qd + e;
      if (m < Q) opart[((size_t(kvh) * nchunk + ch) * Q + m) * HD + 16 * d + n] = o[e];
    }
  }
}

// Merge of the chunks in key order (dattn_reduce): o = Σ e^(m − M)·O / Σ e^(m − M)·l, to the o_proj input (fragment
// layout, column h·HD + d). Grid (B, QH), HD / 8 threads (8 dims each).
__global__ void dattn_reduce_kernel(const float* __restrict__ opart, const float2* __restrict__ ml, int nchunk, int G,
                                    int B, int HD, uint4* __restrict__ frag, int nkb, int ntile) {
  const int t = blockIdx.x, h = blockIdx.y, kvh = h / G, m = t * G + h % G, Q = G * B;
  const int c8 = threadIdx.x;  // dims 8·c8 …
  float M = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < nchunk; ++s) M = fmaxf(M, ml[(size_t(kvh) * nchunk + s) * Q + m].x);
  float L = 0.f, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // Loads without branches (an empty chunk's partial is read and not added), so an unrolled group's requests are in
  // flight together.
#pragma unroll 4
  for (int s = 0; s < nchunk; ++s) {
    const float2 v = ml[(size_t(kvh) * nchunk + s) * Q + m];
    const float4* op = reinterpret_cast<const float4*>(opart + ((size_t(kvh) * nchunk + s) * Q + m) * HD + 8 * c8);
    const float4 p0 = op[0], p1 = op[1];
    const bool live = v.x != -INFINITY;
    const float w = live ? __expf(v.x - M) : 0.f;
    L = live ? L + w * v.y : L;
    const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = live ? o[j] + w * pv[j] : o[j];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = L > 0.f ? o[j] / L : 0.f;
  frag_store_chunk(frag, nkb, ntile, t, (h * HD) / 8 + c8, o);
}

// The greedy selector (dselect, yy_model.metal:569-614): at position t the candidate j with the highest
// val[t][j] + Σ_r pred[prev][r]·hp[t][r]·succ[cand_j][r] (prev = the anchor at t = 0, else the pick at t − 1; the first
// if tied); tok[1 + t] = the pick, conf[t] = its softmax(score/τ) over the 16. rank = 0: the best candidate
// (dpick_top1).
//
// The pick at t − 1 is one of the 16 candidates of t − 1, so the bilinear term depends on the chain only through
// that index: dselect_pairs_kernel computes it for every (t, i, j) — i the index of the previous pick among the
// candidates of t − 1 (only i = 0, the anchor, at t = 0) — in parallel, one workgroup of `rank` threads (a multiple
// of 64, ≤ 1024) per (t, i); dselect_kernel then walks t in one wave over those scores in LDS. Each E[t][i][j] is
// summed in one fixed order (64-lane butterfly, then the waves in order) whatever the chain.
constexpr int DSEL = DTOPK * DTOPK;  // E entries per position
__global__ void dselect_pairs_kernel(const uint32_t* __restrict__ cand, int ldc, const float* __restrict__ hp,
                                     const uint16_t* __restrict__ pred, const uint16_t* __restrict__ succ, int rank,
                                     const uint32_t* __restrict__ tok, float* __restrict__ E) {
  __shared__ float part[16][DTOPK];
  const int t = blockIdx.x, i = blockIdx.y, r = threadIdx.x, wave = r >> 6, lane = r & 63, nw = int(blockDim.x) >> 6;
  if (t == 0 && i > 0) return;  // the anchor is the only previous token at t = 0
  const uint32_t prev = t == 0 ? tok[0] : cand[size_t(t - 1) * ldc + i];
  const float a = dbf16(pred[size_t(prev) * rank + r]) * hp[size_t(t) * rank + r];
  for (int j = 0; j < DTOPK; ++j) {
    float e = a * dbf16(succ[size_t(cand[size_t(t) * ldc + j]) * rank + r]);
    e += lane_xor<32>(e);
    e += lane_xor<16>(e);
    e += lane_xor<8>(e);
    e += lane_xor<4>(e);
    e += lane_xor<2>(e);
    e += lane_xor<1>(e);
    if (lane == 0) part[wave][j] = e;
  }
  __syncthreads();
  if (r < DTOPK) {
    float e = 0.f;
    for (int q = 0; q < nw; ++q) e += part[q][r];
    E[size_t(t) * DSEL + i * DTOPK + r] = e;
  }
}

// 256 threads stage the scores of all positions in LDS (every load issued before the first store), then one wave
// walks the chain (E = nullptr: rank 0).
__global__ __launch_bounds__(256) void dselect_kernel(const uint32_t* __restrict__ cand, const float* __restrict__ val,
                                                      int ldc, const float* __restrict__ E, uint32_t* __restrict__ tok,
                                                      int M, float* __restrict__ conf) {
  constexpr int NE = 16 * DSEL / 4 / 256;  // float4 loads of E per thread
  __shared__ float4 es4[16 * DSEL / 4];
  __shared__ float vs[16][DTOPK];
  __shared__ uint32_t cs[16][DTOPK];
  const int tid = threadIdx.x;
  float4 q[NE];
#pragma unroll
  for (int u = 0; u < NE; ++u) {
    const int k = tid + 256 * u;
    q[u] = E && k < M * DSEL / 4 ? reinterpret_cast<const float4*>(E)[k] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int t0 = tid / DTOPK, j0 = tid % DTOPK;
  float v0 = 0.f;
  uint32_t c0 = 0;
  if (t0 < M) {
    v0 = val[size_t(t0) * ldc + j0];
    c0 = cand[size_t(t0) * ldc + j0];
  }
#pragma unroll
  for (int u = 0; u < NE; ++u) es4[tid + 256 * u] = q[u];
  vs[t0][j0] = v0;
  cs[t0][j0] = c0;
  __syncthreads();
  if (tid >= 64) return;
  // Wave 0 walks the chain, lane j (mod 16) on candidate j: the first maximum by a butterfly over the 16 (NaN scores
  // never picked, as with a strict > from −inf), then Σ exp((s − s_best)/τ) by another.
  const float* es = reinterpret_cast<const float*>(es4);
  const int j = tid & (DTOPK - 1);
  int pi = 0;  // index of the previous pick among the previous position's candidates (0: the anchor)
  for (int t = 0; t < M; ++t) {
    const float sc = vs[t][j] + es[t * DSEL + pi * DTOPK + j];
    float bs = sc != sc ? -INFINITY : sc;
    int best = j;
#define IH_PICK(H)                                                                           \
    {                                                                                        \
      const float ob = lane_xor<H>(bs);                                                      \
      const int oj = __float_as_int(lane_xor<H>(__int_as_float(best)));                      \
      const bool take = (ob > bs) | ((ob == bs) & (oj < best));                              \
      bs = take ? ob : bs;                                                                   \
      best = take ? oj : best;                                                               \
    }
    IH_PICK(1) IH_PICK(2) IH_PICK(4) IH_PICK(8)
#undef IH_PICK
    float z = __expf((sc - bs) / CONF_TAU);
    z += lane_xor<1>(z);
    z += lane_xor<2>(z);
    z += lane_xor<4>(z);
    z += lane_xor<8>(z);
    if (tid == 0) {
      tok[1 + t] = cs[t][best];
      conf[t] = 1.0f / z;
    }
    pi = best;
  }
}

// The block's tokens: [anchor, mask × (block − 1)], the anchor from vtok[0].
__global__ void dtok_kernel(const uint32_t* __restrict__ vtok, uint32_t mask, int B, uint32_t* __restrict__ dtok) {
  const int i = threadIdx.x;
  if (i < B) dtok[i] = i == 0 ? vtok[0] : mask;
}

// ---------------------------------------------------------------------------------------------------------------
static int dalloc(void** p, size_t bytes) {
  if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) return fail(IH_ENOMEM, "drafter: allocation failed");
  return IH_OK;
}
template <typename T>
static int dalloc_t(T** p, size_t n) {
  void* v = nullptr;
  IH_TRY(dalloc(&v, n * sizeof(T)));
  *p = static_cast<T*>(v);
  return IH_OK;
}

// The target model is being freed: its drafters stay allocated for ih_drafter_free but refuse further work.
void model_drafters_orphan(ih_model* m) {
  for (ih_drafter* r : m->drafters) r->target = nullptr;
  m->drafters.clear();
  m->drafter = nullptr;
}

static void drafter_release(ih_drafter* r) {
  if (!r) return;
  for (auto& L : r->layers) {
    for (ih_qmat* q : {L.qkv, L.kv, L.o, L.gu, L.down, L.aproj, L.mproj}) ih_qmat_free(q);
    for (void* p : {(void*)L.n1, (void*)L.n2, (void*)L.qn, (void*)L.kn, (void*)L.abase, (void*)L.mbase, (void*)L.kc,
                    (void*)L.vc})
      if (p) (void)hipFree(p);
  }
  ih_qmat_free(r->fc);
  ih_qmat_free(r->hproj);
  for (void* p : {(void*)r->hnorm, (void*)r->fnorm, (void*)r->pred, (void*)r->succ, (void*)r->caps, (void*)r->dtok, (void*)r->rope,
                  (void*)r->x, (void*)r->proj, (void*)r->dyn, (void*)r->y, (void*)r->gu, (void*)r->logits,
                  (void*)r->hp, (void*)r->xn, (void*)r->q, (void*)r->opart, (void*)r->ml, (void*)r->cidx,
                  (void*)r->cval, (void*)r->cz, (void*)r->conf, (void*)r->esel})
    if (p) (void)hipFree(p);
  for (ActBuf* a : {&r->act_h, &r->act_a, &r->act_i, &r->act_c, &r->act_f}) free_act(*a);
  delete r;
}

// An MLX int4 matrix from the synthetic streams; `rows` (when set) keeps the row range [r0, r0 + n) of an N-row
// tensor (the k|v rows of q|k|v).
static int dsynth_qmat(ih_ctx* c, int N, int K, uint64_t seed, uint64_t tensor, ih_qmat** out, int r0 = 0,
                       int n = -1) {
  uint32_t* w = nullptr;
  uint16_t *s = nullptr, *b = nullptr;
  IH_TRY(dalloc_t(&w, size_t(N) * K / 8));
  int st = dalloc_t(&s, size_t(N) * K / 64);
  if (st == IH_OK) st = dalloc_t(&b, size_t(N) * K / 64);
  if (st == IH_OK) st = synth_int4(c, w, s, b, N, K, seed, tensor, 0.02f);
  if (n < 0) n = N;
  if (st == IH_OK)
    st = qmat_int4_create_dev(c, w + size_t(r0) * K / 8, s + size_t(r0) * K / 64, b + size_t(r0) * K / 64, 1, n, K, 0,
                              out);
  (void)hipStreamSynchronize(c->stream);
  for (void* p : {(void*)w, (void*)s, (void*)b})
    if (p) (void)hipFree(p);
  return st;
}

// The shapes the drafter kernels run (DFlash2Drafter's mismatch rules for the shapes this build supports).
static int drafter_check(const ih_model* target, const ih_drafter_desc& d, const std::string& who) {
  const ih_model_desc& td = target->d;
  IH_CHECK(d.n_layers >= 1 && d.hidden == td.hidden, IH_EINVAL,
           who + "the drafter's hidden size must be the target's (it uses its embedding and head)");
  IH_CHECK(d.head_dim == 64 || d.head_dim == 128, IH_EINVAL, who + "head_dim must be 64 or 128");
  IH_CHECK(d.n_q_heads >= DKVH && d.n_q_heads % DKVH == 0 && d.n_q_heads * d.head_dim % 512 == 0, IH_EINVAL,
           who + "q heads must be a multiple of the 8 KV heads (q heads · head_dim % 512 == 0)");
  IH_CHECK(d.block >= 2 && d.block <= 16 && d.n_q_heads / DKVH * d.block <= 64, IH_EINVAL,
           who + "block must be in 2..16 with (q heads / 8)·block ≤ 64");
  IH_CHECK(d.window >= d.block && d.window % 32 == 0, IH_EINVAL,
           who + "window must be a multiple of 32, at least the block");
  IH_CHECK(d.hidden % 64 == 0 && d.intermediate >= 64 && d.intermediate % 64 == 0, IH_EINVAL,
           who + "hidden and intermediate must be multiples of 64");
  IH_CHECK(d.n_targets >= 1 && d.n_targets <= IH_DRAFTER_MAX_TARGETS, IH_EINVAL, who + "1..8 target layers");
  for (int j = 0; j < d.n_targets; ++j)
    IH_CHECK(d.target_layers[j] >= 0 && d.target_layers[j] < td.n_layers, IH_EINVAL,
             who + "a target layer is outside the target model");
  IH_CHECK(d.rank == 0 || (d.rank % 64 == 0 && d.rank <= 1024), IH_EINVAL,
           who + "rank must be 0 or a multiple of 64 up to 1024");
  IH_CHECK(d.mask_token < uint32_t(td.vocab), IH_EINVAL, who + "mask token beyond the vocabulary");
  return IH_OK;
}

static ih_drafter* drafter_new(ih_model* target, const ih_drafter_desc& d) {
  ih_drafter* r = new ih_drafter();
  r->ctx = target->ctx;
  r->d = d;
  r->target = target;
  r->QP = (d.n_q_heads + 2 * DKVH) * d.head_dim;
  r->G = d.n_q_heads / DKVH;
  r->slots = (d.window + 16 + 31) / 32 * 32;
  r->DYN = 4 * (d.hidden / DCG);
  r->layers.resize(d.n_layers);
  return r;
}

// The context rings and the scratch of one pass, then registration with the target (st: the weights' status).
static int drafter_finish(ih_drafter* r, int st, ih_drafter** out) {
  ih_ctx* c = r->ctx;
  const auto& d = r->d;
  const ih_model_desc& td = r->target->d;
  const int H = d.hidden, HD = d.head_dim, QH = d.n_q_heads, I = d.intermediate, V = td.vocab;
  auto run = [&](int s) { if (st == IH_OK) st = s; };
  for (auto& L : r->layers) {
    run(dalloc_t(&L.kc, size_t(DKVH) * r->slots * HD));
    run(dalloc_t(&L.vc, size_t(DKVH) * r->slots * HD));
    if (st == IH_OK) run(fill(c, L.kc, 0, size_t(DKVH) * r->slots * HD * 2));
    if (st == IH_OK) run(fill(c, L.vc, 0, size_t(DKVH) * r->slots * HD * 2));
  }
  const int nchunk = (r->slots + DCHUNK - 1) / DCHUNK, Q = r->G * d.block;
  run(dalloc_t(&r->caps, size_t(MAX_TOK) * d.n_targets * td.hidden));
  run(dalloc_t(&r->dtok, 16));
  run(dalloc_t(&r->rope, size_t(IH_MAX_ROWS) * HD / 2));
  run(dalloc_t(&r->x, size_t(MAX_TOK) * H));
  run(dalloc_t(&r->proj, size_t(MAX_TOK) * r->QP));
  run(dalloc_t(&r->dyn, size_t(MAX_TOK) * r->DYN));
  run(dalloc_t(&r->y, size_t(MAX_TOK) * H));
  run(dalloc_t(&r->gu, size_t(MAX_TOK) * 2 * I));
  run(dalloc_t(&r->logits, size_t(16) * V));
  run(dalloc_t(&r->hp, size_t(16) * std::max(d.rank, 1)));
  run(dalloc_t(&r->xn, size_t(MAX_TOK) * H));
  run(dalloc_t(&r->q, size_t(DKVH) * Q * HD));
  run(dalloc_t(&r->opart, size_t(DKVH) * nchunk * Q * HD));
  run(dalloc_t(&r->ml, size_t(DKVH) * nchunk * Q));
  run(dalloc_t(&r->cidx, size_t(16) * IH_TOPK));
  run(dalloc_t(&r->cval, size_t(16) * IH_TOPK));
  run(dalloc_t(&r->cz, 32));
  run(dalloc_t(&r->conf, 16));
  run(dalloc_t(&r->esel, size_t(16) * DSEL));
  if (st == IH_OK) run(ensure_act(c, r->act_h, H, false));
  if (st == IH_OK) run(ensure_act(c, r->act_a, QH * HD, false));
  if (st == IH_OK) run(ensure_act(c, r->act_i, I, false));
  if (st == IH_OK) run(ensure_act(c, r->act_c, d.n_targets * td.hidden, false));
  if (st == IH_OK) run(ensure_act(c, r->act_f, H, false));
  if (st == IH_OK) run(fill(c, r->caps, 0, size_t(MAX_TOK) * d.n_targets * td.hidden * 2));
  if (st == IH_OK && hipStreamSynchronize(c->stream) != hipSuccess) st = fail(IH_EDEVICE, "drafter: creation failed");
  if (st != IH_OK) {
    (void)hipStreamSynchronize(c->stream);
    drafter_release(r);
    return st;
  }
  r->target->drafters.push_back(r);  // registered only once complete (a failed creation is released above)
  *out = r;
  return IH_OK;
}

}  // namespace ih

extern "C" {

int ih_drafter_create_synthetic(ih_model* target, const ih_drafter_desc* desc, uint64_t seed, ih_drafter** out) {
  IH_CHECK(target && desc && out, IH_EINVAL, "ih_drafter_create_synthetic: null argument");
  *out = nullptr;
  IH_TRY(drafter_check(target, *desc, "ih_drafter_create_synthetic: "));
  ih_drafter* r = drafter_new(target, *desc);
  ih_ctx* c = target->ctx;
  const auto& d = r->d;
  const int H = d.hidden, HD = d.head_dim, QH = d.n_q_heads, I = d.intermediate, V = target->d.vocab;
  int st = IH_OK;
  auto run = [&](int s) { if (st == IH_OK) st = s; };
  for (int l = 0; l < d.n_layers && st == IH_OK; ++l) {
    ih_drafter_layer& L = r->layers[l];
    run(dalloc_t(&L.n1, H));
    run(dalloc_t(&L.n2, H));
    run(dalloc_t(&L.qn, HD));
    run(dalloc_t(&L.kn, HD));
    if (st != IH_OK) break;
    run(synth_bf16(c, L.n1, H, seed, dl_tensor(l, D_N1), 1.0f, 0.125f));
    run(synth_bf16(c, L.n2, H, seed, dl_tensor(l, D_N2), 1.0f, 0.125f));
    run(synth_bf16(c, L.qn, HD, seed, dl_tensor(l, D_QN), 1.0f, 0.125f));
    run(synth_bf16(c, L.kn, HD, seed, dl_tensor(l, D_KN), 1.0f, 0.125f));
    run(dsynth_qmat(c, r->QP, H, seed, dl_tensor(l, D_QKV), &L.qkv));
    run(dsynth_qmat(c, r->QP, H, seed, dl_tensor(l, D_QKV), &L.kv, QH * HD, 2 * DKVH * HD));
    run(dsynth_qmat(c, H, QH * HD, seed, dl_tensor(l, D_O), &L.o));
    run(dsynth_qmat(c, 2 * I, H, seed, dl_tensor(l, D_GU), &L.gu));
    run(dsynth_qmat(c, H, I, seed, dl_tensor(l, D_DOWN), &L.down));
    if (d.dyn_conv) {
      run(dsynth_qmat(c, r->DYN, H, seed, dl_tensor(l, D_APROJ), &L.aproj));
      run(dsynth_qmat(c, r->DYN, H, seed, dl_tensor(l, D_MPROJ), &L.mproj));
      run(dalloc_t(&L.abase, 4 * H));
      run(dalloc_t(&L.mbase, 4 * H));
      // Taps: [prep|finish][tap][H]; the current tap near 1, the previous near 0.
      for (int k = 0; k < 4 && st == IH_OK; ++k) {
        run(synth_bf16(c, L.abase + k * H, H, seed, dl_tensor(l, D_ABASE) + 100 * k, k % 2 ? 0.0f : 1.0f, 0.1f));
        run(synth_bf16(c, L.mbase + k * H, H, seed, dl_tensor(l, D_MBASE) + 100 * k, k % 2 ? 0.0f : 1.0f, 0.1f));
      }
    }
  }
  run(dsynth_qmat(c, H, d.n_targets * target->d.hidden, seed, dg_tensor(D_FC), &r->fc));
  run(dalloc_t(&r->hnorm, H));
  run(dalloc_t(&r->fnorm, H));
  if (st == IH_OK) run(synth_bf16(c, r->hnorm, H, seed, dg_tensor(D_HNORM), 1.0f, 0.125f));
  if (st == IH_OK) run(synth_bf16(c, r->fnorm, H, seed, dg_tensor(D_FNORM), 1.0f, 0.125f));
  if (d.rank > 0) {
    run(dsynth_qmat(c, d.rank, H, seed, dg_tensor(D_HPROJ), &r->hproj));
    run(dalloc_t(&r->pred, size_t(V) * d.rank));
    run(dalloc_t(&r->succ, size_t(V) * d.rank));
    if (st == IH_OK) run(synth_bf16(c, r->pred, size_t(V) * d.rank, seed, dg_tensor(D_PRED), 0.0f, 0.25f));
    if (st == IH_OK) run(synth_bf16(c, r->succ, size_t(V) * d.rank, seed, dg_tensor(D_SUCC), 0.0f, 0.25f));
  }
  return drafter_finish(r, st, out);
}

int ih_drafter_load_mlx(ih_model* target, const char* dir, ih_drafter** out) {
  IH_CHECK(target && dir && out, IH_EINVAL, "ih_drafter_load_mlx: null argument");
  *out = nullptr;
  DrafterCkpt ck;
  IH_TRY(read_drafter_mlx(dir, target->d, ck));
  IH_TRY(drafter_check(target, ck.d, "ih_drafter_load_mlx: "));
  ih_drafter* r = drafter_new(target, ck.d);
  ih_ctx* c = target->ctx;
  const auto& d = r->d;
  const int QH = d.n_q_heads, HD = d.head_dim;
  int st = IH_OK;
  auto run = [&](int s) { if (st == IH_OK) st = s; };
  auto q4 = [&](const HostQ4& h, ih_qmat** q) {
    run(ih_qmat_int4_create(c, h.w.data(), h.s.data(), h.b.data(), 1, h.N, h.K, q));
  };
  auto vec = [&](const std::vector<uint16_t>& v, uint16_t** p) {
    run(dalloc_t(p, v.size()));
    if (st == IH_OK)
      run(hipMemcpy(*p, v.data(), v.size() * 2, hipMemcpyHostToDevice) == hipSuccess
              ? IH_OK : fail(IH_EDEVICE, "ih_drafter_load_mlx: upload failed"));
  };
  for (int l = 0; l < d.n_layers && st == IH_OK; ++l) {
    ih_drafter_layer& L = r->layers[l];
    const DrafterLayerCkpt& K = ck.layers[l];
    vec(K.n1, &L.n1);
    vec(K.n2, &L.n2);
    vec(K.qn, &L.qn);
    vec(K.kn, &L.kn);
    q4(K.qkv, &L.qkv);
    q4(K.qkv.rows(QH * HD, 2 * DKVH * HD), &L.kv);
    q4(K.o, &L.o);
    q4(K.gu, &L.gu);
    q4(K.down, &L.down);
    if (d.dyn_conv) {
      q4(K.aproj, &L.aproj);
      q4(K.mproj, &L.mproj);
      vec(K.abase, &L.abase);
      vec(K.mbase, &L.mbase);
    }
  }
  q4(ck.fc, &r->fc);
  vec(ck.hnorm, &r->hnorm);
  vec(ck.fnorm, &r->fnorm);
  if (d.rank > 0) {
    q4(ck.hproj, &r->hproj);
    vec(ck.pred, &r->pred);
    vec(ck.succ, &r->succ);
  }
  return drafter_finish(r, st, out);
}

int ih_drafter_free(ih_drafter* r) {
  if (!r) return IH_OK;
  (void)hipStreamSynchronize(r->ctx->stream);
  ++r->ctx->gen;
  if (ih_model* t = r->target) {
    if (t->drafter == r) t->drafter = nullptr;
    t->drafters.erase(std::remove(t->drafters.begin(), t->drafters.end(), r), t->drafters.end());
  }
  drafter_release(r);
  return IH_OK;
}

int ih_model_set_drafter(ih_model* m, ih_drafter* r) {
  IH_CHECK(m, IH_EINVAL, "ih_model_set_drafter: null model");
  IH_CHECK(!r || r->target, IH_EINVAL, "ih_model_set_drafter: the drafter's target model was freed");
  IH_CHECK(!r || r->target == m, IH_EINVAL, "ih_model_set_drafter: the drafter was made for another model");
  if (m->drafter != r) ++m->ctx->gen;
  m->drafter = r;
  return IH_OK;
}

int ih_drafter_context(ih_drafter* r, int rows, int nvalid, int pos0, const uint32_t* st_dev) {
  IH_CHECK(r, IH_EINVAL, "ih_drafter_context: null drafter");
  IH_CHECK(r->target, IH_EINVAL, "ih_drafter_context: the drafter's target model was freed");
  IH_CHECK(rows >= 1 && rows <= IH_MAX_ROWS, IH_EINVAL, "ih_drafter_context: rows must be in 1..17");
  IH_CHECK(st_dev || (nvalid >= 0 && nvalid <= rows && pos0 >= 0), IH_EINVAL, "ih_drafter_context: bad nvalid/pos0");
  ih_ctx* c = r->ctx;
  const auto& d = r->d;
  const int H = d.hidden, HD = d.head_dim, Ht = r->target->d.hidden;
  // fc over the captures, RMSNorm (hidden_norm), then each layer's k|v into its ring.
  IH_TRY(launch_act_from_bf16(c, r->caps, d.n_targets * Ht, rows, r->act_c));
  IH_TRY(launch_qmm(c, r->fc, 0, r->act_c, rows, r->y, H, QM_F32));
  dnorm_kernel<<<rows, 256, 0, c->stream>>>(r->y, H, r->hnorm, d.rms_eps, 0, static_cast<uint4*>(r->act_h.frag),
                                            r->act_h.nkb, r->act_h.ntile, nullptr);
  IH_HIP(hipGetLastError());
  for (auto& L : r->layers) {
    IH_TRY(launch_qmm(c, L.kv, 0, r->act_h, rows, r->proj, 2 * DKVH * HD, QM_F32));
    if (HD == 128)
      dctx_kernel<128><<<dim3(4, rows), 256, 0, c->stream>>>(r->proj, L.kn, L.kc, L.vc, d.window, r->slots, d.rms_eps,
                                                             d.rope_theta, st_dev, nvalid, pos0);
    else
      dctx_kernel<64><<<dim3(4, rows), 256, 0, c->stream>>>(r->proj, L.kn, L.kc, L.vc, d.window, r->slots, d.rms_eps,
                                                            d.rope_theta, st_dev, nvalid, pos0);
    IH_HIP(hipGetLastError());
  }
  return IH_OK;
}

int ih_drafter_block(ih_drafter* r, uint32_t* vtok_dev, int P, const uint32_t* st_dev, float* conf_dev) {
  IH_CHECK(r && vtok_dev, IH_EINVAL, "ih_drafter_block: null argument");
  IH_CHECK(r->target, IH_EINVAL, "ih_drafter_block: the drafter's target model was freed");
  IH_CHECK(st_dev || P >= 0, IH_EINVAL, "ih_drafter_block: negative position");
  ih_ctx* c = r->ctx;
  const auto& d = r->d;
  ih_model* t = r->target;
  const int B = d.block, M = B - 1, H = d.hidden, HD = d.head_dim, QH = d.n_q_heads, I = d.intermediate;
  const int V = t->d.vocab, Q = r->G * B, nchunk = (r->slots + DCHUNK - 1) / DCHUNK, G = H / DCG;
  dtok_kernel<<<1, 64, 0, c->stream>>>(vtok_dev, d.mask_token, B, r->dtok);
  IH_HIP(hipGetLastError());
  // Embedding of the block with the target's table into fp32 rows (the kernel's other outputs, an activation and a
  // RoPE table, go to drafter scratch and are not used).
  IH_TRY(launch_embed_act(c, r->dtok, t->emb_w, t->emb_s, t->emb_b, r->x, B, H, V, r->fnorm, r->act_f, r->rope, 0,
                          d.rope_theta, HD / 2, nullptr, 0));
  DAttn a{};
  a.qkv = r->proj;
  a.QP = r->QP;
  a.QH = QH;
  a.G = r->G;
  a.HD = HD;
  a.B = B;
  a.win = d.window;
  a.slots = r->slots;
  a.q = r->q;
  a.eps = d.rms_eps;
  a.theta = d.rope_theta;
  a.st = st_dev;
  a.P = P;
  const bool conv = d.dyn_conv != 0;
  // The first layer's attention norm; every later norm is launched with the conv that precedes it.
  dnorm_kernel<<<B, 256, 0, c->stream>>>(r->x, H, r->layers[0].n1, d.rms_eps, 0, static_cast<uint4*>(r->act_h.frag),
                                         r->act_h.nkb, r->act_h.ntile, conv ? r->xn : nullptr);
  IH_HIP(hipGetLastError());
  for (size_t li = 0; li < r->layers.size(); ++li) {
    auto& L = r->layers[li];
    const bool last = li + 1 == r->layers.size();
    if (conv) {
      IH_TRY(launch_qmm(c, L.aproj, 0, r->act_h, B, r->dyn, r->DYN, QM_F32));
      dconv_prep_kernel<<<B, 256, 0, c->stream>>>(r->xn, r->dyn, r->DYN, L.abase, H, G,
                                                  static_cast<uint4*>(r->act_h.frag), r->act_h.nkb, r->act_h.ntile);
      IH_HIP(hipGetLastError());
    }
    IH_TRY(launch_qmm(c, L.qkv, 0, r->act_h, B, r->proj, r->QP, QM_F32));
    a.qn = L.qn;
    a.kn = L.kn;
    a.kc = L.kc;
    a.vc = L.vc;
    const dim3 pg((QH + 2 * DKVH + 3) / 4, B);
    if (HD == 128) {
      dprework_kernel<128><<<pg, 256, 0, c->stream>>>(a);
      dattn_kernel<128><<<dim3(nchunk, DKVH), 256, 0, c->stream>>>(a, r->opart, r->ml, nchunk);
    } else {
      dprework_kernel<64><<<pg, 256, 0, c->stream>>>(a);
      dattn_kernel<64><<<dim3(nchunk, DKVH), 256, 0, c->stream>>>(a, r->opart, r->ml, nchunk);
    }
    IH_HIP(hipGetLastError());
    dattn_reduce_kernel<<<dim3(B, QH), HD / 8, 0, c->stream>>>(r->opart, r->ml, nchunk, r->G, B, HD,
                                                                static_cast<uint4*>(r->act_a.frag), r->act_a.nkb,
                                                                r->act_a.ntile);
    IH_HIP(hipGetLastError());
    IH_TRY(launch_qmm(c, L.o, 0, r->act_a, B, r->y, H, QM_F32));
    // The conv into the residual and the MLP sublayer's norm.
    dfin_norm_kernel<<<B, 256, 0, c->stream>>>(r->y, conv ? r->dyn : nullptr, r->DYN, L.abase, H, G, r->x, L.n2,
                                               d.rms_eps, 0, static_cast<uint4*>(r->act_h.frag), r->act_h.nkb,
                                               r->act_h.ntile, conv ? r->xn : nullptr);
    IH_HIP(hipGetLastError());
    if (conv) {
      IH_TRY(launch_qmm(c, L.mproj, 0, r->act_h, B, r->dyn, r->DYN, QM_F32));
      dconv_prep_kernel<<<B, 256, 0, c->stream>>>(r->xn, r->dyn, r->DYN, L.mbase, H, G,
                                                  static_cast<uint4*>(r->act_h.frag), r->act_h.nkb, r->act_h.ntile);
      IH_HIP(hipGetLastError());
    }
    IH_TRY(launch_qmm(c, L.gu, 0, r->act_h, B, r->gu, 2 * I, QM_F32));
    dswiglu_kernel<<<B, 256, 0, c->stream>>>(r->gu, I, static_cast<uint4*>(r->act_i.frag), r->act_i.nkb,
                                             r->act_i.ntile);
    IH_HIP(hipGetLastError());
    IH_TRY(launch_qmm(c, L.down, 0, r->act_i, B, r->y, H, QM_F32));
    // The conv into the residual and the next layer's attention norm, after the last layer the final norm of rows
    // 1 … B − 1.
    if (!last)
      dfin_norm_kernel<<<B, 256, 0, c->stream>>>(r->y, conv ? r->dyn : nullptr, r->DYN, L.mbase, H, G, r->x,
                                                 r->layers[li + 1].n1, d.rms_eps, 0,
                                                 static_cast<uint4*>(r->act_h.frag), r->act_h.nkb, r->act_h.ntile,
                                                 conv ? r->xn : nullptr);
    else
      dfin_norm_kernel<<<B, 256, 0, c->stream>>>(r->y, conv ? r->dyn : nullptr, r->DYN, L.mbase, H, G, r->x,
                                                 r->fnorm, d.rms_eps, 1, static_cast<uint4*>(r->act_f.frag),
                                                 r->act_f.nkb, r->act_f.ntile, nullptr);
    IH_HIP(hipGetLastError());
  }
  // The target's head over rows 1 … B − 1, the top-16 candidates and the selector.
  IH_TRY(launch_qmm(c, t->head, 0, r->act_f, M, r->logits, V, QM_F32));
  IH_TRY(launch_topk64(c, r->logits, V, M, V, 1.0f, r->cidx, r->cval, r->cz));
  if (d.rank > 0) IH_TRY(launch_qmm(c, r->hproj, 0, r->act_f, M, r->hp, d.rank, QM_F32));
  if (d.rank > 0) {
    dselect_pairs_kernel<<<dim3(M, DTOPK), d.rank, 0, c->stream>>>(r->cidx, IH_TOPK, r->hp, r->pred, r->succ, d.rank,
                                                                   vtok_dev, r->esel);
    IH_HIP(hipGetLastError());
  }
  dselect_kernel<<<1, 256, 0, c->stream>>>(r->cidx, r->cval, IH_TOPK, d.rank > 0 ? r->esel : nullptr, vtok_dev, M,
                                          conf_dev ? conf_dev : r->conf);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

const uint16_t* ih_drafter_captures_dev(const ih_drafter* r) { return r ? r->caps : nullptr; }

int ih_drafter_block_rows(const ih_drafter* r) { return r ? r->d.block : 0; }

int ih_drafter_describe(const ih_drafter* r, ih_drafter_desc* out) {
  IH_CHECK(r && out, IH_EINVAL, "ih_drafter_describe: null argument");
  *out = r->d;
  return IH_OK;
}

}  // extern "C"

namespace ih {
// The verify step's captures: the residual rows after each target layer (capture_rows).
int drafter_capture(ih_model* m, int layer, int B) {
  ih_drafter* r = m->drafter;
  if (!r) return IH_OK;
  for (int j = 0; j < r->d.n_targets; ++j) {
    if (r->d.target_layers[j] != layer) continue;
    capture_kernel<<<B, 256, 0, m->ctx->stream>>>(m->h, m->d.hidden, r->caps, r->d.n_targets * m->d.hidden,
                                                  j * m->d.hidden);
    IH_HIP(hipGetLastError());
  }
  return IH_OK;
}
}  // namespace ih
