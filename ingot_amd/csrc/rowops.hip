// Row kernels of the verify round: embedding gather, RMSNorm into the qmm activation layout, the gated activation,
// vocab-wide argmax and greedy acceptance.
#include "act.h"
#include "lanes.h"
#include "ih_internal.h"

namespace ih {

// ---------------------------------------------------------------------------------------------------------------
// Embedding of the block's rows: h[r] = dequant(table[tok[r]]) in fp32 (MLX int4 g64 row; embed_rows,
// Shaders/yy_model.metal:12-49), and the first layer's RMSNorm input: the activation bf16(h ⊙ w) and Σh² per row
// (one partial). Also the step's RoPE table (the rotation angles depend only on the position, so every layer's
// prework reads them): rope[r][i] = (cos, sin)(pos · θ^(−i/RH)), pos = P + r, evaluated in double (a scaled RoPE:
// pos · inv_freq[i] and both times mscale). Grid (2·rows), 256
// threads: workgroup r < rows embeds row r (one thread per 8 values), workgroup rows + r evaluates row r's angles
// (double pow, cos and sin take longer than the embedding, so the two run side by side).
__global__ __launch_bounds__(256) void embed_act_kernel(const uint32_t* __restrict__ tok, const uint32_t* __restrict__ w,
                                                        const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                                                        float* __restrict__ h, int H, int ldh,
                                                        const uint16_t* __restrict__ nw, uint4* __restrict__ frag,
                                                        int nkb, int ntile, float* __restrict__ ss_out, int V,
                                                        float2* __restrict__ rope, int P, float theta, int RH,
                                                        const uint32_t* __restrict__ pos_dev, int pos_max,
                                                        const float* __restrict__ rinv, float rmscale) {
  __shared__ float red[4];
  const int rows = gridDim.x / 2;
  if (int(blockIdx.x) >= rows) {  // workgroup-uniform
    const int row = blockIdx.x - rows;
    if (pos_dev) P = int(min(pos_dev[0], uint32_t(pos_max)));  // chained rounds: the position of the round state
    if (rinv) {
      // A scaled RoPE (RopeTable): the pair's fp32 frequency, the angle in double, cos and sin times mscale.
      for (int i = threadIdx.x; i < RH; i += blockDim.x) {
        const double ang = double(P + row) * double(rinv[i]);
        rope[row * RH + i] = make_float2(float(cos(ang) * double(rmscale)), float(sin(ang) * double(rmscale)));
      }
      return;
    }
    for (int i = threadIdx.x; i < RH; i += blockDim.x) {
      const double ang = double(P + row) * pow(double(theta), -double(i) / double(RH));
      rope[row * RH + i] = make_float2(float(cos(ang)), float(sin(ang)));
    }
    return;
  }
  const int row = blockIdx.x;
  // Ids beyond the vocabulary (the device entry points cannot check them on the host) read the last row instead of
  // memory past the table.
  const uint32_t t = min(tok[row], uint32_t(V - 1));
  const uint32_t* wr = w + size_t(t) * (H / 8);
  float ss = 0.f;
  for (int c = threadIdx.x; c < H / 8; c += blockDim.x) {
    const uint32_t word = wr[c];
    const size_t g = size_t(t) * (H / 64) + c / 8;
    const float sc = dbf16(s[g]), bi = dbf16(b[g]);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = sc * float((word >> (4 * j)) & 15u) + bi;
      h[size_t(row) * ldh + 8 * c + j] = x;
      ss += x * x;
      v[j] = x * dbf16(nw[8 * c + j]);
    }
    frag_store_chunk(frag, nkb, ntile, row, c, v);
  }
  ss += lane_xor<32>(ss);
  ss += lane_xor<16>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<1>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) ss_out[size_t(row) * SS_CAP] = ((red[0] + red[1]) + (red[2] + red[3]));
}

// ---------------------------------------------------------------------------------------------------------------
// argmax per row, ties to the lowest index, NaN never wins: argmax_rows, Shaders/verify.metal:525-547. Two passes: grid
// (rows, ARGMAX_CHUNKS) workgroups of 256 threads each reduce a contiguous chunk of the row with 16-byte loads, four
// in flight per thread (a row per workgroup left 17 CUs to stream 10 MB one load at a time), then one wave per row
// merges the chunks in order.
constexpr int ARGMAX_CHUNKS = 16;

// (v, i) beats (m, mi): larger value, or equal value and lower index. NaN never beats, and −inf never takes an index
// (the reference scans from (−inf, 0) with a strict >, so a row of −inf and NaN gives index 0).
__device__ __forceinline__ bool am_better(float v, uint32_t i, float m, uint32_t mi) {
  return v > m || (v == m && i < mi && v != -INFINITY);
}

// (value, index) maximum over the wave under am_better, partners at distance 32, 16, …, 1 (every lane active).
__device__ __forceinline__ void am_butterfly(float& m, uint32_t& mi) {
  auto step = [&](auto hc) {
    constexpr int H = decltype(hc)::value;
    const float om = lane_xor<H>(m);
    const uint32_t oi = __float_as_uint(lane_xor<H>(__uint_as_float(mi)));
    if (am_better(om, oi, m, mi)) { m = om; mi = oi; }
  };
  step(std::integral_constant<int, 32>{});
  step(std::integral_constant<int, 16>{});
  step(std::integral_constant<int, 8>{});
  step(std::integral_constant<int, 4>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 1>{});
}

__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float* __restrict__ x, int ldx, int N,
                                                           float2* __restrict__ part) {
  __shared__ float bv[4];
  __shared__ uint32_t bi[4];
  const int row = blockIdx.x, ch = blockIdx.y;
  const int per = (N + ARGMAX_CHUNKS - 1) / ARGMAX_CHUNKS;
  const int c0 = ch * per, c1 = min(N, c0 + per);
  const float* xr = x + size_t(row) * ldx;
  float m = -INFINITY;
  uint32_t mi = 0xFFFFFFFFu;
  // Aligned 16-byte body [a0, a1) of the chunk (ldx and the row start are 16-byte aligned when ldx % 4 == 0), scalar
  // head and tail.
  const int a0 = (ldx % 4 == 0) ? min(c1, (c0 + 3) & ~3) : c1, a1 = (ldx % 4 == 0) ? max(a0, c1 & ~3) : c1;
  for (int i = c0 + int(threadIdx.x); i < a0; i += 256) {
    const float v = xr[i];
    if (am_better(v, uint32_t(i), m, mi)) { m = v; mi = uint32_t(i); }
  }
  for (int i0 = a0 + 4 * int(threadIdx.x); i0 < a1; i0 += 4 * 256 * 4) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + 4 * 256 * u;
      v[u] = i < a1 ? *reinterpret_cast<const float4*>(xr + i) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t i = uint32_t(i0 + 4 * 256 * u);
      if (am_better(v[u].x, i, m, mi)) { m = v[u].x; mi = i; }
      if (am_better(v[u].y, i + 1, m, mi)) { m = v[u].y; mi = i + 1; }
      if (am_better(v[u].z, i + 2, m, mi)) { m = v[u].z; mi = i + 2; }
      if (am_better(v[u].w, i + 3, m, mi)) { m = v[u].w; mi = i + 3; }
    }
  }
  for (int i = a1 + int(threadIdx.x); i < c1; i += 256) {
    const float v = xr[i];
    if (am_better(v, uint32_t(i), m, mi)) { m = v; mi = uint32_t(i); }
  }
  am_butterfly(m, mi);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { bv[wave] = m; bi[wave] = mi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = bv[0];
    uint32_t ix = bi[0];
    for (int w = 1; w < 4; ++w)
      if (am_better(bv[w], bi[w], b, ix)) { b = bv[w]; ix = bi[w]; }
    part[row * ARGMAX_CHUNKS + ch] = make_float2(b, __uint_as_float(ix));
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float2* __restrict__ part, uint32_t* __restrict__ out) {
  const int row = blockIdx.x, l = threadIdx.x;
  float m = -INFINITY;
  uint32_t mi = 0xFFFFFFFFu;
  if (l < ARGMAX_CHUNKS) {
    const float2 p = part[row * ARGMAX_CHUNKS + l];
    m = p.x;
    mi = __float_as_uint(p.y);
  }
  am_butterfly(m, mi);
  if (l == 0) out[row] = mi == 0xFFFFFFFFu ? 0u : mi;  // all NaN / −inf: index 0, as the reference
}

// ---------------------------------------------------------------------------------------------------------------
// Greedy acceptance on the device, one thread: m = drafts vtok[1..m] that equal top1[0..m−1]; rec[round % ring] = (m,
// emitted tokens, REC_P = P before, REC_ROWS = rows); st = [P, nacc, pend, pendPos, anchor, round, rows] advanced:
// P += m + 1 (the commit), anchor = top1[m], vtok[0] = anchor. spec_accept, Shaders/yy_model.metal:616-642.
__global__ void accept_kernel(uint32_t* st, uint32_t* vtok, const uint32_t* top1, uint32_t* rec, int ring, int rows,
                              uint32_t* hist, int hist_cap) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  // Rows from the round state (rows = 0) are clamped to 1…IH_MAX_ROWS: vtok, top1 and a record hold at most that many.
  const uint32_t nr = rows ? uint32_t(rows) : min(max(st[6], 1u), uint32_t(IH_MAX_ROWS));
  uint32_t m = 0;
  while (m + 1 < nr && vtok[m + 1] == top1[m]) ++m;
  uint32_t* r = rec + (st[5] % uint32_t(ring)) * IH_REC_STRIDE;
  r[0] = m;
  r[IH_REC_ROWS] = nr;
  for (uint32_t i = 1; i <= m; ++i) r[i] = vtok[i];
  r[m + 1] = top1[m];
  r[IH_REC_P] = st[0];
  st[3] = st[0];
  st[2] = m + 1;
  st[0] += m + 1;
  st[1] = m + 1;
  st[4] = top1[m];
  st[5] += 1;
  vtok[0] = top1[m];
  // The token history of the copy drafter (hist[i] = token at position i, the anchor last): the emitted tokens go to
  // the positions after the old anchor (the dtok write of the reference, the drafter's side of the round).
  if (hist) {
    const uint32_t p0 = st[3];  // P before this round
    for (uint32_t i = 0; i < m; ++i)
      if (p0 + 1 + i < uint32_t(hist_cap)) hist[p0 + 1 + i] = vtok[1 + i];
    if (p0 + 1 + m < uint32_t(hist_cap)) hist[p0 + 1 + m] = top1[m];
  }
}

// ---------------------------------------------------------------------------------------------------------------
int launch_embed_act(ih_ctx* c, const uint32_t* tok, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     float* h, int B, int H, int V, const uint16_t* nw, ActBuf& a, float2* rope, int P, float theta,
                     int RH, const uint32_t* pos_dev, int pos_max, const float* rinv, float rmscale) {
  TimedLaunch tl(c, TC_ROWS, double(B) * H * (0.5625 + 4 + 2));
  tlaunch(tl, embed_act_kernel, dim3(2 * B), dim3(256), 0, c->stream, tok, w, s, b, h, H, H, nw, static_cast<uint4*>(a.frag),
          a.nkb, a.ntile, a.ss, V, rope, P, theta, RH, pos_dev, pos_max, rinv, rmscale);
  IH_HIP(hipGetLastError());
  a.nss = 1;
  return IH_OK;
}

int launch_argmax(ih_ctx* c, const float* x, int ldx, int rows, int N, uint32_t* out) {
  IH_TRY(ensure_part(c, size_t(rows) * ARGMAX_CHUNKS * sizeof(float2)));
  float2* part = reinterpret_cast<float2*>(c->part);
  TimedLaunch tl(c, TC_ARGMAX, double(rows) * N * 4);
  tlaunch(tl, argmax_chunk_kernel, dim3(rows, ARGMAX_CHUNKS), dim3(256), 0, c->stream, x, ldx, N, part);
  IH_HIP(hipGetLastError());
  argmax_final_kernel<<<rows, 64, 0, c->stream>>>(part, out);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

// Chunk partials of ih_argmax_rows_noalloc: a static per-device array instead of the context's allocated scratch. Host
// code never passes `scratch` itself (in host code the name is a stand-in, not a device address): init_noalloc_scratch
// stores its device address, from hipGetSymbolAddress with the context's device current, and the kernels get that.
static __device__ __align__(256) float2 scratch[IH_ARGMAX_NOALLOC_MAX_ROWS * ARGMAX_CHUNKS];

int init_noalloc_scratch(ih_ctx* c) {
  void* p = nullptr;
  IH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  IH_CHECK(p != nullptr, IH_EDEVICE, "ih_init: no device address for the static argmax scratch");
  c->noalloc_scratch = p;
  return IH_OK;
}

int launch_accept(ih_ctx* c, uint32_t* st, uint32_t* vtok, const uint32_t* top1, uint32_t* rec, int ring, int rows,
                  uint32_t* hist, int hist_cap) {
  accept_kernel<<<1, 64, 0, c->stream>>>(st, vtok, top1, rec, ring, rows, hist, hist_cap);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

int ih_argmax_rows(ih_ctx* c, const float* x_dev, int rows, int N, uint32_t* out_dev) {
  IH_CHECK(c && x_dev && out_dev, IH_EINVAL, "ih_argmax_rows: null argument");
  IH_CHECK(rows >= 1 && N >= 1, IH_EINVAL, "ih_argmax_rows: empty input");
  return launch_argmax(c, x_dev, N, rows, N, out_dev);
}

int ih_argmax_rows_noalloc(ih_ctx* c, const float* x_dev, int rows, int N, uint32_t* out_dev) {
  IH_CHECK(c && x_dev && out_dev, IH_EINVAL, "ih_argmax_rows_noalloc: null argument");
  IH_CHECK(rows >= 1 && N >= 1, IH_EINVAL, "ih_argmax_rows_noalloc: empty input");
  IH_CHECK(rows <= IH_ARGMAX_NOALLOC_MAX_ROWS, IH_EINVAL,
           "ih_argmax_rows_noalloc: " + std::to_string(rows) + " rows exceed the static scratch (" +
               std::to_string(IH_ARGMAX_NOALLOC_MAX_ROWS) + " rows)");
  IH_CHECK(c->noalloc_scratch, IH_ESTATE, "ih_argmax_rows_noalloc: the context has no static scratch");
  // Every partial the final pass reads is written by the chunk pass of the same call: nothing to clear.
  float2* part = static_cast<float2*>(c->noalloc_scratch);
  argmax_chunk_kernel<<<dim3(rows, ARGMAX_CHUNKS), 256, 0, c->stream>>>(x_dev, N, N, part);
  IH_HIP(hipGetLastError());
  argmax_final_kernel<<<rows, 64, 0, c->stream>>>(part, out_dev);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int ih_accept(const uint32_t* vtok, const uint32_t* top1, int B, ih_accept_result* out) {
  IH_CHECK(vtok && top1 && out, IH_EINVAL, "ih_accept: null argument");
  IH_CHECK(B >= 1 && B <= IH_MAX_ROWS, IH_EINVAL, "ih_accept: B must be in 1..17");
  int m = 0;
  while (m + 1 < B && vtok[m + 1] == top1[m]) ++m;
  out->m = m;
  out->n_emitted = m + 1;
  for (int i = 1; i <= m; ++i) out->tokens[i - 1] = vtok[i];
  out->tokens[m] = top1[m];
  for (int i = m + 1; i < IH_MAX_ROWS; ++i) out->tokens[i] = 0;
  return IH_OK;
}

int ih_spec_accept_dev(ih_ctx* c, uint32_t* st_dev, uint32_t* vtok_dev, const uint32_t* top1_dev, uint32_t* rec_dev,
                       int ring, int rows) {
  IH_CHECK(c && st_dev && vtok_dev && top1_dev && rec_dev, IH_EINVAL, "ih_spec_accept_dev: null argument");
  IH_CHECK(ring >= 1 && rows >= 0 && rows <= IH_MAX_ROWS, IH_EINVAL, "ih_spec_accept_dev: bad ring or rows");
  return launch_accept(c, st_dev, vtok_dev, top1_dev, rec_dev, ring, rows, nullptr, 0);
}

}  // extern "C"
