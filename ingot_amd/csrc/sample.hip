// Temperature > 0 verification by rejection sampling, and the verify-row chooser, on gfx950.
//
// Reference: Shaders/zz_sample.metal:1-281 (topk64_part / topk64_merge: per row the 64 best logits, ties to the lower
// id, and the max and Σ exp((x − max)/T) over the whole vocabulary; sample_dist: temperature → top-k → min-p → top-p
// over the 64 candidates; spec_accept_sample: draft d of row i accepted with probability p_i(d), otherwise the token is
// drawn from p_i without d, so the emitted tokens follow the target distribution exactly) and spec_rows_choose
// (Shaders/yy_model.metal:644-675, SpecRows.swift: the rows with the best expected tokens per cost).
//
// MI355X design: a 64-entry list is one value per lane of a wave. Each wave keeps its sorted top-64 in registers; a
// batch of 64 new values that holds any candidate better than the list's last entry is sorted by a bitonic network of
// lane exchanges and merged (the better of list[l] and batch[63 − l] is a bitonic sequence holding the 64 best, which
// six exchange stages sort). The workgroup then merges its four waves' lists, and one wave per row merges the 32
// chunk lists the same way.
#include <cfloat>
#include <cmath>

#include "ih_internal.h"
#include "lanes.h"

namespace ih {

constexpr int SK = IH_TOPK;      // candidates per row
constexpr int SPG = 32;          // chunks (workgroups) per row
constexpr int SPT = 256;         // threads per chunk workgroup
constexpr uint32_t NO_ID = 0xFFFFFFFFu;

// (v, i) ranks before (w, j): larger value, ties to the lower id (tk_better, yy_model.metal:503).
__device__ __forceinline__ bool tk_better(float v, uint32_t i, float w, uint32_t j) {
  return (v > w) | ((v == w) & (i < j));  // no short circuit: compares and masks, no branches
}

// Compare-exchange with lane ^ J: the lane ends with the better of the pair if keep_better, else the worse. The
// partner's value and id come through DPP / row-swap lane patterns (lane_xor), not an LDS round trip; every lane of
// the wave is active wherever these run.
template <int J>
__device__ __forceinline__ void cx(float& v, uint32_t& id, bool keep_better) {
  const float ov = lane_xor<J>(v);
  const uint32_t oi = __float_as_uint(lane_xor<J>(__uint_as_float(id)));
  const bool take = (keep_better & tk_better(ov, oi, v, id)) | (!keep_better & tk_better(v, id, ov, oi));
  v = take ? ov : v;
  id = take ? oi : id;
}

// Bitonic sort of one value per lane into descending rank order (lane 0 the best).
__device__ __forceinline__ void sort64(float& v, uint32_t& id, int lane) {
#define IH_CX(K, J) cx<J>(v, id, (((lane & (J)) == 0) == ((lane & (K)) == 0)))
  IH_CX(2, 1);
  IH_CX(4, 2); IH_CX(4, 1);
  IH_CX(8, 4); IH_CX(8, 2); IH_CX(8, 1);
  IH_CX(16, 8); IH_CX(16, 4); IH_CX(16, 2); IH_CX(16, 1);
  IH_CX(32, 16); IH_CX(32, 8); IH_CX(32, 4); IH_CX(32, 2); IH_CX(32, 1);
  IH_CX(64, 32); IH_CX(64, 16); IH_CX(64, 8); IH_CX(64, 4); IH_CX(64, 2); IH_CX(64, 1);
#undef IH_CX
}

// The 64 best of two descending lists (the list in v/id, the other in bv/bi), descending, in v/id.
// x of lane 63 − lane (= lane ^ 63): the row mirror (i ^ 15 within 16 lanes), then the row swaps 16 and 32.
__device__ __forceinline__ float rev64(float x) {
  return lane_xor<32>(lane_xor<16>(__int_as_float(dpp_mov<0x140>(__float_as_int(x)))));
}

__device__ __forceinline__ void merge64(float& v, uint32_t& id, float bv, uint32_t bi, int lane) {
  const float rv = rev64(bv);
  const uint32_t ri = __float_as_uint(rev64(__uint_as_float(bi)));
  const bool take = tk_better(rv, ri, v, id);
  v = take ? rv : v;
  id = take ? ri : id;
  // v is now bitonic (descending, then ascending); six half-cleaners sort it.
  cx<32>(v, id, (lane & 32) == 0);
  cx<16>(v, id, (lane & 16) == 0);
  cx<8>(v, id, (lane & 8) == 0);
  cx<4>(v, id, (lane & 4) == 0);
  cx<2>(v, id, (lane & 2) == 0);
  cx<1>(v, id, (lane & 1) == 0);
}

// Online (max, Σ exp((x − max)/T)) of one lane, and their combination (the max starts at −FLT_MAX, as the
// reference's, so −inf logits add exp(−inf) = 0). NaN logits are left out.
__device__ __forceinline__ void lse_add(float c, float it, float& mt, float& s) {
  // Written with selects: exp(0) is taken as exactly 1 where either operand is the new max.
  const float nm = fmaxf(mt, c);  // NaN c leaves the max
  const float add = c != c ? 0.f : (c == nm ? 1.0f : __expf((c - nm) * it));
  s = (mt == nm ? s : s * __expf((mt - nm) * it)) + add;
  mt = nm;
}

// A chunk's 64 best (value, id) and its (max, Σ exp((x − max)/T)). Each wave keeps its sorted list in registers and
// a buffer of pending candidates in LDS: an element enters the buffer only if it beats the list's 64th entry (which
// only rises), and the buffer is sorted and merged into the list whenever it holds 64 — a few times per wave instead
// of once per batch of 64 elements. The list is exactly the 64 best of the wave's elements: an element that does not
// beat the 64th best seen so far is not among the 64 best of all.
__global__ __launch_bounds__(SPT) void topk64_part_kernel(const float* __restrict__ x, int ldx, int V, float temp,
                                                          uint32_t* __restrict__ pidx, float* __restrict__ pval,
                                                          float2* __restrict__ pz) {
  __shared__ float sv[SPT / 64][SK];
  __shared__ uint32_t si[SPT / 64][SK];
  __shared__ float bv[SPT / 64][2 * SK];
  __shared__ uint32_t bi[SPT / 64][2 * SK];
  __shared__ float rm[SPT / 64], rs[SPT / 64];
  const int g = blockIdx.x, row = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float it = 1.0f / temp;
  const float* xr = x + size_t(row) * ldx;
  const int C = (V + SPG - 1) / SPG, lo = g * C, hi = min(V, lo + C);
  float v = -FLT_MAX, mt = -FLT_MAX, s = 0.f;
  uint32_t id = NO_ID;
  int pend = 0;  // candidates in the wave's buffer (uniform)
  // Sort the buffer's first 64 and merge them into the list; the rest (fewer than 64) move to the front.
  auto flush = [&]() {
    float c = lane < pend ? bv[wave][lane] : -FLT_MAX;
    uint32_t cid = lane < pend ? bi[wave][lane] : NO_ID;
    sort64(c, cid, lane);
    merge64(v, id, c, cid, lane);
    const int rest = max(0, pend - SK);
    float nv = 0.f;
    uint32_t ni = 0;
    if (lane < rest) {
      nv = bv[wave][SK + lane];
      ni = bi[wave][SK + lane];
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < rest) {
      bv[wave][lane] = nv;
      bi[wave][lane] = ni;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    pend = rest;
  };
  auto process = [&](float c, int ci) {
    const bool ok = ci < hi;
    if (ok) lse_add(c, it, mt, s);
    uint32_t cid = ok && c == c ? uint32_t(ci) : NO_ID;
    if (cid == NO_ID) c = -FLT_MAX;
    const float tv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    const uint32_t ti = uint32_t(__builtin_amdgcn_readlane(int(id), 63));
    const bool take = tk_better(c, cid, tv, ti);
    const unsigned long long m = __ballot(take);
    if (m == 0ull) return;  // wave-uniform
    const int at = pend + int(__popcll(m & ((1ull << lane) - 1ull)));
    if (take) {
      bv[wave][at] = c;
      bi[wave][at] = cid;
    }
    pend += int(__popcll(m));
    if (pend >= SK) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the other lanes' buffer writes, in order
      __builtin_amdgcn_wave_barrier();
      flush();
    }
  };
  // The wave's tiles of 256: element base + 64k + lane for k < 4 (coalesced loads, the next tile's requested before
  // this one is processed; indices clamped to the chunk, so the loads need no branches).
  auto ld = [&](int i) { return xr[min(i, hi - 1)]; };
  int base = lo + wave * 256;
  float c0 = 0.f, c1 = 0.f, c2 = 0.f, c3 = 0.f;
  if (base < hi) {
    c0 = ld(base + lane);
    c1 = ld(base + 64 + lane);
    c2 = ld(base + 128 + lane);
    c3 = ld(base + 192 + lane);
  }
  for (; base < hi; base += SPT * 4) {
    const int nb = base + SPT * 4;
    const float n0 = ld(nb + lane), n1 = ld(nb + 64 + lane), n2 = ld(nb + 128 + lane), n3 = ld(nb + 192 + lane);
    process(c0, base + lane);
    process(c1, base + 64 + lane);
    process(c2, base + 128 + lane);
    process(c3, base + 192 + lane);
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  if (pend > 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    flush();
  }
  // The wave's (max, sum), then the workgroup's lists and sums.
  float m = mt;
  m = fmaxf(m, lane_xor<32>(m));
  m = fmaxf(m, lane_xor<16>(m));
  m = fmaxf(m, lane_xor<8>(m));
  m = fmaxf(m, lane_xor<4>(m));
  m = fmaxf(m, lane_xor<2>(m));
  m = fmaxf(m, lane_xor<1>(m));
  float ss = s * __expf((mt - m) * it);
  ss += lane_xor<32>(ss);
  ss += lane_xor<16>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<1>(ss);
  sv[wave][lane] = v;
  si[wave][lane] = id;
  if (lane == 0) {
    rm[wave] = m;
    rs[wave] = ss;
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < SPT / 64; ++w) merge64(v, id, sv[w][lane], si[w][lane], lane);
  const size_t o = (size_t(row) * SPG + g) * SK;
  pval[o + lane] = v;
  pidx[o + lane] = id;
  if (lane == 0) {
    float M = rm[0];
    for (int w = 1; w < SPT / 64; ++w) M = fmaxf(M, rm[w]);
    float Z = 0.f;
    for (int w = 0; w < SPT / 64; ++w) Z += rs[w] * __expf((rm[w] - M) * it);
    pz[size_t(row) * SPG + g] = make_float2(M, Z);
  }
}

// One workgroup of 4 waves per row: wave w merges the chunk lists 8w … 8w + 7, then wave 0 merges the four results
// (the merge is exact, so its order does not change the list); lane 0 combines the chunks' (max, sum) in chunk order.
__global__ __launch_bounds__(256) void topk64_merge_kernel(const uint32_t* __restrict__ pidx,
                                                           const float* __restrict__ pval,
                                                           const float2* __restrict__ pz, float temp,
                                                           uint32_t* __restrict__ idx, float* __restrict__ val,
                                                           float* __restrict__ z) {
  constexpr int NW = 4, PER = SPG / NW;
  __shared__ float wv[NW][SK];
  __shared__ uint32_t wi[NW][SK];
  const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float it = 1.0f / temp;
  const size_t o = size_t(row) * SPG * SK;
  const int g0 = wave * PER;
  float v = pval[o + g0 * SK + lane];
  uint32_t id = pidx[o + g0 * SK + lane];
  for (int g = g0 + 1; g < g0 + PER; ++g) merge64(v, id, pval[o + g * SK + lane], pidx[o + g * SK + lane], lane);
  wv[wave][lane] = v;
  wi[wave][lane] = id;
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < NW; ++w) merge64(v, id, wv[w][lane], wi[w][lane], lane);
  idx[size_t(row) * SK + lane] = id;
  val[size_t(row) * SK + lane] = v;
  if (lane == 0) {
    const float2* p = pz + size_t(row) * SPG;
    float M = p[0].x;
    for (int g = 1; g < SPG; ++g) M = fmaxf(M, p[g].x);
    float Z = 0.f;
    for (int g = 0; g < SPG; ++g) Z += p[g].y * __expf((p[g].x - M) * it);
    z[2 * row] = M;
    z[2 * row + 1] = Z;
  }
}

// Probabilities of a row's candidates after temperature, top-k, min-p and top-p, renormalised; returns how many
// remain (sample_dist, zz_sample.metal:196-226). The loops run over all SK slots, unrolled, with the slots past the
// count predicated off, so pr stays in registers; every sum still runs over j = 0, 1, … in order.
__device__ __forceinline__ int sample_dist(const uint32_t* ci, const float* cv, float M, float Z,
                                           const ih_sample_params& p, float (&pr)[SK]) {
  const float it = 1.0f / p.temp;
  float e[SK];
  int n = 0;
#pragma unroll
  for (int j = 0; j < SK; ++j) {
    n += int((n == j) & (ci[j] != NO_ID));  // the leading candidates that exist
    e[j] = __expf((cv[j] - M) * it);
  }
  float tot = Z;
  if (p.top_k > 0 && p.top_k < n) n = p.top_k;
  if (p.top_k > 0) {
    tot = 0.f;
#pragma unroll
    for (int j = 0; j < SK; ++j)
      if (j < n) tot += e[j];
  }
#pragma unroll
  for (int j = 0; j < SK; ++j) pr[j] = j < n ? e[j] / tot : 0.f;
  if (p.min_p > 0.f) {
    const float thr = p.min_p * pr[0];
    int k = 1;
#pragma unroll
    for (int j = 1; j < SK; ++j) k += int((k == j) & (j < n) & (pr[j] >= thr));
    n = k;
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < SK; ++j)
      if (j < n) sm += pr[j];
#pragma unroll
    for (int j = 0; j < SK; ++j)
      if (j < n) pr[j] /= sm;
  }
  if (p.top_p < 1.f) {
    float c = 0.f;
    int k = n;
    bool done = false;
#pragma unroll
    for (int j = 0; j < SK; ++j) {
      if (j < n && !done) {
        c += pr[j];
        if (c >= p.top_p) {
          k = j + 1;
          done = true;
        }
      }
    }
    n = max(k, 1);
  }
  float sm = 0.f;
#pragma unroll
  for (int j = 0; j < SK; ++j)
    if (j < n) sm += pr[j];
#pragma unroll
  for (int j = 0; j < SK; ++j) pr[j] = j < n ? pr[j] / sm : 0.f;
  return n;
}

// A token from pr[0 … n) without `skip` (whose mass is q), with the uniform u (sample_pick, zz_sample.metal:228-239).
__device__ uint32_t sample_pick(const uint32_t* ci, const float* pr, int n, uint32_t skip, float q, float u) {
  const float target = u * (1.0f - q);
  float acc = 0.f;
  uint32_t last = NO_ID;
  for (int j = 0; j < n; ++j) {
    if (ci[j] == skip) continue;
    acc += pr[j];
    last = ci[j];
    if (acc > target) return ci[j];
  }
  return last == NO_ID ? ci[0] : last;
}

// Acceptance by rejection (spec_accept_sample, zz_sample.metal:241-281): rows' candidates idx/val [rows][64] and
// (max, Z) [rows][2]; uniforms rnd[round · IH_RND_PER_ROUND + 2i] (accept) and [… + 2i + 1] (resample) of row i. Writes the record
// and advances the state as the greedy acceptance does (vtok[0] = the new anchor; the history as in accept_kernel).
// One wave: every row's distribution is computed at once, one lane per row (each in the same sequential order as
// before, so the results do not change), into LDS; lane 0 then walks the rows in order.
__global__ __launch_bounds__(64) void accept_sample_kernel(uint32_t* st, uint32_t* vtok, const uint32_t* cidx,
                                                           const float* cval, const float* z, uint32_t* rec,
                                                           const float* rnd, ih_sample_params p, int ring, int rows,
                                                           uint32_t* hist, int hist_cap) {
  __shared__ float prs[IH_MAX_ROWS][SK];
  __shared__ int ns[IH_MAX_ROWS];
  __shared__ float qs[IH_MAX_ROWS];
  __shared__ float us[IH_RND_PER_ROUND];   // the round's uniforms
  __shared__ uint32_t vts[IH_MAX_ROWS];    // the verify block
  const int lane = threadIdx.x;
  const uint32_t nr = rows ? uint32_t(rows) : min(max(st[6], 1u), uint32_t(IH_MAX_ROWS));
  const uint32_t round = st[5], p0 = st[0];
  // The walk below reads the uniforms and the block in LDS: loaded here by all lanes at once, not one dependent read
  // per row.
  if (lane < 2 * int(nr)) us[lane] = rnd[size_t(round) * IH_RND_PER_ROUND + lane];
  if (lane < int(nr)) vts[lane] = vtok[lane];
  if (lane < int(nr)) {
    const uint32_t* ci = cidx + lane * SK;
    float pr[SK];
    const int n = sample_dist(ci, cval + lane * SK, z[2 * lane], z[2 * lane + 1], p, pr);
    float q = 0.f;
    const uint32_t d = lane + 1 < int(nr) ? vtok[lane + 1] : NO_ID;
#pragma unroll
    for (int j = 0; j < SK; ++j) {
      if (j < n && ci[j] == d) q = pr[j];
      prs[lane][j] = pr[j];
    }
    ns[lane] = n;
    qs[lane] = q;
  }
  __syncthreads();
  if (lane != 0) return;
  uint32_t m = 0, next = 0;
  for (uint32_t i = 0; i < nr; ++i) {
    const uint32_t* ci = cidx + i * SK;
    const int n = ns[i];
    if (i + 1 < nr) {
      const uint32_t d = vts[i + 1];
      const float q = qs[i];
      if (us[2 * i] < q) {
        ++m;
        continue;
      }
      next = sample_pick(ci, prs[i], n, d, q, us[2 * i + 1]);
    } else {
      next = sample_pick(ci, prs[i], n, NO_ID, 0.f, us[2 * i + 1]);
    }
    break;
  }
  uint32_t* r = rec + (round % uint32_t(ring)) * IH_REC_STRIDE;
  r[0] = m;
  r[IH_REC_ROWS] = nr;
  for (uint32_t i = 1; i <= m; ++i) r[i] = vts[i];
  r[m + 1] = next;
  r[IH_REC_P] = p0;
  st[3] = p0;
  st[2] = m + 1;
  st[0] = p0 + m + 1;
  st[1] = m + 1;
  st[4] = next;
  st[5] = round + 1;
  if (hist) {
    for (uint32_t i = 0; i < m; ++i)
      if (p0 + 1 + i < uint32_t(hist_cap)) hist[p0 + 1 + i] = vts[1 + i];
    if (p0 + 1 + m < uint32_t(hist_cap)) hist[p0 + 1 + m] = next;
  }
  vtok[0] = next;
}

// Verification rows of the round (spec_rows_choose, yy_model.metal:654-675): with draft t's calibrated acceptance
// q_t = sigmoid(a_g · logit(conf_t) + b_g) (g = min(t, 3)), expected tokens E(k) = 1 + Σ_{i<k−1} Π_{t≤i} q_t, the
// k in [kmin, kmax] with the highest E(k) / cost(k) goes to st[6].
__global__ void rows_choose_kernel(uint32_t* st, const float* conf, ih_rows_params p) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float acc = 1.f, lp = 1.f, bv = -1.f;
  uint32_t best = uint32_t(p.kmax);
  for (int t = 0; t + 1 < p.kmax; ++t) {
    const int g = min(t, 3);
    const float c = fminf(fmaxf(conf[t], 1e-6f), 1.0f - 1e-6f);
    const float q = 1.0f / (1.0f + __expf(-(p.a[g] * __logf(c / (1.0f - c)) + p.b[g])));
    lp *= q;
    acc += lp;
    const int k = t + 2;
    if (k >= p.kmin) {
      const float v = acc / p.cost[k];
      if (v > bv) {
        bv = v;
        best = uint32_t(k);
      }
    }
  }
  st[6] = best;
}

int ensure_samp(ih_ctx* c, size_t bytes) {
  if (c->samp_bytes >= bytes) return IH_OK;
  ++c->gen;
  IH_HIP(hipStreamSynchronize(c->stream));
  if (c->samp) IH_HIP(hipFree(c->samp));
  c->samp = nullptr;
  c->samp_bytes = 0;
  if (hipMalloc(&c->samp, bytes) != hipSuccess) return fail(IH_ENOMEM, "sampling scratch allocation failed");
  c->samp_bytes = bytes;
  return IH_OK;
}

int launch_topk64(ih_ctx* c, const float* x, int ldx, int rows, int V, float temp, uint32_t* idx, float* val,
                  float* z) {
  const size_t n = size_t(rows) * SPG * SK;
  IH_TRY(ensure_samp(c, n * 8 + size_t(rows) * SPG * sizeof(float2)));
  uint32_t* pidx = static_cast<uint32_t*>(c->samp);
  float* pval = reinterpret_cast<float*>(pidx + n);
  float2* pz = reinterpret_cast<float2*>(pval + n);
  {
    TimedLaunch tl(c, TC_ARGMAX, double(rows) * V * 4);
    tlaunch(tl, topk64_part_kernel, dim3(SPG, rows), dim3(SPT), 0, c->stream, x, ldx, V, temp, pidx, pval, pz);
    IH_HIP(hipGetLastError());
  }
  topk64_merge_kernel<<<rows, 256, 0, c->stream>>>(pidx, pval, pz, temp, idx, val, z);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_accept_sample(ih_ctx* c, uint32_t* st, uint32_t* vtok, const uint32_t* idx, const float* val,
                         const float* z, uint32_t* rec, const float* rnd, const ih_sample_params& p, int ring, int rows,
                         uint32_t* hist, int hist_cap) {
  accept_sample_kernel<<<1, 64, 0, c->stream>>>(st, vtok, idx, val, z, rec, rnd, p, ring, rows, hist, hist_cap);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

int ih_topk64_dev(ih_ctx* c, const float* logits_dev, int ldl, int rows, int V, float temp, uint32_t* idx_dev,
                  float* val_dev, float* z_dev) {
  IH_CHECK(c && logits_dev && idx_dev && val_dev && z_dev, IH_EINVAL, "ih_topk64_dev: null argument");
  IH_CHECK(rows >= 1 && rows <= 256 && V >= 1 && ldl >= V, IH_EINVAL, "ih_topk64_dev: bad shape");
  IH_CHECK(temp > 0.f && std::isfinite(temp), IH_EINVAL, "ih_topk64_dev: temperature must be positive");
  return launch_topk64(c, logits_dev, ldl, rows, V, temp, idx_dev, val_dev, z_dev);
}

int ih_spec_accept_sample_dev(ih_ctx* c, uint32_t* st_dev, uint32_t* vtok_dev, const uint32_t* idx_dev,
                              const float* val_dev, const float* z_dev, uint32_t* rec_dev, const float* rnd_dev,
                              const ih_sample_params* p, int ring, int rows) {
  IH_CHECK(c && st_dev && vtok_dev && idx_dev && val_dev && z_dev && rec_dev && rnd_dev && p, IH_EINVAL,
           "ih_spec_accept_sample_dev: null argument");
  IH_CHECK(ring >= 1 && rows >= 0 && rows <= IH_MAX_ROWS, IH_EINVAL, "ih_spec_accept_sample_dev: bad ring or rows");
  IH_CHECK(p->temp > 0.f && p->top_p > 0.f && p->top_k >= 0 && p->min_p >= 0.f, IH_EINVAL,
           "ih_spec_accept_sample_dev: need temp > 0, top_p > 0, top_k >= 0, min_p >= 0");
  return launch_accept_sample(c, st_dev, vtok_dev, idx_dev, val_dev, z_dev, rec_dev, rnd_dev, *p, ring, rows, nullptr,
                              0);
}

int ih_spec_rows_choose_dev(ih_ctx* c, uint32_t* st_dev, const float* conf_dev, const ih_rows_params* p) {
  IH_CHECK(c && st_dev && conf_dev && p, IH_EINVAL, "ih_spec_rows_choose_dev: null argument");
  IH_CHECK(p->kmin >= 2 && p->kmin <= p->kmax && p->kmax <= IH_MAX_ROWS, IH_EINVAL,
           "ih_spec_rows_choose_dev: need 2 <= kmin <= kmax <= 17");
  rows_choose_kernel<<<1, 64, 0, c->stream>>>(st_dev, conf_dev, *p);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // extern "C"
