// Copy-from-context drafting: the trigram index of the history on the host and a scan of the int32 context on the
// device. Both follow CopyIndex (Sources/Ingot/CopySpec.swift:15-139): the current trigram is the last three tokens
// (ending at cur = n − 1); among the three most recent earlier ends p < cur of the same trigram, take the one with
// the longest backward match h[p − i] == h[cur − i] (i < maxMatch, i ≤ p), ties to the more recent; a match shorter
// than minMatch proposes nothing; otherwise propose h[p + 1 … min(cur, p + maxK)].
//
// The host table is keyed by the trigram itself, not by a 64-bit hash of it, so two trigrams never share a slot.
#include "ih_internal.h"

#include <algorithm>
#include <cstring>
#include <vector>

struct ih_copy_index {
  struct Slot {
    uint32_t a, b, c;
    uint32_t n;        // stored ends (0 = empty slot), at most WAYS
    uint32_t end[4];   // most recent first
  };
  static constexpr int WAYS = 4;
  int min_match = 3, max_match = 64;
  std::vector<uint32_t> hist;
  std::vector<Slot> tab;
  size_t used = 0;

  static uint64_t hash3(uint32_t a, uint32_t b, uint32_t c) {
    uint64_t x = (uint64_t(a) << 32 | b) * 0xD6E8FEB86659FD93ull;
    x ^= (x >> 29) ^ (uint64_t(c) * 0x9FB21C651E98DF25ull);
    x *= 0xC2B2AE3D27D4EB4Full;
    return x ^ (x >> 31);
  }
  size_t slot_of(uint32_t a, uint32_t b, uint32_t c) const {
    const size_t mask = tab.size() - 1;
    size_t i = hash3(a, b, c) & mask;
    while (tab[i].n && !(tab[i].a == a && tab[i].b == b && tab[i].c == c)) i = (i + 1) & mask;
    return i;
  }
  void grow(size_t cap) {
    std::vector<Slot> old;
    old.swap(tab);
    tab.assign(cap, Slot{0, 0, 0, 0, {0, 0, 0, 0}});
    for (const Slot& s : old)
      if (s.n) tab[slot_of(s.a, s.b, s.c)] = s;
  }
  void index_end(size_t e) {
    if ((used + 1) * 2 > tab.size()) grow(tab.size() * 2);
    Slot& s = tab[slot_of(hist[e - 2], hist[e - 1], hist[e])];
    if (!s.n) {
      s.a = hist[e - 2];
      s.b = hist[e - 1];
      s.c = hist[e];
      ++used;
    }
    std::memmove(s.end + 1, s.end, sizeof(uint32_t) * (WAYS - 1));
    s.end[0] = uint32_t(e);
    s.n = std::min<uint32_t>(s.n + 1, WAYS);
  }
  void push(uint32_t t) {
    hist.push_back(t);
    if (hist.size() >= 3) index_end(hist.size() - 1);
  }
  void clear() {
    hist.clear();
    std::fill(tab.begin(), tab.end(), Slot{0, 0, 0, 0, {0, 0, 0, 0}});
    used = 0;
  }
  int propose(int max_k, uint32_t* out, int* match) const {
    *match = 0;
    const size_t n = hist.size();
    if (n < 4 || max_k <= 0) return 0;
    const size_t cur = n - 1;
    const Slot& s = tab[slot_of(hist[cur - 2], hist[cur - 1], hist[cur])];
    size_t best = 0;
    int best_len = 0;
    for (uint32_t w = 0; w < s.n; ++w) {
      const size_t p = s.end[w];
      if (p >= cur) continue;
      int len = 0;
      while (len < max_match && size_t(len) <= p && hist[p - len] == hist[cur - len]) ++len;
      if (len > best_len) {
        best_len = len;
        best = p;
      }
    }
    if (best_len < min_match) return 0;
    *match = best_len;
    const size_t last = std::min(cur, best + size_t(max_k));
    for (size_t i = best + 1; i <= last; ++i) out[i - best - 1] = hist[i];
    return int(last - best);
  }
};

namespace ih {

// ---------------------------------------------------------------------------------------------------------------
// Device scan. Pass 1: each workgroup takes CH consecutive end positions and keeps the three largest ends p (2 ≤ p <
// cur) whose trigram equals the current one; lists are merged lane to lane (sorted descending, −1 = none). Pass 2:
// one wave merges the workgroups' lists, measures the backward match of the ≤ 3 candidates and writes the proposal.
constexpr int COPY_CH = 1024;
constexpr int COPY_THREADS = 256;

struct Top3 {
  int v[3];
};

__device__ __forceinline__ Top3 top3_merge(const Top3& x, const Top3& y) {
  // Both lists hold distinct positions in descending order, −1 for none.
  Top3 r;
  int i = 0, j = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int xv = i == 0 ? x.v[0] : i == 1 ? x.v[1] : i == 2 ? x.v[2] : -1;
    const int yv = j == 0 ? y.v[0] : j == 1 ? y.v[1] : j == 2 ? y.v[2] : -1;
    if (xv >= yv) {
      r.v[k] = xv;
      ++i;
    } else {
      r.v[k] = yv;
      ++j;
    }
  }
  return r;
}

__device__ __forceinline__ Top3 top3_wave(Top3 t) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    Top3 u;
#pragma unroll
    for (int k = 0; k < 3; ++k) u.v[k] = __shfl_xor(t.v[k], o);
    t = top3_merge(t, u);
  }
  return t;
}

// The history length n of a chained round is the round state's position + 1 (hist[P] is the anchor), read on the
// device: pos_dev non-null gives n = min(pos_dev[0] + 1, n); a history shorter than 4 proposes nothing.
__device__ __forceinline__ int copy_len(int n, const uint32_t* pos_dev) {
  return pos_dev ? int(min(pos_dev[0] + 1u, uint32_t(n))) : n;
}

__global__ __launch_bounds__(COPY_THREADS) void copy_scan_kernel(const uint32_t* __restrict__ h, int n,
                                                                 int* __restrict__ part,
                                                                 const uint32_t* __restrict__ pos_dev) {
  __shared__ int red[COPY_THREADS / 64][3];
  n = copy_len(n, pos_dev);
  const int cur = n - 1;
  const uint32_t t0 = h[max(cur - 2, 0)], t1 = h[max(cur - 1, 0)], t2 = h[max(cur, 0)];
  const int lo = blockIdx.x * COPY_CH;
  Top3 t{{-1, -1, -1}};
  // Ascending positions per thread: a new match is always the largest so far.
  for (int p = lo + threadIdx.x; p < lo + COPY_CH && p < cur && n >= 4; p += COPY_THREADS) {
    if (p < 2) continue;
    if (h[p] == t2 && h[p - 1] == t1 && h[p - 2] == t0) {
      t.v[2] = t.v[1];
      t.v[1] = t.v[0];
      t.v[0] = p;
    }
  }
  t = top3_wave(t);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0)
    for (int k = 0; k < 3; ++k) red[wave][k] = t.v[k];
  __syncthreads();
  if (threadIdx.x == 0) {
    Top3 r{{red[0][0], red[0][1], red[0][2]}};
    for (int w = 1; w < COPY_THREADS / 64; ++w) r = top3_merge(r, Top3{{red[w][0], red[w][1], red[w][2]}});
    for (int k = 0; k < 3; ++k) part[blockIdx.x * 3 + k] = r.v[k];
  }
}

// out: [0] proposal length, [1] match length, [2] chosen end p (or −1), [3] reserved, [4 …] proposed tokens.
// vtok (optional): the verify block [anchor = h[cur], proposal…, padding = h[cur]] of `rows` entries.
__global__ __launch_bounds__(64) void copy_pick_kernel(const uint32_t* __restrict__ h, int n, const int* __restrict__ part,
                                                       int nparts, int max_k, int min_match, int max_match,
                                                       uint32_t* __restrict__ out, uint32_t* __restrict__ vtok, int rows,
                                                       const uint32_t* __restrict__ pos_dev) {
  const int lane = threadIdx.x;
  n = copy_len(n, pos_dev);
  const int cur = n - 1;
  Top3 t{{-1, -1, -1}};
  for (int i = lane; i < nparts; i += 64) t = top3_merge(t, Top3{{part[3 * i], part[3 * i + 1], part[3 * i + 2]}});
  t = top3_wave(t);
  // Backward match of candidate k on lane k (k < 3).
  int len = 0;
  const int mine = lane == 0 ? t.v[0] : lane == 1 ? t.v[1] : lane == 2 ? t.v[2] : -1;
  if (mine >= 0) {
    const int p = mine;
    while (len < max_match && len <= p && h[p - len] == h[cur - len]) ++len;
  }
  const int l0 = __shfl(len, 0), l1 = __shfl(len, 1), l2 = __shfl(len, 2);
  int best = -1, best_len = 0;
  if (l0 > best_len) { best_len = l0; best = t.v[0]; }
  if (l1 > best_len) { best_len = l1; best = t.v[1]; }
  if (l2 > best_len) { best_len = l2; best = t.v[2]; }
  int cnt = 0;
  if (best_len >= min_match) cnt = min(cur, best + max_k) - best;
  else best_len = 0;
  for (int i = lane; i < max_k; i += 64) out[4 + i] = i < cnt ? h[best + 1 + i] : 0u;
  if (vtok && cur >= 0)
    for (int i = lane; i < rows; i += 64) vtok[i] = (i >= 1 && i <= cnt) ? h[best + i] : h[cur];
  if (lane == 0) {
    out[0] = uint32_t(cnt);
    out[1] = uint32_t(best_len);
    out[2] = uint32_t(cnt ? best : -1);
    out[3] = 0u;
  }
}

int launch_copy_lookup(ih_ctx* c, const uint32_t* h, int n, int max_k, int min_match, int max_match, uint32_t* out,
                       uint32_t* vtok, int rows, const uint32_t* pos_dev) {
  const int nparts = std::max(1, (n - 1 + COPY_CH - 1) / COPY_CH);
  const size_t need = size_t(nparts) * 3 * sizeof(int);
  IH_TRY(ensure_part(c, need));
  int* part = reinterpret_cast<int*>(c->part);
  {
    TimedLaunch tl(c, TC_OTHER, double(n) * 4);
    tlaunch(tl, copy_scan_kernel, dim3(nparts), dim3(COPY_THREADS), 0, c->stream, h, n, part, pos_dev);
    IH_HIP(hipGetLastError());
  }
  copy_pick_kernel<<<1, 64, 0, c->stream>>>(h, n, part, nparts, max_k, min_match, max_match, out, vtok, rows, pos_dev);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

int ih_copy_index_create(int min_match, int max_match, int capacity, ih_copy_index** out) {
  IH_CHECK(out, IH_EINVAL, "ih_copy_index_create: out is null");
  *out = nullptr;
  IH_CHECK(capacity >= 0, IH_EINVAL, "ih_copy_index_create: negative capacity");
  auto* x = new (std::nothrow) ih_copy_index();
  if (!x) return fail(IH_ENOMEM, "ih_copy_index_create: out of host memory");
  x->min_match = std::max(3, min_match);
  x->max_match = std::max(x->min_match, max_match);
  size_t cap = 16;
  while (cap < size_t(capacity) * 2) cap <<= 1;
  x->tab.assign(cap, ih_copy_index::Slot{0, 0, 0, 0, {0, 0, 0, 0}});
  x->hist.reserve(size_t(capacity));
  *out = x;
  return IH_OK;
}

int ih_copy_index_free(ih_copy_index* x) {
  delete x;
  return IH_OK;
}

int ih_copy_index_append(ih_copy_index* x, const uint32_t* toks, int n) {
  IH_CHECK(x && (n == 0 || toks) && n >= 0, IH_EINVAL, "ih_copy_index_append: bad argument");
  for (int i = 0; i < n; ++i) x->push(toks[i]);
  return IH_OK;
}

int ih_copy_index_sync(ih_copy_index* x, const uint32_t* toks, int n) {
  IH_CHECK(x && (n == 0 || toks) && n >= 0, IH_EINVAL, "ih_copy_index_sync: bad argument");
  const size_t have = x->hist.size();
  const bool prefix = have <= size_t(n) && (have == 0 || std::memcmp(x->hist.data(), toks, have * 4) == 0);
  if (!prefix) x->clear();
  for (size_t i = x->hist.size(); i < size_t(n); ++i) x->push(toks[i]);
  return IH_OK;
}

int ih_copy_index_reset(ih_copy_index* x) {
  IH_CHECK(x, IH_EINVAL, "ih_copy_index_reset: null index");
  x->clear();
  return IH_OK;
}

int ih_copy_index_len(const ih_copy_index* x) { return x ? int(x->hist.size()) : 0; }

int ih_copy_index_propose(const ih_copy_index* x, int max_k, uint32_t* out, int* n_out, int* match_out) {
  IH_CHECK(x && n_out && match_out && (max_k <= 0 || out), IH_EINVAL, "ih_copy_index_propose: bad argument");
  *n_out = x->propose(max_k, out, match_out);
  return IH_OK;
}

int ih_copy_lookup_dev(ih_ctx* c, const uint32_t* hist_dev, int n, int max_k, int min_match, int max_match,
                       uint32_t* out_dev, uint32_t* vtok_dev, int rows) {
  IH_CHECK(c && hist_dev && out_dev, IH_EINVAL, "ih_copy_lookup_dev: null argument");
  IH_CHECK(n >= 4, IH_EINVAL, "ih_copy_lookup_dev: the history needs at least 4 tokens");
  IH_CHECK(max_k >= 1 && max_k <= 4096, IH_EINVAL, "ih_copy_lookup_dev: max_k must be in 1..4096");
  IH_CHECK(!vtok_dev || (rows >= 1 && rows <= IH_MAX_ROWS), IH_EINVAL, "ih_copy_lookup_dev: rows must be in 1..17");
  min_match = std::max(3, min_match);
  max_match = std::max(min_match, max_match);
  return launch_copy_lookup(c, hist_dev, n, max_k, min_match, max_match, out_dev, vtok_dev, rows, nullptr);
}

}  // extern "C"
