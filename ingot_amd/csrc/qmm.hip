// Few-row quantized matmul of the verify step on gfx950: Y[M ≤ 32, N] (+)= X[M, K] · dequant(W)ᵀ, with the epilogues
// of the round fused in (RMSNorm scale, residual add, gated activation, next activation's layout).
//
// Reference: VQMV.encode → vnax_qmv_nf1_sg32 (Sources/Ingot/Layers/Linear.swift:263-445,
// Sources/Ingot/Shaders/verify_nax.metal:102-176); the arithmetic it stands for is qmv_acc
// (Sources/Ingot/Shaders/verify.metal:89-105): y = Σ_groups s·Σ x·q + b·Σ x.
//
// MI355X design (not a translation of the Metal kernel):
//   - HBM-bound at M ≤ 17 (≈ 2·M / 0.5625 ≤ 60 FLOP/B). Each wave streams its weight tiles with one contiguous
//     1024-byte dwordx4 buffer load per 16×128 tile (layout in ih_internal.h), the next K-block in flight while the
//     current one is multiplied, and dequantizes in registers.
//   - The products run on MFMA v_mfma_f32_16x16x32_bf16 with the tokens as the A operand (16 tokens × 32 K) and the
//     weights as B (32 K × 16 rows). A nibble q becomes the bf16 128 + q with one v_and_or_b32 per pair
//     ((w >> 4c) & 0x000F000F | 0x43004300), so the MFMA sums Σ x·(128 + q) exactly in fp32 per group of 64; one more
//     MFMA against a ones operand gives Σ x per group and token in the same layout, and the affine map is applied
//     once per group and output: y += s·acc + (b − 128·s)·Σx. No rounding of the dequantised weight.
//   - Token 16 (the 17th row of a k = 16 block) is the only live row of a second MFMA token tile whose A operand
//     comes from LDS (token 16 staged once per workgroup, zeros for the other rows), so it costs no extra
//     vector-memory instructions and one output element of VALU work. Each MFMA output element depends only on its
//     own A row, so its bits are those of the M > 17 path (two full token tiles) and never depend on M.
//   - K is split over the waves of a workgroup (a split chosen from (N, K) only, never from M) and the partial sums are
//     added in wave order in LDS: deterministic and row-invariant (row r's bits do not depend on M).
#include "act.h"
#include "ih_internal.h"
#include "qmm_common.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <cstdlib>

namespace ih {

// ---------------------------------------------------------------------------------------------------------------
// Repack an MLX int4 g64 matrix ([E][N][K/8] words, [E][N][K/64] bf16 scales and biases) into the tile layout.
// Grid (Npad/16 · nkb, E), 64 threads: lane L = 16·qd + n. With il8, rows are interleaved by eights for a gate|up pair
// (N = 2I, gate rows 0…I−1, up rows I…2I−1): tile t holds gate rows 8t…8t+7 then up rows 8t…8t+7, so one tile's
// outputs are the gate and up of the same 8 columns.
__global__ void pack_int4_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                 const uint16_t* __restrict__ b, uint4* __restrict__ wp, uint2* __restrict__ sp, int N,
                                 int K, int Npad, int nkb, int il8) {
  const int lane = threadIdx.x, n = lane & 15, qd = lane >> 4;
  const int tile = blockIdx.x / nkb, kb = blockIdx.x % nkb, e = blockIdx.y;
  const int prow = tile * 16 + n;
  const int row = il8 ? (n < 8 ? 8 * tile + n : N / 2 + 8 * tile + n - 8) : prow;
  const bool live = il8 ? (8 * tile + (n & 7) < N / 2) : row < N;
  const int wpr = K / 8, gpr = K / 64;
  const size_t ebase_w = size_t(e) * N * wpr, ebase_s = size_t(e) * N * gpr;
  unsigned v[4];
  for (int t = 0; t < 4; ++t) {
    int wi = kb * 16 + 4 * t + qd;
    v[t] = (live && wi < wpr) ? w[ebase_w + size_t(row) * wpr + wi] : 0u;
  }
  const size_t tb = (size_t(e) * (Npad / 16) + tile) * nkb + kb;
  wp[tb * 64 + lane] = make_uint4(v[0], v[1], v[2], v[3]);
  if (qd == 0) {
    unsigned s0 = 0, b0 = 0, s1 = 0, b1 = 0;
    if (live) {
      int g0 = 2 * kb, g1 = 2 * kb + 1;
      if (g0 < gpr) { s0 = s[ebase_s + size_t(row) * gpr + g0]; b0 = b[ebase_s + size_t(row) * gpr + g0]; }
      if (g1 < gpr) { s1 = s[ebase_s + size_t(row) * gpr + g1]; b1 = b[ebase_s + size_t(row) * gpr + g1]; }
    }
    sp[tb * 16 + n] = make_uint2(s0 | (b0 << 16), s1 | (b1 << 16));
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Natural-layout activations → fragment layout. Grid (MAX_TOK), 256 threads; one thread per 8 values. Rows ≥ M are
// written as zeros.
template <typename TIn>
__global__ void act_kernel(const TIn* __restrict__ x, int ldx, int M, int K, int nkb, int ntile, uint4* __restrict__ frag) {
  const int i = blockIdx.x;
  const int nchunk = nkb * 16;
  for (int c = threadIdx.x; c < nchunk; c += blockDim.x) {
    float v[8];
    const bool valid = i < M && c < K / 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float f = 0.f;
      if (valid) {
        if constexpr (sizeof(TIn) == 2) f = bf16f(x[size_t(i) * ldx + 8 * c + e]);
        else f = x[size_t(i) * ldx + 8 * c + e];
      }
      v[e] = f;
    }
    frag_store_chunk(frag, nkb, ntile, i, c, v);
  }
}

// ---------------------------------------------------------------------------------------------------------------
struct QmmParams {
  const uint4* w;          // packed words of the expert
  const uint2* s;          // packed scale/bias of the expert
  const uint4* xa;         // activation fragments
  void* y;
  int ldy, M, N, Npad, nkb, mode;
  // The nibble-decode constants 0x000F000F and 0x43004300, passed as arguments so that they live in SGPRs and the
  // compiler can use the three-operand v_and_or_b32 (gfx9 VOP3 takes no literal constants).
  unsigned kmask, kbias;
  // RMSNorm factor of the input rows (modes QM_F32_SCALE, QM_GLU_ACT): r_t = 1/sqrt(Σ ss_in[t][j] / D + eps).
  const float* ss_in;
  int nss_in, D;
  float eps;
  // QM_RESID_ACT: h[m][n] += v (fp32, the y pointer), then the next activation bf16(h ⊙ nw) and the sum-of-squares
  // partial of this workgroup's columns, ss_out[t][blockIdx.x].
  const uint16_t* nw;
  const float* bias;  // QM_RESID_ACT: h += v + bias[n] when not null
  uint4* act_out;
  int act_nkb;
  float* ss_out;
  // QM_GLU_ACT: gated activation kind and clip.
  int glu;
  float limit;
  int act_f16;  // the next activation in fp16 (the input of MXFP4 experts) instead of bf16
  // K split over workgroups (gridDim.y > 1): partial sums [split][MAX_TOK][Npad], added in split order by
  // qmm_finish_kernel, which then runs the epilogue.
  float* part;
  int nsplit;
  // K split over workgroups with a fused epilogue: arrival counters, one per row group (zero between launches).
  unsigned* ctr;
};

// The epilogue of the R tiles tile0 … tile0+R−1 of a workgroup of nthr threads, given val(m, r, rn) = the finished
// product of token m and row rn of tile r. rsc holds the RMSNorm factors (modes QM_F32_SCALE, QM_GLU_ACT); ssu is
// LDS scratch of MAX_TOK·2R floats; wg indexes this workgroup's sum-of-squares partial (QM_RESID_ACT).
// QM_RESID_ACT: a thread's first work item (token m, 8 columns) of the residual epilogue, its h and norm weights
// loaded at kernel entry so that their latency overlaps the main loop.
struct ResidPrefetch {
  float h[8];
  float nw[8];
};
template <int R>
__device__ __forceinline__ void resid_prefetch(ResidPrefetch& pf, const QmmParams& p, int tile0) {
  constexpr int nch = 2 * R;
  const int u = threadIdx.x;
  if (u >= p.M * nch) return;
  const int m = u / nch, cl = u % nch, col0 = (tile0 + (cl >> 1)) * 16 + 8 * (cl & 1);
  const float* hrow = static_cast<const float*>(p.y) + size_t(m) * p.ldy;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int col = min(col0 + j, p.N - 1);
    pf.h[j] = hrow[col];
    pf.nw[j] = bf16f(p.nw[col]);
  }
}

template <int R, int MODE, typename V>
__device__ __forceinline__ void qmm_epilogue(const QmmParams& p, int tile0, V val, const float* rsc, float* ssu,
                                             int nthr, int wg, const ResidPrefetch* rpf = nullptr) {
  if constexpr (MODE == QM_RESID_ACT) {
    // h += v for the 16R columns, the next activation bf16(h ⊙ nw) in 8-column chunks, and Σh² per token.
    constexpr int nch = 2 * R;
    for (int u = threadIdx.x; u < p.M * nch; u += nthr) {
      const int m = u / nch, cl = u % nch, r = cl >> 1, half = cl & 1;
      const int col0 = (tile0 + r) * 16 + 8 * half;
      const bool pre = rpf && u == int(threadIdx.x);
      float v[8], ss = 0.f;
      float* hrow = static_cast<float*>(p.y) + size_t(m) * p.ldy;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int col = col0 + j;
        float hv = 0.f;
        if (col < p.N) {
          hv = (pre ? rpf->h[j] : hrow[col]) + (p.bias ? val(m, r, 8 * half + j) + p.bias[col] : val(m, r, 8 * half + j));
          hrow[col] = hv;
        }
        ss += hv * hv;
        v[j] = col < p.N ? hv * (pre ? rpf->nw[j] : bf16f(p.nw[col])) : 0.f;
      }
      ssu[m * nch + cl] = ss;
      if (col0 < p.N) frag_store(p.act_f16 != 0, p.act_out, p.act_nkb, MAX_TOK / 16, m, col0 / 8, v);
    }
    __syncthreads();
    if (int(threadIdx.x) < p.M) {
      float ss = 0.f;
      for (int cl = 0; cl < nch; ++cl) ss += ssu[threadIdx.x * nch + cl];
      p.ss_out[threadIdx.x * SS_CAP + wg] = ss;
    }
    return;
  }
  if constexpr (MODE == QM_GLU_ACT) {
    // Interleaved gate|up tiles: rows 0–7 gate, 8–15 up of the same 8 columns (chunk tile0 + r of the output).
    for (int u = threadIdx.x; u < p.M * R; u += nthr) {
      const int m = u / R, r = u % R;
      const float rs_ = rsc[m];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = glu_f(val(m, r, j) * rs_, val(m, r, 8 + j) * rs_, p.glu, p.limit);
      const int chunk = tile0 + r;
      if (chunk * 8 < p.N / 2) frag_store(p.act_f16 != 0, p.act_out, p.act_nkb, MAX_TOK / 16, m, chunk, v);
    }
    return;
  }
  for (int u = threadIdx.x; u < p.M * 16 * R; u += nthr) {
    const int m = u / (16 * R), rr = u % (16 * R), r = rr >> 4, rn = rr & 15;
    const int row = (tile0 + r) * 16 + rn;
    if (row >= p.N) continue;
    float v = val(m, r, rn);
    if constexpr (MODE == QM_F32_SCALE) v *= rsc[m];
    if constexpr (MODE == QM_BF16) {
      static_cast<unsigned short*>(p.y)[size_t(m) * p.ldy + row] = f2bf(v);
    } else if constexpr (MODE == QM_F32_ADD) {
      float* o = static_cast<float*>(p.y) + size_t(m) * p.ldy + row;
      *o = *o + v;
    } else {
      static_cast<float*>(p.y)[size_t(m) * p.ldy + row] = v;
    }
  }
}

// T: MFMA token tiles loaded from memory (tokens 0–15, and 16–31 when T = 2); X16 (with T = 1, M = 17): token 16 as
// a second tile whose A operand comes from LDS.
//
// Workgroup (blockIdx.x, blockIdx.y) = KW waves over the 16·R rows of tiles R·blockIdx.x …; the K range is split over
// gridDim.y workgroups and, inside one, over its waves: wave w streams the KPW consecutive K-blocks from
// (blockIdx.y·KW + w)·KPW through a D-deep register ring (the loads of K-block i + D go out as K-block i is
// multiplied). R tiles per wave share each x fragment, so x traffic per weight byte falls as 1/R (one tile per wave
// re-reads x ~4× the weight bytes from L2).
// VALU budget. At M = 17 the products are cheap on MFMA; the VALU work per 16 × 128 tile (nibble decode 28, the
// per-group affine map 20, scale words 6) is ~55 % of the tile's HBM time at full speed, so nothing else may run on
// the VALU in the loop: every K-dependent offset is a scalar (buffer loads take the K-block as soffset, the LDS reads
// as an immediate of an unrolled trip), and the ring's last D K-blocks are peeled rather than guarded.
// The KW partial sums are added in wave order through LDS; with gridDim.y > 1 each workgroup writes its sum to
// p.part and qmm_finish_kernel adds the splits in order. No atomics and no cross-workgroup fences (an agent-scope
// release on MI355X writes back the XCD's L2: ~15 µs per launch), and a row's summation order depends only on
// (N, K), never on M.
// KPW1 > 0: the second half of the waves (the second wave of each SIMD at KW = 8) take KPW1 K-blocks each instead of
// KPW. A CU's loads come back roughly in issue order, so those waves receive their first stage after the first half's
// first two stages; with fewer K-blocks they still end with the first half.
template <int T, int R, int KW, bool X16, int D, int KPW, int MODE, int KPW1 = 0>
__global__ __launch_bounds__(64 * KW) void qmm_int4_kernel(QmmParams p) {
  static_assert(KPW % D == 0 && KPW1 % D == 0, "the ring depth divides the K-blocks of a wave");
  // The wave index is uniform: readfirstlane keeps it (and everything derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, qd = lane >> 4;
  const int tile0 = blockIdx.x * R;
  constexpr int nk = KPW;                                // K-blocks of a wave of the first half (the LDS stride)
  constexpr int HALF = KW / 2;
  const int nkr = (KPW1 == 0 || wave < HALF) ? KPW : KPW1;  // K-blocks of this wave
  const int kwg = int(blockIdx.y) * (KPW1 ? HALF * (KPW + KPW1) : KW * nk);  // first K-block of the workgroup
  const int kb0 = kwg + (KPW1 == 0 ? wave * nk : wave < HALF ? wave * KPW : HALF * KPW + (wave - HALF) * KPW1);
  const unsigned tiles_total = unsigned(p.Npad / 16) * unsigned(p.nkb);
  const unsigned wlim = tiles_total * 1024u, xlim = unsigned(MAX_TOK) * p.nkb * 256u;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, wlim), rsb = make_rsrc(p.s, tiles_total * 128u),
                               rx = make_rsrc(p.xa, xlim);
  const unsigned km = vgpr_of(p.kmask), kbias = p.kbias;
  const unsigned shv[3] = {vgpr_of(4u), vgpr_of(8u), vgpr_of(12u)};  // 64-bit nibble shifts (nib_bf16_pair)

  // Epilogue inputs that another kernel just wrote, requested ahead of the weight stages (consumed after the main loop).
  // Rows per wave of the RMSNorm prefetch: M ≤ 16 (T = 1), 17 (X16) or 32 (T = 2); more than eight (one-wave
  // workgroups) are read after the loop instead.
  constexpr int NR = ((T == 2 ? 32 : X16 ? 17 : 16) + KW - 1) / KW;
  constexpr bool RMS = MODE == QM_F32_SCALE || MODE == QM_GLU_ACT, RMS_PRE = RMS && NR <= 8;
  RmsPrefetch<RMS_PRE ? NR : 1> rpf;
  ResidPrefetch hpf;
  unsigned xoff[T];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
    xoff[tt] = (16 * tt + n < p.M) ? (unsigned(tt) * 4096u + n * 64u + qd * 16u) : OOB;
  const unsigned woff = unsigned(lane) * 16u;

  u32x4 wv[D][R], xv[D][T][4];
  // One ring stage: the weight tiles and x of K-block kb. Every offset that depends on kb is a scalar.
  auto load_stage = [&](int d, int kb) {
    kb = kb < p.nkb ? kb : p.nkb - 1;  // a ragged last wave re-reads the last K-block; its scales are zero
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xv[d][tt][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rx, xoff[tt], kb * (MAX_TOK / 16) * 4096 + 1024 * t, 0));
#pragma unroll
    for (int r = 0; r < R; ++r)
      wv[d][r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rw, woff, ((tile0 + r) * p.nkb + kb) * 1024, 0));
    __builtin_amdgcn_sched_barrier(0);
  };
  // With the asymmetric split (two waves per SIMD), every wave's first stage goes out before anything else of the
  // workgroup: a CU's loads come back roughly in issue order at its share of the bandwidth, and the second half's
  // first stages would otherwise queue behind the first half's staging loads and second stages. The barrier orders
  // only the issue. (With one wave per SIMD the staging loads go first: they are small and the first products wait
  // for them.)
  // The same for the seven-wave split-K shapes (down at K = 14336: 2.318 → 2.310 ms per step); at 16 waves (qkv, o) it
  // loses (2.347).
  constexpr bool FS = KPW1 > 0 || KW == 7;
  if constexpr (FS) {
    load_stage(0, kb0);
    __syncthreads();
  }
  if constexpr (RMS_PRE)
    if (p.ss_in) rms_prefetch(rpf, p.ss_in, SS_CAP, p.M, wave, KW, lane);
  if constexpr (MODE == QM_RESID_ACT) resid_prefetch<R>(hpf, p, tile0);

  // Wave-private staging in LDS: the scale/bias words of the R tiles over this wave's K-blocks ([r][i][row] 8 bytes)
  // and token 16 of those K-blocks as [i][t][row ∈ {token 16, zeros}][qd] 16 bytes, so that lane (n, qd) reads
  // row n ≠ 0 ? zeros : token 16 from an address that depends on the K-block only through an immediate. The loads go
  // out first and only they are waited for before the LDS writes; no barrier: one wave's LDS operations complete in
  // order and no other wave reads the region (a workgroup barrier here made every wave wait for the slowest wave's
  // staging, queued behind all of the workgroup's first weight stages).
  __shared__ u32x4 ssb[KW][R * nk * 8];
  __shared__ u32x4 s16[KW][X16 ? nk * 32 : 1];
  __shared__ float rsc[MAX_TOK];
  constexpr int nsb = R * nk * 8;
  constexpr int NSB = (nsb + 63) / 64, N16 = X16 ? (nk * 16 + 63) / 64 : 1;
  u32x4 vsb[NSB], v16[N16];
#pragma unroll
  for (int j = 0; j < NSB; ++j) {
    const int e = j * 64 + lane, r = e / (nk * 8), i = (e >> 3) % nk;
    const unsigned off = (unsigned(tile0 + r) * unsigned(p.nkb) + unsigned(kb0 + i)) * 128u + unsigned(e & 7) * 16u;
    const bool in = e < nsb && i < nkr && kb0 + i < p.nkb;  // K-blocks past the matrix: zero scale and bias
    vsb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsb, in ? off : OOB, 0, 0));
  }
  if constexpr (X16) {
#pragma unroll
    for (int j = 0; j < N16; ++j) {
      const int e = j * 64 + lane, i = e >> 4, t = (e >> 2) & 3, q = e & 3;
      const unsigned off = unsigned(kb0 + i) * unsigned(MAX_TOK / 16) * 4096u + 4096u + 1024u * t + 16u * q;
      v16[j] = __builtin_bit_cast(u32x4,
                                  __builtin_amdgcn_raw_buffer_load_b128(rx, i < nkr && kb0 + i < p.nkb ? off : OOB, 0, 0));
    }
  }

#pragma unroll
  for (int d = FS ? 1 : 0; d < D; ++d) load_stage(d, kb0 + d);

  // The RMSNorm factors of the input rows, while the first stages are on their way: their partials were requested
  // first, so waiting for them does not wait for the weights, and no accumulator is live yet.
  if constexpr (RMS_PRE) {
    if (p.ss_in) rms_finish(rpf, p.ss_in, SS_CAP, p.nss_in, p.D, p.eps, p.M, rsc, wave, KW, lane);
  }

#pragma unroll
  for (int j = 0; j < NSB; ++j) {
    const int e = j * 64 + lane;
    if (e < nsb) ssb[wave][e] = vsb[j];
  }
  if constexpr (X16) {
#pragma unroll
    for (int j = 0; j < N16; ++j) {
      const int e = j * 64 + lane, i = e >> 4, t = (e >> 2) & 3, q = e & 3;
      if (i < nk) {
        s16[wave][(i * 4 + t) * 8 + q] = v16[j];
        s16[wave][(i * 4 + t) * 8 + 4 + q] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  f32x4 acc[R][T];
  float acc16[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc16[r] = 0.f;
#pragma unroll
    for (int tt = 0; tt < T; ++tt) acc[r][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4* const s16l = &s16[wave][0] + (n ? 4 : 0) + qd;  // this lane's row of the token-16 staging
  const uint2* const sbl = reinterpret_cast<const uint2*>(&ssb[wave][0]) + n;  // row n of the staged scale words

  // Products of ring stage d (K-block kl of this wave, 0 ≤ kl < nk).
  auto compute = [&](int d, int kl) {
    u32x4 x16[X16 ? 4 : 1];
    if constexpr (X16) {
#pragma unroll
      for (int t = 0; t < 4; ++t) x16[t] = s16l[(kl * 4 + t) * 8];
    }
    // Σx per group and token (ones operand), in the D layout of the products: lane (n, qd) gets tokens 4qd … 4qd+3.
    f32x4 xs[T][2];
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        f32x4 z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[d][tt][2 * g]), ones, zero4,
                                                          0, 0, 0);
        xs[tt][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[d][tt][2 * g + 1]), ones,
                                                            z, 0, 0, 0);
      }
    // Token 16: a second token tile whose only live row is token 16; its Σx per group lands in element 0 of the
    // qd = 0 lanes, like every other output of that token.
    float xs16[2] = {0.f, 0.f};
    if constexpr (X16) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        f32x4 z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x16[2 * g]), ones, zero4, 0, 0,
                                                          0);
        z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x16[2 * g + 1]), ones, z, 0, 0, 0);
        xs16[g] = z[0];
      }
    }
    // The scale/bias words of all R tiles, requested together before the first product so that one LDS latency per
    // K-block is exposed instead of one per tile (the fence after each tile keeps later reads from being hoisted).
    uint2 sbv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) sbv[r] = sbl[(r * nk + kl) * 16];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint2 sb = sbv[r];
      const float s0 = __uint_as_float(sb.x << 16), s1 = __uint_as_float(sb.y << 16);
      const float c0 = fmaf(-128.f, s0, __uint_as_float(sb.x & 0xFFFF0000u));
      const float c1 = fmaf(-128.f, s1, __uint_as_float(sb.y & 0xFFFF0000u));
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        bf16x8 w0, w1;
        nib_bf16_pair(wv[d][r][2 * g], wv[d][r][2 * g + 1], km, kbias, shv, w0, w1);
        const float sg = g ? s1 : s0, cg = g ? c1 : c0;
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
          f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[d][tt][2 * g]), w0,
                                                              zero4, 0, 0, 0);
          tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv[d][tt][2 * g + 1]), w1, tmp, 0,
                                                        0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][tt][e] = fmaf(sg, tmp[e], fmaf(cg, xs[tt][g][e], acc[r][tt][e]));
        }
        if constexpr (X16) {
          f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x16[2 * g]), w0, zero4, 0,
                                                              0, 0);
          tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x16[2 * g + 1]), w1, tmp, 0, 0,
                                                        0);
          acc16[r] = fmaf(sg, tmp[0], fmaf(cg, xs16[g], acc16[r]));
        }
      }
      // One tile at a time: without the fence the scheduler decodes every tile's nibbles ahead of the products and
      // the decoded operands (16 VGPRs per tile) exhaust the register file at R = 7.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The ring: trips of D K-blocks, each multiplied from its stage and the stage refilled D K-blocks ahead, then the
  // last D K-blocks without refills (nk is a multiple of D, which the launch checks; nk = D loads everything at
  // entry).
  int i = 0;
#pragma unroll 1
  for (; i < nkr - D; i += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      compute(d, i + d);
      load_stage(d, kb0 + i + d + D);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) {
    compute(d, i + d);
  }

  // Partial sums of every wave → LDS [wave][r][tt][e][lane] (+ token 16 [wave][r][row]), then fixed-order sums.
  constexpr int NEL = R * T * 4 * 64;
  constexpr int NEL16 = X16 ? R * 16 : 0;
  constexpr int WST = NEL + NEL16;
  __shared__ float red[KW * WST];
  __shared__ float ssu[MAX_TOK * 2 * R];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave * WST + ((r * T + tt) * 4 + e) * 64 + lane] = acc[r][tt][e];
  if constexpr (X16) {
    if (lane < 16) {
#pragma unroll
      for (int r = 0; r < R; ++r) red[wave * WST + NEL + r * 16 + lane] = acc16[r];
    }
  }
  // Without the entry prefetch (one-wave workgroups, more rows than a wave prefetches): the RMSNorm factors once the
  // accumulators are in LDS (their loads and shuffles would otherwise keep every accumulator live across them).
  if constexpr (RMS && !RMS_PRE) {
    if (p.ss_in) rms_factors(p.ss_in, SS_CAP, p.nss_in, p.D, p.eps, p.M, rsc, wave, KW, lane);
  }
  __syncthreads();
  // Sum over waves, in wave order, of every partial at once (independent, coalesced LDS reads spread over the whole
  // workgroup), into wave 0's slots; the epilogue then reads one value per output.
  if constexpr (KW > 1) {
    for (int i = threadIdx.x; i < WST; i += 64 * KW) {
      float v = red[i];
#pragma unroll
      for (int w = 1; w < KW; ++w) v += red[w * WST + i];
      red[i] = v;
    }
    __syncthreads();
  }
  // The finished output (token m, tile r, row rn of the tile).
  auto val = [&](int m, int r, int rn) -> float {
    int i;
    if (X16 && m == 16) {
      i = NEL + r * 16 + rn;
    } else {
      const int tt = m >> 4, mm = m & 15;
      i = ((r * T + tt) * 4 + (mm & 3)) * 64 + 16 * (mm >> 2) + rn;
    }
    return red[i];
  };
  if constexpr (MODE == QM_PART) {
    float* part = p.part + size_t(blockIdx.y) * MAX_TOK * p.Npad;
    for (int u = threadIdx.x; u < p.M * 16 * R; u += 64 * KW) {
      const int m = u / (16 * R), rr = u % (16 * R);
      part[size_t(m) * p.Npad + tile0 * 16 + rr] = val(m, rr >> 4, rr & 15);
    }
  } else {
    if (gridDim.y > 1) {
      // K split over gridDim.y workgroups: each writes its partial sums with agent-coherent stores (they bypass the
      // XCD's L2, so no cache write-back is needed), then counts itself in on the row group's counter; the last to
      // arrive adds the partials in split order (its own from LDS) and runs the epilogue, the others exit. No
      // workgroup waits for another, and the sum's order depends only on the split, not on who arrives last.
      const int nsp = int(gridDim.y), me = int(blockIdx.y);
      const unsigned sstride = unsigned(MAX_TOK) * unsigned(p.Npad);  // floats per split
      const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.part, unsigned(nsp) * sstride * 4u);
      // Quads of 4 consecutive rows of one token: slot of (m, 4q) in red, byte offset in a split's partials.
      auto quad = [&](int u, int& i, unsigned& off) {
        const int m = u / (4 * R), rr = 4 * (u % (4 * R)), r = rr >> 4, rn = rr & 15;
        if (X16 && m == 16) {
          i = NEL + r * 16 + rn;
        } else {
          const int tt = m >> 4, mm = m & 15;
          i = ((r * T + tt) * 4 + (mm & 3)) * 64 + 16 * (mm >> 2) + rn;
        }
        off = (unsigned(m) * unsigned(p.Npad) + unsigned(tile0 * 16 + rr)) * 4u;
      };
      constexpr int SC1 = 16;  // cache policy: agent-coherent (sc1)
      for (int u = threadIdx.x; u < p.M * 4 * R; u += 64 * KW) {
        int i;
        unsigned off;
        quad(u, i, off);
        const f32x4 v = f32x4{red[i], red[i + 1], red[i + 2], red[i + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, off, unsigned(me) * sstride * 4u,
                                               SC1);
      }
      __builtin_amdgcn_s_waitcnt(0);  // every partial store of this thread has completed
      __syncthreads();
      __shared__ unsigned arrived;
      if (threadIdx.x == 0) {
        arrived = __hip_atomic_fetch_add(p.ctr + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == unsigned(nsp - 1))
          __hip_atomic_store(p.ctr + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (arrived != unsigned(nsp - 1)) return;  // workgroup-uniform
      // Ordering without agent-scope fences (an agent-scope release writes back the XCD's L2, ~15 µs per launch; an
      // acquire, which invalidates the CU's caches, measured 0.14 ms per configuration-1 step): every writer's
      // partials are agent-coherent stores (sc1: they bypass the XCD's L2), completed (waitcnt 0) before its barrier
      // and its count, so they are at the coherence point before the count that reports them; the reads below are
      // sc1 loads (they do not hit stale lines of this CU's caches), issued after the workgroup barrier that follows
      // the count (a workgroup-scope acquire: the compiler cannot hoist them above it) and under the branch on the
      // count's value (the hardware issues no load of a branch before the branch resolves).
      // The sums, in split order, into wave 0's partial slots (each thread reads back only slots it owns).
      for (int u = threadIdx.x; u < p.M * 4 * R; u += 64 * KW) {
        int i;
        unsigned off;
        quad(u, i, off);
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < nsp; ++sp) {
          const f32x4 x = sp == me ? f32x4{red[i], red[i + 1], red[i + 2], red[i + 3]}
                                   : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                   rp, off, unsigned(sp) * sstride * 4u, SC1));
          v += x;
        }
        red[i] = v[0];
        red[i + 1] = v[1];
        red[i + 2] = v[2];
        red[i + 3] = v[3];
      }
      __syncthreads();
    }
    qmm_epilogue<R, MODE>(p, tile0, val, rsc, ssu, 64 * KW, blockIdx.x, &hpf);
  }
}

// Adds the split partial sums in split order and runs the epilogue: workgroup = 4 tiles (64 rows), 256 threads.
constexpr int FIN_R = 4;
__global__ __launch_bounds__(256) void qmm_finish_kernel(QmmParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tile0 = blockIdx.x * FIN_R;
  __shared__ float rsc[MAX_TOK];
  __shared__ float ssu[MAX_TOK * 2 * FIN_R];
  if (p.ss_in) rms_factors(p.ss_in, SS_CAP, p.nss_in, p.D, p.eps, p.M, rsc, wave, 4, lane);
  __syncthreads();
  const size_t sstride = size_t(MAX_TOK) * p.Npad;
  auto val = [&](int m, int r, int rn) -> float {
    const float* q = p.part + size_t(m) * p.Npad + (tile0 + r) * 16 + rn;
    float v = q[0];
    for (int s = 1; s < p.nsplit; ++s) v += q[s * sstride];
    return v;
  };
  switch (p.mode) {
    case QM_F32: qmm_epilogue<FIN_R, QM_F32>(p, tile0, val, rsc, ssu, 256, blockIdx.x); break;
    case QM_F32_ADD: qmm_epilogue<FIN_R, QM_F32_ADD>(p, tile0, val, rsc, ssu, 256, blockIdx.x); break;
    case QM_BF16: qmm_epilogue<FIN_R, QM_BF16>(p, tile0, val, rsc, ssu, 256, blockIdx.x); break;
    case QM_F32_SCALE: qmm_epilogue<FIN_R, QM_F32_SCALE>(p, tile0, val, rsc, ssu, 256, blockIdx.x); break;
    case QM_RESID_ACT: qmm_epilogue<FIN_R, QM_RESID_ACT>(p, tile0, val, rsc, ssu, 256, blockIdx.x); break;
    case QM_GLU_ACT: qmm_epilogue<FIN_R, QM_GLU_ACT>(p, tile0, val, rsc, ssu, 256, blockIdx.x); break;
    default: break;
  }
}

// Launch shape for an (Npad, nkb) matrix: R row tiles per wave, KW waves per workgroup, ring depth D, kpw K-blocks per
// wave, and ks = nkb / (KW·kpw) workgroups splitting K. Chosen from the shape only, never from M, so each row's
// summation order is fixed. The K range tiles exactly (ks·KW·kpw = nkb, kpw a multiple of D), or, in one split, the
// last wave runs past the end by less than its kpw: its K-blocks past the matrix re-stream the last block (clamped,
// so every load stays inside the matrix) with zero scale and bias words, which add exactly nothing.
struct QmmShape { int R, KW, D, kpw, ks, kpw1 = 0; };
constexpr int qmm_ring_depth(int kpw) { return kpw % 2 == 0 ? 2 : kpw <= 3 ? kpw : 1; }
static bool qmm_shape_ok(const QmmShape& sh, int Npad, int nkb) {
  const int span = sh.kpw1 ? sh.KW / 2 * (sh.kpw + sh.kpw1) : sh.KW * sh.kpw;
  return sh.R >= 1 && sh.KW >= 1 && sh.D >= 1 && sh.kpw >= sh.D && sh.kpw % sh.D == 0 && sh.kpw <= 32 &&
         sh.R * sh.kpw <= 64 && (Npad / 16) % sh.R == 0 &&
         (sh.ks * span == nkb || (sh.ks == 1 && span > nkb && span - nkb < sh.kpw));
}
// The instantiated (R, KW, KPW) shapes (qmm_dispatch_mode lists the same set).
static constexpr int kQmmShapes[][3] = {{1, 16, 2}, {2, 16, 2}, {2, 8, 4}, {4, 4, 8}, {4, 8, 4}, {7, 4, 8},
                                        {1, 8, 14}, {1, 14, 8}, {4, 4, 2}, {2, 8, 2}, {4, 8, 2}, {1, 1, 1},
                                        {2, 1, 1},  {4, 1, 1},  {7, 1, 1},  {2, 8, 3},  {4, 8, 3}};
static QmmShape qmm_shape_sym(int Npad, int nkb);
// The symmetric choice below, except that seven-tile workgroups over 32 K-blocks (gate|up at K = 4096) run at two
// waves per SIMD with the asymmetric split (7,8,6,2): the loop's VALU work issues ~2× faster per SIMD with two waves,
// and the second wave of each SIMD, whose first stage arrives ~3 µs later, takes a third of the K-blocks of the first.
static QmmShape qmm_shape(int Npad, int nkb) {
  const QmmShape sh = qmm_shape_sym(Npad, nkb);
  if (sh.R == 7 && sh.KW == 4 && sh.kpw == 8 && sh.ks == 1) return QmmShape{7, 8, 2, 6, 1, 2};
  // One-tile workgroups over 112 K-blocks (down at K = 14336): every workgroup reads the whole 487 KB activation from
  // L2, which bounds the kernel; two-tile workgroups with K split in two read half as much per CU, and the split's
  // reduction in the last-arriving workgroup costs less than that saves (config 1: 2.375 → 2.342 ms per step).
  if (sh.R == 1 && sh.KW == 8 && sh.kpw == 14 && sh.ks == 1 && nkb == 112 && Npad % 32 == 0) {
    const QmmShape s2{2, 7, qmm_ring_depth(8), 8, 2};
    if (qmm_shape_ok(s2, Npad, nkb)) return s2;
  }
  return sh;
}
static QmmShape qmm_shape_sym(int Npad, int nkb) {
  const int NT = Npad / 16;
  // Rows: R tiles per wave share x, and the workgroup count NT / R should be about one round over the 256 CUs (a
  // partial second round doubles the time of the CUs that run it): 7 for gate|up (1792 tiles → 256 workgroups), 4
  // for the vocabulary head (~9 rounds), 2 for qkv (192), 1 for o and down (256).
  int rp[4] = {1, 2, 0, 0};
  if (NT % 7 == 0 && NT / 7 >= 192 && NT / 7 <= 320) { rp[0] = 7; rp[1] = 4; rp[2] = 2; rp[3] = 1; }
  else if (NT >= 2048) { rp[0] = 4; rp[1] = 2; rp[2] = 1; }
  else if (NT > 256) { rp[0] = 2; rp[1] = 1; }
  // K: the whole range in one workgroup when a shape tiles it (16 waves × 2 K-blocks at K = 4096; a ring of 8 or 14
  // K-blocks per wave for longer K), else split over workgroups.
  for (int pass = 0; pass < 2; ++pass)
    for (int R : rp) {
      if (R == 0) continue;
      for (const auto& c : kQmmShapes) {
        if (c[0] != R || c[1] == 1) continue;
        const int span = c[1] * c[2];
        if (nkb % span) continue;
        const QmmShape sh{R, c[1], qmm_ring_depth(c[2]), c[2], nkb / span};
        if ((pass == 0 && sh.ks != 1) || !qmm_shape_ok(sh, Npad, nkb)) continue;
        return sh;
      }
    }
  // K-block counts without a fitting factor: one split whose last wave runs past the end by less than its kpw.
  for (int R : rp)
    if (R)
      for (const auto& c : kQmmShapes) {
        if (c[0] != R || c[1] == 1) continue;
        const QmmShape sh{R, c[1], qmm_ring_depth(c[2]), c[2], 1};
        if (c[1] * c[2] > nkb && qmm_shape_ok(sh, Npad, nkb)) return sh;
      }
  // Otherwise one wave per workgroup, one K-block per wave.
  for (int R : rp)
    if (R && (Npad / 16) % R == 0) return QmmShape{R, 1, 1, 1, nkb};
  return QmmShape{1, 1, 1, 1, nkb};
}

template <int T, int R, int KW, bool X16, int KPW>
constexpr bool qmm_fits() {
  return 4 * KW * (R * T * 256 + (X16 ? R * 16 : 0)) + 4 * MAX_TOK * (2 * R + 1) + R * KW * KPW * 128 +
             (X16 ? KW * KPW * 512 : 0) <= 128 * 1024;
}

// Instantiated launch shapes (R, KW, KPW; ring depth qmm_ring_depth(KPW)) for each epilogue. Epilogues are compile-time:
// the code of every mode in one kernel raised its register demand past the ring's (302 VGPRs at R = 7, KW = 4).
// The kernel-level modes QM_F32_ADD and QM_BF16 run as QM_PART + qmm_finish_kernel; QM_F32 and the fused modes run in
// the kernel itself.
template <int T, bool X16, int MODE>
static bool qmm_dispatch_mode(const TimedLaunch& tl, QmmShape sh, dim3 grid, hipStream_t st, const QmmParams& p) {
#define IH_QMM_CASE(R_, KW_, KPW_)                                                                          \
  if constexpr (qmm_fits<T, R_, KW_, X16, KPW_>()) {                                                        \
    if (sh.R == R_ && sh.KW == KW_ && sh.kpw == KPW_ && sh.kpw1 == 0) {                                     \
      tlaunch(tl, qmm_int4_kernel<T, R_, KW_, X16, qmm_ring_depth(KPW_), KPW_, MODE>, grid, dim3(64 * KW_), 0, \
              st, p);                                                                                       \
      return true;                                                                                          \
    }                                                                                                       \
  }
  // K = 4096 (32 K-blocks); K = 14336 (112; (4,7,4) and (2,7,8) split it over 4 and 2 workgroups); K = 2048 (16);
  // K = 2880 (23, ragged); and the one-wave fallback.
  IH_QMM_CASE(1, 16, 2) IH_QMM_CASE(2, 16, 2) IH_QMM_CASE(2, 8, 4) IH_QMM_CASE(4, 8, 4) IH_QMM_CASE(4, 4, 8)
  IH_QMM_CASE(7, 4, 8) IH_QMM_CASE(1, 14, 8) IH_QMM_CASE(1, 8, 14) IH_QMM_CASE(4, 4, 2) IH_QMM_CASE(2, 8, 2)
  IH_QMM_CASE(4, 8, 2) IH_QMM_CASE(2, 8, 3) IH_QMM_CASE(4, 8, 3) IH_QMM_CASE(4, 7, 4) IH_QMM_CASE(2, 7, 8)
  IH_QMM_CASE(1, 1, 1) IH_QMM_CASE(2, 1, 1) IH_QMM_CASE(4, 1, 1) IH_QMM_CASE(7, 1, 1)
#undef IH_QMM_CASE
  // Asymmetric K split (KPW for the first half of the waves, KPW1 for the second): gate|up at two waves per SIMD.
#define IH_QMM_CASE1(R_, KW_, KPW_, KPW1_)                                                                       \
  if constexpr (qmm_fits<T, R_, KW_, X16, KPW_>()) {                                                        \
    if (sh.R == R_ && sh.KW == KW_ && sh.kpw == KPW_ && sh.kpw1 == KPW1_) {                                \
      tlaunch(tl, qmm_int4_kernel<T, R_, KW_, X16, 2, KPW_, MODE, KPW1_>, grid, dim3(64 * KW_), 0, st, p);   \
      return true;                                                                                          \
    }                                                                                                       \
  }
  IH_QMM_CASE1(7, 8, 6, 2)
#undef IH_QMM_CASE1
  return false;  // not an instantiated shape
}

template <int T, bool X16>
static bool qmm_dispatch(const TimedLaunch& tl, QmmShape sh, dim3 grid, hipStream_t st, const QmmParams& p,
                         int mode) {
  switch (mode) {
    case QM_F32: return qmm_dispatch_mode<T, X16, QM_F32>(tl, sh, grid, st, p);
    case QM_F32_SCALE: return qmm_dispatch_mode<T, X16, QM_F32_SCALE>(tl, sh, grid, st, p);
    case QM_RESID_ACT: return qmm_dispatch_mode<T, X16, QM_RESID_ACT>(tl, sh, grid, st, p);
    case QM_GLU_ACT: return qmm_dispatch_mode<T, X16, QM_GLU_ACT>(tl, sh, grid, st, p);
    case QM_PART: return qmm_dispatch_mode<T, X16, QM_PART>(tl, sh, grid, st, p);
    default: return false;
  }
}

int launch_act_from_bf16(ih_ctx* c, const uint16_t* x, int ldx, int M, ActBuf& a) {
  act_kernel<uint16_t><<<MAX_TOK, 256, 0, c->stream>>>(x, ldx, M, a.K, a.nkb, a.ntile, static_cast<uint4*>(a.frag));
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_act_from_f32(ih_ctx* c, const float* x, int ldx, int M, ActBuf& a) {
  act_kernel<float><<<MAX_TOK, 256, 0, c->stream>>>(x, ldx, M, a.K, a.nkb, a.ntile, static_cast<uint4*>(a.frag));
  IH_HIP(hipGetLastError());
  return IH_OK;
}


int qmm_grid(const ih_qmat* W) {
  const QmmShape sh = qmm_shape(W->Npad, W->nkb);
  return W->Npad / (16 * sh.R);
}

// Split-K partial sums: grown on demand, the stream drained before an old buffer is freed.
static int ensure_qpart(ih_ctx* c, size_t bytes) {
  if (!c->qctr) {
    // Arrival counters of the in-kernel split-K reduction: zeroed once; the last workgroup of a row group resets its
    // counter, so they are zero between launches.
    ++c->gen;
    if (hipMalloc(&c->qctr, QCTR_CAP * sizeof(unsigned)) != hipSuccess)
      return fail(IH_ENOMEM, "qmm: split-K counter allocation failed");
    IH_TRY(fill(c, c->qctr, 0, QCTR_CAP * sizeof(unsigned)));
  }
  if (c->qpart_bytes >= bytes) return IH_OK;
  ++c->gen;
  IH_HIP(hipStreamSynchronize(c->stream));
  if (c->qpart) IH_HIP(hipFree(c->qpart));
  c->qpart = nullptr;
  c->qpart_bytes = 0;
  if (hipMalloc(&c->qpart, bytes) != hipSuccess) return fail(IH_ENOMEM, "qmm: split-K partial allocation failed");
  c->qpart_bytes = bytes;
  return IH_OK;
}

int launch_qmm_ex(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, const QmmEpilogue& ep) {
  IH_CHECK(W->format == QF_INT4, IH_EINVAL, "qmm: int4 matrix expected");
  IH_CHECK(M >= 1 && M <= MAX_TOK, IH_EINVAL, "qmm: M must be in 1..32");
  IH_CHECK(a.nkb == W->nkb && !a.f16, IH_EINVAL, "qmm: activation K does not match the matrix");
  QmmShape sh = qmm_shape(W->Npad, W->nkb);
  for (const auto& o : c->qmm_shapes) {
    if (o[0] != W->N || o[1] != W->K) continue;
    const int span = o[5] ? o[3] / 2 * (o[4] + o[5]) : o[3] * o[4];
    sh = QmmShape{o[2], o[3], o[5] ? 2 : qmm_ring_depth(o[4]), o[4], std::max(1, W->nkb / std::max(1, span)), o[5]};
  }
  IH_CHECK(qmm_shape_ok(sh, W->Npad, W->nkb), IH_EINVAL, "qmm: launch shape does not tile the matrix");
  const int ks = sh.ks;
  // The kernel runs the step's fused epilogues and the plain fp32 output itself (with K split over workgroups, in the
  // last workgroup of each row group to arrive); the other kernel-level modes (accumulate, bf16) write partial sums
  // that qmm_finish_kernel adds and applies.
  const bool fused = ep.mode == QM_F32_SCALE || ep.mode == QM_RESID_ACT || ep.mode == QM_GLU_ACT || ep.mode == QM_F32;
  const bool finish = !fused;
  const int kmode = finish ? int(QM_PART) : ep.mode;
  QmmParams p{};
  const size_t tiles_per_e = size_t(W->Npad / 16) * W->nkb;
  p.w = static_cast<const uint4*>(W->w) + tiles_per_e * 64 * expert;
  p.s = static_cast<const uint2*>(W->s) + tiles_per_e * 16 * expert;
  p.xa = static_cast<const uint4*>(a.frag);
  p.y = ep.y;
  p.ldy = ep.ldy;
  p.M = M;
  p.N = W->N;
  p.Npad = W->Npad;
  p.nkb = W->nkb;
  p.mode = ep.mode;
  p.kmask = 0x000F000Fu;
  p.kbias = 0x43004300u;
  p.nsplit = ks;
  if (ep.mode == QM_F32_SCALE || ep.mode == QM_GLU_ACT) {
    IH_CHECK(a.ss && a.nss > 0, IH_EINVAL, "qmm: the input activation carries no RMSNorm sums");
    p.ss_in = a.ss;
    p.nss_in = a.nss;
    p.D = a.K;
    p.eps = ep.eps;
  }
  // Workgroups that write the epilogue: the qmm's own (one split) or the finisher's (4 tiles each).
  const int grid_x = W->Npad / (16 * sh.R);
  const int egrid = finish ? W->Npad / (16 * FIN_R) : grid_x;
  if (ep.mode == QM_RESID_ACT) {
    IH_CHECK(ep.act_out && ep.act_out->nkb * KBLK >= W->N && ep.nw, IH_EINVAL, "qmm: residual epilogue needs an output");
    IH_CHECK(egrid <= ep.act_out->ss_cap, IH_EINVAL, "qmm: too many workgroups for the RMSNorm partials");
    p.nw = ep.nw;
    p.bias = ep.bias;
    p.act_out = static_cast<uint4*>(ep.act_out->frag);
    p.act_nkb = ep.act_out->nkb;
    p.act_f16 = ep.act_out->f16 ? 1 : 0;
    p.ss_out = ep.act_out->ss;
    ep.act_out->nss = egrid;
  }
  if (ep.mode == QM_GLU_ACT) {
    IH_CHECK(ep.act_out && ep.act_out->nkb * KBLK >= W->N / 2 && W->il8, IH_EINVAL,
             "qmm: gated epilogue needs an interleaved gate|up matrix and an output");
    p.act_out = static_cast<uint4*>(ep.act_out->frag);
    p.act_nkb = ep.act_out->nkb;
    p.act_f16 = ep.act_out->f16 ? 1 : 0;
    p.glu = ep.glu;
    p.limit = ep.limit;
  }
  if (finish || ks > 1) {
    IH_TRY(ensure_qpart(c, size_t(ks) * MAX_TOK * W->Npad * sizeof(float)));
    p.part = c->qpart;
  }
  if (!finish && ks > 1) {
    IH_CHECK(grid_x <= QCTR_CAP, IH_EINVAL, "qmm: too many row groups for the split-K counters");
    p.ctr = c->qctr;
  }
  // Algorithmic bytes: the matrix in its MLX format, x (bf16) read, y written (read too when accumulating).
  const double ybytes = double(M) * W->N *
                        (ep.mode == QM_BF16 ? 2 : (ep.mode == QM_F32_ADD || ep.mode == QM_RESID_ACT ? 8 : 4));
  {
    TimedLaunch tl(c, TC_QMM, double(W->algo_bytes) + double(M) * W->K * 2 + (finish ? 0.0 : ybytes));
    const dim3 grid(grid_x, ks);
    bool ok;
    if (M > 17) ok = qmm_dispatch<2, false>(tl, sh, grid, c->stream, p, kmode);
    else if (M == 17) ok = qmm_dispatch<1, true>(tl, sh, grid, c->stream, p, kmode);
    else ok = qmm_dispatch<1, false>(tl, sh, grid, c->stream, p, kmode);
    IH_CHECK(ok, IH_EINVAL, "qmm: launch shape not instantiated");
    IH_HIP(hipGetLastError());
  }
  if (finish) {
    TimedLaunch tl(c, TC_QMM_FINISH, double(ks) * M * W->N * 4 + ybytes);
    tlaunch(tl, qmm_finish_kernel, dim3(egrid), dim3(256), 0, c->stream, p);
    IH_HIP(hipGetLastError());
  }
  return IH_OK;
}

int launch_qmm(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, void* y, int ldy, int out_mode) {
  QmmEpilogue ep;
  ep.mode = out_mode;
  ep.y = y;
  ep.ldy = ldy;
  return launch_qmm_ex(c, W, expert, a, M, ep);
}

static int qmat_alloc(ih_ctx* c, ih_qmat* q) {
  const size_t tiles = size_t(q->E) * (q->Npad / 16) * q->nkb;
  q->wbytes = tiles * 1024;
  q->sbytes = tiles * (q->format == QF_INT4 ? 128 : 64);
  if (hipMalloc(&q->w, q->wbytes) != hipSuccess) return fail(IH_ENOMEM, "qmat: weight allocation failed");
  if (hipMalloc(&q->s, q->sbytes) != hipSuccess) return fail(IH_ENOMEM, "qmat: scale allocation failed");
  return IH_OK;
}

int pack_int4(ih_ctx* c, ih_qmat* q, const uint32_t* w, const uint16_t* s, const uint16_t* b) {
  dim3 grid((q->Npad / 16) * q->nkb, q->E);
  pack_int4_kernel<<<grid, 64, 0, c->stream>>>(w, s, b, static_cast<uint4*>(q->w), static_cast<uint2*>(q->s), q->N,
                                               q->K, q->Npad, q->nkb, q->il8);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

static ih_qmat* new_qmat_int4(ih_ctx* c, int E, int N, int K) {
  ih_qmat* q = new ih_qmat();
  q->ctx = c;
  q->format = QF_INT4;
  q->E = E;
  q->N = N;
  q->K = K;
  q->Npad = (N + 255) / 256 * 256;
  q->nkb = (K + KBLK - 1) / KBLK;
  q->ktail = (K % KBLK) ? 1 : 0;
  q->algo_bytes = size_t(N) * K / 2 + size_t(N) * (K / 64) * 4;
  return q;
}

int qmat_int4_create_dev(ih_ctx* c, const void* w, const void* s, const void* b, int E, int N, int K, int il8,
                         ih_qmat** out) {
  IH_CHECK(c && w && s && b && out, IH_EINVAL, "ih_qmat_int4_create_dev: null argument");
  IH_CHECK(E >= 1 && N >= 1 && K >= 64 && K % 64 == 0, IH_EINVAL,
           "ih_qmat_int4_create_dev: need E, N >= 1 and K a positive multiple of 64");
  IH_CHECK(!il8 || N % 16 == 0, IH_EINVAL, "qmat: an interleaved gate|up matrix needs N a multiple of 16");
  *out = nullptr;
  ih_qmat* q = new_qmat_int4(c, E, N, K);
  q->il8 = il8;
  int st = qmat_alloc(c, q);
  if (st == IH_OK) st = pack_int4(c, q, static_cast<const uint32_t*>(w), static_cast<const uint16_t*>(s),
                                  static_cast<const uint16_t*>(b));
  if (st != IH_OK) {
    ih_qmat_free(q);
    return st;
  }
  *out = q;
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

int ih_qmat_int4_create_dev(ih_ctx* c, const void* w, const void* s, const void* b, int E, int N, int K,
                            ih_qmat** out) {
  return qmat_int4_create_dev(c, w, s, b, E, N, K, 0, out);
}

int ih_qmat_int4_create(ih_ctx* c, const uint32_t* w, const uint16_t* s, const uint16_t* b, int E, int N, int K,
                        ih_qmat** out) {
  IH_CHECK(c && w && s && b && out, IH_EINVAL, "ih_qmat_int4_create: null argument");
  IH_CHECK(E >= 1 && N >= 1 && K >= 64 && K % 64 == 0, IH_EINVAL,
           "ih_qmat_int4_create: need E, N >= 1 and K a positive multiple of 64");
  const size_t wb = size_t(E) * N * (K / 8) * 4, sb = size_t(E) * N * (K / 64) * 2;
  void *dw = nullptr, *ds = nullptr, *db = nullptr;
  int st = IH_OK;
  if (hipMalloc(&dw, wb) != hipSuccess || hipMalloc(&ds, sb) != hipSuccess || hipMalloc(&db, sb) != hipSuccess)
    st = fail(IH_ENOMEM, "ih_qmat_int4_create: staging allocation failed");
  if (st == IH_OK && (hipMemcpyAsync(dw, w, wb, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
                      hipMemcpyAsync(ds, s, sb, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
                      hipMemcpyAsync(db, b, sb, hipMemcpyHostToDevice, c->stream) != hipSuccess))
    st = fail(IH_EDEVICE, "ih_qmat_int4_create: upload failed");
  if (st == IH_OK) st = ih_qmat_int4_create_dev(c, dw, ds, db, E, N, K, out);
  (void)hipStreamSynchronize(c->stream);
  if (dw) (void)hipFree(dw);
  if (ds) (void)hipFree(ds);
  if (db) (void)hipFree(db);
  return st;
}

int ih_qmat_free(ih_qmat* q) {
  if (!q) return IH_OK;
  if (q->ctx) (void)hipStreamSynchronize(q->ctx->stream);
  if (q->w) (void)hipFree(q->w);
  if (q->s) (void)hipFree(q->s);
  delete q;
  return IH_OK;
}

size_t ih_qmat_bytes(const ih_qmat* q) { return q ? q->algo_bytes * q->E : 0; }

int ih_qmm_shape_override(ih_ctx* c, int N, int K, int R, int KW, int kpw) {
  IH_CHECK(c && N >= 1 && K >= 64, IH_EINVAL, "ih_qmm_shape_override: null context or empty matrix");
  IH_CHECK(R >= 0 && KW >= 0 && kpw >= 0, IH_EINVAL, "ih_qmm_shape_override: negative shape");
  auto& v = c->qmm_shapes;
  for (size_t i = 0; i < v.size();) {
    if (v[i][0] == N && v[i][1] == K) v.erase(v.begin() + i);
    else ++i;
  }
  if (R > 0) v.push_back({N, K, R, KW, kpw, 0});
  ++c->gen;  // recorded steps launched the previous shapes
  return IH_OK;
}

int ih_qmm_int4(ih_ctx* c, const ih_qmat* W, const void* x, int ldx, int M, void* y, int ldy, int out_mode) {
  IH_CHECK(c && W && x && y, IH_EINVAL, "ih_qmm_int4: null argument");
  IH_CHECK(M >= 1 && M <= MAX_TOK, IH_EINVAL, "ih_qmm_int4: M must be in 1..32");
  IH_CHECK(ldx >= W->K && ldy >= W->N, IH_EINVAL, "ih_qmm_int4: leading dimension smaller than the row");
  IH_CHECK(out_mode >= 0 && out_mode <= 2, IH_EINVAL, "ih_qmm_int4: out_mode must be 0, 1 or 2");
  IH_CHECK(W->E == 1, IH_EINVAL, "ih_qmm_int4: stacked experts need the gathered entry point");
  IH_TRY(ensure_act(c, c->act, W->K, false));
  IH_TRY(launch_act_from_bf16(c, static_cast<const uint16_t*>(x), ldx, M, c->act));
  return launch_qmm(c, W, 0, c->act, M, y, ldy, out_mode);
}

}  // extern "C"
