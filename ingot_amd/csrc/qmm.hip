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

#include <cstdio>
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
  // RMSNorm factor of the input rows (modes QM_F32_SCALE, QM_GLU_ACT): r_t = 1/sqrt(Σ ss_in[j][t] / D + eps).
  const float* ss_in;
  int nss_in, D;
  float eps;
  // QM_RESID_ACT: h[m][n] += v (fp32, the y pointer), then the next activation bf16(h ⊙ nw) and the sum-of-squares
  // partial of this workgroup's columns, ss_out[blockIdx.x][t].
  const uint16_t* nw;
  uint4* act_out;
  int act_nkb;
  float* ss_out;
  // QM_GLU_ACT: gated activation kind and clip.
  int glu;
  float limit;
  int act_f16;  // the next activation in fp16 (the input of MXFP4 experts) instead of bf16
};

// One K-block's operands of a wave, in two rings of different depth: the weight tiles come from HBM and are
// prefetched far ahead; the token fragments of x (L2 hits) and the LDS-staged token 16 and scale/bias words need only
// a short lead.
template <int R>
struct QmmW {
  u32x4 w[R];
};
template <int T, int R, bool X16>
struct QmmX {
  u32x4 x[T][4];
  u32x4 x16[X16 ? 4 : 1];   // token 16's A operand (rows 1–15 zero), from LDS
  uint2 sb[R];              // scale | bias << 16 of the two groups of the K-block, row n of each tile, from LDS
};

struct QmmRsrc {
  __amdgpu_buffer_rsrc_t w, s, x;
  unsigned xoff[2];   // this lane's offset in a K-block's fragments (OOB for dead tokens), per token tile
};

// Past the last K-block every offset is forced out of range (offsets stay below 2^31, so OR-ing OOB keeps them out):
// the loads are issued unconditionally, read zeros without touching memory, and the loop body is one basic block
// with a fixed number of loads in flight, so the wait before each multiply covers only the stage it reads.
// The scheduling barriers keep a stage's loads together, ahead of the multiply that follows (LLVM's scheduler
// otherwise sinks them toward their use and the prefetch distance collapses).
template <int R>
__device__ __forceinline__ void qmm_load_w(QmmW<R>& st, const QmmParams& p, const QmmRsrc& rs, int tile0, int kb,
                                           int lane, int n) {
  const unsigned oob = kb < p.nkb ? 0u : OOB;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const unsigned tb = unsigned(tile0 + r) * unsigned(p.nkb) + unsigned(kb);
    st.w[r] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.w, (tb * 1024u + lane * 16u) | oob, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Token 16 is staged in LDS once per workgroup (x16s: [kb][t][qd] 16 bytes, block nkb all zeros): all 16 row lanes of
// a lane group read the same 16 bytes, a broadcast read, where a buffer load would spend a full vector-memory
// instruction per MFMA step on 64 distinct bytes.
template <int T, int R, bool X16>
__device__ __forceinline__ void qmm_load_x(QmmX<T, R, X16>& st, const QmmParams& p, const QmmRsrc& rs, int kb,
                                           const u32x4* x16s, const uint2* sbs, int n, int qd) {
  const unsigned oob = kb < p.nkb ? 0u : OOB;
  const unsigned kx = unsigned(kb) * unsigned(MAX_TOK / 16) * 4096u;  // [kb][tile][t][1 KB]
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      st.x[tt][t] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.x, (rs.xoff[tt] + kx + 1024 * t) | oob, 0, 0));
  if constexpr (X16) {
    // The A operand of the second token tile: row 0 (lanes n = 0) is token 16, rows 1–15 read the zero block.
    const int kq = (kb < p.nkb && n == 0) ? kb : p.nkb;
#pragma unroll
    for (int t = 0; t < 4; ++t) st.x16[t] = x16s[(kq * 4 + t) * 4 + qd];
  }
  // Past the last K-block the scales read the zero block that follows the staged words (the weights are zero there
  // too, and the bias term must not add c·Σx): an address select, so the loop body stays one basic block.
  const bool kin = kb < p.nkb;
#pragma unroll
  for (int r = 0; r < R; ++r) st.sb[r] = sbs[(kin ? (r * p.nkb + kb) * 16 : R * p.nkb * 16) + n];
  __builtin_amdgcn_sched_barrier(0);
}

// Workgroup staging in LDS, loaded once for all KW waves: token 16 of every K-block (X16; entries
// e = (kb·4 + t)·4 + qd, 16 bytes each, the fragment bytes at kb·(MAX_TOK/16)·4096 + 4096 + 1024·t + 16·qd, then a
// zero block nkb) and the scale/bias words of the workgroup's R tiles (contiguous in the packed layout:
// [tile][kb][row] 8 bytes, from tile0·nkb·128). Eight loads per thread for each, issued before the weight prologue so
// that their latency overlaps it, stored after it. Straight-line code with a fixed number of loads: a loop here would
// make the wait counts of everything after it conservative. The launch checks that both fit in 8·NTHR entries.
template <int NTHR, bool X16>
struct QmmStage {
  u32x4 v16[X16 ? 8 : 1];
  u32x4 vsb[8];
};

template <int NTHR, bool X16>
__device__ __forceinline__ void qmm_stage_issue(QmmStage<NTHR, X16>& st, const QmmParams& p, const QmmRsrc& rs,
                                                int tile0, int R) {
  if constexpr (X16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = j * NTHR + int(threadIdx.x);
      const int kb = e >> 4, t = (e >> 2) & 3, qd = e & 3;
      const unsigned off = unsigned(kb) * unsigned(MAX_TOK / 16) * 4096u + 4096u + 1024u * t + 16u * qd;
      st.v16[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.x, kb < p.nkb ? off : OOB, 0, 0));
    }
  }
  const unsigned nsb = unsigned(R) * unsigned(p.nkb) * 8u, base = unsigned(tile0) * unsigned(p.nkb) * 128u;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const unsigned e = unsigned(j * NTHR) + threadIdx.x;
    st.vsb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.s, e < nsb ? base + e * 16u : OOB, 0, 0));
  }
}

template <int NTHR, bool X16>
__device__ __forceinline__ void qmm_stage_commit(const QmmStage<NTHR, X16>& st, u32x4* x16s, u32x4* sbs,
                                                 const QmmParams& p, int R) {
  if constexpr (X16) {
    const int ne = (p.nkb + 1) * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = j * NTHR + int(threadIdx.x);
      if (e < ne) x16s[e] = st.v16[j];
    }
  }
  const int nsb = R * p.nkb * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = j * NTHR + int(threadIdx.x);
    if (e < nsb) sbs[e] = st.vsb[j];
  }
  if (threadIdx.x < 8) sbs[nsb + threadIdx.x] = u32x4{0u, 0u, 0u, 0u};  // the zero block (16 rows × 8 bytes)
}

template <int T, int R, bool X16>
__device__ __forceinline__ void qmm_compute(f32x4 (&acc)[R][T], float (&acc16)[R], const QmmW<R>& sw,
                                            const QmmX<T, R, X16>& st, unsigned km, unsigned kbias) {
  // Σx per group and token (ones operand), in the D layout of the products: lane (n, qd) gets tokens 4qd … 4qd+3.
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  f32x4 xs[T][2];
#pragma unroll
  for (int tt = 0; tt < T; ++tt)
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      f32x4 z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[tt][2 * g]), ones,
                                                        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      xs[tt][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[tt][2 * g + 1]), ones, z, 0,
                                                          0, 0);
    }
  // Token 16 (X16): a second token tile whose only live row is token 16; Σx per group lands in element 0 of the
  // qd = 0 lanes, like every other output of that token.
  float xs16[2] = {0.f, 0.f};
  if constexpr (X16) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      f32x4 z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x16[2 * g]), ones,
                                                        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x16[2 * g + 1]), ones, z, 0, 0, 0);
      xs16[g] = z[0];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s0 = bf16f(st.sb[r].x & 0xFFFFu), s1 = bf16f(st.sb[r].y & 0xFFFFu);
    const float c0 = fmaf(-128.f, s0, bf16f(st.sb[r].x >> 16)), c1 = fmaf(-128.f, s1, bf16f(st.sb[r].y >> 16));
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const bf16x8 w0 = nib_bf16(sw.w[r][2 * g], km, kbias), w1 = nib_bf16(sw.w[r][2 * g + 1], km, kbias);
      const float sg = g ? s1 : s0, cg = g ? c1 : c0;
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[tt][2 * g]), w0,
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[tt][2 * g + 1]), w1, tmp, 0,
                                                      0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][tt][e] = fmaf(sg, tmp[e], fmaf(cg, xs[tt][g][e], acc[r][tt][e]));
      }
      if constexpr (X16) {
        f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x16[2 * g]), w0,
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x16[2 * g + 1]), w1, tmp, 0, 0,
                                                      0);
        acc16[r] = fmaf(sg, tmp[0], fmaf(cg, xs16[g], acc16[r]));
      }
    }
  }
}


// T: MFMA token tiles loaded from memory (tokens 0–15, and 16–31 when T = 2); X16 (with T = 1, M = 17): token 16
// as a second tile from LDS.
// Workgroup = KW waves over the same 16·R rows; wave w takes K-blocks w, w + KW, … (adjacent waves read adjacent
// 1 KB blocks), with the next block's loads in flight while the current one is multiplied. The KW partial sums are
// added in wave order through LDS: no cross-workgroup synchronisation (an agent-scope fence on MI355X writes the
// XCD's L2 back and costs tens of µs) and a summation order that depends only on (N, K).
template <int T, int R, int KW, bool X16, int DW, int DX>
__global__ __launch_bounds__(64 * KW) void qmm_int4_kernel(QmmParams p) {
  static_assert(DW % DX == 0, "the x ring depth divides the weight ring depth");
  // The wave index is uniform: readfirstlane keeps it (and the K-block loop) in scalar registers and scalar branches.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, qd = lane >> 4;
  const int tile0 = blockIdx.x * R;
  __shared__ float rsc[MAX_TOK];
  f32x4 acc[R][T];
  float acc16[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc16[r] = 0.f;
#pragma unroll
    for (int tt = 0; tt < T; ++tt) acc[r][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  QmmRsrc rs;
  const unsigned tiles_total = unsigned(p.Npad / 16) * unsigned(p.nkb);
  rs.w = make_rsrc(p.w, tiles_total * 1024u);
  rs.s = make_rsrc(p.s, tiles_total * 128u);
  rs.x = make_rsrc(p.xa, unsigned(MAX_TOK) * p.nkb * 256u);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tok = 16 * tt + n;
    const bool live = tt < T && tok < p.M;
    rs.xoff[tt] = live ? (unsigned(tt) * 4096u + n * 64u + qd * 16u) : OOB;
  }
  const unsigned km = vgpr_of(p.kmask), kbias = p.kbias;

  // DW K-blocks of weights and DX of x in flight. This wave's K-blocks are wave, wave + KW, … (nk of them), DW per
  // trip of a loop with a single exit (a loop with two exits is structurized into a join that the wait-count pass
  // treats as a back edge with other stages' loads still pending, which serialises every trip). Stages past the end
  // are loaded out of range: zero weights and scales, so their products add exact zeros (the count depends only on
  // the shape).
  // Prologue in the order of the steady state (x(j) issued DX stages ahead of its use, w(j) DW stages ahead, x before
  // w within a stage), so the wait counts at the loop head are those of every later trip.
  extern __shared__ u32x4 stage_lds[];
  u32x4* const x16s = stage_lds;
  u32x4* const sbs = stage_lds + (X16 ? (p.nkb + 1) * 16 : 0);
  QmmStage<64 * KW, X16> stg;
  qmm_stage_issue(stg, p, rs, tile0, R);
  QmmW<R> sw[DW];
  QmmX<T, R, X16> sx[DX];
  int kb = wave;
#pragma unroll
  for (int t = -DW; t < -DX; ++t) qmm_load_w(sw[t + DW], p, rs, tile0, kb + (t + DW) * KW, lane, n);
  qmm_stage_commit(stg, x16s, sbs, p, R);
  __syncthreads();
  const uint2* const sbv = reinterpret_cast<const uint2*>(sbs);
#pragma unroll
  for (int t = -DX; t < 0; ++t) {
    qmm_load_x(sx[t + DX], p, rs, kb + (t + DX) * KW, x16s, sbv, n, qd);
    qmm_load_w(sw[t + DW], p, rs, tile0, kb + (t + DW) * KW, lane, n);
  }
  const int nk = kb < p.nkb ? (p.nkb - kb + KW - 1) / KW : 0;
  const int trips = (nk + DW - 1) / DW;
  for (int it = 0; it < trips; ++it) {
#pragma unroll
    for (int s = 0; s < DW; ++s) {
      qmm_compute(acc, acc16, sw[s], sx[s % DX], km, kbias);
      qmm_load_x(sx[s % DX], p, rs, kb + (s + DX) * KW, x16s, sbv, n, qd);
      qmm_load_w(sw[s], p, rs, tile0, kb + (s + DW) * KW, lane, n);
    }
    kb += DW * KW;
  }

  // RMSNorm factors of the input rows (the norm's sums of squares come in as partials of the producer's workgroups,
  // added here in a fixed order). After the K loop: loads with a data-dependent count ahead of it would make the
  // compiler's wait counts at the loop head conservative.
  // Wave w takes tokens w, w + KW, …; lane l adds partials l, l + 64, … and the lanes are combined by a fixed
  // butterfly, so a token's factor does not depend on M or on the launch shape.
  if (p.ss_in) {
    for (int t = wave; t < p.M; t += KW) {
      float ss = 0.f;
      for (int j = lane; j < p.nss_in; j += 64) ss += p.ss_in[j * MAX_TOK + t];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
      if (lane == 0) rsc[t] = 1.0f / sqrtf(ss / float(p.D) + p.eps);
    }
  }

  // Partial sums of every wave → LDS [wave][r][tt][e][lane] (+ token 16 [wave][r][row]), then fixed-order sums.
  constexpr int NEL = R * T * 4 * 64;
  constexpr int NEL16 = X16 ? R * 16 : 0;
  constexpr int WST = NEL + NEL16;
  __shared__ float red[KW * WST];
  __shared__ float ssu[MAX_TOK * 8];
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
  __syncthreads();
  // Sum over waves of output (token m, tile r, row rn of the tile).
  auto val = [&](int m, int r, int rn) -> float {
    int i;
    if (X16 && m == 16) {
      i = NEL + r * 16 + rn;
    } else {
      const int tt = m >> 4, mm = m & 15;
      i = ((r * T + tt) * 4 + (mm & 3)) * 64 + 16 * (mm >> 2) + rn;
    }
    float v = red[i];
#pragma unroll
    for (int w = 1; w < KW; ++w) v += red[w * WST + i];
    return v;
  };

  const int nthr = 64 * KW;
  if (p.mode == QM_RESID_ACT) {
    // h += v for this workgroup's 16R columns, the next activation bf16(h ⊙ nw) in 8-column chunks, and Σh² per token.
    const int nch = 2 * R;
    for (int u = threadIdx.x; u < p.M * nch; u += nthr) {
      const int m = u / nch, cl = u % nch, r = cl >> 1, half = cl & 1;
      const int col0 = (tile0 + r) * 16 + 8 * half;
      float v[8], ss = 0.f;
      float* hrow = static_cast<float*>(p.y) + size_t(m) * p.ldy;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int col = col0 + j;
        float hv = 0.f;
        if (col < p.N) {
          hv = hrow[col] + val(m, r, 8 * half + j);
          hrow[col] = hv;
        }
        ss += hv * hv;
        v[j] = col < p.N ? hv * bf16f(p.nw[col]) : 0.f;
      }
      ssu[m * 8 + cl] = ss;
      if (col0 < p.N) frag_store(p.act_f16 != 0, p.act_out, p.act_nkb, MAX_TOK / 16, m, col0 / 8, v);
    }
    __syncthreads();
    if (threadIdx.x < p.M) {
      float ss = 0.f;
      for (int cl = 0; cl < nch; ++cl) ss += ssu[threadIdx.x * 8 + cl];
      p.ss_out[blockIdx.x * MAX_TOK + threadIdx.x] = ss;
    }
    return;
  }
  if (p.mode == QM_GLU_ACT) {
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
    if (p.mode == QM_F32_SCALE) v *= rsc[m];
    if (p.mode == QM_BF16) {
      static_cast<unsigned short*>(p.y)[size_t(m) * p.ldy + row] = f2bf(v);
    } else if (p.mode == QM_F32_ADD) {
      float* o = static_cast<float*>(p.y) + size_t(m) * p.ldy + row;
      *o = *o + v;
    } else {
      static_cast<float*>(p.y)[size_t(m) * p.ldy + row] = v;
    }
  }
}

// Launch shape for an (Npad, nkb) matrix: rows per workgroup (16·R) and waves per workgroup (KW, the intra-workgroup
// split of K). Chosen from the shape only, never from M, so each row's summation order is fixed.
struct QmmShape { int R, KW, DW, DX; };
static QmmShape qmm_shape(int Npad, int nkb) {
  // Measured at M = 16/17 on gfx950, cold weights (8B shapes): four row tiles per wave when there are enough tiles
  // to fill the chip (fewer activation bytes per weight byte), two for mid-sized N, one for N ≤ 4096.
  const int NT = Npad / 16;
  QmmShape sh = NT >= 1536 ? QmmShape{4, 4, 2, 1} : NT >= 384 ? QmmShape{2, 4, 4, 2} : QmmShape{1, 4, 4, 2};
  // The workgroup's scale/bias words (R·nkb·128 bytes) are staged in LDS by eight 16-byte loads per thread.
  while (sh.R > 1 && sh.R * nkb > 64 * sh.KW) sh.R /= 2;
  if (sh.R * nkb > 64 * sh.KW) sh = QmmShape{1, 16, 4, 2};
  return sh;
}

template <int T, bool X16>
static bool qmm_dispatch(const TimedLaunch& tl, QmmShape sh, int grid, hipStream_t st, const QmmParams& p) {
  // LDS staging: token 16 (X16) and the scale/bias words of the workgroup's R tiles.
  const size_t shm16 = (X16 ? size_t(p.nkb + 1) * 256 : 0) + 128, shsb = size_t(p.nkb) * 128;
#define IH_QMM_CASE(R_, KW_, DW_, DX_)                                                                \
  if (sh.R == R_ && sh.KW == KW_ && sh.DW == DW_ && sh.DX == DX_) {                                  \
    tlaunch(tl, qmm_int4_kernel<T, R_, KW_, X16, DW_, DX_>, dim3(grid), dim3(64 * KW_), shm16 + R_ * shsb, st, p); \
    return true;                                                                                          \
  }
  IH_QMM_CASE(1, 4, 1, 1) IH_QMM_CASE(1, 4, 2, 1) IH_QMM_CASE(1, 4, 2, 2) IH_QMM_CASE(1, 4, 4, 2)
  IH_QMM_CASE(1, 8, 1, 1) IH_QMM_CASE(1, 8, 2, 1) IH_QMM_CASE(1, 8, 4, 2) IH_QMM_CASE(1, 16, 4, 2)
  IH_QMM_CASE(2, 4, 1, 1) IH_QMM_CASE(2, 4, 2, 1) IH_QMM_CASE(2, 4, 2, 2) IH_QMM_CASE(2, 4, 4, 2)
  IH_QMM_CASE(2, 8, 1, 1) IH_QMM_CASE(2, 8, 2, 1)
  IH_QMM_CASE(4, 4, 1, 1) IH_QMM_CASE(4, 4, 2, 1) IH_QMM_CASE(4, 4, 2, 2) IH_QMM_CASE(4, 2, 1, 1)
  IH_QMM_CASE(8, 4, 1, 1) IH_QMM_CASE(8, 2, 1, 1)
#undef IH_QMM_CASE
  return false;  // not an instantiated shape
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

int launch_qmm_ex(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, const QmmEpilogue& ep) {
  IH_CHECK(W->format == QF_INT4, IH_EINVAL, "qmm: int4 matrix expected");
  IH_CHECK(M >= 1 && M <= MAX_TOK, IH_EINVAL, "qmm: M must be in 1..32");
  IH_CHECK(a.nkb == W->nkb && !a.f16, IH_EINVAL, "qmm: activation K does not match the matrix");
  QmmShape sh = qmm_shape(W->Npad, W->nkb);
  if (const char* ov = getenv("IH_QMM_SHAPE")) sscanf(ov, "%d,%d,%d,%d", &sh.R, &sh.KW, &sh.DW, &sh.DX);  // tuning override
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
  if (ep.mode == QM_F32_SCALE || ep.mode == QM_GLU_ACT) {
    IH_CHECK(a.ss && a.nss > 0, IH_EINVAL, "qmm: the input activation carries no RMSNorm sums");
    p.ss_in = a.ss;
    p.nss_in = a.nss;
    p.D = a.K;
    p.eps = ep.eps;
  }
  IH_CHECK(sh.R * W->nkb <= 64 * sh.KW, IH_EINVAL, "qmm: the scale/bias staging does not fit this launch shape");
  const int grid = W->Npad / (16 * sh.R);
  if (ep.mode == QM_RESID_ACT) {
    IH_CHECK(ep.act_out && ep.act_out->nkb * KBLK >= W->N && ep.nw, IH_EINVAL, "qmm: residual epilogue needs an output");
    IH_CHECK(grid <= ep.act_out->ss_cap, IH_EINVAL, "qmm: too many workgroups for the RMSNorm partials");
    IH_CHECK(2 * sh.R <= 8, IH_EINVAL, "qmm: residual epilogue supports R ≤ 4");
    p.nw = ep.nw;
    p.act_out = static_cast<uint4*>(ep.act_out->frag);
    p.act_nkb = ep.act_out->nkb;
    p.act_f16 = ep.act_out->f16 ? 1 : 0;
    p.ss_out = ep.act_out->ss;
    ep.act_out->nss = grid;
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
  // Algorithmic bytes: the matrix in its MLX format, x (bf16) read, y written (read too when accumulating).
  const double ybytes = double(M) * W->N *
                        (ep.mode == QM_BF16 ? 2 : (ep.mode == QM_F32_ADD || ep.mode == QM_RESID_ACT ? 8 : 4));
  TimedLaunch tl(c, TC_QMM, double(W->algo_bytes) + double(M) * W->K * 2 + ybytes);
  bool ok;
  if (M > 17) ok = qmm_dispatch<2, false>(tl, sh, grid, c->stream, p);
  else if (M == 17 && (W->nkb + 1) * 16 <= 8 * 64 * sh.KW) ok = qmm_dispatch<1, true>(tl, sh, grid, c->stream, p);
  else if (M == 17) ok = qmm_dispatch<2, false>(tl, sh, grid, c->stream, p);  // K too long to stage token 16 in LDS
  else ok = qmm_dispatch<1, false>(tl, sh, grid, c->stream, p);
  IH_CHECK(ok, IH_EINVAL, "qmm: launch shape not instantiated");
  IH_HIP(hipGetLastError());
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
