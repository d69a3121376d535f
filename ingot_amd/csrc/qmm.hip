// Few-row quantized matmul of the verify step on gfx950: Y[M ≤ 32, N] (+)= X[M, K] · dequant(W)ᵀ.
//
// Reference: VQMV.encode → vnax_qmv_nf1_sg32 (Sources/Ingot/Layers/Linear.swift:263-445,
// Sources/Ingot/Shaders/verify_nax.metal:102-176); the arithmetic it stands for is qmv_acc
// (Sources/Ingot/Shaders/verify.metal:89-105): y = Σ_groups s·Σ x·q + b·Σ x.
//
// MI355X design (not a translation of the Metal kernel):
//   - HBM-bound at M ≤ 17 (≈ 2·M / 0.5625 ≤ 60 FLOP/B). Each wave streams its weight tiles with one contiguous
//     1024-byte dwordx4 load per 16×128 tile (layout in ih_internal.h) and dequantizes in registers.
//   - The products run on MFMA v_mfma_f32_16x16x32_bf16 with the tokens as the A operand (16 tokens × 32 K) and the
//     weights as B (32 K × 16 rows). A nibble q becomes the bf16 128 + q with one and-or per pair
//     ((w >> 4c) & 0x000F000F | 0x43004300), so the MFMA sums Σ x·(128 + q) exactly in fp32 per group of 64, and the
//     affine map is applied once per group and output: y += s·acc + (b − 128·s)·Σx. No rounding of the dequantised
//     weight (the reference rounds it to half); the only rounding is fp32 accumulation.
//   - K is split over the waves of a workgroup (a split chosen from (N, K) only, never from M) and the partial sums are
//     added in wave order in LDS: deterministic and row-invariant (row r's bits do not depend on M).
#include "ih_internal.h"

#include <cstdio>
#include <cstdlib>

namespace ih {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
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

// ---------------------------------------------------------------------------------------------------------------
// Repack an MLX int4 g64 matrix ([E][N][K/8] words, [E][N][K/64] bf16 scales and biases) into the tile layout.
// Grid (Npad/16 · nkb, E), 64 threads: lane L = 16·qd + n.
__global__ void pack_int4_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                 const uint16_t* __restrict__ b, uint4* __restrict__ wp, uint2* __restrict__ sp, int N,
                                 int K, int Npad, int nkb) {
  const int lane = threadIdx.x, n = lane & 15, qd = lane >> 4;
  const int tile = blockIdx.x / nkb, kb = blockIdx.x % nkb, e = blockIdx.y;
  const int row = tile * 16 + n, wpr = K / 8, gpr = K / 64;
  const size_t ebase_w = size_t(e) * N * wpr, ebase_s = size_t(e) * N * gpr;
  unsigned v[4];
  for (int t = 0; t < 4; ++t) {
    int wi = kb * 16 + 4 * t + qd;
    v[t] = (row < N && wi < wpr) ? w[ebase_w + size_t(row) * wpr + wi] : 0u;
  }
  const size_t tb = (size_t(e) * (Npad / 16) + tile) * nkb + kb;
  wp[tb * 64 + lane] = make_uint4(v[0], v[1], v[2], v[3]);
  if (qd == 0) {
    unsigned s0 = 0, b0 = 0, s1 = 0, b1 = 0;
    if (row < N) {
      int g0 = 2 * kb, g1 = 2 * kb + 1;
      if (g0 < gpr) { s0 = s[ebase_s + size_t(row) * gpr + g0]; b0 = b[ebase_s + size_t(row) * gpr + g0]; }
      if (g1 < gpr) { s1 = s[ebase_s + size_t(row) * gpr + g1]; b1 = b[ebase_s + size_t(row) * gpr + g1]; }
    }
    sp[tb * 16 + n] = make_uint2(s0 | (b0 << 16), s1 | (b1 << 16));
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Natural-layout activations → fragment layout + per-group sums. Grid (MAX_TOK), 256 threads; one thread per 8
// values. Rows ≥ M are written as zeros so every MFMA operand is finite.
template <typename TIn>
__global__ void act_kernel(const TIn* __restrict__ x, int ldx, int M, int K, int nkb, uint4* __restrict__ frag,
                           float* __restrict__ xsum) {
  const int i = blockIdx.x;
  const int nchunk = nkb * 16;
  for (int c0 = 0; c0 < nchunk; c0 += blockDim.x) {
    const int c = c0 + threadIdx.x;
    float v[8];
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
    if (i < M && c < K / 8) {
      for (int e = 0; e < 8; ++e) {
        float f;
        if constexpr (sizeof(TIn) == 2) f = bf16f(x[size_t(i) * ldx + 8 * c + e]);
        else f = bf16f(f2bf(x[size_t(i) * ldx + 8 * c + e]));
        v[e] = f;
      }
    }
    // Group sum (64 values = 8 threads), fixed order: own 8 values in order, then a butterfly over the 8 threads.
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    if (c < nchunk) {
      const int kb = c / 16, w = c % 16, t = w / 4, qd = w % 4;
      const int pe[8] = {0, 4, 1, 5, 2, 6, 3, 7};
      unsigned u[4];
      for (int j = 0; j < 4; ++j) {
        unsigned lo = f2bf(v[pe[2 * j]]), hi = f2bf(v[pe[2 * j + 1]]);
        u[j] = lo | (hi << 16);
      }
      frag[((size_t(i) * nkb + kb) * 4 + qd) * 4 + t] = make_uint4(u[0], u[1], u[2], u[3]);
      if ((c & 7) == 0) xsum[(c / 8) * MAX_TOK + i] = sum;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
struct QmmParams {
  const uint4* w;          // packed words of the expert
  const uint2* s;          // packed scale/bias of the expert
  const uint4* xa;         // activation fragments
  const float* xs;         // activation group sums [2·nkb][MAX_TOK]
  void* y;
  int ldy, M, N, Npad, nkb, out_mode;
  // The nibble-decode constants 0x000F000F and 0x43004300, passed as arguments so that they live in SGPRs and the
  // compiler can use the three-operand v_and_or_b32 (gfx9 VOP3 takes no literal constants).
  unsigned kmask, kbias;
};

// Buffer resources (base in SGPRs, 32-bit offsets; an offset past num_records reads as zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr unsigned OOB = 0x80000000u;  // offset that reads as zero

__device__ __forceinline__ void qmm_store(const QmmParams& p, int m, int row, float v) {
  if (p.out_mode == QO_F32) {
    static_cast<float*>(p.y)[size_t(m) * p.ldy + row] = v;
  } else if (p.out_mode == QO_F32_ADD) {
    float* o = static_cast<float*>(p.y) + size_t(m) * p.ldy + row;
    *o = *o + v;
  } else {
    static_cast<unsigned short*>(p.y)[size_t(m) * p.ldy + row] = f2bf(v);
  }
}

// One K-block's operands of a wave: R weight tiles (+ scale/bias) and the T token tiles of x (+ group sums).
template <int T, int R, bool X16>
struct QmmStage {
  u32x4 w[R];
  uint2 sb[R];
  u32x4 x[T][4];
  f32x4 xs[T][2];
  u32x4 x16[X16 ? 4 : 1];   // token 16 (VALU path): this lane's 64 bytes of it
  float xs16[2];
};

// Buffer resources of one launch and the per-lane offsets that do not change along K.
struct QmmRsrc {
  __amdgpu_buffer_rsrc_t w, s, x, xs;
  unsigned xoff[2];   // token row offset of this lane's A operand (OOB for dead tokens), per token tile
  unsigned xsoff[2];  // group-sum offset of this lane's 4 output tokens (OOB if none live)
  unsigned x16off, xs16off;
};

template <int T, int R, bool X16>
__device__ __forceinline__ void qmm_load(QmmStage<T, R, X16>& st, const QmmParams& p, const QmmRsrc& rs, int tile0,
                                         int kb, int lane, int n) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const unsigned tb = unsigned(tile0 + r) * unsigned(p.nkb) + unsigned(kb);
    st.w[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.w, tb * 1024u + lane * 16u, 0, 0));
    st.sb[r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs.s, tb * 128u + n * 8u, 0, 0));
  }
  const unsigned kx = unsigned(kb) * 256u, kxs = unsigned(kb) * (2 * MAX_TOK * 4);
#pragma unroll
  for (int tt = 0; tt < T; ++tt) {
    // Dead token lanes point past the buffer and read zeros (their MFMA outputs are discarded).
#pragma unroll
    for (int t = 0; t < 4; ++t)
      st.x[tt][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.x, rs.xoff[tt] + kx + 16 * t, 0, 0));
#pragma unroll
    for (int g = 0; g < 2; ++g)
      st.xs[tt][g] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.xs, rs.xsoff[tt] + kxs + g * (MAX_TOK * 4), 0, 0));
  }
  if constexpr (X16) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      st.x16[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.x, rs.x16off + kx + 16 * t, 0, 0));
    st.xs16[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs.xs, rs.xs16off + kxs, 0, 0));
    st.xs16[1] = __builtin_bit_cast(float,
                                    __builtin_amdgcn_raw_buffer_load_b32(rs.xs, rs.xs16off + kxs + MAX_TOK * 4, 0, 0));
  }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int T, int R, bool X16>
__device__ __forceinline__ void qmm_compute(f32x4 (&acc)[R][T], float (&acc16)[R], const QmmStage<T, R, X16>& st,
                                            float qd0, unsigned km, unsigned kbias) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s0 = bf16f(st.sb[r].x & 0xFFFFu), s1 = bf16f(st.sb[r].y & 0xFFFFu);
    const float c0 = fmaf(-128.f, s0, bf16f(st.sb[r].x >> 16)), c1 = fmaf(-128.f, s1, bf16f(st.sb[r].y >> 16));
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const bf16x8 w0 = nib_bf16(st.w[r][2 * g], km, kbias), w1 = nib_bf16(st.w[r][2 * g + 1], km, kbias);
      const float sg = g ? s1 : s0, cg = g ? c1 : c0;
#pragma unroll
      for (int tt = 0; tt < T; ++tt) {
        f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[tt][2 * g]), w0,
                                                            f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[tt][2 * g + 1]), w1, tmp, 0,
                                                      0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][tt][e] = fmaf(sg, tmp[e], fmaf(cg, st.xs[tt][g][e], acc[r][tt][e]));
      }
      if constexpr (X16) {
        // Token 16 by packed bf16 dot products: this lane's 16 values of the group (its row n, K slice qd); the
        // group's bias term is added by the qd = 0 lanes only (qd0 = 1 there, 0 elsewhere), the four K slices are
        // summed across lanes at the end.
        float d = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const unsigned wr = st.w[r][2 * g + h];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const unsigned wp = and_or(wr >> (4 * j), km, kbias);
            const unsigned xp = st.x16[2 * g + h][j];
            d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wp), __builtin_bit_cast(bf16x2, xp), d,
                                                false);
          }
        }
        acc16[r] = fmaf(sg, d, fmaf(cg * qd0, st.xs16[g], acc16[r]));
      }
    }
  }
}

// Workgroup = KW waves over the same 16·R rows; wave w takes K-blocks w, w + KW, … (adjacent waves read adjacent
// 1 KB blocks), with the next block's loads in flight while the current one is multiplied. The KW partial sums are
// added in wave order through LDS: no cross-workgroup synchronisation (an agent-scope fence on MI355X writes the
// XCD's L2 back and costs tens of µs) and a summation order that depends only on (N, K).
// T: MFMA token tiles (tokens 0–15, and 17–31 when T = 2); X16: token 16 present (M ≥ 17), done on VALU.
template <int T, int R, int KW, bool X16>
__global__ __launch_bounds__(64 * KW) void qmm_int4_kernel(QmmParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, qd = lane >> 4;
  const int tile0 = blockIdx.x * R;
  const float qd0 = qd == 0 ? 1.f : 0.f;
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
  rs.xs = make_rsrc(p.xs, unsigned(2 * p.nkb) * MAX_TOK * 4u);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tok = 16 * tt + n;
    const bool live = tt < T && tok < p.M && !(X16 && tok == 16);
    rs.xoff[tt] = live ? (unsigned(tok) * p.nkb * 256u + qd * 64u) : OOB;
    rs.xsoff[tt] = (tt < T && 16 * tt + 4 * qd < p.M) ? unsigned(16 * tt + 4 * qd) * 4u : OOB;
  }
  rs.x16off = 16u * p.nkb * 256u + qd * 64u;
  rs.xs16off = 16u * 4u;
  const unsigned km = vgpr_of(p.kmask), kbias = p.kbias;

  QmmStage<T, R, X16> a, b;
  int kb = wave;
  if (kb < p.nkb) {
    qmm_load(a, p, rs, tile0, kb, lane, n);
    while (true) {
      if (kb + KW < p.nkb) qmm_load(b, p, rs, tile0, kb + KW, lane, n);
      qmm_compute(acc, acc16, a, qd0, km, kbias);
      kb += KW;
      if (kb >= p.nkb) break;
      if (kb + KW < p.nkb) qmm_load(a, p, rs, tile0, kb + KW, lane, n);
      qmm_compute(acc, acc16, b, qd0, km, kbias);
      kb += KW;
      if (kb >= p.nkb) break;
    }
  }

  // Partial sums of every wave → LDS [wave][r][tt][e][lane], then a fixed-order sum over the waves.
  // Token 16: sum the four K slices of each row across lanes (qd = lane bits 4–5), fixed order.
  if constexpr (X16) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc16[r] += __shfl_xor(acc16[r], 16);
      acc16[r] += __shfl_xor(acc16[r], 32);
    }
  }
  constexpr int NEL = R * T * 4 * 64;
  constexpr int NEL16 = X16 ? R * 16 : 0;
  __shared__ float red[KW * (NEL + NEL16)];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave * (NEL + NEL16) + ((r * T + tt) * 4 + e) * 64 + lane] = acc[r][tt][e];
  if constexpr (X16) {
    if (lane < 16) {
#pragma unroll
      for (int r = 0; r < R; ++r) red[wave * (NEL + NEL16) + NEL + r * 16 + lane] = acc16[r];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NEL + NEL16; i += 64 * KW) {
    int m, row;
    if (i < NEL) {
      const int l = i & 63, e = (i >> 6) & 3, tt = (i >> 8) % T, r = (i >> 8) / T;
      m = 16 * tt + 4 * (l >> 4) + e;
      row = (tile0 + r) * 16 + (l & 15);
      if (X16 && m == 16) continue;
    } else {
      m = 16;
      row = tile0 * 16 + (i - NEL);
    }
    if (m >= p.M || row >= p.N) continue;
    float v = red[i];
#pragma unroll
    for (int w = 1; w < KW; ++w) v += red[w * (NEL + NEL16) + i];
    qmm_store(p, m, row, v);
  }
}

int launch_act_from_bf16(ih_ctx* c, const uint16_t* x, int ldx, int M, ActBuf& a) {
  act_kernel<uint16_t><<<MAX_TOK, 256, 0, c->stream>>>(x, ldx, M, a.K, a.nkb, static_cast<uint4*>(a.frag), a.xsum);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_act_from_f32(ih_ctx* c, const float* x, int ldx, int M, ActBuf& a) {
  act_kernel<float><<<MAX_TOK, 256, 0, c->stream>>>(x, ldx, M, a.K, a.nkb, static_cast<uint4*>(a.frag), a.xsum);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

// Launch shape for an (Npad, nkb) matrix: rows per workgroup (16·R) and waves per workgroup (KW, the intra-workgroup
// split of K). Chosen from the shape only, never from M, so each row's summation order is fixed.
struct QmmShape { int R, KW; };
static QmmShape qmm_shape(int Npad, int nkb) {
  const int NT = Npad / 16;
  if (NT >= 4096) return {4, 4};
  if (NT >= 1024) return {2, 4};
  if (NT >= 512 || nkb < 16) return {1, 4};
  if (nkb < 64) return {1, 8};
  return {1, 16};
}

template <int T, bool X16>
static void qmm_dispatch(QmmShape sh, int grid, hipStream_t st, const QmmParams& p) {
  if (sh.R == 4) qmm_int4_kernel<T, 4, 4, X16><<<grid, 256, 0, st>>>(p);
  else if (sh.R == 2) qmm_int4_kernel<T, 2, 4, X16><<<grid, 256, 0, st>>>(p);
  else if (sh.KW == 4) qmm_int4_kernel<T, 1, 4, X16><<<grid, 256, 0, st>>>(p);
  else if (sh.KW == 8) qmm_int4_kernel<T, 1, 8, X16><<<grid, 512, 0, st>>>(p);
  else qmm_int4_kernel<T, 1, 16, X16><<<grid, 1024, 0, st>>>(p);
}

int launch_qmm(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, void* y, int ldy, int out_mode) {
  IH_CHECK(W->format == QF_INT4, IH_EINVAL, "qmm: int4 matrix expected");
  IH_CHECK(M >= 1 && M <= MAX_TOK, IH_EINVAL, "qmm: M must be in 1..32");
  IH_CHECK(a.nkb == W->nkb && !a.f16, IH_EINVAL, "qmm: activation K does not match the matrix");
  QmmShape sh = qmm_shape(W->Npad, W->nkb);
  if (const char* ov = getenv("IH_QMM_SHAPE")) sscanf(ov, "%d,%d", &sh.R, &sh.KW);  // tuning override
  QmmParams p;
  const size_t tiles_per_e = size_t(W->Npad / 16) * W->nkb;
  p.w = static_cast<const uint4*>(W->w) + tiles_per_e * 64 * expert;
  p.s = static_cast<const uint2*>(W->s) + tiles_per_e * 16 * expert;
  p.xa = static_cast<const uint4*>(a.frag);
  p.xs = a.xsum;
  p.y = y;
  p.ldy = ldy;
  p.M = M;
  p.N = W->N;
  p.Npad = W->Npad;
  p.nkb = W->nkb;
  p.out_mode = out_mode;
  p.kmask = 0x000F000Fu;
  p.kbias = 0x43004300u;
  const int grid = W->Npad / (16 * sh.R);
  // Algorithmic bytes: the matrix in its MLX format, x (bf16) read, y written (read too when accumulating).
  const double ybytes = double(M) * W->N * (out_mode == QO_BF16 ? 2 : (out_mode == QO_F32_ADD ? 8 : 4));
  TimedLaunch tl(c, TC_QMM, double(W->algo_bytes) + double(M) * W->K * 2 + ybytes);
  if (M > 17) qmm_dispatch<2, true>(sh, grid, c->stream, p);
  else if (M == 17) qmm_dispatch<1, true>(sh, grid, c->stream, p);
  else qmm_dispatch<1, false>(sh, grid, c->stream, p);
  IH_HIP(hipGetLastError());
  return IH_OK;
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
                                               q->K, q->Npad, q->nkb);
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

}  // namespace ih

using namespace ih;

extern "C" {

int ih_qmat_int4_create_dev(ih_ctx* c, const void* w, const void* s, const void* b, int E, int N, int K,
                            ih_qmat** out) {
  IH_CHECK(c && w && s && b && out, IH_EINVAL, "ih_qmat_int4_create_dev: null argument");
  IH_CHECK(E >= 1 && N >= 1 && K >= 64 && K % 64 == 0, IH_EINVAL,
           "ih_qmat_int4_create_dev: need E, N >= 1 and K a positive multiple of 64");
  *out = nullptr;
  ih_qmat* q = new_qmat_int4(c, E, N, K);
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
