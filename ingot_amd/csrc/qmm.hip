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
//   - Split-K over a fixed number of slices chosen from (N, K) only, never from M, and the slices are summed in slice
//     order by the last workgroup to arrive: deterministic and row-invariant (row r's bits do not depend on M).
#include "ih_internal.h"

namespace ih {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16f(unsigned v16) { return __uint_as_float(v16 << 16); }

__device__ __forceinline__ unsigned short f2bf(float f) {
  unsigned u = __float_as_uint(f);
  return (unsigned short)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Eight nibbles of one word → eight bf16 values 128 + q in the element order {0,4,1,5,2,6,3,7}.
__device__ __forceinline__ bf16x8 nib_bf16(unsigned w) {
  u32x4 v;
  v.x = (w & 0x000F000Fu) | 0x43004300u;
  v.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  v.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  v.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
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
  float* part;             // split-K partials [splits][MAX_TOK][Npad]
  unsigned* counters;      // one per workgroup column
  void* y;
  int ldy, M, N, Npad, nkb, kps, out_mode;
};

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

// T: 16-token tiles (1 or 2); R: 16-row weight tiles per wave. Workgroup = 4 waves = 64·R rows, one K slice.
template <int T, int R>
__global__ __launch_bounds__(256) void qmm_int4_kernel(QmmParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, qd = lane >> 4;
  const int tile0 = (blockIdx.x * 4 + wave) * R;
  const int kb0 = blockIdx.y * p.kps;
  const int kb1 = min(p.nkb, kb0 + p.kps);
  f32x4 acc[R][T];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tt = 0; tt < T; ++tt) acc[r][tt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = kb0; kb < kb1; ++kb) {
    bf16x8 xa[T][4];
    f32x4 xs[T][2];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
      const uint4* src = p.xa + ((size_t(16 * tt + n) * p.nkb + kb) * 4 + qd) * 4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint4 u = src[t];
        xa[tt][t] = __builtin_bit_cast(bf16x8, u32x4{u.x, u.y, u.z, u.w});
      }
#pragma unroll
      for (int g = 0; g < 2; ++g)
        xs[tt][g] = *reinterpret_cast<const f32x4*>(p.xs + (2 * kb + g) * MAX_TOK + 16 * tt + 4 * qd);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t tb = size_t(tile0 + r) * p.nkb + kb;
      const u32x4 wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.w) + tb * 64 + lane);
      const uint2 sb = p.s[tb * 16 + n];
      const float s0 = bf16f(sb.x & 0xFFFFu), s1 = bf16f(sb.y & 0xFFFFu);
      const float c0 = fmaf(-128.f, s0, bf16f(sb.x >> 16)), c1 = fmaf(-128.f, s1, bf16f(sb.y >> 16));
      const unsigned ww[4] = {wv[0], wv[1], wv[2], wv[3]};
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const bf16x8 w0 = nib_bf16(ww[2 * g]), w1 = nib_bf16(ww[2 * g + 1]);
        const float sg = g ? s1 : s0, cg = g ? c1 : c0;
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
          f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[tt][2 * g], w0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[tt][2 * g + 1], w1, tmp, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][tt][e] = fmaf(sg, tmp[e], fmaf(cg, xs[tt][g][e], acc[r][tt][e]));
        }
      }
    }
  }

  // Output element (token m = 16·tt + 4·qd + e, row = 16·tile + n).
  if (gridDim.y == 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = (tile0 + r) * 16 + n;
#pragma unroll
      for (int tt = 0; tt < T; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = 16 * tt + 4 * qd + e;
          if (m < p.M && row < p.N) qmm_store(p, m, row, acc[r][tt][e]);
        }
    }
    return;
  }
  float* part = p.part + size_t(blockIdx.y) * MAX_TOK * p.Npad;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = (tile0 + r) * 16 + n;
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * tt + 4 * qd + e;
        if (m < p.M) part[size_t(m) * p.Npad + row] = acc[r][tt][e];
      }
  }
  __threadfence();
  __syncthreads();
  __shared__ unsigned s_last;
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&p.counters[blockIdx.x], 1u);
    s_last = (prev == gridDim.y - 1) ? 1u : 0u;
    if (s_last) p.counters[blockIdx.x] = 0u;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int rows = 64 * R, base = blockIdx.x * rows;
  for (int idx = threadIdx.x; idx < p.M * rows; idx += 256) {
    const int m = idx / rows, row = base + idx % rows;
    if (row >= p.N) continue;
    float v = 0.f;
    for (int sl = 0; sl < (int)gridDim.y; ++sl) v += p.part[(size_t(sl) * MAX_TOK + m) * p.Npad + row];
    qmm_store(p, m, row, v);
  }
}

// Split-K slices for an (Npad, nkb) launch: enough workgroups to cover the device about twice, at least two K-blocks
// per slice. Depends only on the matrix shape and the device, never on M.
static void qmm_plan(const ih_ctx* c, int Npad, int nkb, int R, int* splits, int* kps) {
  const int wgx = Npad / (64 * R);
  const int target = 2 * c->cu_count;
  int s = (target + wgx - 1) / wgx;
  s = std::max(1, std::min(s, nkb / 2 > 0 ? nkb / 2 : 1));
  int k = (nkb + s - 1) / s;
  *kps = k;
  *splits = (nkb + k - 1) / k;
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

int launch_qmm(ih_ctx* c, const ih_qmat* W, int expert, const ActBuf& a, int M, void* y, int ldy, int out_mode) {
  IH_CHECK(W->format == QF_INT4, IH_EINVAL, "qmm: int4 matrix expected");
  IH_CHECK(M >= 1 && M <= MAX_TOK, IH_EINVAL, "qmm: M must be in 1..32");
  IH_CHECK(a.nkb == W->nkb && !a.f16, IH_EINVAL, "qmm: activation K does not match the matrix");
  const int R = 2;
  int splits, kps;
  qmm_plan(c, W->Npad, W->nkb, R, &splits, &kps);
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
  p.kps = kps;
  p.out_mode = out_mode;
  const int wgx = W->Npad / (64 * R);
  if (splits > 1) {
    IH_TRY(ensure_part(c, size_t(splits) * MAX_TOK * W->Npad * 4));
    IH_CHECK(size_t(wgx) <= c->n_counters, IH_EINVAL, "qmm: too many workgroups for the counter array");
  }
  p.part = c->part;
  p.counters = c->counters;
  dim3 grid(wgx, splits);
  if (M > 16) qmm_int4_kernel<2, R><<<grid, 256, 0, c->stream>>>(p);
  else qmm_int4_kernel<1, R><<<grid, 256, 0, c->stream>>>(p);
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
