// MoE block of the verify round on gfx950: MXFP4 weights, the router's top-k and expert union, the gathered per-expert
// quantized matmuls (gate|up with the gated activation, down) and the slot-ordered combine with the residual.
//
// Reference: MoELayer.encode (Sources/Ingot/Layers/MoE.swift:346-428): router qmv → vmoe_route
// (Sources/Ingot/Shaders/verify.metal:160-319) → vnax_moe_gateup (Shaders/verify_nax.metal:258-359) →
// vnax_moe_down_split (:419-509) → vmoe_combine9 (:527-540); MXFP4 decode lab_e8m0x / lab_fp4x2
// (Shaders/qmm_nax_moe.metal:280-288).
//
// MI355X design:
//   - One launch covers every expert of the round: the grid is (row tiles, expert slots) with as many slots as the
//     union can have (min(E, B·k)); a workgroup reads its slot's record (written by the routing on the device) and
//     returns when the slot is unused, so the host never waits for the routing. A slot's tokens are gathered through
//     a row map: the round's rows for gate|up, the expert's own pair rows for down.
//   - Weights stream as 16-row × 128-K tiles, one 1024-byte dwordx4 load per wave and tile (the dense qmm's layout);
//     a workgroup of one wave takes four tiles over all of K (few K-blocks), or four waves split K over two tiles,
//     added in wave order in LDS (many K-blocks).
//   - int4 g64: bf16 MFMA on 128 + q with the affine map applied per group (as the dense qmm). MXFP4: an e2m1 code
//     becomes its exact fp16 value with one v_perm_b32 table lookup per pair and the sign OR-ed in; the MFMA runs in
//     fp16 against fp16 activations, and one e8m0 scale per 32 K (= one MFMA step) multiplies the step's products.
#include "act.h"
#include "ih_internal.h"
#include "qmm_common.h"

namespace ih {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------------------------------------------
// Repack an MLX mxfp4 matrix (codes [E][N][K/8] u32, low nibble first; e8m0 scales [E][N][K/32] u8) into the tile
// layout: codes exactly as the int4 tiles (pack_int4_kernel), scales one u32 per row and K-block holding the four
// e8m0 bytes of its 32-K groups. Rows past N and groups past K read 0 (code 0 is +0). il8: interleave a gate|up pair
// by eights as the int4 pack does. Grid (Npad/16 · nkb, E), 64 threads.
__global__ void pack_mxfp4_kernel(const uint32_t* __restrict__ w, const uint8_t* __restrict__ s, uint4* __restrict__ wp,
                                  uint32_t* __restrict__ sp, int N, int K, int Npad, int nkb, int il8) {
  const int lane = threadIdx.x, n = lane & 15, qd = lane >> 4;
  const int tile = blockIdx.x / nkb, kb = blockIdx.x % nkb, e = blockIdx.y;
  const int prow = tile * 16 + n;
  const int row = il8 ? (n < 8 ? 8 * tile + n : N / 2 + 8 * tile + n - 8) : prow;
  const bool live = il8 ? (8 * tile + (n & 7) < N / 2) : row < N;
  const int wpr = K / 8, gpr = K / 32;
  const size_t ebase_w = size_t(e) * N * wpr, ebase_s = size_t(e) * N * gpr;
  unsigned v[4];
  for (int t = 0; t < 4; ++t) {
    const int wi = kb * 16 + 4 * t + qd;
    v[t] = (live && wi < wpr) ? w[ebase_w + size_t(row) * wpr + wi] : 0u;
  }
  const size_t tb = (size_t(e) * (Npad / 16) + tile) * nkb + kb;
  wp[tb * 64 + lane] = make_uint4(v[0], v[1], v[2], v[3]);
  if (qd == 0) {
    unsigned sc = 0;
    for (int g = 0; g < 4; ++g) {
      const int gi = 4 * kb + g;
      if (live && gi < gpr) sc |= unsigned(s[ebase_s + size_t(row) * gpr + gi]) << (8 * g);
    }
    sp[tb * 16 + n] = sc;
  }
}

// Eight e2m1 codes of one word → eight fp16 values in the element order {0,4,1,5,2,6,3,7}: pair c = (code c, code
// c+4) = bits (4c, 4c+16) of w >> 4c. The magnitude (3 bits) selects the fp16 high byte from the table {0x00, 0x38,
// 0x3C, 0x3E, 0x40, 0x42, 0x44, 0x46} (0, .5, 1, 1.5, 2, 3, 4, 6; low bytes are 0) with one v_perm_b32; the sign bit
// goes to bit 15.
__device__ __forceinline__ f16x8 e2m1_f16(unsigned w) {
  u32x4 v;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const unsigned x = w >> (4 * c);
    const unsigned sel = ((x & 0x00070007u) << 8) | 0x000C000Cu;  // bytes 1, 3 ← table[m]; bytes 0, 2 ← 0
    const unsigned mag = __builtin_amdgcn_perm(0x46444240u, 0x3E3C3800u, sel);
    v[c] = mag | ((x & 0x00080008u) << 12);
  }
  return __builtin_bit_cast(f16x8, v);
}

// 2^(e − 127) for an e8m0 byte (255 → NaN), exact in fp32 (e = 0 → 2^-127, a subnormal).
__device__ __forceinline__ float e8m0f(unsigned e) {
  return e == 0 ? __uint_as_float(0x00400000u) : (e == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float(e << 23));
}

// ---------------------------------------------------------------------------------------------------------------
enum GatherMode : int {
  GM_F32 = 0,   // y[pair][row] = r · v
  GM_GLU = 1,   // gated activation of the interleaved gate|up pair (r · v + bias) → h fragment of the pair
  GM_DOWN = 2,  // y[pair][row] = v + bias
};

struct GatherParams {
  const uint4* w;          // all experts' tiles
  const void* s;           // all experts' scales (int4: uint2 per row, mxfp4: u32 per row)
  unsigned tiles_per_e;    // (Npad / 16) · nkb
  unsigned E;
  const uint4* xa;         // activation fragments (bf16 for int4, fp16 for mxfp4)
  int x_nkb, x_tokens;     // fragment K-blocks; tokens the fragment buffer holds (a multiple of 16)
  const int* x_row;        // pair → activation row (null: the pair index itself)
  const int* entries;      // [U][3] (expert, first pair, pairs); null: one entry (dense_e, 0, M)
  const int* nent;         // U on the device (null: 1)
  const int4* slots;       // one record per possible slot, (expert, first pair, pairs, live); null: entries + nent
  int dense_e, M;
  int N, Npad, nkb, mode;
  void* y;
  int ldy;
  // RMSNorm factor of the activation rows (router and gate|up): r_t = 1/sqrt(Σ ss_in[t][j] / D + eps).
  const float* ss_in;
  int nss_in, D, nrows;
  float eps;
  uint4* h_out;            // GM_GLU: next activation (fragments), by pair
  int h_nkb, h_ntile, h_f16, glu;
  float limit;
  const uint16_t* bias;    // bf16; GM_GLU: [E][2·(N/2)] gate then up; GM_DOWN: [E][N]; null: none
  unsigned kmask, kbias;
  int trips;               // ring trips of D K-blocks per wave: ⌈⌈nkb / GKW⌉ / D⌉ (set by the launch)
};

// Kernel format of the gathered product: the matrix formats, plus int4 codes against fp16 activations (an affine
// router in front of MXFP4 experts, whose activation rows are fp16: a nibble becomes the exact fp16 1024 + q, the MFMA
// runs in fp16 and the affine map is y = s·acc + (b − 1024·s)·Σx).
constexpr int GF_INT4_F16 = 2;

template <int FMT, int R>
struct GStage {
  u32x4 w[R];
  uint2 s[R];  // int4 (both kernel formats): (s0|b0<<16, s1|b1<<16); mxfp4: .x = four e8m0 bytes
  u32x4 x[4];  // one token tile's activation fragments of the K-block
};

// R row tiles × (one slot of the round): grid (⌈N/16/R⌉, slots), 64·GKW threads (GKW waves splitting K). The R
// tiles of a wave share each x fragment, and a workgroup streams R times the bytes behind its one read of the slot's
// routing entry.
//
// Wave w takes K-blocks w, w + GKW, w + 2·GKW, … through a ring of D stages, all D requested at entry, and the stage
// just multiplied refilled D·GKW K-blocks ahead. Many slots run at D = 1: the registers of deeper rings cost waves
// per SIMD, and other workgroups' waves hide a stage's latency better (the launch picks GKW, R and D). K-blocks past
// the matrix load as zeros (out-of-range buffer offsets: no memory traffic) and add exactly nothing. A slot with more
// than 16 pairs (one expert chosen by more than 16 rows) runs the K loop again for its second token tile, so the ring
// holds one token tile's activations.
template <int FMT, int R, int D, int GKW>
__global__ __launch_bounds__(64 * GKW) void qmm_gather_kernel(GatherParams p) {
  constexpr bool I4 = FMT != QF_MXFP4, XH = FMT == GF_INT4_F16;  // int4 codes; fp16 activations for them
  const int u = blockIdx.y;
  int e, start, cnt;
  if (p.slots) {
    // One 16-byte read names the slot's expert and pairs, or that it is unused (one memory latency, not two).
    const int4 r = p.slots[u];
    if (!r.w) return;
    e = r.x;
    start = r.y;
    cnt = r.z;
  } else if (p.entries) {
    const int U = p.nent ? __builtin_amdgcn_readfirstlane(p.nent[0]) : 1;
    if (u >= U) return;
    e = p.entries[3 * u];
    start = p.entries[3 * u + 1];
    cnt = p.entries[3 * u + 2];
  } else {
    e = p.dense_e;
    start = 0;
    cnt = p.M;
  }
  e = __builtin_amdgcn_readfirstlane(e);
  start = __builtin_amdgcn_readfirstlane(start);
  cnt = __builtin_amdgcn_readfirstlane(cnt);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, qd = lane >> 4;
  const int tile0 = blockIdx.x * R;
  const int ntt = cnt > 16 ? 2 : 1;  // token tiles (uniform)
  __shared__ float rsc[MAX_TOK];
  __shared__ int arow_s[MAX_TOK];

  const size_t tb0 = size_t(e) * p.tiles_per_e + size_t(tile0) * p.nkb;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w + tb0 * 64, unsigned(R * p.nkb) * 1024u);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.s) + tb0 * (I4 ? 128 : 64),
                                              unsigned(R * p.nkb) * (I4 ? 128u : 64u));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.xa, unsigned(p.x_tokens) * p.x_nkb * 256u);
  unsigned xoff[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int j = 16 * tt + n;
    const int ar = j < cnt ? (p.x_row ? p.x_row[start + j] : start + j) : -1;
    xoff[tt] = ar >= 0 ? unsigned(ar >> 4) * 4096u + unsigned(ar & 15) * 64u + qd * 16u : OOB;
  }
  if (threadIdx.x < MAX_TOK) {
    const int j = threadIdx.x;
    arow_s[j] = j < cnt ? (p.x_row ? p.x_row[start + j] : start + j) : 0;
  }

  auto load = [&](GStage<FMT, R>& st, int kb, unsigned xo) {
    const unsigned oob = kb < p.nkb ? 0u : OOB;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const unsigned tk = unsigned(r * p.nkb + kb);
      st.w[r] =
          __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, (tk * 1024u + lane * 16u) | oob, 0, 0));
      if constexpr (I4)
        st.s[r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, (tk * 128u + n * 8u) | oob, 0, 0));
      else
        st.s[r].x = __builtin_amdgcn_raw_buffer_load_b32(rs, (tk * 64u + n * 4u) | oob, 0, 0);
    }
    const unsigned kx = unsigned(kb) * unsigned(p.x_tokens / 16) * 4096u;  // [kb][tile][t][1 KB]
#pragma unroll
    for (int t = 0; t < 4; ++t)
      st.x[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (xo + kx + 1024 * t) | oob, 0, 0));
  };

  f32x4 acc[R];
  const unsigned km = vgpr_of(p.kmask), kbias = p.kbias;
  const unsigned shv[3] = {vgpr_of(4u), vgpr_of(8u), vgpr_of(12u)};  // 64-bit nibble shifts (nib_bf16_pair)
  // One MFMA step in the activations' type (bf16, or fp16 for XH); the operands travel as raw 32-bit words.
  auto mma = [](const u32x4& a, const u32x4& b, f32x4 c) -> f32x4 {
    if constexpr (XH)
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                    0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                     0, 0, 0);
  };
  auto compute = [&](const GStage<FMT, R>& st) {
    if constexpr (I4) {
      // 1.0 in the activations' type; a nibble q decodes to the exact 128 + q (bf16) or 1024 + q (fp16).
      const unsigned one = XH ? 0x3C003C00u : 0x3F803F80u;
      const u32x4 ones = u32x4{one, one, one, one};
      constexpr float OFF = XH ? 1024.f : 128.f;
      // Σx per group, shared by the R tiles.
      f32x4 xs[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) xs[g] = mma(st.x[2 * g + 1], ones, mma(st.x[2 * g], ones, f32x4{0.f, 0.f, 0.f, 0.f}));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float s0 = bf16f(st.s[r].x & 0xFFFFu), s1 = bf16f(st.s[r].y & 0xFFFFu);
        const float c0 = fmaf(-OFF, s0, bf16f(st.s[r].x >> 16)), c1 = fmaf(-OFF, s1, bf16f(st.s[r].y >> 16));
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          bf16x8 w0, w1;
          nib_bf16_pair(st.w[r][2 * g], st.w[r][2 * g + 1], km, kbias, shv, w0, w1);
          const float sg = g ? s1 : s0, cg = g ? c1 : c0;
          f32x4 tmp = mma(st.x[2 * g], __builtin_bit_cast(u32x4, w0), f32x4{0.f, 0.f, 0.f, 0.f});
          tmp = mma(st.x[2 * g + 1], __builtin_bit_cast(u32x4, w1), tmp);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[r][q] = fmaf(sg, tmp[q], fmaf(cg, xs[g][q], acc[r][q]));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f16x8 wf = e2m1_f16(st.w[r][t]);
          const float sc = e8m0f((st.s[r].x >> (8 * t)) & 0xFFu);
          const f32x4 tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, st.x[t]), wf,
                                                                   f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[r][q] = fmaf(sc, tmp[q], acc[r][q]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Waves' partial sums → LDS [wave][r][tt][q][lane], then added in wave order.
  constexpr int WST = R * 2 * 4 * 64;
  __shared__ float red[GKW * WST];
#pragma unroll 1
  for (int tt = 0; tt < ntt; ++tt) {
    const unsigned xo = tt ? xoff[1] : xoff[0];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    GStage<FMT, R> st[D];
#pragma unroll
    for (int d = 0; d < D; ++d) load(st[d], wave + d * GKW, xo);
    int kb = wave + D * GKW;
#pragma unroll 1
    for (int t = 0; t < p.trips; ++t) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        compute(st[d]);
        // The last trip's refills lie past the matrix (trips·D·GKW ≥ nkb): zeros, no memory traffic.
        load(st[d], kb + d * GKW, xo);
      }
      kb += D * GKW;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave * WST + ((r * 2 + tt) * 4 + q) * 64 + lane] = acc[r][q];
  }

  // RMSNorm factors of the activation rows.
  if (p.ss_in) rms_factors(p.ss_in, SS_CAP, p.nss_in, p.D, p.eps, p.nrows, rsc, wave, GKW, lane);

  __syncthreads();
  auto val = [&](int r, int j, int rn) {
    const int tt = j >> 4, jj = j & 15;
    const int i = ((r * 2 + tt) * 4 + (jj & 3)) * 64 + 16 * (jj >> 2) + rn;
    float v = red[i];
#pragma unroll
    for (int w = 1; w < GKW; ++w) v += red[w * WST + i];
    return v;
  };
  const int nthr = 64 * GKW;
  if (p.mode == GM_GLU) {
    // Interleaved tiles: rows 0–7 gate, 8–15 up of the same 8 columns (output chunk tile0 + r).
    const int I = p.N / 2;
    for (int u2 = threadIdx.x; u2 < cnt * R; u2 += nthr) {
      const int j = u2 / R, r = u2 % R, tile = tile0 + r;
      const float rr = p.ss_in ? rsc[arow_s[j]] : 1.f;
      float v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int col = 8 * tile + c;
        float g = val(r, j, c) * rr, uu = val(r, j, 8 + c) * rr;
        if (p.bias && col < I) {
          g += bf16f(p.bias[size_t(e) * 2 * I + col]);
          uu += bf16f(p.bias[size_t(e) * 2 * I + I + col]);
        }
        v[c] = col < I ? glu_f(g, uu, p.glu, p.limit) : 0.f;
      }
      if (8 * tile < I) frag_store(p.h_f16 != 0, p.h_out, p.h_nkb, p.h_ntile, start + j, tile, v);
    }
    return;
  }
  for (int q = threadIdx.x; q < cnt * 16 * R; q += nthr) {
    const int j = q / (16 * R), rr = q % (16 * R), r = rr >> 4, rn = rr & 15;
    const int row = (tile0 + r) * 16 + rn;
    if (row >= p.N) continue;
    float v = val(r, j, rn);
    if (p.mode == GM_F32 && p.ss_in) v *= rsc[arow_s[j]];
    if (p.mode == GM_DOWN && p.bias) v += bf16f(p.bias[size_t(e) * p.N + row]);
    static_cast<float*>(p.y)[size_t(start + j) * p.ldy + row] = v;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Routing of the round (vmoe_route, verify.metal:160-319; RouterVector.reference, KernelCaseRouter.swift:54-80):
// logits + router bias (NaN → −inf); top-k by value, ties to the lower expert index; weights = softmax over the chosen
// logits, times an optional per-expert scale. Then the expert union by counting sort: entries (expert, first pair,
// pairs) in increasing expert order, pairs in row order inside an expert; x_row[pair] = its row, pair_w[pair] = its
// weight, row_pair[row·k + slot] = its pair. One workgroup of 1024 threads (E ≤ 256, k ≤ 16, rows ≤ 32).
//
// The top-k takes k rounds of a 32-lane (value, index) reduction per row, lanes 0-31 and 32-63 of a wave holding two
// rows, so the 16 waves cover every row at once; the reductions are register-to-register (DPP within 16 lanes, then
// a swap of the two 16-lane rows). A row picks an expert at most once, so an expert's rows fit one 32-bit mask (rows
// ≤ 32): its pair count is the mask's population and a pair's place among the expert's pairs is the population below
// its row. The exclusive scans over experts (first pair, entry slot) come from wave ballots of the count's bits.
namespace {
// Top-k key: the logit in the high word, mapped so that unsigned order is float order (−0 taken as +0; −inf maps
// above 0, so 0 means "taken"), and ~expert in the low word, so that the larger key is the larger logit, then the
// lower expert.
__device__ __forceinline__ unsigned long long topk_key(float x, int ex) {
  const unsigned b = __float_as_uint(x == 0.f ? 0.f : x);
  const unsigned u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<unsigned long long>(u) << 32) | unsigned(~ex);
}
__device__ __forceinline__ float topk_value(unsigned long long k) {
  const unsigned u = unsigned(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}
__device__ __forceinline__ unsigned long long kmax(unsigned long long a, unsigned long long b) { return a > b ? a : b; }
// Partner key of a DPP lane pattern (all 64 lanes active).
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_k(unsigned long long k) {
  const int lo = __builtin_amdgcn_update_dpp(int(unsigned(k)), int(unsigned(k)), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(int(unsigned(k >> 32)), int(unsigned(k >> 32)), CTRL, 0xF, 0xF, false);
  return (static_cast<unsigned long long>(unsigned(hi)) << 32) | unsigned(lo);
}
// Largest key over each 32-lane half of the wave; every lane of the half ends with it.
__device__ __forceinline__ unsigned long long best32(unsigned long long k) {
  k = kmax(k, dpp_k<0xB1>(k));   // quad_perm [1,0,3,2]
  k = kmax(k, dpp_k<0x4E>(k));   // quad_perm [2,3,0,1]
  k = kmax(k, dpp_k<0x141>(k));  // row_half_mirror
  k = kmax(k, dpp_k<0x140>(k));  // row_mirror
  // Rows 0↔1 and 2↔3: each lane gets its own key and its partner row's, in an order it cannot tell apart.
  const auto lo = __builtin_amdgcn_permlane16_swap(unsigned(k), unsigned(k), false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(unsigned(k >> 32), unsigned(k >> 32), false, false);
  return kmax((static_cast<unsigned long long>(hi[0]) << 32) | lo[0],
              (static_cast<unsigned long long>(hi[1]) << 32) | lo[1]);
}
}  // namespace

template <int NE>
__global__ __launch_bounds__(1024) void moe_route_kernel(const float* __restrict__ logits, int ldl, int rows, int E,
                                                         int K, const float* __restrict__ bias,
                                                         const float* __restrict__ pes, int* __restrict__ nent,
                                                         int* __restrict__ entries, int4* __restrict__ slots,
                                                         int nslots, int* __restrict__ x_row,
                                                         float* __restrict__ pair_w, int* __restrict__ row_pair,
                                                         MoeIid iid) {
  __shared__ float lg[MAX_TOK][256];
  __shared__ int inds[MAX_TOK * 16];
  __shared__ float chosen[MAX_TOK * 16];
  __shared__ unsigned rmask[256];  // bit r: row r chose the expert
  __shared__ int lstart[256], lslot[256], wpairs[4], wslots[4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
  const int nrk = rows * K;
  // Logits (+ router bias), NaN → −inf, one row per wave at a time. With synthetic i.i.d. routing the router's logit
  // of (row, expert) is replaced by the N(0,1) draw of (position, expert).
  const int pos0 = iid.pos_dev ? int(min(iid.pos_dev[0], uint32_t(iid.pos_max))) : iid.pos;
  for (int r = wave; r < rows; r += nw)
    for (int ex = lane; ex < E; ex += 64) {
      const float lv = iid.key ? sm_normal(iid.key, uint64_t(pos0 + r) * uint64_t(E) + uint64_t(ex))
                               : logits[size_t(r) * ldl + ex];
      float x = lv + (bias ? bias[ex] : 0.f);
      lg[r][ex] = x != x ? -INFINITY : x;
    }
  if (tid < 256) rmask[tid] = 0u;
  __syncthreads();
  // Top-k: k rounds of "largest logit, then lowest index" among the experts not yet chosen (a −inf logit still ranks,
  // so a row with fewer than k finite logits takes the lowest remaining indices). Lane l of a half holds experts
  // l + 32·i (NE of them: E ≤ 32·NE). Both halves of a wave run every round (a row past the last repeats the last
  // row and writes nothing); waves past the rows skip it.
  if (2 * wave < rows) {
    const int r = 2 * wave + (lane >> 5), hl = lane & 31, rr = min(r, rows - 1);
    unsigned long long key[NE];  // 0: out of range or already chosen
#pragma unroll
    for (int i = 0; i < NE; ++i) key[i] = hl + 32 * i < E ? topk_key(lg[rr][hl + 32 * i], hl + 32 * i) : 0ull;
    for (int k = 0; k < K; ++k) {
      unsigned long long bk = key[0];
#pragma unroll
      for (int i = 1; i < NE; ++i) bk = kmax(bk, key[i]);
      bk = best32(bk);
      const int bi = int(~unsigned(bk));
      if (hl == 0 && r < rows) {
        inds[r * K + k] = bi;
        chosen[r * K + k] = topk_value(bk);
        atomicOr(&rmask[bi], 1u << r);
      }
#pragma unroll
      for (int i = 0; i < NE; ++i)
        if (hl + 32 * i == bi) key[i] = 0ull;
    }
  }
  __syncthreads();
  // Weights: softmax over the row's k chosen logits (summed in slot order from the largest), × the per-expert scale.
  float wgt = 0.f;
  if (tid < nrk) {
    const int r = tid / K;
    float sum = 0.f;
    for (int kk = 0; kk < K; ++kk) sum += expf(chosen[r * K + kk] - chosen[r * K]);
    wgt = expf(chosen[tid] - chosen[r * K]) / sum * (pes ? pes[inds[tid]] : 1.0f);
  }
  // Expert tid (waves 0-3): pairs c ≤ 32; the exclusive scans of c and of (c > 0) inside the wave from ballots of
  // c's six bits, the wave totals through LDS.
  int c = 0;
  if (wave < 4) {
    c = tid < E ? __popc(rmask[tid]) : 0;
    const unsigned long long below = (1ull << lane) - 1ull;
    int off = 0, tot = 0;
#pragma unroll
    for (int bit = 0; bit < 6; ++bit) {
      const unsigned long long m = __ballot((c >> bit) & 1);
      off += __popcll(m & below) << bit;
      tot += __popcll(m) << bit;
    }
    const unsigned long long nz = __ballot(c > 0);
    lstart[tid] = off;
    lslot[tid] = __popcll(nz & below);
    if (lane == 0) {
      wpairs[wave] = tot;
      wslots[wave] = __popcll(nz);
    }
  }
  __syncthreads();
  if (tid < E && c > 0) {
    int sl = lslot[tid], st = lstart[tid];
    for (int w = 0; w < wave; ++w) {
      sl += wslots[w];
      st += wpairs[w];
    }
    entries[3 * sl] = tid;
    entries[3 * sl + 1] = st;
    entries[3 * sl + 2] = c;
    if (slots) slots[sl] = make_int4(tid, st, c, 1);
  }
  const int U = (wslots[0] + wslots[1]) + (wslots[2] + wslots[3]);
  if (tid == 0) nent[0] = U;
  if (slots && tid >= U && tid < nslots) slots[tid] = make_int4(0, 0, 0, 0);
  // Pair (row r, slot) of expert e goes to first[e] + #{rows r' < r that chose e}.
  if (tid < nrk) {
    const int e = inds[tid], r = tid / K;
    int st = lstart[e] + __popc(rmask[e] & ((1u << r) - 1u));
    for (int w = 0; w < (e >> 6); ++w) st += wpairs[w];
    x_row[st] = r;
    pair_w[st] = wgt;
    row_pair[tid] = st;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Combine (vmoe_combine9, verify_nax.metal:527-540) fused with the residual and the next RMSNorm input: for row r,
// y = Σ_slot w·o[pair(r, slot)] in slot order, h[r] += y, the next activation (h ⊙ nw, bf16 or fp16) and Σh² (one
// partial per row). Grid (rows), one thread per 8 columns (up to 1024; a thread takes further chunks past that). The
// row's pair numbers and weights are read once into LDS; h and o move 16 bytes at a time.
__global__ __launch_bounds__(1024) void moe_combine_kernel(const float* __restrict__ o, int ldo,
                                                           const int* __restrict__ row_pair,
                                                           const float* __restrict__ pair_w, int K,
                                                           float* __restrict__ h, int ldh, int H,
                                                           const uint16_t* __restrict__ nw, uint4* __restrict__ act,
                                                           int act_nkb, int act_ntile, int act_f16,
                                                           float* __restrict__ ss_out) {
  __shared__ float red[16];
  __shared__ int prs[16];
  __shared__ float ws[16];
  const int r = blockIdx.x, tid = threadIdx.x;
  if (tid < K) {
    const int pr = row_pair[r * K + tid];
    prs[tid] = pr;
    ws[tid] = pair_w[pr];
  }
  __syncthreads();
  float ss = 0.f;
  for (int c = tid; c < H / 8; c += blockDim.x) {
    float4* hp = reinterpret_cast<float4*>(h + size_t(r) * ldh + 8 * c);
    const float4 h0 = hp[0], h1 = hp[1];
    float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int k = 0; k < K; ++k) {
      const float w = ws[k];
      const float4* op = reinterpret_cast<const float4*>(o + size_t(prs[k]) * ldo + 8 * c);
      const float4 a = op[0], b = op[1];
      y[0] += w * a.x;
      y[1] += w * a.y;
      y[2] += w * a.z;
      y[3] += w * a.w;
      y[4] += w * b.x;
      y[5] += w * b.y;
      y[6] += w * b.z;
      y[7] += w * b.w;
    }
    const float hv[8] = {h0.x + y[0], h0.y + y[1], h0.z + y[2], h0.w + y[3],
                         h1.x + y[4], h1.y + y[5], h1.z + y[6], h1.w + y[7]};
    hp[0] = float4{hv[0], hv[1], hv[2], hv[3]};
    hp[1] = float4{hv[4], hv[5], hv[6], hv[7]};
    const uint4 nv = reinterpret_cast<const uint4*>(nw)[c];
    const unsigned nwu[4] = {nv.x, nv.y, nv.z, nv.w};
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss += hv[j] * hv[j];
      v[j] = hv[j] * bf16f(uint16_t(nwu[j >> 1] >> (16 * (j & 1))));
    }
    frag_store(act_f16 != 0, act, act_nkb, act_ntile, r, c, v);
  }
  ss += lane_xor<32>(ss);
  ss += lane_xor<16>(ss);
  ss += lane_xor<8>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<1>(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < int(blockDim.x >> 6); ++w) t += red[w];
    ss_out[size_t(r) * SS_CAP] = t;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Host side.

// x_f16: the activation fragments are fp16 (MXFP4 matrices always take fp16; an int4 matrix then runs the fp16 decode).
int launch_gather(ih_ctx* c, const ih_qmat* W, const GatherParams& base, int slots, double bytes, bool x_f16) {
  GatherParams p = base;
  p.w = static_cast<const uint4*>(W->w);
  p.s = W->s;
  p.tiles_per_e = unsigned(W->Npad / 16) * unsigned(W->nkb);
  p.E = unsigned(W->E);
  p.N = W->N;
  p.Npad = W->Npad;
  p.nkb = W->nkb;
  p.kmask = 0x000F000Fu;
  p.kbias = x_f16 && W->format == QF_INT4 ? 0x64006400u : 0x43004300u;  // nibble → fp16 1024 + q / bf16 128 + q
  IH_CHECK(p.x_nkb == W->nkb, IH_EINVAL, "gathered qmm: activation K does not match the matrix");
  IH_CHECK(size_t(W->E) * p.tiles_per_e * 1024u < (size_t(1) << 31), IH_EINVAL,
           "gathered qmm: stacked matrix above 2 GiB");
  TimedLaunch tl(c, TC_MOE, bytes);
  // Waves per workgroup (K split), row tiles per workgroup and ring depth, measured on the MoE configurations (i.i.d.
  // routing, MoE kernels per step). Many slots: with K at most 16 K-blocks (E128 top-8, K = 2048 and 768) one wave
  // per workgroup over four tiles (3.27 ms) beats two waves over four tiles (3.30), over two tiles (3.72) and four
  // waves over two (3.95) or one (5.13); with more K-blocks (E32 top-4, K = 2880) four waves over two tiles (2.22)
  // beat two waves (2.52), eight (2.46), and four tiles (2.43). A slot holds few pairs, so a workgroup's life is a
  // few memory latencies and the rate is set by how much each wave streams behind them: longer waves win until the
  // registers cost waves per SIMD (eight tiles: 171 VGPRs, 3.53 ms; a ring of two or three stages: 4.47, 5.70). A
  // single slot (a router, or one expert) has few workgroups; there K is split over waves and every K-block of a
  // wave is requested at entry.
  // Only tiles with a live row are launched (rows are padded to 256 in memory, so the tiles of a group past N stay
  // inside the matrix: their rows read as the zero padding and are not stored).
  const int tiles = (W->N + 15) / 16;
  int GKW, R = 1, D = 1;
  if (slots == 1) {
    GKW = W->nkb <= 16 ? 2 : 4;
    const int kpw = (W->nkb + GKW - 1) / GKW;
    D = kpw <= 1 ? 1 : (kpw <= 2 ? 2 : 4);
  } else if (W->nkb <= 16) {
    GKW = 1;
    R = 4;
  } else {
    GKW = 4;
    if (((tiles + 1) / 2) * slots >= 2 * c->cu_count) R = 2;
  }
  const int kpw = (W->nkb + GKW - 1) / GKW;
  p.trips = (kpw + D - 1) / D;
  const dim3 grid((tiles + R - 1) / R, slots);
#define IH_GATHER_LAUNCH(R_, D_, W_)                                                                                \
  if (R == R_ && D == D_ && GKW == W_) {                                                                          \
    if (W->format == QF_MXFP4)                                                                                    \
      tlaunch(tl, qmm_gather_kernel<QF_MXFP4, R_, D_, W_>, grid, dim3(64 * W_), 0, c->stream, p);                 \
    else if (x_f16)                                                                                               \
      tlaunch(tl, qmm_gather_kernel<GF_INT4_F16, R_, D_, W_>, grid, dim3(64 * W_), 0, c->stream, p);              \
    else                                                                                                          \
      tlaunch(tl, qmm_gather_kernel<QF_INT4, R_, D_, W_>, grid, dim3(64 * W_), 0, c->stream, p);                  \
  }
  IH_GATHER_LAUNCH(1, 1, 2) IH_GATHER_LAUNCH(1, 2, 2) IH_GATHER_LAUNCH(1, 4, 2) IH_GATHER_LAUNCH(1, 1, 4)
  IH_GATHER_LAUNCH(1, 2, 4) IH_GATHER_LAUNCH(1, 4, 4) IH_GATHER_LAUNCH(2, 1, 4) IH_GATHER_LAUNCH(4, 1, 1)
#undef IH_GATHER_LAUNCH
  IH_HIP(hipGetLastError());
  return IH_OK;
}

// slots (may be null): the one-record slot table of the gathered launches, min(E, rows·K) records.
int launch_moe_route(ih_ctx* c, const float* logits, int ldl, int rows, int E, int K, const float* bias,
                     const float* pes, int* nent, int* entries, int4* slots, int* x_row, float* pair_w, int* row_pair,
                     const MoeIid& iid) {
  IH_CHECK(E >= 1 && E <= 256 && K >= 1 && K <= 16 && K <= E && rows >= 1 && rows <= MAX_TOK, IH_EINVAL,
           "moe route: need E ≤ 256, 1 ≤ k ≤ min(16, E), 1 ≤ rows ≤ 32");
  TimedLaunch tl(c, TC_MOE, double(rows) * E * 4);
  auto kern = E <= 128 ? moe_route_kernel<4> : moe_route_kernel<8>;
  tlaunch(tl, kern, dim3(1), dim3(1024), 0, c->stream, logits, ldl, rows, E, K, bias, pes, nent, entries, slots,
          std::min(E, rows * K), x_row, pair_w, row_pair, iid);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int launch_moe_combine(ih_ctx* c, const float* o, int ldo, const int* row_pair, const float* pair_w, int K, int rows,
                       float* h, int H, const uint16_t* nw, ActBuf& act) {
  IH_CHECK(H % 8 == 0, IH_EINVAL, "moe combine: hidden size must be a multiple of 8");
  TimedLaunch tl(c, TC_MOE, double(rows) * H * (4.0 * K + 8 + 2));
  IH_CHECK(ldo % 4 == 0 && K <= 16 && reinterpret_cast<uintptr_t>(o) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(h) % 16 == 0 && reinterpret_cast<uintptr_t>(nw) % 16 == 0,
           IH_EINVAL, "moe combine: o, h and the norm weights must be 16-byte aligned, k ≤ 16");
  const int threads = std::min(1024, (H / 8 + 63) / 64 * 64);
  tlaunch(tl, moe_combine_kernel, dim3(rows), dim3(threads), 0, c->stream, o, ldo, row_pair, pair_w, K, h, H, H, nw,
          static_cast<uint4*>(act.frag), act.nkb, act.ntile, act.f16 ? 1 : 0, act.ss);
  IH_HIP(hipGetLastError());
  act.nss = 1;
  return IH_OK;
}

// The model's MoE launches. Router: logits fp32 [rows][ldl] = r · (x · Wᵀ) (one dense slot).
int launch_moe_router(ih_ctx* c, const ih_qmat* W, const ActBuf& x, int rows, float eps, float* logits, int ldl) {
  // An int4 router runs on the dense qmm, whose workgroups split K across waves (the matrix is a few hundred KB:
  // one memory round trip instead of a walk over its K-blocks).
  if (W->format == QF_INT4 && W->E == 1 && !x.f16) {
    QmmEpilogue ep;
    ep.mode = QM_F32_SCALE;
    ep.y = logits;
    ep.ldy = ldl;
    ep.eps = eps;
    return launch_qmm_ex(c, W, 0, x, rows, ep);
  }
  GatherParams p{};
  p.xa = static_cast<const uint4*>(x.frag);
  p.x_nkb = x.nkb;
  p.x_tokens = MAX_TOK;
  p.dense_e = 0;
  p.M = rows;
  p.mode = GM_F32;
  p.y = logits;
  p.ldy = ldl;
  p.ss_in = x.ss;
  p.nss_in = x.nss;
  p.D = x.K;
  p.nrows = rows;
  p.eps = eps;
  return launch_gather(c, W, p, 1, double(W->algo_bytes) + double(rows) * W->N * 4, x.f16);
}

// Gate|up of every pair: h[pair] = act(r·g + bg, r·u + bu) as fragments (one token per pair).
int launch_moe_gate_up(ih_ctx* c, const ih_qmat* W, const ActBuf& x, int rows, int K_top, float eps, const int* nent,
                       const int* entries, const int4* slot_tab, const int* x_row, const uint16_t* bias, int glu,
                       float limit, void* h_frag, int h_nkb, int h_tokens, bool h_f16) {
  IH_CHECK(W->il8, IH_EINVAL, "moe gate|up: the matrix must be interleaved by eights");
  GatherParams p{};
  p.xa = static_cast<const uint4*>(x.frag);
  p.x_nkb = x.nkb;
  p.x_tokens = MAX_TOK;
  p.x_row = x_row;
  p.entries = entries;
  p.nent = nent;
  p.slots = slot_tab;
  p.mode = GM_GLU;
  p.ss_in = x.ss;
  p.nss_in = x.nss;
  p.D = x.K;
  p.nrows = rows;
  p.eps = eps;
  p.h_out = static_cast<uint4*>(h_frag);
  p.h_nkb = h_nkb;
  p.h_ntile = h_tokens / 16;
  p.h_f16 = h_f16 ? 1 : 0;
  p.glu = glu;
  p.limit = limit;
  p.bias = bias;
  const int slots = std::min(W->E, rows * K_top);
  return launch_gather(c, W, p, slots, double(W->algo_bytes) * slots, x.f16);
}

// Down of every pair: o[pair] = h[pair] · Wdᵀ + bd (fp32).
int launch_moe_down(ih_ctx* c, const ih_qmat* W, const void* h_frag, int h_nkb, int h_tokens, bool h_f16, int rows,
                    int K_top, const int* nent, const int* entries, const int4* slot_tab, const uint16_t* bias, float* o,
                    int ldo) {
  GatherParams p{};
  p.xa = static_cast<const uint4*>(h_frag);
  p.x_nkb = h_nkb;
  p.x_tokens = h_tokens;
  p.entries = entries;
  p.nent = nent;
  p.slots = slot_tab;
  p.mode = GM_DOWN;
  p.y = o;
  p.ldy = ldo;
  p.bias = bias;
  const int slots = std::min(W->E, rows * K_top);
  return launch_gather(c, W, p, slots, double(W->algo_bytes) * slots, h_f16);
}

int pack_mxfp4(ih_ctx* c, ih_qmat* q, const uint32_t* w, const uint8_t* s) {
  dim3 grid((q->Npad / 16) * q->nkb, q->E);
  pack_mxfp4_kernel<<<grid, 64, 0, c->stream>>>(w, s, static_cast<uint4*>(q->w), static_cast<uint32_t*>(q->s), q->N,
                                                q->K, q->Npad, q->nkb, q->il8);
  IH_HIP(hipGetLastError());
  return IH_OK;
}

int qmat_mxfp4_create_dev(ih_ctx* c, const void* w, const void* s, int E, int N, int K, int il8, ih_qmat** out) {
  IH_CHECK(c && w && s && out, IH_EINVAL, "ih_qmat_mxfp4_create_dev: null argument");
  IH_CHECK(E >= 1 && N >= 1 && K >= 32 && K % 32 == 0, IH_EINVAL,
           "ih_qmat_mxfp4_create_dev: need E, N ≥ 1 and K a positive multiple of 32");
  IH_CHECK(!il8 || N % 16 == 0, IH_EINVAL, "qmat: an interleaved gate|up matrix needs N a multiple of 16");
  *out = nullptr;
  ih_qmat* q = new ih_qmat();
  q->ctx = c;
  q->format = QF_MXFP4;
  q->E = E;
  q->N = N;
  q->K = K;
  q->Npad = (N + 255) / 256 * 256;
  q->nkb = (K + KBLK - 1) / KBLK;
  q->ktail = (K % KBLK) ? 1 : 0;
  q->il8 = il8;
  q->algo_bytes = size_t(N) * K / 2 + size_t(N) * (K / 32);
  const size_t tiles = size_t(E) * (q->Npad / 16) * q->nkb;
  q->wbytes = tiles * 1024;
  q->sbytes = tiles * 64;
  int st = IH_OK;
  if (hipMalloc(&q->w, q->wbytes) != hipSuccess || hipMalloc(&q->s, q->sbytes) != hipSuccess)
    st = fail(IH_ENOMEM, "ih_qmat_mxfp4_create_dev: allocation failed");
  if (st == IH_OK) st = pack_mxfp4(c, q, static_cast<const uint32_t*>(w), static_cast<const uint8_t*>(s));
  if (st != IH_OK) {
    ih_qmat_free(q);
    return st;
  }
  *out = q;
  return IH_OK;
}

// Natural bf16 rows → fragments (bf16 or fp16 elements). Grid (tokens), 256 threads.
__global__ void act_gather_kernel(const uint16_t* __restrict__ x, int ldx, int M, int K, int nkb, int ntile, int f16,
                                  uint4* __restrict__ frag) {
  const int i = blockIdx.x;
  for (int cc = threadIdx.x; cc < nkb * 16; cc += blockDim.x) {
    float v[8];
    const bool valid = i < M && cc < K / 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = valid ? bf16f(x[size_t(i) * ldx + 8 * cc + e]) : 0.f;
    frag_store(f16 != 0, frag, nkb, ntile, i, cc, v);
  }
}

int stage_act_bf16(ih_ctx* c, const uint16_t* x, int ldx, int M, int K, bool f16, ActBuf& a) {
  IH_TRY(ensure_act(c, a, K, f16));
  act_gather_kernel<<<MAX_TOK, 256, 0, c->stream>>>(x, ldx, M, K, a.nkb, a.ntile, f16 ? 1 : 0,
                                                    static_cast<uint4*>(a.frag));
  IH_HIP(hipGetLastError());
  return IH_OK;
}

}  // namespace ih

using namespace ih;

extern "C" {

int ih_qmat_mxfp4_create_dev(ih_ctx* c, const void* w, const void* s, int E, int N, int K, ih_qmat** out) {
  return qmat_mxfp4_create_dev(c, w, s, E, N, K, 0, out);
}

int ih_qmat_mxfp4_create(ih_ctx* c, const uint32_t* w, const uint8_t* s, int E, int N, int K, ih_qmat** out) {
  IH_CHECK(c && w && s && out, IH_EINVAL, "ih_qmat_mxfp4_create: null argument");
  IH_CHECK(E >= 1 && N >= 1 && K >= 32 && K % 32 == 0, IH_EINVAL,
           "ih_qmat_mxfp4_create: need E, N ≥ 1 and K a positive multiple of 32");
  const size_t wb = size_t(E) * N * (K / 8) * 4, sb = size_t(E) * N * (K / 32);
  void *dw = nullptr, *ds = nullptr;
  int st = IH_OK;
  if (hipMalloc(&dw, wb) != hipSuccess || hipMalloc(&ds, sb) != hipSuccess)
    st = fail(IH_ENOMEM, "ih_qmat_mxfp4_create: staging allocation failed");
  if (st == IH_OK && (hipMemcpyAsync(dw, w, wb, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
                      hipMemcpyAsync(ds, s, sb, hipMemcpyHostToDevice, c->stream) != hipSuccess))
    st = fail(IH_EDEVICE, "ih_qmat_mxfp4_create: upload failed");
  if (st == IH_OK) st = ih_qmat_mxfp4_create_dev(c, dw, ds, E, N, K, out);
  (void)hipStreamSynchronize(c->stream);
  if (dw) (void)hipFree(dw);
  if (ds) (void)hipFree(ds);
  return st;
}

int ih_qmat_format(const ih_qmat* q) { return q ? q->format : -1; }

int ih_qmm_expert(ih_ctx* c, const ih_qmat* W, int expert, const void* x, int ldx, int M, float* y, int ldy) {
  IH_CHECK(c && W && x && y, IH_EINVAL, "ih_qmm_expert: null argument");
  IH_CHECK(M >= 1 && M <= MAX_TOK, IH_EINVAL, "ih_qmm_expert: M must be in 1..32");
  IH_CHECK(expert >= 0 && expert < W->E, IH_EINVAL, "ih_qmm_expert: expert out of range");
  IH_CHECK(ldx >= W->K && ldy >= W->N, IH_EINVAL, "ih_qmm_expert: leading dimension smaller than the row");
  const bool f16 = W->format == QF_MXFP4;
  IH_TRY(stage_act_bf16(c, static_cast<const uint16_t*>(x), ldx, M, W->K, f16, c->act));
  GatherParams p{};
  p.xa = static_cast<const uint4*>(c->act.frag);
  p.x_nkb = c->act.nkb;
  p.x_tokens = MAX_TOK;
  p.dense_e = expert;
  p.M = M;
  p.mode = GM_F32;
  p.y = y;
  p.ldy = ldy;
  return launch_gather(c, W, p, 1, double(W->algo_bytes) + double(M) * W->K * 2 + double(M) * W->N * 4, f16);
}

int ih_moe_route(ih_ctx* c, const float* logits, int ldl, int rows, int E, int K, const float* bias, const float* pes,
                 int* nent, int* entries, int* x_row, float* pair_w, int* row_pair) {
  IH_CHECK(c && logits && nent && entries && x_row && pair_w && row_pair, IH_EINVAL, "ih_moe_route: null argument");
  IH_CHECK(ldl >= E, IH_EINVAL, "ih_moe_route: ldl < E");
  return launch_moe_route(c, logits, ldl, rows, E, K, bias, pes, nent, entries, nullptr, x_row, pair_w, row_pair,
                          MoeIid{});
}

int ih_qmm_gathered(ih_ctx* c, const ih_qmat* W, const void* x, int ldx, int rows, int K_top, const int* nent,
                    const int* entries, const int* x_row, float* y, int ldy) {
  IH_CHECK(c && W && x && nent && entries && x_row && y, IH_EINVAL, "ih_qmm_gathered: null argument");
  IH_CHECK(rows >= 1 && rows <= MAX_TOK && K_top >= 1 && K_top <= 16, IH_EINVAL,
           "ih_qmm_gathered: rows must be in 1..32 and k in 1..16");
  IH_CHECK(ldx >= W->K && ldy >= W->N, IH_EINVAL, "ih_qmm_gathered: leading dimension smaller than the row");
  const bool f16 = W->format == QF_MXFP4;
  IH_TRY(stage_act_bf16(c, static_cast<const uint16_t*>(x), ldx, rows, W->K, f16, c->act));
  GatherParams p{};
  p.xa = static_cast<const uint4*>(c->act.frag);
  p.x_nkb = c->act.nkb;
  p.x_tokens = MAX_TOK;
  p.x_row = x_row;
  p.entries = entries;
  p.nent = nent;
  p.mode = GM_F32;
  p.y = y;
  p.ldy = ldy;
  const int slots = std::min(W->E, rows * K_top);
  return launch_gather(c, W, p, slots, double(W->algo_bytes) * slots, f16);
}

}  // extern "C"
